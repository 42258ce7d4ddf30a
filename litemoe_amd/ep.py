"""Expert dispatch for one GPU (EP1), litemoe/ep.py:7-53.

The lean branch hands router outputs straight to ``backend.operation`` (the
fused gfx950 experts), as ep.py:39-41; the masked branch zeroes inactive rows,
maps ids through the placement and writes into a preallocated output
(ep.py:42-53). Expert parallelism over several GPUs (ep.py:54-72) is not part
of this single-GPU build.
"""
import torch


class ExpertParallel:
    def __init__(self, world, rank, capacity, hidden, topk, dtype, device, backend, combine="partial"):
        if combine not in ("partial", "routes"):
            raise ValueError("Unknown EP combine policy")
        if world != 1 or rank != 0:
            raise ValueError("This build runs on one GPU: expert parallelism needs world == 1")
        self.world, self.rank, self.backend = world, rank, backend
        self.prefill_backend = None
        self.decode_lean = False
        self.combine = "local"
        self.buffers = {}
        self.capacity, self.hidden, self.topk = capacity, hidden, topk
        self.dtype, self.device = dtype, device

    def prepare(self, tokens):
        if tokens > self.capacity:
            raise ValueError("Communication capacity exceeded")
        if tokens not in self.buffers:
            self.buffers[tokens] = torch.empty(tokens, self.hidden, dtype=self.dtype, device=self.device)

    def __call__(self, x, ids, weights, valid, physical, w1, w2, logical=None, decode=False, tokens=None):
        if decode and self.decode_lean:  # identity placement; stopped rows need no zero scales
            return self.backend.operation(x.contiguous(), w1, w2, weights.float().contiguous(),
                                          ids.int().contiguous(), apply_router_weight_on_input=False,
                                          global_num_experts=w1.shape[0])
        rows = x.shape[0]
        out = self.buffers.get(rows)
        if out is None:
            out = torch.empty(rows, self.hidden, dtype=self.dtype, device=x.device)
        x = torch.where(valid[:, None], x, 0).contiguous()
        ids = physical[ids.long()].to(torch.int32).contiguous()
        scales = (weights.float() * valid[:, None]).contiguous()
        options = {"logical": logical} if logical is not None and logical.numel() else {}
        backend = self.backend if decode or self.prefill_backend is None else self.prefill_backend
        backend(x, ids, scales, w1, w2, 0, 1, out, **options)
        return out
