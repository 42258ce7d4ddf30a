"""Expert dispatch on one GPU (EP1): litemoe/ep.py:7-53's call contract.

``ExpertParallel(world, rank, capacity, hidden, topk, dtype, device, backend,
combine)`` and ``__call__(x, ids, weights, valid, physical, w1, w2,
logical=None, decode=False, tokens=None)`` are the reference's. Two routes:

* lean (decode under the fast-path policy, identity placement): the router
  outputs go to ``backend.operation`` unchanged (ep.py:39-41);
* masked: rows that are not ``valid`` enter as zeros with zero scales, so
  they add exactly nothing; router ids are mapped to weight slots through
  ``physical``, and ``logical`` keeps the combine in checkpoint-expert
  order; the result lands in an output buffer owned by this object, one
  per row count (``prepare``), as the reference's does (ep.py:22-36).

Several GPUs (the reference's EP2 all-gather / reduce-scatter, ep.py:54-72)
are not part of this single-GPU build.
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
        self.capacity, self.hidden, self.topk = capacity, hidden, topk
        self.dtype, self.device = dtype, device
        self.buffers = {}   # row count -> output [rows, hidden]

    def prepare(self, tokens):
        """Own an output buffer for calls of ``tokens`` rows."""
        if tokens > self.capacity:
            raise ValueError("Communication capacity exceeded")
        if tokens not in self.buffers:
            self.buffers[tokens] = torch.empty(tokens, self.hidden, dtype=self.dtype, device=self.device)
        return self.buffers[tokens]

    def _output(self, rows, device):
        out = self.buffers.get(rows)
        return out if out is not None else torch.empty(rows, self.hidden, dtype=self.dtype, device=device)

    def __call__(self, x, ids, weights, valid, physical, w1, w2, logical=None, decode=False, tokens=None):
        experts = w1.shape[0]
        if decode and self.decode_lean:
            return self.backend.operation(x.contiguous(), w1, w2, weights.float().contiguous(),
                                          ids.int().contiguous(), apply_router_weight_on_input=False,
                                          global_num_experts=experts)
        keep = valid.reshape(-1, 1)
        rows_in = torch.where(keep, x, torch.zeros((), dtype=x.dtype, device=x.device)).contiguous()
        slot_ids = physical.index_select(0, ids.reshape(-1).long()).view_as(ids).to(torch.int32).contiguous()
        scales = weights.float().mul(keep).contiguous()
        out = self._output(x.shape[0], x.device)
        backend = self.backend if decode or self.prefill_backend is None else self.prefill_backend
        extra = {} if logical is None or logical.numel() == 0 else {"logical": logical}
        backend(rows_in, slot_ids, scales, w1, w2, 0, 1, out, **extra)
        return out
