"""Expert backend on the gfx950 kernels: the drop-in for vLLM ``fused_experts``.

``HipFusedExperts`` follows the reference's backend protocol
(litemoe/vllm_moe.py:6-27, ops.py:59-61): attributes ``graph_safe``, ``name``,
``fused_combine``; ``operation(x, w1, w2, topk_weights, topk_ids,
apply_router_weight_on_input=False, global_num_experts=E)`` as the lean EP1
path calls it (ep.py:40-41); ``__call__(x, ids, scales, w1, w2, rank, world,
out, logical=None)`` writing into ``out``. The model gates its fused decode
path on the ``native`` capability attribute instead of a type check.
"""
import torch

from . import _lib


def _check_weights(x, w1, w2):
    if any(t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous() for t in (x, w1, w2)):
        raise ValueError('Contiguous CUDA BF16 activations/weights/output required')
    experts, two_inter, hidden = w1.shape
    if x.shape[-1] != hidden or w2.shape != (experts, hidden, two_inter // 2) or two_inter % 2:
        raise ValueError('Expert weight shapes must be w1 [E, 2I, H] and w2 [E, H, I]')
    return experts, hidden, two_inter // 2


class _Workspace:
    """Grow-only device scratch.

    A captured HIP graph keeps the address of every buffer its kernels were
    given, so a buffer is never released once handed out: growing allocates
    a larger one and keeps the old one referenced (``retired``) for the
    workspace's lifetime. Growth is geometric, so the retired buffers add at
    most the size of the current one."""

    def __init__(self):
        self.buffers = {}
        self.retired = []

    def get(self, device, nbytes):
        key = str(torch.device(device))
        buf = self.buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 256, 0 if buf is None else 2 * buf.numel())
            if buf is not None:
                self.retired.append(buf)
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            self.buffers[key] = buf
        return buf


_SHARED = _Workspace()


def fused_experts(x, w1, w2, topk_weights, topk_ids, apply_router_weight_on_input=False,
                  global_num_experts=None, out=None, logical=None, block_rows=0, workspace=None,
                  packed=False):
    """``out[t] = sum_j w[t,j] * W2[e] (silu(W13[e,:I] x_t) * W13[e,I:] x_t)``
    (``packed``: weights from :func:`pack_expert_weights`)."""
    if apply_router_weight_on_input:
        raise ValueError('apply_router_weight_on_input=True is not implemented')
    experts, hidden, inter = _check_weights(x, w1, w2)
    if global_num_experts is not None and global_num_experts != experts:
        raise ValueError('Expert parallelism is not part of this single-GPU path')
    tokens = x.numel() // hidden
    topk = topk_ids.shape[-1]
    if topk_ids.shape[0] != tokens or topk_weights.shape != topk_ids.shape:
        raise ValueError('Router outputs must be [tokens, topk]')
    ids = topk_ids.to(torch.int32).contiguous()
    weights = topk_weights.to(torch.float32).contiguous()
    out = torch.empty_like(x) if out is None else out
    if out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError('Output must match x')
    remap = logical is not None and logical.numel() != 0
    logical64 = logical.to(torch.int64).contiguous() if remap else None
    nbytes = _lib.size_query("lm_fused_experts_workspace_size", tokens, topk, hidden, inter, experts)
    ws = (workspace or _SHARED).get(x.device, nbytes)
    _lib.call("lm_fused_experts_packed" if packed else "lm_fused_experts", x.data_ptr(), w1.data_ptr(),
              w2.data_ptr(), weights.data_ptr(),
              ids.data_ptr(), _lib.ptr(logical64), tokens, hidden, inter, experts, topk, block_rows,
              out.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream(x.device))
    return out


class HipFusedExperts:
    graph_safe = True
    name = 'hip-gfx950-fused-experts'
    fused_combine = True
    native = True  # capability the model's fused decode path is gated on

    def __init__(self, block_rows=0):
        self.block_rows = block_rows
        self.workspace = _Workspace()

    def operation(self, x, w1, w2, topk_weights, topk_ids, apply_router_weight_on_input=False,
                  global_num_experts=None, out=None):
        return fused_experts(x, w1, w2, topk_weights, topk_ids, apply_router_weight_on_input,
                             global_num_experts, out=out, block_rows=self.block_rows,
                             workspace=self.workspace)

    def routes_combine(self, x, w1, w2, topk_ids, topk_weights, residual=None, alpha=1.0, sumsq=None,
                       packed=False):
        """:func:`moe_routes_combine` on this backend's workspace."""
        return moe_routes_combine(x, w1, w2, topk_ids, topk_weights, residual, alpha, sumsq,
                                  workspace=self.workspace, packed=packed)

    def routes(self, x, w1, w2, topk_ids, packed=False):
        """Unweighted per-route expert outputs ``[M*k, H]`` in route order
        (``packed``: weights from :func:`pack_expert_weights`)."""
        return moe_routes(x, w1, w2, topk_ids, block_rows=self.block_rows, workspace=self.workspace,
                          packed=packed)

    def __call__(self, x, ids, scales, w1, w2, rank, world, out, logical=None):
        if rank != 0 or world != 1:
            raise ValueError('The fused-expert backend supports EP1 only')
        if any(t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous() for t in (x, w1, w2, out)):
            raise ValueError('Contiguous CUDA BF16 activations/weights/output required')
        return fused_experts(x, w1, w2, scales.float(), ids.int(), out=out, logical=logical,
                             block_rows=self.block_rows, workspace=self.workspace)


def scan_path(tokens, topk):
    """Whether a call of ``tokens`` rows takes the decode scan path (each
    expert's workgroups collect their routes from topk_ids): the rule of
    the library's expert kernels."""
    return tokens <= 256 and tokens * topk <= 2048


def pack_expert_weights(w1, w2):
    """The expert weights in MFMA fragment order (``lm_expert_pack``), for
    the ``packed`` forms of :func:`moe_routes` and :func:`fused_experts`:
    tensors of the same shapes whose 16-byte chunk (tile, k-step, lane)
    holds ``M[16*tile + lane%16, 32*k-step + 8*(lane//16):+8]`` of each
    matrix ``M`` (w1 as ``[E*2I, H]``, w2 as ``[E*H, I]``). Done once at
    load time; the reference keeps the checkpoint layout for vLLM
    (litemoe/weights.py:80-108)."""
    experts, hidden, inter = _check_weights(torch.empty(1, w1.shape[2], dtype=w1.dtype, device=w1.device),
                                            w1, w2)
    p1, p2 = torch.empty_like(w1), torch.empty_like(w2)
    _lib.call("lm_expert_pack", w1.data_ptr(), w2.data_ptr(), experts, hidden, inter, p1.data_ptr(),
              p2.data_ptr(), _lib.stream(w1.device))
    return p1, p2


def moe_routes(x, w1, w2, topk_ids, block_rows=0, workspace=None, y=None, packed=False):
    """``y[t*k + j] = W2[e] (silu(W13[e,:I] x_t) * W13[e,I:] x_t)`` (bf16
    roundings as lm_fused_experts), unweighted, in route order. ``packed``:
    w1/w2 come from :func:`pack_expert_weights` (same kernels and results)."""
    experts, hidden, inter = _check_weights(x, w1, w2)
    tokens = x.numel() // hidden
    ids = topk_ids.to(torch.int32).contiguous()
    topk = ids.shape[-1]
    if ids.shape[0] != tokens:
        raise ValueError('Router outputs must be [tokens, topk]')
    y = torch.empty(tokens * topk, hidden, device=x.device, dtype=x.dtype) if y is None else y
    nbytes = _lib.size_query("lm_moe_routes_workspace_size", tokens, topk, hidden, inter, experts)
    ws = (workspace or _SHARED).get(x.device, nbytes)
    _lib.call("lm_moe_routes_packed" if packed else "lm_moe_routes", x.data_ptr(), w1.data_ptr(), w2.data_ptr(),
              ids.data_ptr(), tokens, hidden, inter, experts, topk, block_rows, y.data_ptr(), ws.data_ptr(),
              ws.numel(), _lib.stream(x.device))
    return y


def moe_routes_combine(x, w1, w2, topk_ids, topk_weights, residual=None, alpha=1.0, sumsq=None, out=None,
                       workspace=None, packed=False):
    """The decode MoE in two launches, the combine fused into the down
    projection (``lm_moe_routes_combine``). Each token's ids must be in
    ascending expert id (the router's ``id_order``). Without ``residual``:
    returns ``out [M, H] = bf16(sum_j bf16(bf16(y_tj) * bf16(w_tj)))``
    (equal to :func:`moe_routes` + ``moe_finish``). With ``residual``:
    ``residual <- bf16(residual + alpha * out)`` in place, and returns
    ``sumsq [M, H/64]`` fp32, the per-64-column sums of squares of the new
    residual that :func:`linear.linear_splitk_rmsnorm` finishes the next
    RMSNorm from."""
    experts, hidden, inter = _check_weights(x, w1, w2)
    tokens = x.numel() // hidden
    ids = topk_ids.to(torch.int32).contiguous()
    weights = topk_weights.to(torch.float32).contiguous()
    topk = ids.shape[-1]
    if ids.shape[0] != tokens or weights.shape != ids.shape:
        raise ValueError('Router outputs must be [tokens, topk]')
    if residual is not None:
        if residual.shape != (tokens, hidden) or residual.dtype != torch.bfloat16 or not residual.is_contiguous():
            raise ValueError('Residual must be contiguous bf16 [tokens, hidden]')
        if sumsq is None:
            sumsq = torch.empty(tokens, hidden // 64, device=x.device, dtype=torch.float32)
        elif sumsq.shape != (tokens, hidden // 64) or sumsq.dtype != torch.float32 or not sumsq.is_contiguous():
            raise ValueError('sumsq must be contiguous fp32 [tokens, hidden/64]')
        target = None
    else:
        target = torch.empty_like(x) if out is None else out
    nbytes = _lib.size_query("lm_moe_routes_combine_workspace_size", tokens, topk, hidden, inter, experts)
    ws = (workspace or _SHARED).get(x.device, nbytes)
    _lib.call("lm_moe_routes_combine_packed" if packed else "lm_moe_routes_combine", x.data_ptr(),
              w1.data_ptr(), w2.data_ptr(), ids.data_ptr(), weights.data_ptr(), tokens, hidden, inter, experts,
              topk, _lib.ptr(residual), float(alpha), _lib.ptr(sumsq if residual is not None else None),
              _lib.ptr(target), ws.data_ptr(), ws.numel(), _lib.stream(x.device))
    return sumsq if residual is not None else target


def combine_supported(tokens, topk, hidden, inter):
    """Whether :func:`moe_routes_combine` has kernels for this call."""
    return (scan_path(tokens, topk) and topk <= 8 and hidden % 64 == 0 and hidden // 64 <= 256
            and inter <= 1024 and hidden % 128 == 0 and inter % 128 == 0)


def finish_add_rmsnorm(y, ids, scales, x, alpha, norm_weight, eps, z=None, logical=None):
    """Combine route outputs (moe_finish order and rounding), then
    ``x <- bf16(x + alpha * out)`` and ``z = rmsnorm(x)`` in one kernel."""
    _lib.require_cuda(y, ids, scales, x, norm_weight, what="combine inputs")
    tokens, hidden = x.shape
    topk = ids.shape[-1]
    if y.shape != (tokens * topk, hidden) or scales.shape != ids.shape or not y.is_contiguous():
        raise ValueError('Route outputs must be [tokens*topk, hidden] with [tokens, topk] ids/scales')
    z = torch.empty_like(x) if z is None else z
    ids32 = ids.to(torch.int32).contiguous()
    w32 = scales.to(torch.float32).contiguous()
    remap = logical is not None and logical.numel() != 0
    logical64 = logical.to(torch.int64).contiguous() if remap else None
    _lib.call("lm_moe_finish_add_rmsnorm", y.data_ptr(), ids32.data_ptr(), w32.data_ptr(), _lib.ptr(logical64),
              x.data_ptr(), float(alpha), norm_weight.data_ptr(), float(eps), z.data_ptr(), tokens, hidden,
              topk, _lib.stream(x.device))
    return z


def moe_align(topk_ids, local_experts, first_expert=0, inverse=True):
    """Stable expert-sorted permutation of the flat routes.

    Returns ``offsets [E+1]`` (int32), ``sorted_routes`` (int32, equal to
    ``argsort(key, stable=True)``) and optionally ``inverse``; non-local routes
    sort into the tail after ``offsets[E]`` (litemoe/ops.py:163-173).
    """
    _lib.require_cuda(topk_ids, what="expert ids")
    ids = topk_ids.to(torch.int32).contiguous().view(-1)
    routes = ids.numel()
    offsets = torch.empty(local_experts + 1, device=ids.device, dtype=torch.int32)
    order = torch.empty(routes, device=ids.device, dtype=torch.int32)
    inv = torch.empty(routes, device=ids.device, dtype=torch.int32) if inverse else None
    _lib.call("lm_moe_align", ids.data_ptr(), routes, first_expert, local_experts, offsets.data_ptr(),
              order.data_ptr(), _lib.ptr(inv), _lib.stream(ids.device))
    return offsets, order, inv


def gate_up(x, w1, offsets, sorted_routes, topk, block_rows=0, topk_ids=None, act=None):
    """Stage 1: ``act[r] = bf16(silu(bf16(g)) * bf16(u))`` per route (route
    order). Routes from ``lm_moe_align`` (offsets, sorted_routes) or, with
    ``topk_ids``, collected by each expert's workgroups (decode path)."""
    experts, two_inter, hidden = w1.shape
    inter = two_inter // 2
    routes = topk_ids.numel() if topk_ids is not None else sorted_routes.numel()
    act = torch.zeros(routes, inter, device=x.device, dtype=x.dtype) if act is None else act
    _lib.call("lm_moe_gate_up", x.data_ptr(), w1.data_ptr(), _lib.ptr(offsets), _lib.ptr(sorted_routes),
              _lib.ptr(topk_ids), routes, topk, hidden, inter, experts, block_rows, act.data_ptr(),
              _lib.stream(x.device))
    return act


def down(act, w2, offsets, sorted_routes, block_rows=0, topk_ids=None, y=None):
    """Stage 2: ``y[r] = bf16(W2[e] . act[r])`` in route order."""
    experts, hidden, inter = w2.shape
    routes = topk_ids.numel() if topk_ids is not None else sorted_routes.numel()
    y = torch.zeros(routes, hidden, device=act.device, dtype=act.dtype) if y is None else y
    _lib.call("lm_moe_down", act.data_ptr(), w2.data_ptr(), _lib.ptr(offsets), _lib.ptr(sorted_routes),
              _lib.ptr(topk_ids), routes, hidden, inter, experts, block_rows, y.data_ptr(),
              _lib.stream(act.device))
    return y
