"""Router: gate GEMV, top-k and softmax on the gfx950 kernel.

``fused_topk`` keeps vLLM's signature as the reference calls it
(litemoe/model.py:112-113): ``fused_topk(hidden, gating_output, topk,
renormalize=True) -> (weights fp32 [M,k], ids int32 [M,k], indices)``.
``route`` fuses the router GEMV ``linear_rows(z, router.layer)``
(model.py:110) in front of it. Selection: descending logits, equal logits by
ascending expert id.
"""
import torch

from . import _lib


def _outputs(m, topk, device):
    return (torch.empty(m, topk, device=device, dtype=torch.float32),
            torch.empty(m, topk, device=device, dtype=torch.int32))


def fused_topk(hidden_states, gating_output, topk, renormalize=True):
    """Top-k of bf16 logits ``gating_output [M, E]``. The third output is the
    flat route index ``t * topk + j`` of each selection."""
    _lib.require_cuda(gating_output, what="router logits")
    if gating_output.dtype != torch.bfloat16 or gating_output.ndim != 2:
        raise ValueError('Router logits must be a BF16 [tokens, experts] tensor')
    if hidden_states is not None and hidden_states.shape[0] != gating_output.shape[0]:
        raise ValueError('Hidden states and logits disagree on the token count')
    logits = gating_output.contiguous()
    m, experts = logits.shape
    weights, ids = _outputs(m, topk, logits.device)
    _lib.call("lm_topk_softmax", logits.data_ptr(), m, experts, topk, int(bool(renormalize)),
              weights.data_ptr(), ids.data_ptr(), _lib.stream(logits.device))
    indices = torch.arange(m * topk, device=logits.device, dtype=torch.int32).view(m, topk)
    return weights, ids, indices


def route(z, gate_weight, topk, renormalize=True, logits_out=None, id_order=False):
    """Fused ``logits = bf16(z . W_r^T)`` then ``fused_topk``; ``z [M, H]``,
    ``gate_weight [E, H]``. Optionally writes the bf16 logits. ``id_order``:
    each token's experts (and weights) in ascending id instead of descending
    logit."""
    _lib.require_cuda(z, gate_weight, what="router inputs")
    if z.dtype != torch.bfloat16 or gate_weight.dtype != torch.bfloat16:
        raise ValueError('Router supports BF16')
    if not z.is_contiguous() or not gate_weight.is_contiguous() or z.shape[-1] != gate_weight.shape[1]:
        raise ValueError('Router needs contiguous [M, H] input and [E, H] weight')
    m, hidden = z.numel() // z.shape[-1], z.shape[-1]
    experts = gate_weight.shape[0]
    weights, ids = _outputs(m, topk, z.device)
    if logits_out is not None and (logits_out.shape != (m, experts) or logits_out.dtype != torch.bfloat16):
        raise ValueError('logits_out must be BF16 [tokens, experts]')
    _lib.call("lm_router", z.data_ptr(), gate_weight.data_ptr(), m, hidden, experts, topk,
              int(bool(renormalize)) | (2 if id_order else 0), _lib.ptr(logits_out), weights.data_ptr(),
              ids.data_ptr(), _lib.stream(z.device))
    return weights, ids


def add_rmsnorm_route(x, a, alpha, norm_weight, eps, gate_weight, topk, z=None, renormalize=True,
                      logits_out=None):
    """``x <- bf16(x + alpha * a)``, ``z = rmsnorm(x)``, then :func:`route` on z,
    in one kernel (litemoe/model.py:108-113). Returns (weights, ids, z)."""
    _lib.require_cuda(x, norm_weight, gate_weight, what="router inputs")
    if x.dtype != torch.bfloat16 or not x.is_contiguous() or gate_weight.shape[1] != x.shape[-1]:
        raise ValueError('Router needs a contiguous BF16 [M, H] residual and [E, H] weight')
    if a is not None and (a.shape != x.shape or a.dtype != x.dtype or not a.is_contiguous()):
        raise ValueError('Residual input must match x and be contiguous')
    m, hidden = x.numel() // x.shape[-1], x.shape[-1]
    experts = gate_weight.shape[0]
    z = torch.empty_like(x) if z is None else z
    weights, ids = _outputs(m, topk, x.device)
    _lib.call("lm_add_rmsnorm_router", x.data_ptr(), _lib.ptr(a), float(alpha), norm_weight.data_ptr(),
              float(eps), z.data_ptr(), gate_weight.data_ptr(), m, hidden, experts, topk,
              int(bool(renormalize)), _lib.ptr(logits_out), weights.data_ptr(), ids.data_ptr(),
              _lib.stream(x.device))
    return weights, ids, z


def add_rmsnorm_route_splitk(x, partials, alpha, norm_weight, eps, gate_weight, topk, z=None,
                             renormalize=True, logits_out=None, id_order=False):
    """:func:`add_rmsnorm_route` with the residual branch given as split-K
    partials ``[S, M, H]`` of the attention output projection
    (``a = bf16(sum of slices)``, litemoe/model.py:73 then :108-113).
    ``id_order``: each token's experts (and weights) in ascending id, the
    order :func:`experts.moe_routes_combine` sums in."""
    _lib.require_cuda(x, partials, norm_weight, gate_weight, what="router inputs")
    if x.dtype != torch.bfloat16 or not x.is_contiguous() or gate_weight.shape[1] != x.shape[-1]:
        raise ValueError('Router needs a contiguous BF16 [M, H] residual and [E, H] weight')
    m, hidden = x.numel() // x.shape[-1], x.shape[-1]
    if partials.dtype != torch.float32 or not partials.is_contiguous() or partials.shape[1:] != (m, hidden):
        raise ValueError('Residual partials must be contiguous fp32 [S, M, H]')
    experts = gate_weight.shape[0]
    z = torch.empty_like(x) if z is None else z
    weights, ids = _outputs(m, topk, x.device)
    _lib.call("lm_add_rmsnorm_router_splitk", x.data_ptr(), partials.data_ptr(), partials.shape[0],
              float(alpha), norm_weight.data_ptr(), float(eps), z.data_ptr(), gate_weight.data_ptr(), m,
              hidden, experts, topk, int(bool(renormalize)) | (2 if id_order else 0), _lib.ptr(logits_out),
              weights.data_ptr(),
              ids.data_ptr(), _lib.stream(x.device))
    return weights, ids, z
