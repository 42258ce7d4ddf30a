"""Split-K projections for decode-sized row counts.

The dense projections of the reference layer (packed q|k|v,
litemoe/model.py:47-49, and o_proj, :73) are ``F.linear`` calls. For a decode
batch (rows <= 128) they are computed by ``lm_linear_splitk`` as fp32
partial sums over K slices; ``bf16(sum of slices)`` is F.linear's bf16
output. The decode layer hands the partials straight to the consumer kernel
(``FlashDecode.fused_qkv``, ``router.add_rmsnorm_route_splitk``), which sums
them on load; :func:`linear` is the stand-alone form (projection + reduce).
"""
import torch

from . import _lib

MAX_ROWS = 128
MAX_CONSUMER_SPLITS = 8
_KW = (1, 2, 3, 4, 6, 8)


def pick_splits(rows, out_features, in_features, target_workgroups=192, max_splits=MAX_CONSUMER_SPLITS):
    """Fewest K slices giving about ``target_workgroups`` workgroups
    (out_features / 32 column tiles per slice), or None when the shape has no
    kernel. Slices are K / (128 * kw) for the compiled kw values."""
    if not 1 <= rows <= MAX_ROWS or out_features % 32 or in_features % 128:
        return None
    steps = in_features // 128
    valid = [s for s in range(1, max_splits + 1) if steps % s == 0 and steps // s in _KW]
    if not valid:
        return None
    for s in valid:
        if (out_features // 32) * s >= target_workgroups:
            return s
    return valid[-1]


def linear_splitk(a, weight, splits, out=None):
    """fp32 partials ``[splits, rows, out_features]`` of ``a @ weight.T``."""
    _lib.require_cuda(a, weight, what="projection operands")
    if a.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("Split-K projection supports BF16 operands")
    if a.dim() != 2 or a.stride(1) != 1 or not weight.is_contiguous() or weight.shape[1] != a.shape[1]:
        raise ValueError("Split-K projection needs a [rows, K] input with contiguous rows and a contiguous [N, K] weight")
    rows, k = a.shape
    n = weight.shape[0]
    if out is None:
        out = torch.empty(splits, rows, n, device=a.device, dtype=torch.float32)
    elif out.shape != (splits, rows, n) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("Partials buffer must be contiguous fp32 [splits, rows, out_features]")
    _lib.call("lm_linear_splitk", a.data_ptr(), a.stride(0), weight.data_ptr(), rows, n, k, splits,
              out.data_ptr(), _lib.stream(a.device))
    return out


def linear_splitk_rmsnorm(x, sumsq, norm_weight, eps, weight, splits, out=None):
    """fp32 partials ``[splits, rows, out_features]`` of ``rmsnorm(x) @
    weight.T``, the norm formed in the kernel from ``sumsq`` (the
    per-64-column sums of squares of ``x`` that
    :func:`experts.moe_routes_combine` writes): bitwise
    ``linear_splitk(lm_rmsnorm(x), weight, splits)``."""
    _lib.require_cuda(x, sumsq, norm_weight, weight, what="projection operands")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or norm_weight.dtype != torch.bfloat16:
        raise ValueError("Split-K projection supports BF16 operands")
    if x.dim() != 2 or not x.is_contiguous() or not weight.is_contiguous() or weight.shape[1] != x.shape[1]:
        raise ValueError("Split-K projection needs a contiguous [rows, K] input and a contiguous [N, K] weight")
    rows, k = x.shape
    if sumsq.shape != (rows, k // 64) or sumsq.dtype != torch.float32 or not sumsq.is_contiguous():
        raise ValueError("sumsq must be contiguous fp32 [rows, K/64]")
    n = weight.shape[0]
    if out is None:
        out = torch.empty(splits, rows, n, device=x.device, dtype=torch.float32)
    _lib.call("lm_linear_splitk_rmsnorm", x.data_ptr(), sumsq.data_ptr(), norm_weight.data_ptr(), float(eps),
              weight.data_ptr(), rows, n, k, splits, out.data_ptr(), _lib.stream(x.device))
    return out


def frag_row_blocks(rows):
    """16-row blocks of the fragment order for ``rows`` rows: the smallest of
    1, 2, 4, 8 covering them (the split-K kernel's row-block count)."""
    if not 1 <= rows <= MAX_ROWS:
        raise ValueError(f"Fragment order holds 1..{MAX_ROWS} rows, got {rows}")
    return 1 if rows <= 16 else 2 if rows <= 32 else 4 if rows <= 64 else 8


class FragRows:
    """A bf16 ``[rows, cols]`` matrix in MFMA A-fragment order, the layout
    ``lm_linear_splitk_frag`` reads and ``lm_flash_decode_qkv_frag`` writes
    (the decode attention output, o_proj's input): rows padded to ``16 * mb``;
    element ``(r, k)`` at ``((k//32)*mb + r//16)*512 + ((k%32)//8)*128 +
    (r%16)*8 + k%8``, so one 64-lane load of 16 bytes reads 1 KB contiguously.
    Padding rows are never written and only feed outputs that are dropped."""

    def __init__(self, rows, cols, device, data=None):
        if cols % 32:
            raise ValueError("Fragment order needs a multiple of 32 columns")
        self.rows, self.cols, self.mb = rows, cols, frag_row_blocks(rows)
        size = 16 * self.mb * cols
        if data is None:
            data = torch.empty(size, device=device, dtype=torch.bfloat16)
        elif data.numel() != size or data.dtype != torch.bfloat16 or not data.is_contiguous():
            raise ValueError("Fragment buffer must be contiguous bf16 of 16*mb*cols elements")
        self.data = data

    @property
    def device(self):
        return self.data.device

    @classmethod
    def from_rows(cls, a):
        """The fragment order of a row-major ``[rows, cols]`` matrix (padding rows zero)."""
        rows, cols = a.shape
        out = cls(rows, cols, a.device)
        padded = torch.zeros(16 * out.mb, cols, device=a.device, dtype=torch.bfloat16)
        padded[:rows] = a
        out.data.copy_(padded.view(out.mb, 16, cols // 32, 4, 8).permute(2, 0, 3, 1, 4).reshape(-1))
        return out

    def to_rows(self):
        """The row-major ``[rows, cols]`` matrix."""
        c = self.cols // 32
        return self.data.view(c, self.mb, 4, 16, 8).permute(1, 3, 0, 2, 4).reshape(16 * self.mb, self.cols)[:self.rows]


def linear_splitk_frag(a, weight, splits, out=None):
    """:func:`linear_splitk` with ``a`` a :class:`FragRows` (same partials)."""
    _lib.require_cuda(a.data, weight, what="projection operands")
    if weight.dtype != torch.bfloat16 or not weight.is_contiguous() or weight.shape[1] != a.cols:
        raise ValueError("Split-K projection needs a contiguous BF16 [N, K] weight matching the input")
    n = weight.shape[0]
    if out is None:
        out = torch.empty(splits, a.rows, n, device=a.device, dtype=torch.float32)
    elif out.shape != (splits, a.rows, n) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("Partials buffer must be contiguous fp32 [splits, rows, out_features]")
    _lib.call("lm_linear_splitk_frag", a.data.data_ptr(), weight.data_ptr(), a.rows, n, a.cols, splits,
              out.data_ptr(), _lib.stream(a.device))
    return out


def reduce(partials, out=None):
    """``bf16(sum over slices)``, slices in ascending order."""
    splits, rows, n = partials.shape
    if out is None:
        out = torch.empty(rows, n, device=partials.device, dtype=torch.bfloat16)
    _lib.call("lm_linear_splitk_reduce", partials.data_ptr(), splits, rows, n, out.data_ptr(),
              out.stride(0), _lib.stream(partials.device))
    return out


def linear(a, weight, splits=None):
    """``F.linear(a, weight)`` for decode-sized ``a`` (bf16, no bias)."""
    splits = splits or pick_splits(a.shape[0], weight.shape[0], weight.shape[1])
    if splits is None:
        raise ValueError(f"No split-K kernel for rows={a.shape[0]}, weight {tuple(weight.shape)}")
    return reduce(linear_splitk(a, weight, splits))


def linear_dense(a, weight, out=None):
    """``F.linear(a, weight)`` (bf16, no bias) for any row count on
    ``lm_linear``: one workgroup reduces each output over all of K in
    ascending order, so a row's bits do not depend on the batch or the
    launch. ``a [rows, K]`` with contiguous rows (any row stride),
    ``weight [N, K]`` with contiguous rows; ``out [rows, N]`` (optional, any
    row stride) receives the result."""
    _lib.require_cuda(a, weight, what="projection operands")
    if a.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("Dense projection supports BF16 operands")
    if a.dim() != 2 or weight.dim() != 2 or a.shape[1] != weight.shape[1]:
        raise ValueError("Dense projection needs a [rows, K] input and an [N, K] weight")
    rows, k = a.shape
    n = weight.shape[0]
    if k % 64:
        raise ValueError("Dense projection needs in_features a multiple of 64")
    if rows and (a.stride(1) != 1 or a.stride(0) % 8 or a.data_ptr() % 16):
        raise ValueError("Dense projection needs 16-byte aligned input rows with a stride a multiple of 8")
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        raise ValueError("Dense projection needs 16-byte aligned weight rows with a stride a multiple of 8")
    if out is None:
        out = torch.empty(rows, n, device=a.device, dtype=torch.bfloat16)
    elif out.shape != (rows, n) or out.dtype != torch.bfloat16 or out.stride(1) != 1:
        raise ValueError("Output must be bf16 [rows, out_features] with unit column stride")
    if rows:
        _lib.call("lm_linear", a.data_ptr(), max(a.stride(0), k), weight.data_ptr(), max(weight.stride(0), k),
                  rows, n, k, out.data_ptr(), max(out.stride(0), n), _lib.stream(a.device))
    return out


def linear_rope_kv(a, weight, q_heads, kv_heads, positions, active, cos_sin, cache, layer, slots=None):
    """``linear_dense(a, weight)`` of the packed q|k|v weight followed by
    ``rope_kv_write(q, k, v, ..., write_k=True)`` in one launch
    (``lm_linear_rope_kv``): returns ``qkv [rows, (q_heads + 2*kv_heads)*64]``
    with q and k rotated; k and v stored into ``cache`` layer ``layer`` at
    ``(slots[r], h, positions[r])`` for active rows. Bitwise the two-call
    result. Replaces litemoe/model.py:47-49 with :58-59 / :63-70."""
    _lib.require_cuda(a, weight, cos_sin, positions, what="projection operands")
    if a.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or cos_sin.dtype != torch.bfloat16:
        raise ValueError("Fused QKV projection supports BF16 operands")
    rows, k = a.shape
    n = (q_heads + 2 * kv_heads) * 64
    if weight.shape != (n, k) or not weight.is_contiguous() or k % 64:
        raise ValueError("Fused QKV projection needs a contiguous [(q+2kv)*64, K] weight, K a multiple of 64")
    if cos_sin.shape[-1] != 64 or not cos_sin.is_contiguous():
        raise ValueError("Fused QKV projection needs a contiguous [table_len, 64] cos/sin table")
    if rows and (a.stride(1) != 1 or a.stride(0) % 8 or a.data_ptr() % 16):
        raise ValueError("Dense projection needs 16-byte aligned input rows with a stride a multiple of 8")
    kc, vc = cache.k[layer], cache.v[layer]
    if kc.dtype != torch.bfloat16 or kc.shape[1] != kv_heads or kc.shape[-1] != 64:
        raise ValueError("Fused QKV projection needs a bf16 cache with head_dim 64")
    out = torch.empty(rows, n, device=a.device, dtype=torch.bfloat16)
    if rows:
        positions = positions.to(torch.int64).contiguous()
        active = None if active is None else active.to(torch.bool).contiguous()
        slots = None if slots is None else slots.to(torch.int64).contiguous()
        _lib.call("lm_linear_rope_kv", a.data_ptr(), max(a.stride(0), k), weight.data_ptr(), rows, q_heads,
                  kv_heads, k, out.data_ptr(), n, positions.data_ptr(), _lib.ptr(active), _lib.ptr(slots),
                  cos_sin.data_ptr(), cos_sin.shape[0], kc.data_ptr(), vc.data_ptr(), cache.capacity,
                  kc.shape[0], _lib.stream(a.device))
    return out
