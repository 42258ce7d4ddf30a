"""The two ends of a greedy decode step, each one gfx950 launch.

``decode_prologue`` replaces the step's set-up (litemoe/engine.py:89-91,
model.py:103-106): valid rows, positions, the attention's ``used`` lengths,
the scaled embedding and the first layer's RMSNorm. ``greedy_epilogue``
replaces the logits scaling and everything after the forward
(model.py:127, engine.py:92-102): the argmax, the emit row and the state
update. Both keep the reference's arithmetic, so a step through them emits
the same tokens and leaves the same state as the reference's torch ops.
``greedy_head`` folds the LM head product into the epilogue: the head
weights are streamed once with the argmax in the product's epilogue, and
the logits are not materialised unless asked for.
"""
import torch

from . import _lib


def _bool_bytes(t):
    if t.dtype != torch.bool or not t.is_contiguous():
        raise ValueError("expected a contiguous bool tensor")
    return t.view(torch.uint8)


def decode_prologue(active, length, next_tokens, embedding, multiplier, norm_weight, eps, row_order=None,
                    step_counter=None):
    """Returns ``(x, z, valid, positions, used)`` for one decode step.

    ``valid = active``; ``positions = where(valid, length, 0)``;
    ``used = int32(positions + 1)``; ``x = embedding[next] * multiplier``
    (bf16); ``z = rmsnorm(x, norm_weight, eps)``. With ``row_order`` (int32
    ``[rows]``) also the rows by descending ``used`` (ties by row), the
    dispatch order for :meth:`FlashDecode.fused_qkv`. ``step_counter``
    (int64 ``[1]``) is incremented: the step count an emit ring is indexed by.
    """
    _lib.require_cuda(active, length, next_tokens, embedding, norm_weight, what="decode prologue inputs")
    rows = active.shape[0]
    vocab, hidden = embedding.shape
    if length.dtype != torch.int64 or next_tokens.dtype != torch.int64:
        raise ValueError("length and next must be int64")
    if embedding.dtype != torch.bfloat16 or norm_weight.dtype != torch.bfloat16:
        raise ValueError("embedding and norm weight must be bf16")
    if not (embedding.is_contiguous() and norm_weight.is_contiguous() and length.is_contiguous()
            and next_tokens.is_contiguous()) or norm_weight.numel() != hidden:
        raise ValueError("contiguous [vocab, hidden] embedding and [hidden] norm weight required")
    dev = embedding.device
    x = torch.empty(rows, hidden, dtype=torch.bfloat16, device=dev)
    z = torch.empty_like(x)
    valid = torch.empty(rows, dtype=torch.bool, device=dev)
    positions = torch.empty(rows, dtype=torch.int64, device=dev)
    used = torch.empty(rows, dtype=torch.int32, device=dev)
    if row_order is not None and (row_order.dtype != torch.int32 or row_order.shape != (rows,)
                                  or not row_order.is_contiguous()):
        raise ValueError("row_order must be a contiguous int32 [rows] tensor")
    if step_counter is not None and (step_counter.dtype != torch.int64 or step_counter.numel() != 1):
        raise ValueError("step_counter must be an int64 [1] tensor")
    _lib.call("lm_decode_prologue", _bool_bytes(active).data_ptr(), length.data_ptr(),
              next_tokens.data_ptr(), embedding.data_ptr(), float(multiplier), norm_weight.data_ptr(),
              float(eps), x.data_ptr(), z.data_ptr(), valid.view(torch.uint8).data_ptr(),
              positions.data_ptr(), used.data_ptr(), _lib.ptr(row_order), _lib.ptr(step_counter), rows,
              hidden, vocab, _lib.stream(dev))
    return x, z, valid, positions, used


def greedy_epilogue(logits, logits_scaling, valid, state, emit, eos, ignore_eos, ring_target=None):
    """Greedy token choice and the engine's state update, in place.

    ``logits`` is the raw head output ``[rows, vocab]`` (before
    ``/ logits_scaling``); ``state`` holds the engine's ``next``,
    ``length``, ``generated``, ``budget`` (int64) and ``active`` (bool);
    ``emit`` is ``[rows, 3]`` int64; ``eos`` an int64 tensor of stop ids.
    ``ring_target`` (``OutputRing.device_target(rows)``: the ring's device
    address, depth and step counter) also receives the emit rows, in slot
    ``(counter - 1) % depth``.
    """
    _lib.require_cuda(logits, valid, emit, eos, what="greedy epilogue inputs")
    rows, vocab = logits.shape
    if logits.dtype != torch.bfloat16 or logits.stride(1) != 1:
        raise ValueError("logits must be bf16 with unit column stride")
    for name in ("next", "length", "generated", "budget"):
        t = state[name]
        if t.dtype != torch.int64 or not t.is_contiguous() or t.shape != (rows,):
            raise ValueError(f"state[{name!r}] must be contiguous int64 [rows]")
    if emit.dtype != torch.int64 or emit.shape != (rows, 3) or not emit.is_contiguous():
        raise ValueError("emit must be contiguous int64 [rows, 3]")
    if eos.dtype != torch.int64 or not eos.is_contiguous():
        raise ValueError("eos must be a contiguous int64 tensor")
    ring_ptr, depth, counter = (None, 0, None) if ring_target is None else ring_target
    nbytes = _lib.size_query("lm_greedy_epilogue_workspace_size", rows, vocab)
    ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=logits.device)
    _lib.call("lm_greedy_epilogue", logits.data_ptr(), logits.stride(0), float(logits_scaling), vocab,
              rows, _bool_bytes(valid).data_ptr(), state["next"].data_ptr(), state["length"].data_ptr(),
              state["generated"].data_ptr(), state["budget"].data_ptr(),
              _bool_bytes(state["active"]).data_ptr(), emit.data_ptr(),
              eos.data_ptr() if eos.numel() else None, eos.numel(), int(bool(ignore_eos)),
              ring_ptr, depth, _lib.ptr(counter), ws.data_ptr(), ws.numel(), _lib.stream(logits.device))


def head_supported(rows, vocab, hidden):
    """Whether :func:`greedy_head` has a kernel for this shape (rows <= 128,
    hidden 512/1024/1536/2048)."""
    return 1 <= rows <= 128 and 0 < vocab < 2 ** 31 and hidden in (512, 1024, 1536, 2048)


class PackedHead:
    """The LM head ``[vocab, hidden]`` in MFMA fragment order
    (``lm_head_pack``): what :func:`greedy_head` streams."""

    def __init__(self, head):
        _lib.require_cuda(head, what="head")
        if head.dtype != torch.bfloat16 or head.dim() != 2 or not head.is_contiguous():
            raise ValueError("head must be a contiguous bf16 [vocab, hidden] tensor")
        self.vocab, self.hidden = head.shape
        nbytes = _lib.size_query("lm_head_pack_size", self.vocab, self.hidden)
        self.packed = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=head.device)
        _lib.call("lm_head_pack", head.data_ptr(), self.vocab, self.hidden, self.packed.data_ptr(),
                  _lib.stream(head.device))


def greedy_head(z, head, logits_scaling, valid, state, emit, eos, ignore_eos, ring_target=None,
                logits_out=None):
    """The LM head product and :func:`greedy_epilogue` in two launches: the
    packed head (:class:`PackedHead`) is streamed once with the argmax in the
    product's epilogue, then the state update. Same candidate, emit rows and
    state as ``greedy_epilogue(F.linear(z, head), ...)`` given the same bf16
    logits; ``logits_out`` (bf16 ``[rows, vocab]``, optional) receives them
    (litemoe/model.py:127 and litemoe/engine.py:92-102)."""
    _lib.require_cuda(z, head.packed, valid, emit, eos, what="greedy head inputs")
    rows, hidden = z.shape
    vocab = head.vocab
    if z.dtype != torch.bfloat16:
        raise ValueError("z must be bf16")
    if z.stride(1) != 1 or head.hidden != hidden:
        raise ValueError("z must have unit column stride and the head's hidden size")
    if not head_supported(rows, vocab, hidden):
        raise ValueError(f"no fused head kernel for rows={rows}, hidden={hidden}")
    for name in ("next", "length", "generated", "budget"):
        t = state[name]
        if t.dtype != torch.int64 or not t.is_contiguous() or t.shape != (rows,):
            raise ValueError(f"state[{name!r}] must be contiguous int64 [rows]")
    if emit.dtype != torch.int64 or emit.shape != (rows, 3) or not emit.is_contiguous():
        raise ValueError("emit must be contiguous int64 [rows, 3]")
    if eos.dtype != torch.int64 or not eos.is_contiguous():
        raise ValueError("eos must be a contiguous int64 tensor")
    if logits_out is not None and (logits_out.dtype != torch.bfloat16 or logits_out.shape != (rows, vocab)
                                   or logits_out.stride(1) != 1):
        raise ValueError("logits_out must be bf16 [rows, vocab] with unit column stride")
    ring_ptr, depth, counter = (None, 0, None) if ring_target is None else ring_target
    nbytes = _lib.size_query("lm_head_greedy_workspace_size", rows, vocab, hidden)
    ws = torch.empty(max(nbytes, 8), dtype=torch.uint8, device=z.device)
    _lib.call("lm_head_greedy", z.data_ptr(), z.stride(0), head.packed.data_ptr(), rows, vocab, hidden,
              float(logits_scaling), _lib.ptr(logits_out), 0 if logits_out is None else logits_out.stride(0),
              _bool_bytes(valid).data_ptr(), state["next"].data_ptr(), state["length"].data_ptr(),
              state["generated"].data_ptr(), state["budget"].data_ptr(),
              _bool_bytes(state["active"]).data_ptr(), emit.data_ptr(),
              eos.data_ptr() if eos.numel() else None, eos.numel(), int(bool(ignore_eos)),
              ring_ptr, depth, _lib.ptr(counter), ws.data_ptr(), ws.numel(), _lib.stream(z.device))
