"""Granite MoE forward on the gfx950 kernels (litemoe/model.py:17-127).

``Granite(cfg, weights, ep, capacity).forward(tokens, positions, valid, cache,
slot=None, last=None, communication_tokens=None)`` keeps the reference's
signature and tensor layouts. Per layer (decode and packed prefill alike):

    x += r * y_prev; z = rmsnorm(x)          lm_add_rmsnorm (layer 0: plain norm)
    qkv = z . Wqkv^T                         lm_linear (packed q|k|v, model.py:37-40,47-49)
    rope(q, k); k, v -> cache                lm_rope_kv_write
    a = attention(q, cache or packed k/v)    lm_flash_decode | lm_prefill_attention
    a = a . Wo^T                             lm_linear
    x += r * a; z = rmsnorm(x)               lm_add_rmsnorm
    w, ids = router(z)                       lm_router (GEMV + top-k + softmax)
    y = experts(z, ids, w)                   lm_fused_experts (align, gate_up, down, finish)

then ``x += r * y; logits = rmsnorm(x) . head^T / logits_scaling``. With
the library's experts, identity placement and no masked rows (lean decode,
packed prefill) the layer tail is fused further into three launches:
``lm_add_rmsnorm_router`` (x += r*a, norm, router), ``lm_moe_routes`` (expert
GEMMs, route order) and ``lm_moe_finish_add_rmsnorm`` (combine, x += r*y,
next layer's norm). In lean decode (rows <= 128) the dense projections are
split-K MFMA kernels (``lm_linear_splitk``) whose fp32 partials are summed
by their consumers: ``lm_flash_decode_qkv`` (QKV reduction, RoPE, KV store
and attention in one launch) and ``lm_add_rmsnorm_router_splitk``; a decode
layer is then seven hand-written launches. Every other projection (packed
prefill, decode above 128 rows, the LM head of ``forward``) is ``lm_linear``,
which reduces each output over K in one fixed order: no vendor BLAS runs on
the path, and a row's bits do not depend on the batch. There is no CPU path.
"""
import torch
import torch.nn.functional as F

from . import _lib
from .config import validate_config
from .flash_decode import FlashDecode
from .experts import combine_supported, finish_add_rmsnorm, pack_expert_weights, scan_path
from .linear import (linear_dense, linear_rope_kv, linear_splitk, linear_splitk_frag, linear_splitk_rmsnorm,
                     pick_splits)
from .norm import add_rmsnorm, rmsnorm
from .packed import PackedPrefill, build_packed, varlen_attention
from .rope import rope_kv_write
from .router import add_rmsnorm_route as route_add_rmsnorm
from .router import add_rmsnorm_route_splitk as route_add_rmsnorm_splitk
from .router import route
from .step import PackedHead, decode_prologue, greedy_epilogue, greedy_head, head_supported


class Granite:
    """The reference's ``Granite(cfg, weights, ep, capacity)``.

    ``pack_weights`` (default True) makes the decode copies of the expert
    weights and the LM head in MFMA fragment order once at construction
    (``lm_expert_pack``, ``lm_head_pack``): about 6 GB for the 32-layer 3B
    model plus 151 MB for its head. With False no copy is made; decode then
    reads the checkpoint layout (the same scan kernels on row-major weights)
    and takes the LM head through ``lm_linear`` and the greedy epilogue."""

    def __init__(self, cfg, weights, ep, capacity, pack_weights=True):
        validate_config(cfg)
        self.pack_weights = bool(pack_weights)
        self.cfg, self.w, self.ep = cfg, weights, ep
        self.trace = None
        self.decode_flash = None   # FlashDecode set by the execution policy
        self.decode_lean = False   # positions pre-zeroed for stopped rows; outputs unmasked
        self.prefill_lean = False  # set by the optimized policy: batched prefill is packed
        # decode option: the combine in the down projection, the next norm in
        # the QKV projection (bitwise the same results; measured slower)
        self.chain_combine = False
        # attention(): RoPE and the KV store in the QKV projection's epilogue
        # (lm_linear_rope_kv) rather than a separate lm_rope_kv_write pass
        self.qkv_epilogue = True
        self.used = None
        self._row_order = None     # the decode prologue's row order, during greedy_step only
        self.fused_head = True     # greedy_step: LM head with the argmax in its epilogue (lm_head_greedy)
        self._flash = {}
        device, dtype = weights["embedding"].device, weights["embedding"].dtype
        dim = cfg.hidden_size // cfg.num_attention_heads
        self.capacity = capacity
        # RoPE tables as litemoe/model.py:31-36: inverse frequencies on the CPU
        # in fp32 (HF's initialisation), positions on the device.
        inv = 1.0 / cfg.rope_theta ** (torch.arange(0, dim, 2, device="cpu").float() / dim)
        freq = torch.outer(torch.arange(capacity, device=device).float(), inv.to(device))
        self.cos_sin = torch.cat((freq.cos(), freq.sin()), -1).to(dtype)
        self.cos, self.sin = [half.repeat(1, 2) for half in self.cos_sin.chunk(2, -1)]
        self.prepare_packed_qkv()
        self.packed_head = None
        if self.pack_weights:
            self.prepare_packed_experts()
            # The head in the fused greedy head's fragment order (a second
            # copy, made once; the embedding keeps the checkpoint layout).
            head = weights["head"]
            self.packed_head = (PackedHead(head) if head.is_cuda and head.is_contiguous() and
                                head_supported(1, head.shape[0], cfg.hidden_size) else None)

    def prepare_packed_qkv(self):
        for w in self.w["layers"]:
            if "self_attn.qkv_proj" not in w:
                w["self_attn.qkv_proj"] = torch.cat([w[f"self_attn.{p}_proj"] for p in ("q", "k", "v")])

    def prepare_packed_experts(self):
        """Expert weights in MFMA fragment order (``lm_expert_pack``) for the
        decode steps of the fused layer tail, made once next to the
        checkpoint layout: decode then loads every weight fragment as 1 KB
        contiguous (gate/up 29.0 -> 27.3 us per layer at the 3B decode
        shape), while the prefill expert GEMM and the masked expert path
        keep the checkpoint layout (the GEMM's 128-byte row runs measured
        15% faster there)."""
        if not getattr(self.ep.backend, "native", False):
            return
        for w in self.w["layers"]:
            w1, w2 = w["input_linear"], w["output_linear"]
            if "input_linear_packed" not in w and w1.is_cuda and w1.is_contiguous() and w2.is_contiguous():
                w["input_linear_packed"], w["output_linear_packed"] = pack_expert_weights(w1, w2)

    def _decode_attention(self, batch, cache):
        if self.decode_flash is not None:
            return self.decode_flash
        key = (batch, cache.capacity)
        if key not in self._flash:
            cfg = self.cfg
            self._flash[key] = FlashDecode(batch, cfg.num_key_value_heads,
                                           cfg.num_attention_heads // cfg.num_key_value_heads,
                                           cache.capacity, cache.k.device)
        return self._flash[key]

    def attention(self, z, w, cache, layer, rope_positions, active, positions, slot):
        """Packed QKV projection, RoPE + KV store, attention, output projection
        (litemoe/model.py:42-73). ``z [rows, H]`` -> ``[rows, H]``."""
        cfg = self.cfg
        rows = z.shape[0]
        d = cfg.hidden_size // cfg.num_attention_heads
        hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads
        packed = isinstance(slot, PackedPrefill)
        slots = slot.slots if packed else None
        if self.qkv_epilogue:
            qkv = linear_rope_kv(z, w["self_attn.qkv_proj"], hq, hkv, rope_positions, active, self.cos_sin,
                                 cache, layer, slots)
        else:
            qkv = linear_dense(z, w["self_attn.qkv_proj"])
        q = qkv[:, :hq * d].view(rows, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].view(rows, hkv, d)
        v = qkv[:, (hq + hkv) * d:].view(rows, hkv, d)
        if not self.qkv_epilogue:
            rope_kv_write(q, k, v, rope_positions, active, self.cos_sin, cache, layer, slots=slots,
                          write_k=packed)
        if packed:
            a = varlen_attention(q, k, v, slot.cu, slot.maximum, cfg.attention_multiplier)
        else:
            flash = self._decode_attention(rows, cache)
            a = flash(q.unsqueeze(2), cache.k[layer], cache.v[layer], positions, active,
                      cfg.attention_multiplier, self.used)
        return linear_dense(a.reshape(rows, hq * d), w["self_attn.o_proj"])

    def decode_splits(self, rows):
        """K-slice counts (qkv, o_proj) of the split-K decode projections, or
        None when a shape has no kernel (the layer then uses lm_linear)."""
        cfg = self.cfg
        d = cfg.hidden_size // cfg.num_attention_heads
        # lm_add_rmsnorm_router_splitk: hidden 512*{1..4}, at most 4 slices
        if d != 64 or cfg.hidden_size % 512 or cfg.hidden_size > 2048:
            return None
        nqkv = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * d
        sq = pick_splits(rows, nqkv, cfg.hidden_size)
        so = pick_splits(rows, cfg.hidden_size, cfg.num_attention_heads * d, max_splits=4)
        return (sq, so) if sq and so else None

    def attention_splitk(self, z, w, cache, layer, rope_positions, active, splits, part=None):
        """Decode layer attention on the split-K projections: the packed QKV
        partials go to lm_flash_decode_qkv (reduction, RoPE, KV store and
        attention in one launch), and the o_proj partials are returned for
        the router's residual add (litemoe/model.py:47-73). The attention
        output goes to o_proj in the split-K kernel's fragment order (1 KB
        per activation load; o_proj 5.48 -> 4.84 us at cfg 3). z stays
        row-major: its combine kernel writes whole rows, and the scattered
        fragment-order stores there cost more than the QKV projection gains.
        ``part``: the QKV partials, when the caller formed them (e.g. with the
        input norm fused in, :func:`linear_splitk_rmsnorm`)."""
        cfg = self.cfg
        rows = z.shape[0]
        if part is None:
            part = linear_splitk(z, w["self_attn.qkv_proj"], splits[0])
        flash = self._decode_attention(rows, cache)
        order = self._row_order if self._row_order is not None and self._row_order.shape[0] == rows else None
        a = flash.fused_qkv(part, self.cos_sin, rope_positions, active, cache.k[layer], cache.v[layer],
                            cfg.attention_multiplier, self.used, cfg.num_attention_heads, row_order=order,
                            frag_out=True)
        return linear_splitk_frag(a, w["self_attn.o_proj"], splits[1])

    def _fused_moe(self):
        """The fused layer tail (add+norm+router, route GEMMs, combine+add+norm)
        applies when the experts run on this library with identity placement
        and no row needs masking (lean decode or packed prefill)."""
        return getattr(self.ep.backend, "native", False) and all(
            w["logical"].numel() == 0 for w in self.w["layers"])

    def _fused_layers(self, x, z, cache, rope_positions, valid_rows, flat_positions, slot):
        """The layer stack on the fused tail: per layer attention, then
        add+norm+router, the route GEMMs and combine+add+next norm. ``x`` is
        the residual stream and ``z`` the normalised input of the first
        layer; on return ``z`` holds the final norm's output."""
        cfg = self.cfg
        layers = self.w["layers"]
        r, eps, k = cfg.residual_multiplier, cfg.rms_norm_eps, cfg.num_experts_per_tok
        splits = None if isinstance(slot, PackedPrefill) else self.decode_splits(x.shape[0])
        if splits and self._combine_chain(x.shape[0]):
            return self._chained_layers(x, z, cache, rope_positions, valid_rows, splits)
        for layer, w in enumerate(layers):
            if splits:
                o_part = self.attention_splitk(z, w, cache, layer, rope_positions, valid_rows, splits)
                weights, ids, z = route_add_rmsnorm_splitk(x, o_part, r, w["post_attention_layernorm"],
                                                           eps, w["block_sparse_moe.router.layer"], k, z)
            else:
                a = self.attention(z, w, cache, layer, rope_positions, valid_rows, flat_positions, slot)
                weights, ids, z = route_add_rmsnorm(x, a, r, w["post_attention_layernorm"], eps,
                                                    w["block_sparse_moe.router.layer"], k, z)
            if self.pack_weights and "input_linear_packed" in w and scan_path(x.shape[0], k):
                # decode: the fragment layout (1 KB per weight-fragment load)
                y = self.ep.backend.routes(z, w["input_linear_packed"], w["output_linear_packed"], ids,
                                           packed=True)
            else:
                # prefill GEMM: measured faster on the checkpoint layout's 128-byte row runs
                y = self.ep.backend.routes(z, w["input_linear"], w["output_linear"], ids)
            nxt = layers[layer + 1]["input_layernorm"] if layer + 1 < len(layers) else self.w["norm"]
            finish_add_rmsnorm(y, ids, weights, x, r, nxt, eps, z)
        return z

    def _combine_chain(self, rows):
        """Whether the decode layers run chained: the combine and the residual
        add fused into the down projection (``lm_moe_routes_combine``) and
        the next layer's input norm into its QKV projection
        (``lm_linear_splitk_rmsnorm``). Off by default: at the 3B decode
        shape the chained step measured 3.03-3.04 ms against 2.965-2.968 ms
        (the last arriver's combine adds 2.6 us per layer at the end of the
        down launch, forming the norm adds 1.6 us to the QKV projection,
        against the 5.1 us combine launch they replace)."""
        cfg = self.cfg
        h, i = cfg.hidden_size, cfg.intermediate_size
        return (self.chain_combine and self.pack_weights and "input_linear_packed" in self.w["layers"][0]
                and h % 512 == 0 and h <= 2048 and combine_supported(rows, cfg.num_experts_per_tok, h, i))

    def _chained_layers(self, x, z, cache, rope_positions, valid_rows, splits):
        """The decode layers with four launches between attentions instead of
        five: per layer the QKV projection (layer 0 from the prologue's z,
        then with the input norm formed from ``x`` and the previous layer's
        sums of squares), the attention, o_proj, add+norm+router (each
        token's experts in id order), gate/up, and down with the combine and
        the residual add. Bitwise the same x, z, KV cache and logits as the
        unchained layers; the final norm is one lm_rmsnorm."""
        cfg = self.cfg
        r, eps, k = cfg.residual_multiplier, cfg.rms_norm_eps, cfg.num_experts_per_tok
        sumsq = None
        for layer, w in enumerate(self.w["layers"]):
            part = None
            if layer:
                part = linear_splitk_rmsnorm(x, sumsq, w["input_layernorm"], eps, w["self_attn.qkv_proj"],
                                             splits[0])
            o_part = self.attention_splitk(z, w, cache, layer, rope_positions, valid_rows, splits, part=part)
            weights, ids, z = route_add_rmsnorm_splitk(x, o_part, r, w["post_attention_layernorm"], eps,
                                                       w["block_sparse_moe.router.layer"], k, z, id_order=True)
            sumsq = self.ep.backend.routes_combine(z, w["input_linear_packed"], w["output_linear_packed"], ids,
                                                   weights, residual=x, alpha=r, sumsq=sumsq, packed=True)
        return rmsnorm(x, self.w["norm"], eps, out=z)

    def greedy_supported(self):
        """Whether :meth:`greedy_step` applies: lean decode on the fused tail,
        and a hidden size the prologue kernel takes."""
        h = self.cfg.hidden_size
        return bool(self.decode_lean) and self._fused_moe() and h % 8 == 0 and h <= 4096

    def greedy_step(self, state, emit, eos, ignore_eos, cache, ring=None):
        """One lean greedy decode step from the engine's state to its update:
        prologue kernel (valid, positions, ``used``, embedding, first norm),
        the fused layers, the raw head product and the epilogue kernel
        (argmax of ``logits / logits_scaling``, emit row, state update).
        Same tokens and state as litemoe/engine.py:87-102 around this model's
        forward (model.py:95-127) in lean decode. With an asynchronous
        ``ring`` the epilogue also stores the emit rows into the ring's slot
        for this step (counted by the prologue)."""
        cfg = self.cfg
        rows = state["active"].shape[0]
        order = getattr(self.decode_flash, "row_order", None)
        if order is not None and order.shape[0] != rows:
            order = None
        target = ring.device_target(rows) if ring is not None else None
        x, z, valid, positions, used = decode_prologue(
            state["active"], state["length"], state["next"], self.w["embedding"],
            cfg.embedding_multiplier, self.w["layers"][0]["input_layernorm"], cfg.rms_norm_eps,
            row_order=order, step_counter=None if target is None else target[2])
        self.used = used
        self._row_order = order  # valid for this step only: the prologue just wrote it
        try:
            z = self._fused_layers(x, z, cache, positions, valid, positions, None)
        finally:
            self._row_order = None
        head = self.w["head"]
        if self.fused_head and self.packed_head is not None and head_supported(rows, head.shape[0],
                                                                               cfg.hidden_size):
            greedy_head(z, self.packed_head, cfg.logits_scaling, valid, state, emit, eos, ignore_eos,
                        ring_target=target)
        else:
            greedy_epilogue(linear_dense(z, head), cfg.logits_scaling, valid, state, emit, eos,
                            ignore_eos, ring_target=target)

    def forward(self, tokens, positions, valid, cache, slot=None, last=None, communication_tokens=None):
        """Logits ``[rows, positions, V] / logits_scaling`` (litemoe/model.py:95-127).

        ``slot=None``: one decode step, ``tokens [B, 1]``. ``slot`` a
        :class:`PackedPrefill`: the packed ragged prefill, one row of all
        prompts. ``slot`` an int or a slice: a right-padded prefill of
        ``tokens [b, s]`` into cache rows ``slot`` (``valid`` a prefix of each
        row, ``positions`` the column index), run on the packed kernels
        (:meth:`_padded_prefill`). ``last`` keeps one position per row (an
        int, or a tensor of per-row positions; for a packed row, flat token
        indices). ``communication_tokens`` sizes the reference's EP2
        exchange and is not used on one GPU."""
        if slot is not None and not isinstance(slot, PackedPrefill):
            return self._padded_prefill(tokens, positions, valid, cache, slot, last)
        cfg = self.cfg
        packed = isinstance(slot, PackedPrefill)
        _lib.require_cuda(tokens, positions, valid, cache.k, what="model inputs")
        b, s = tokens.shape
        hidden = cfg.hidden_size
        valid_rows = valid.reshape(-1)
        if packed:
            rope_positions, flat_positions = slot.positions, slot.positions
            self.used = None
        else:
            if s != 1:
                raise ValueError("Decode takes one token per row")
            flat_positions = positions[:, 0]
            lean = self.decode_lean
            rope_positions = flat_positions if lean else torch.where(valid_rows, flat_positions, 0)
            # seqused_k of flash_decode.py:21 / model.py:103
            self.used = ((rope_positions + 1) if lean else
                         torch.where(valid_rows, flat_positions + 1, 1)).to(torch.int32)
        x = (F.embedding(tokens, self.w["embedding"]) * cfg.embedding_multiplier).reshape(b * s, hidden)
        x = x.contiguous()
        z = self._layers(x, cache, rope_positions, valid_rows, flat_positions, slot, communication_tokens)
        if last is not None:
            # row i keeps position last[i] (litemoe/model.py:123-125); a packed
            # batch is one row, so its `last` are flat token indices
            last = last.long() if isinstance(last, torch.Tensor) else torch.tensor(last, device=x.device)
            z = z[torch.arange(b, device=x.device) * s + last]
            out_rows = (z.shape[0], 1)
        else:
            out_rows = (b, s)
        return (linear_dense(z, self.w["head"]) / cfg.logits_scaling).view(*out_rows, -1)

    def _layers(self, x, cache, rope_positions, valid_rows, flat_positions, slot, communication_tokens=None):
        """The layer stack over the rows of ``x [rows, H]`` (the residual
        stream, updated in place); returns the final norm's output."""
        cfg = self.cfg
        eps, r = cfg.rms_norm_eps, cfg.residual_multiplier
        packed = isinstance(slot, PackedPrefill)
        masked = not packed and not self.decode_lean
        layers = self.w["layers"]
        z = add_rmsnorm(x, None, r, layers[0]["input_layernorm"], eps)
        if not masked and self._fused_moe():
            return self._fused_layers(x, z, cache, rope_positions, valid_rows, flat_positions, slot)
        y = None
        for layer, w in enumerate(layers):
            if layer:
                add_rmsnorm(x, y, r, w["input_layernorm"], eps, out=z)
            a = self.attention(z, w, cache, layer, rope_positions, valid_rows, flat_positions, slot)
            if masked:
                a = a * valid_rows[:, None]
            add_rmsnorm(x, a, r, w["post_attention_layernorm"], eps, out=z)
            scales, ids = route(z, w["block_sparse_moe.router.layer"], cfg.num_experts_per_tok)
            if packed or not self.decode_lean:
                # outside the fused paths the reference hands the experts
                # bf16 scales (litemoe/model.py:117-118)
                scales = scales.to(torch.bfloat16)
            y = self.ep(z, ids, scales, valid_rows, w["physical"], w["input_linear"], w["output_linear"],
                        w["logical"], decode=True, tokens=communication_tokens)
        return add_rmsnorm(x, y, r, self.w["norm"], eps, out=z)

    def _padded_prefill(self, tokens, positions, valid, cache, slot, last):
        """Right-padded prefill into cache rows ``slot`` (an int: one row; a
        slice: ``b`` rows), litemoe/model.py:95-127 with ``slot`` not None.

        The reference runs every position through SDPA with a padding mask
        and stores ``k * valid`` in cache positions ``0 .. s-1``
        (litemoe/cache.py:21-33). Here each row's valid prefix becomes one
        sequence of a packed batch (the same kernels as the packed prefill,
        so padding costs no work), and its KV lands in the row's cache
        positions ``0 .. n-1``; positions ``n .. s-1`` are zeroed. A padding
        position's residual stream keeps its scaled embedding, as in the
        reference, where its attention output is masked to zero and its
        expert rows enter as zeros: its logits (``last`` may point there)
        are those of ``norm(embedding * multiplier)``."""
        cfg = self.cfg
        _lib.require_cuda(tokens, positions, valid, cache.k, what="model inputs")
        b, s = tokens.shape
        if isinstance(slot, slice):
            rows = list(range(*slot.indices(cache.k.shape[1])))
        else:
            rows = [int(slot)]
        if len(rows) != b or not all(0 <= row < cache.k.shape[1] for row in rows):
            raise ValueError("Prefill slots must name one cache row per batch row")
        if tuple(positions.shape) != (b, s) or tuple(valid.shape) != (b, s):
            raise ValueError("tokens, positions and valid must all be [rows, width]")
        device = tokens.device
        valid = valid.to(torch.bool)
        columns = torch.arange(s, device=device)
        counts = valid.sum(1)
        right_padded = (valid == (columns[None] < counts[:, None])).all()
        in_order = ((positions == columns[None]) | ~valid).all()
        host = torch.cat((counts, torch.stack((right_padded, in_order)).long())).tolist()
        counts, ok = host[:b], all(host[b:])
        if not ok:
            raise ValueError("Padded prefill needs right-padded rows: valid a prefix of each row "
                             "and positions equal to the column index")
        if s > cache.capacity:
            raise ValueError("Prompt width exceeds the KV capacity")
        for row, n in zip(rows, counts):  # cache.py:28-29 stores k * valid: zeros past the prompt
            if n < s:
                cache.k[:, row, :, n:s].zero_()
                cache.v[:, row, :, n:s].zero_()
        x = (F.embedding(tokens, self.w["embedding"]) * cfg.embedding_multiplier).reshape(b * s, cfg.hidden_size)
        x = x.contiguous()
        live = [i for i, n in enumerate(counts) if n]
        if live:
            packed, _ = build_packed([counts[i] for i in live], device, slots=[rows[i] for i in live])
            index = valid.reshape(-1).nonzero().flatten()  # row-major: each row's prefix in order
            xv = x.index_select(0, index)
            self._layers(xv, cache, packed.positions, torch.ones(xv.shape[0], dtype=torch.bool, device=device),
                         packed.positions, packed)
            x.index_copy_(0, index, xv)
        if last is not None:
            last = last.long().to(device) if isinstance(last, torch.Tensor) else torch.tensor(last, device=device)
            x = x[torch.arange(b, device=device) * s + last]
            out_rows = (b, 1)
        else:
            out_rows = (b, s)
        z = add_rmsnorm(x.contiguous(), None, cfg.residual_multiplier, self.w["norm"], cfg.rms_norm_eps)
        return (linear_dense(z, self.w["head"]) / cfg.logits_scaling).view(*out_rows, -1)
