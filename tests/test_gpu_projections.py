"""Split-K decode projections and their fused consumers.

Bars: the projection against an fp32 product of the same bf16 operands
(within fp32 accumulation-order error; the bf16 output within one ulp); the
fused consumers bitwise against the unfused kernels they replace
(reduce -> rope_kv_write -> flash_decode, reduce -> add_rmsnorm_route).
"""
import pytest
import torch

from litemoe_amd import _lib, flash_decode, linear, rope, router
from litemoe_amd.cache import KVCache
from litemoe_amd.config import ModelConfig
from litemoe_amd.synth import normal_bf16
from oracle import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(shape, std=1.0, seed=0):
    return normal_bf16(shape, std, seed)


def ordered(t):
    i = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(i >= 0, i, -(i & 0x7FFF))


def within_ulp_or_abs(a, b, ulps, floor):
    """Every element within ``ulps`` bf16 ulps or ``floor`` absolutely (sums
    that cancel to near zero lose relative accuracy)."""
    close = (ordered(a) - ordered(b)).abs() <= ulps
    return bool((close | ((a.float() - b.float()).abs() <= floor)).all())


@pytest.mark.parametrize("rows", [1, 7, 16, 33, 64, 128])
@pytest.mark.parametrize("n,k", [(2560, 1536), (1536, 1536), (2048, 1024), (64, 512)])
@torch.inference_mode()
def test_linear_splitk_matches_fp32_product(rows, n, k):
    a = bf((rows, k), 1.0, rows + n)
    w = bf((n, k), 0.02, k + 1)
    exp = a.float() @ w.float().T
    for splits in sorted({s for s in (1, 2, 3, 4, 6, 8) if (k // 128) % s == 0 and (k // 128) // s in (1, 2, 3, 4, 6, 8)}):
        part = linear.linear_splitk(a.to(DEV), w.to(DEV), splits)
        assert part.shape == (splits, rows, n)
        got = part.sum(0).cpu()
        torch.testing.assert_close(got, exp, atol=2e-5 * k ** 0.5, rtol=1e-5)
        out = linear.reduce(part).cpu()
        assert within_ulp_or_abs(out, exp.to(torch.bfloat16), 1, 1e-3)


@torch.inference_mode()
def test_linear_splitk_strided_rows_and_unsupported_shapes():
    a = bf((16, 2048), 1.0, 3).to(DEV)
    w = bf((512, 1024), 0.02, 4).to(DEV)
    view = a[:, 512:1536]  # row stride 2048
    got = linear.linear(view, w).cpu()
    exp = (view.float().cpu() @ w.float().cpu().T).to(torch.bfloat16)
    assert within_ulp_or_abs(got, exp, 1, 1e-3)
    assert linear.pick_splits(129, 512, 1024) is None
    assert linear.pick_splits(64, 500, 1024) is None
    with pytest.raises(_lib.NativeError):
        linear.linear_splitk(bf((129, 1024)).to(DEV), w, 2)
    with pytest.raises(_lib.NativeError):
        linear.linear_splitk(bf((16, 1024)).to(DEV), w, 5)  # 8 k steps do not split in 5


@pytest.mark.parametrize("rows", [1, 7, 16, 33, 64, 100, 128])
@pytest.mark.parametrize("n,k", [(2560, 1536), (1536, 1536), (64, 512)])
@torch.inference_mode()
def test_linear_splitk_frag_equals_row_major(rows, n, k):
    """The fragment-order input gives the row-major kernel's partials, bit for
    bit (the same MFMA operands in the same order; padding rows dropped)."""
    a = bf((rows, k), 1.0, 7 * rows + n).to(DEV)
    w = bf((n, k), 0.02, k + 3).to(DEV)
    fa = linear.FragRows.from_rows(a)
    for splits in sorted({s for s in (1, 2, 3, 4, 6, 8) if (k // 128) % s == 0 and (k // 128) // s in (1, 2, 3, 4, 6, 8)}):
        exp = linear.linear_splitk(a, w, splits)
        got = linear.linear_splitk_frag(fa, w, splits)
        assert torch.equal(got, exp)
    # padding rows are never written in the decode step: NaN there reaches no valid row
    if rows % 16:
        mb = fa.mb
        padded = torch.full((16 * mb, k), float("nan"), device=DEV, dtype=torch.bfloat16)
        padded[:rows] = a
        data = padded.view(mb, 16, k // 32, 4, 8).permute(2, 0, 3, 1, 4).contiguous().view(-1)
        junk = linear.FragRows(rows, k, DEV, data)
        splits = 1 if k == 512 else 3
        assert torch.equal(linear.linear_splitk_frag(junk, w, splits), linear.linear_splitk(a, w, splits))


def _fp32_product(a, w, chunk=8192):
    """fp32 product of the same bf16 operands (on the device, in row chunks)."""
    wt = w.float().T
    return torch.cat([a[i:i + chunk].float() @ wt for i in range(0, a.shape[0], chunk)])


@pytest.mark.parametrize("rows,n,k", [
    (46990, 2560, 1536),   # cfg 4 packed QKV (46,990 prefill tokens)
    (46990, 1536, 1536),   # cfg 4 o_proj
    (65536, 2560, 1536),   # cfg 3 prefill QKV (64 prompts of 1024)
    (48, 49155, 1536),     # prefill LM head at the last positions: odd vocabulary, 2-byte stores
    (1, 512, 1024), (17, 200, 256), (130, 2560, 1536), (257, 1536, 1536),
    # one k step (K = 64) on both tile sizes, an odd column count on the 256-row tiles, two k steps
    (2049, 100, 64), (5, 8, 64), (3000, 4100, 128), (2048, 2560, 192)])
@torch.inference_mode()
def test_linear_dense_matches_fp32_product(rows, n, k):
    """lm_linear against an fp32 product of the same bf16 operands: the bf16
    output within one ulp (or 1e-3 absolutely where the sum cancels)."""
    g = torch.Generator(device=DEV).manual_seed(rows + n + k)
    a = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    got = linear.linear_dense(a, w)
    exp = _fp32_product(a, w)
    assert torch.isfinite(got.float()).all()
    # fp32 accumulation-order error of a K-long sum of products of magnitude ~0.02
    assert (got.float() - exp).abs().max() <= 1e-2 * exp.abs().max() or within_ulp_or_abs(
        got, exp.to(torch.bfloat16), 1, 1e-3)
    assert within_ulp_or_abs(got, exp.to(torch.bfloat16), 1, 1e-3)


@torch.inference_mode()
def test_linear_dense_is_batch_and_launch_invariant():
    """A row's output is the same bits alone, inside any batch, at any row
    position, through strided views, and on every launch (one workgroup
    reduces each output over K in one order)."""
    g = torch.Generator(device=DEV).manual_seed(5)
    a = torch.randn(3000, 1536, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(2560, 1536, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    full = linear.linear_dense(a, w)
    for _ in range(3):
        assert torch.equal(linear.linear_dense(a, w), full)
    for start, stop in ((0, 1), (5, 6), (100, 229), (2999, 3000), (1000, 2500)):
        assert torch.equal(linear.linear_dense(a[start:stop], w), full[start:stop])
    # strided input and output, and a weight that is a row range of a larger matrix
    wide = torch.zeros(64, 2048, device=DEV, dtype=torch.bfloat16)
    wide[:, 256:1792] = a[:64]
    out = torch.full((64, 3000), float("nan"), device=DEV, dtype=torch.bfloat16)
    linear.linear_dense(wide[:, 256:1792], w[512:2048], out=out[:, 100:1636])
    assert torch.equal(out[:, 100:1636], full[:64, 512:2048])
    assert out[:, :100].isnan().all() and out[:, 1636:].isnan().all()


@torch.inference_mode()
def test_linear_dense_rejections():
    a = bf((16, 96)).to(DEV)
    with pytest.raises(ValueError):
        linear.linear_dense(a, bf((32, 96)).to(DEV))  # K not a multiple of 64
    with pytest.raises(ValueError):
        linear.linear_dense(bf((16, 128)).to(DEV), bf((32, 64)).to(DEV))
    assert linear.linear_dense(bf((0, 128)).to(DEV), bf((32, 128)).to(DEV)).shape == (0, 32)


class _Cache:
    def __init__(self, layers, batch, hkv, cap):
        self.capacity = cap
        shape = (layers, batch, hkv, cap, 64)
        self.k = torch.full(shape, 7.0, device=DEV, dtype=torch.bfloat16)
        self.v = torch.full(shape, -3.0, device=DEV, dtype=torch.bfloat16)


@pytest.mark.parametrize("rows,hq,hkv,k,batch,cap,table,masked", [
    (5000, 24, 8, 1536, 6, 1024, 1024, False),   # cfg 3/4 layer shape, 256 x 256 tiles
    (3001, 16, 8, 1024, 4, 1024, 900, True),     # cfg 2 shape; positions past the table
    (700, 24, 8, 1536, 3, 512, 512, True),       # 128 x 128 tiles
    (37, 8, 4, 512, 2, 64, 64, False), (1, 24, 8, 1536, 1, 16, 16, False)])
@torch.inference_mode()
def test_linear_rope_kv_equals_projection_then_rope_kv_write(rows, hq, hkv, k, batch, cap, table, masked):
    """lm_linear_rope_kv against lm_linear then lm_rope_kv_write(write_k=1):
    the rotated qkv and both cache layers bit for bit, with packed-prefill
    slots and positions, inactive rows, rows whose position or slot is out
    of range (not stored) and positions past the RoPE table (not rotated)."""
    g = torch.Generator(device=DEV).manual_seed(rows + k)
    a = torch.randn(rows, k, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn((hq + 2 * hkv) * 64, k, generator=g, device=DEV) * 0.03).to(torch.bfloat16)
    cos_sin, _, _ = ops.rope_tables(1e4, 64, table, torch.bfloat16)
    cos_sin = cos_sin.to(DEV)
    # distinct (slot, position) pairs: one writer per cache entry
    cell = torch.randperm(batch * cap, generator=g, device=DEV)[:rows]
    slots, pos = cell // cap, cell % cap
    active = torch.ones(rows, dtype=torch.bool, device=DEV)
    if masked:
        active = torch.rand(rows, generator=g, device=DEV) > 0.2
        pos[::7] = cap + 3          # past capacity (and past the table)
        pos[::11] = -1
        slots[::13] = batch         # past the cache batch
    layer = 1
    ref_cache, got_cache = _Cache(3, batch, hkv, cap), _Cache(3, batch, hkv, cap)
    ref = linear.linear_dense(a, w)
    q = ref[:, :hq * 64].view(rows, hq, 64)
    kk = ref[:, hq * 64:(hq + hkv) * 64].view(rows, hkv, 64)
    v = ref[:, (hq + hkv) * 64:].view(rows, hkv, 64)
    rope.rope_kv_write(q, kk, v, pos, active, cos_sin, ref_cache, layer, slots=slots, write_k=True)
    for rep in range(2):
        got = linear.linear_rope_kv(a, w, hq, hkv, pos, None if not masked and rep else active, cos_sin,
                                    got_cache, layer, slots)
        assert torch.equal(got, ref), rep
        assert torch.equal(got_cache.k, ref_cache.k) and torch.equal(got_cache.v, ref_cache.v), rep
    # a row range alone: the same rows
    got = linear.linear_rope_kv(a[:3], w, hq, hkv, pos[:3], None, cos_sin, got_cache, layer, slots[:3])
    assert torch.equal(got, ref[:3])


def _qkv_case(b, hq, hkv, cap, splits, seed):
    g = torch.Generator().manual_seed(seed)
    ncols = (hq + 2 * hkv) * 64
    part = (torch.randn(splits, b, ncols, generator=g) * 0.7).to(DEV)
    cos_sin, _, _ = ops.rope_tables(1e4, 64, cap, torch.bfloat16)
    pos = torch.randint(0, cap, (b,), generator=g)
    pos[0] = 0
    pos[-1] = cap - 1
    return part, cos_sin.to(DEV), pos.to(DEV)


@pytest.mark.parametrize("b,hq,hkv,cap,attn_splits,qkv_splits", [
    (64, 24, 8, 1280, 1, 3), (5, 24, 8, 1024, 4, 3), (3, 16, 8, 300, 3, 2), (7, 8, 8, 64, 1, 8),
    (2, 32, 4, 2048, 16, 1), (9, 24, 6, 512, 2, 3), (4, 24, 4, 700, 1, 2)])
@torch.inference_mode()
def test_flash_decode_qkv_equals_unfused(b, hq, hkv, cap, attn_splits, qkv_splits):
    part, cos_sin, pos = _qkv_case(b, hq, hkv, cap, qkv_splits, b * cap)
    active = torch.ones(b, dtype=torch.bool, device=DEV)
    if b > 2:
        active[1] = False
    used = torch.where(active, pos + 1, 1).to(torch.int32)
    cfg = ModelConfig(num_key_value_heads=hkv, hidden_size=hq * 64, num_attention_heads=hq, num_hidden_layers=1)
    caches = [KVCache(cfg, b, cap, DEV, torch.bfloat16) for _ in range(2)]
    caches[0].k.normal_()
    caches[0].v.normal_()
    caches[1].k.copy_(caches[0].k)
    caches[1].v.copy_(caches[0].v)
    fd = flash_decode.FlashDecode(b, hkv, hq // hkv, cap, DEV, num_splits=attn_splits)
    # unfused: reduce -> rope + kv store -> attention over the cache
    qkv = linear.reduce(part)
    q = qkv[:, :hq * 64].view(b, hq, 64)
    k = qkv[:, hq * 64:(hq + hkv) * 64].view(b, hkv, 64)
    v = qkv[:, (hq + hkv) * 64:].view(b, hkv, 64)
    rope.rope_kv_write(q, k, v, pos, active, cos_sin, caches[0], 0)
    exp = fd(q.unsqueeze(2), caches[0].k[0], caches[0].v[0], None, None, 0.125, used=used)
    got = fd.fused_qkv(part, cos_sin, pos, active, caches[1].k[0], caches[1].v[0], 0.125, used, hq)
    assert torch.equal(got, exp)
    assert torch.equal(caches[1].k, caches[0].k) and torch.equal(caches[1].v, caches[0].v)
    # any dispatch order of the rows gives the same bits (a fresh copy of the
    # cache: the fused call writes the new keys again)
    g = torch.Generator().manual_seed(b)
    order = torch.randperm(b, generator=g).to(torch.int32).to(DEV)
    caches[1].k.copy_(caches[0].k)
    caches[1].v.copy_(caches[0].v)
    got2 = fd.fused_qkv(part, cos_sin, pos, active, caches[1].k[0], caches[1].v[0], 0.125, used, hq,
                        row_order=order)
    assert torch.equal(got2, got)
    assert torch.equal(caches[1].k, caches[0].k) and torch.equal(caches[1].v, caches[0].v)
    # and against the oracle's attention over the updated cache
    rows = list(range(min(b, 8)))
    ref = ops.decode_attention(q.cpu()[rows], caches[0].k[0].cpu()[rows], caches[0].v[0].cpu()[rows],
                               used.cpu()[rows], 0.125)
    torch.testing.assert_close(got[rows, :, 0].cpu(), ref, atol=.004, rtol=.03)


@torch.inference_mode()
def test_flash_decode_qkv_in_a_graph_replays_like_eager():
    b, hq, hkv, cap = 16, 24, 8, 512
    part, cos_sin, pos = _qkv_case(b, hq, hkv, cap, 3, 5)
    used = (pos + 1).to(torch.int32)
    cfg = ModelConfig(num_key_value_heads=hkv, hidden_size=hq * 64, num_attention_heads=hq, num_hidden_layers=1)
    cache = KVCache(cfg, b, cap, DEV, torch.bfloat16)
    cache.k.normal_()
    cache.v.normal_()
    fd = flash_decode.FlashDecode(b, hkv, hq // hkv, cap, DEV, num_splits=2)
    eager = fd.fused_qkv(part, cos_sin, pos, None, cache.k[0], cache.v[0], 0.125, used, hq).clone()
    k_after = cache.k.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            out = fd.fused_qkv(part, cos_sin, pos, None, cache.k[0], cache.v[0], 0.125, used, hq)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager) and torch.equal(cache.k, k_after)


@pytest.mark.parametrize("splits", [1, 2, 3, 4])
@torch.inference_mode()
def test_add_rmsnorm_route_splitk_equals_unfused(splits):
    m, h, e, k = 64, 1536, 40, 8
    g = torch.Generator().manual_seed(40 + splits)
    part = (torch.randn(splits, m, h, generator=g) * 0.5).to(DEV)
    x = torch.randn(m, h, generator=g).to(torch.bfloat16).to(DEV)
    w = (1 + 0.2 * torch.randn(h, generator=g)).to(torch.bfloat16).to(DEV)
    wr = (0.02 * torch.randn(e, h, generator=g)).to(torch.bfloat16).to(DEV)
    x1, x2 = x.clone(), x.clone()
    l1 = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    l2 = torch.empty(m, e, device=DEV, dtype=torch.bfloat16)
    w1, i1, z1 = router.add_rmsnorm_route_splitk(x1, part, 0.22, w, 1e-6, wr, k, logits_out=l1)
    a = linear.reduce(part)
    w2, i2, z2 = router.add_rmsnorm_route(x2, a, 0.22, w, 1e-6, wr, k, logits_out=l2)
    assert torch.equal(x1, x2) and torch.equal(z1, z2) and torch.equal(l1, l2)
    assert torch.equal(i1, i2) and torch.equal(w1, w2)


@torch.inference_mode()
def test_add_rmsnorm_route_splitk_limits():
    x = torch.zeros(4, 1536, dtype=torch.bfloat16, device=DEV)
    w = torch.ones(1536, dtype=torch.bfloat16, device=DEV)
    wr = torch.zeros(40, 1536, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.NativeError):  # more than 4 slices
        router.add_rmsnorm_route_splitk(x, torch.zeros(5, 4, 1536, device=DEV), 0.2, w, 1e-6, wr, 8)
    x3 = torch.zeros(4, 3072, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_lib.NativeError):  # hidden above 2048
        router.add_rmsnorm_route_splitk(x3, torch.zeros(2, 4, 3072, device=DEV), 0.2,
                                        torch.ones(3072, dtype=torch.bfloat16, device=DEV), 1e-6,
                                        torch.zeros(40, 3072, dtype=torch.bfloat16, device=DEV), 8)


@torch.inference_mode()
def test_bf16_rounding_of_every_float():
    """Every kernel rounds fp32 to bf16 with one helper (the hardware
    conversion plus NaN canonicalisation). The split-K reduce with one slice
    writes bf16(0 + p), i.e. that rounding of p (p = -0 gives +0), so all
    2^32 bit patterns go through it: against round-to-nearest-even with NaN ->
    0x7fc0 computed in integers, and against torch's CPU conversion on a
    sample of every chunk (non-NaN inputs: torch's own NaN patterns differ
    between its scalar conversion, 0x7fc0, and its vectorised one, 0xffff)."""
    rows, n = 1 << 16, 1 << 12
    chunk = rows * n
    for base in range(0, 1 << 32, chunk):
        u = torch.arange(base, base + chunk, device=DEV, dtype=torch.int64)
        p = u.to(torch.int32).view(torch.float32)
        out = linear.reduce(p.view(1, rows, n)).view(-1).view(torch.int16).to(torch.int64) & 0xFFFF
        rne = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
        exp = torch.where(torch.isnan(p), torch.full_like(u, 0x7FC0), rne & 0xFFFF)
        exp = torch.where(u == 0x80000000, torch.zeros_like(exp), exp)
        assert torch.equal(out, exp), hex(base)
        idx = torch.randint(0, chunk, (1 << 16,), device=DEV)
        sample = p[idx].cpu()
        got = out[idx].cpu()
        ref = sample.to(torch.bfloat16).view(torch.int16).to(torch.int64) & 0xFFFF
        ref = torch.where(sample.view(torch.int32) == -0x80000000, torch.zeros_like(ref), ref)
        nan = torch.isnan(sample)
        assert torch.equal(got[~nan], ref[~nan]), hex(base)
        assert bool((got[nan] == 0x7FC0).all()), hex(base)


@pytest.mark.parametrize("b,hq,hkv,cap,attn_splits,qkv_splits", [
    (64, 24, 8, 1280, 1, 3), (5, 24, 8, 1024, 4, 3), (100, 16, 8, 300, 1, 2), (33, 24, 8, 512, 2, 3)])
@torch.inference_mode()
def test_flash_decode_qkv_frag_output_equals_row_major(b, hq, hkv, cap, attn_splits, qkv_splits):
    part, cos_sin, pos = _qkv_case(b, hq, hkv, cap, qkv_splits, 3 * b + cap)
    used = (pos + 1).to(torch.int32)
    cfg = ModelConfig(num_key_value_heads=hkv, hidden_size=hq * 64, num_attention_heads=hq, num_hidden_layers=1)
    caches = [KVCache(cfg, b, cap, DEV, torch.bfloat16) for _ in range(2)]
    caches[0].k.normal_()
    caches[0].v.normal_()
    caches[1].k.copy_(caches[0].k)
    caches[1].v.copy_(caches[0].v)
    fd = flash_decode.FlashDecode(b, hkv, hq // hkv, cap, DEV, num_splits=attn_splits)
    exp = fd.fused_qkv(part, cos_sin, pos, None, caches[0].k[0], caches[0].v[0], 0.125, used, hq)
    got = fd.fused_qkv(part, cos_sin, pos, None, caches[1].k[0], caches[1].v[0], 0.125, used, hq, frag_out=True)
    assert isinstance(got, linear.FragRows) and (got.rows, got.cols) == (b, hq * 64)
    assert torch.equal(got.to_rows(), exp.view(b, -1))
    assert torch.equal(caches[1].k, caches[0].k) and torch.equal(caches[1].v, caches[0].v)
    # o_proj reads it as it reads the row-major output
    wo = bf((hq * 64, hq * 64), 0.02, 11).to(DEV)
    splits = linear.pick_splits(b, hq * 64, hq * 64, max_splits=4)
    assert torch.equal(linear.linear_splitk_frag(got, wo, splits), linear.linear_splitk(exp.view(b, -1), wo, splits))
