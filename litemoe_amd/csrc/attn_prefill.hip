// Packed variable-length (causal) attention on MFMA, head_dim 64.
//
// Workgroup (query block of 128, q head, sequence); wave w owns two 16-query
// sub-blocks. Keys stream in tiles of 64 through two LDS stages, K and V both
// row-major, copied straight from global memory (global_load_lds_dwordx4)
// into one stage while the other is computed.
// Scores are computed transposed, S^T = K . Q^T, so each lane's C fragment
// (keys 16h + 4*(l/16) + i, query l%16) is directly the A operand of P . V:
// the eight keys a lane holds become the eight k slots of one
// v_mfma_f32_16x16x32_bf16. The matching B slots (four keys of one channel
// per 64-bit half) come from row-major V through gfx950's transposing LDS
// read, ds_read_b64_tr_b16: within each 16-lane group, lanes 4j..4j+3 point
// at 16 consecutive channels of key row j, and lane p receives channel p of
// rows 0..3. Online softmax (fp32, exp2 with the scale folded in) per query;
// P is rounded to bf16 for the MFMA. The row sum l is a fifth P.V product with
// an all-ones V block (the sum of the same bf16 P that O accumulates, in O's
// lane layout), and the running maximum moves only when a tile raises it by
// more than kLazy (log2 units): until then p <= 2^kLazy, which bf16 P and the
// fp32 sums carry as exactly as p <= 1, and O is not rescaled.
//
// Reference semantics: litemoe/packed.py:12-16 (aten varlen flash attention,
// causal, q and k share cu_seqlens).
#include "common.h"

namespace lm {
namespace {

constexpr int kD = 64;
constexpr int kThreads = 256;
constexpr int kBK = 64;
constexpr int kRowBytes = kD * 2;  // one key row in LDS (no padding: rows are XOR-swizzled)
constexpr float kLazy = 8.f;
constexpr uint32_t kOnes = 0x3F803F80u;  // two bf16 1.0

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

// Scores and running maxima in log2 units: scale * log2(e) is folded into
// the q.k product, so each exponential is one v_exp_f32.
__device__ __forceinline__ float factor(float m, float mnew) {
  return m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
}

// Four bf16 of one channel from four key rows (see the header).
__device__ __forceinline__ uint2 read_tr(const bf16 *p) {
  const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4 *)p);
  return uint2{(uint32_t)(uint16_t)r[0] | ((uint32_t)(uint16_t)r[1] << 16),
               (uint32_t)(uint16_t)r[2] | ((uint32_t)(uint16_t)r[3] << 16)};
}

// kQS 16-query sub-blocks per wave (kBQ = 64 * kQS queries per workgroup):
// every K fragment and transposed V read feeds kQS MFMAs, and the sub-blocks'
// softmax chains are independent, so a wave has kQS chains to interleave.
// Per query the arithmetic is the same for every kQS (a tile that is fully
// masked for one sub-block adds exact zeros to its state).
template <int kQS>
// Four waves per SIMD (<= 128 registers). With the K/V tiles staged through
// registers the Q fragments had to live in LDS to fit (0.350 -> 0.328 ms per
// layer at cfg 4 against three waves); the direct copies free those
// registers, so Q is back in registers, and the second LDS stage takes Q's
// LDS: 0.311 -> 0.282 ms per layer at cfg 4.
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
prefill_kernel(const bf16 *__restrict__ q, int64_t qs0, int64_t qs1, const bf16 *__restrict__ k,
               int64_t ks0, int64_t ks1, const bf16 *__restrict__ v, int64_t vs0, int64_t vs1,
               const int32_t *__restrict__ cu, int q_heads, int kv_heads, float scale, int causal,
               bf16 *__restrict__ out) {
  constexpr int kBQ = 64 * kQS;
  // Two stages of one key tile each: K rows (64 x 128 bytes) then V rows,
  // filled by direct global -> LDS copies. 16-byte chunk c of K row r sits at
  // c ^ (r & 7) (the 8 rows of a fragment read hit 8 different bank groups);
  // of V row r at c ^ 2(r & 3) (the 4 rows of one transposing read group hit
  // 4 different 32-byte bank groups).
  __shared__ __attribute__((aligned(16))) char kv_lds[2][2 * kBK * kRowBytes];
  const int qb = blockIdx.x, hq = blockIdx.y, seq = blockIdx.z;
  const int start = cu[seq];
  const int len = cu[seq + 1] - start;
  const int q0 = qb * kBQ;
  if (q0 >= len) return;
  const int hk = hq / (q_heads / kv_heads);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  const int wq0 = q0 + wave * 16 * kQS;  // the wave's first query
  const float sl2 = scale * 1.4426950408889634f;

  // Sub-block qs: queries wq0 + 16 qs + (0..15); lane col owns query
  // wq0 + 16 qs + col's softmax state and holds its Q fragments.
  float m[kQS];
  f32x4 o[kQS][4], lsum[kQS];  // lsum: C layout of o, every column the row sum
  u32x4 qf0[kQS], qf1[kQS];
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs) {
    const int qi = wq0 + 16 * qs + col;
    qf0[qs] = u32x4{0u, 0u, 0u, 0u};
    qf1[qs] = qf0[qs];
    if (qi < len) {
      const bf16 *qp = q + (int64_t)(start + qi) * qs0 + (int64_t)hq * qs1 + grp * 8;
      qf0[qs] = *reinterpret_cast<const u32x4 *>(qp);
      qf1[qs] = *reinterpret_cast<const u32x4 *>(qp + 32);
    }
    m[qs] = -INFINITY;
    lsum[qs] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < 4; ++d) o[qs][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int kend = causal ? min(len, q0 + kBQ) : len;
  const bool wave_live = wq0 < len;
  // Copy instruction i of wave w fills LDS rows 8*(2w+i) .. +7 of the K (V)
  // tile: lane l writes row 8*(2w+i) + l/8 at position l%8, so it fetches
  // the chunk that position holds. Keys past the sequence repeat its last
  // key (finite values; their scores are masked). Byte offsets from the
  // tile's first key stay below 64 row strides.
  const uint32_t uw = __builtin_amdgcn_readfirstlane(wave);
  const int crow = lane / 8;  // row within the 8-row group; (row & 7) == crow
  const int kchunk = (lane % 8) ^ crow, vchunk = (lane % 8) ^ (2 * (crow & 3));
  const bf16 *kseq = k + (int64_t)start * ks0 + (int64_t)hk * ks1;
  const bf16 *vseq = v + (int64_t)start * vs0 + (int64_t)hk * vs1;
  auto issue = [&](int kt, int stage) {
    const bf16 *kb = kseq + (int64_t)kt * ks0, *vb = vseq + (int64_t)kt * vs0;
    const uint32_t lk = lds_address(kv_lds[stage]) + uw * 2 * 1024, lv = lk + kBK * kRowBytes;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = min(8 * (2 * wave + i) + crow, len - 1 - kt);
      lds_copy16(kb, (uint32_t)(row * ks0 + kchunk * 8) * 2, lk + i * 1024);
      lds_copy16(vb, (uint32_t)(row * vs0 + vchunk * 8) * 2, lv + i * 1024);
    }
  };
  // Transposing-read addresses: lane 16g + 4j + t reads channels 4t..4t+3
  // (plus 16 per channel block) of key row 4g + j (slots 0-3) or
  // 16 + 4g + j (slots 4-7), matching the keys of the P fragment. Channel
  // block d's bytes of that row are chunk 2d + t/2, offset 8 (t & 1).
  const int trow = 4 * grp + (col / 4), tsub = (col % 4) / 2, toff = 8 * (col & 1);
  int it = 0;
  issue(0, 0);
  for (int kt = 0; kt < kend; kt += kBK, ++it) {
    // Tile it has landed in every wave, and every wave has left tile it - 1,
    // whose stage the next copy overwrites.
    lds_copy_wait();
    __syncthreads();
    if (kt + kBK < kend) issue(kt + kBK, (it + 1) & 1);
    if (!wave_live || (causal && kt > wq0 + 16 * kQS - 1)) continue;
    const char *ks = kv_lds[it & 1];
    const char *vs = ks + kBK * kRowBytes;
    constexpr int kH = kBK / 16;  // 16-key blocks of the tile
    f32x4 st[kQS][kH];
#pragma unroll
    for (int h = 0; h < kH; ++h) {
      const char *krow = ks + (16 * h + col) * kRowBytes;
      const u32x4 a0 = *reinterpret_cast<const u32x4 *>(krow + ((grp ^ (col & 7)) << 4));
      const u32x4 a1 = *reinterpret_cast<const u32x4 *>(krow + (((4 + grp) ^ (col & 7)) << 4));
#pragma unroll
      for (int qs = 0; qs < kQS; ++qs) {
        st[qs][h] = mfma16x16x32(a0, qf0[qs], f32x4{0.f, 0.f, 0.f, 0.f});
        st[qs][h] = mfma16x16x32(a1, qf1[qs], st[qs][h]);
      }
    }
    // Only a tile crossing the causal diagonal of this wave's queries, or the
    // sequence's last tile, has masked scores. Key j = kt + 16h + 4grp + i
    // against query q = wq0 + 16qs + col: j - q = base + 16(h - qs) + i.
    if (causal && kt + kBK - 1 > wq0) {
      const int base = kt - wq0 + 4 * grp - col;
#pragma unroll
      for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
        for (int h = 0; h < kH; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (base + 16 * (h - qs) + i > 0) st[qs][h][i] = -INFINITY;
    }
    if (kt + kBK > len) {
      const int room = len - kt - 4 * grp;  // j < len  <=>  16h + i < room
#pragma unroll
      for (int qs = 0; qs < kQS; ++qs)
#pragma unroll
        for (int h = 0; h < kH; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (16 * h + i >= room) st[qs][h][i] = -INFINITY;
    }
    uint32_t pw[kQS][2 * kH];
#pragma unroll
    for (int qs = 0; qs < kQS; ++qs) {
      // The maximum is taken on the raw dot products (the scale is
      // positive), and exp2(s * scale*log2e - m) is one FMA and one v_exp_f32.
      float mt = -INFINITY;
#pragma unroll
      for (int h = 0; h < kH; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) mt = fmaxf(mt, st[qs][h][i]);
      mt = fmaxf(mt, xor_lanes<16>(mt));  // the four lane groups hold a query's keys
      mt = fmaxf(mt, xor_lanes<32>(mt));
      // The first tile always sets the maximum (m = -inf; key 0 is visible to
      // every query); a tile fully masked for a query has mt = -inf and keeps it.
      const float cand = mt * sl2;
      const bool raise = cand > m[qs] + kLazy;
      if (__ballot(raise)) {
        const float mn = raise ? cand : m[qs];
        const float corr = factor(m[qs], mn);  // 1 for the queries that keep theirs
        m[qs] = mn;
        // O and lsum rows held by this lane are queries 4*grp + i
        float rc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) rc[i] = __shfl(corr, grp * 4 + i, kWave);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lsum[qs][i] *= rc[i];
#pragma unroll
          for (int d = 0; d < 4; ++d) o[qs][d][i] *= rc[i];
        }
      }
      const float mq = m[qs];  // finite from the first tile on
#pragma unroll
      for (int h = 0; h < kH; ++h) {
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[qs][h][i], sl2, -mq));  // exp2(-inf) = 0
        pw[qs][2 * h] = pack_bf16_finite(p[0], p[1]);  // p = exp2(finite or -inf): never NaN
        pw[qs][2 * h + 1] = pack_bf16_finite(p[2], p[3]);
      }
    }
    // Each 32 keys of the tile are one P.V step: keys 32c + (the two
    // 16-key blocks' rows) as the eight k slots.
    constexpr u32x4 kOnesB = {kOnes, kOnes, kOnes, kOnes};
#pragma unroll
    for (int c = 0; c < kBK / 32; ++c) {
#pragma unroll
      for (int qs = 0; qs < kQS; ++qs) {
        const u32x4 pa = {pw[qs][4 * c], pw[qs][4 * c + 1], pw[qs][4 * c + 2], pw[qs][4 * c + 3]};
        lsum[qs] = mfma16x16x32(pa, kOnesB, lsum[qs]);
      }
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int r0 = 32 * c + trow, r1 = r0 + 16;  // (r & 3) == (col / 4) for both
        const int pos = ((2 * d + tsub) ^ (2 * (col / 4))) << 4;
        const uint2 lo = read_tr(reinterpret_cast<const bf16 *>(vs + r0 * kRowBytes + pos + toff));
        const uint2 hi = read_tr(reinterpret_cast<const bf16 *>(vs + r1 * kRowBytes + pos + toff));
        const u32x4 vb = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int qs = 0; qs < kQS; ++qs) {
          const u32x4 pa = {pw[qs][4 * c], pw[qs][4 * c + 1], pw[qs][4 * c + 2], pw[qs][4 * c + 3]};
          o[qs][d] = mfma16x16x32(pa, vb, o[qs][d]);
        }
      }
    }
  }
  if (!wave_live) return;
  // O / l, written through the wave's own Q staging area (2 KB per sub-block:
  // its 16 * kQS output rows of 128 bytes; only this wave uses it, and the
  // fence below keeps its last Q reads ahead of these writes), then read back
  // row-contiguous so every row leaves as eight 16-byte stores instead of 64
  // 2-byte ones. The 16-byte chunk c of row r sits at c ^ 2((r / 4) % 4): the
  // four lane groups of one write (rows 4 apart) then hit different banks.
  // l >= 1 for every query that has a key (its maximum key has p >= 1), and
  // the reciprocal (within one ulp) times O replaces a division per output.
  // The stage the last tile did not use: every wave left it at the barrier
  // of the last tile, and no copy targets it. 4 KB per wave.
  uint16_t *tile = reinterpret_cast<uint16_t *>(kv_lds[it & 1] + wave * (16 * kQS * kD * 2));
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
  for (int qs = 0; qs < kQS; ++qs) {
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = lsum[qs][i] > 0.f ? __builtin_amdgcn_rcpf(lsum[qs][i]) : 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int chunk = (2 * d + col / 8) ^ (2 * grp);  // rows 16 qs + 4 grp + i: (r / 4) % 4 = grp
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const uint32_t w = pack_bf16(o[qs][d][i] * r[i], o[qs][d][i + 1] * r[i + 1]);
        const int at = (16 * qs + 4 * grp + i) * 64 + chunk * 8 + col % 8;
        tile[at] = (uint16_t)w;
        tile[at + 64] = (uint16_t)(w >> 16);
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  const u32x4 *rows = reinterpret_cast<const u32x4 *>(tile);
#pragma unroll
  for (int j = 0; j < 2 * kQS; ++j) {
    const int row = 8 * j + lane / 8, c = lane % 8;
    const u32x4 val = rows[row * 8 + (c ^ (2 * ((row / 4) % 4)))];
    if (wq0 + row < len)
      *reinterpret_cast<u32x4 *>(out + ((int64_t)(start + wq0 + row) * q_heads + hq) * kD + c * 8) = val;
  }
}

}  // namespace
}  // namespace lm

using namespace lm;

extern "C" int lm_prefill_attention(const void *q, int64_t qs0, int64_t qs1, const void *k,
                                    int64_t ks0, int64_t ks1, const void *v, int64_t vs0,
                                    int64_t vs1, const int32_t *cu_seqlens, int64_t num_seqs,
                                    int64_t tokens, int64_t max_len, int64_t q_heads,
                                    int64_t kv_heads, int64_t head_dim, float scale, int causal,
                                    void *out, void *stream) {
  LM_REQUIRE(num_seqs >= 0 && tokens >= 0 && max_len >= 0 && q_heads > 0 && kv_heads > 0 &&
             q_heads % kv_heads == 0 && num_seqs < 65536 && q_heads < 65536);
  if (head_dim != kD) return LM_EUNSUPPORTED;
  if (num_seqs == 0 || tokens == 0 || max_len == 0) return LM_OK;
  LM_REQUIRE(q && k && v && cu_seqlens && out);
  // 16-byte loads of q/k/v rows and 16-byte stores of output rows.
  const auto aligned = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
  LM_REQUIRE(aligned(q) && aligned(k) && aligned(v) && aligned(out));
  LM_REQUIRE(qs0 % 8 == 0 && qs1 % 8 == 0 && ks0 % 8 == 0 && ks1 % 8 == 0 && vs0 % 8 == 0 &&
             vs1 % 8 == 0);
// Two sub-blocks per wave: 0.46 -> 0.41 ms per layer at cfg 4 with the
// accumulators in VGPRs (built that way); in the AGPR form the second
// sub-block costs occupancy and is slower than one.
#ifndef LM_PREFILL_QSUB
#define LM_PREFILL_QSUB 2
#endif
  constexpr int kQS = LM_PREFILL_QSUB;
  const dim3 grid((unsigned)cdiv(max_len, 64 * kQS), (unsigned)q_heads, (unsigned)num_seqs);
  prefill_kernel<kQS><<<grid, kThreads, 0, (hipStream_t)stream>>>(
      (const bf16 *)q, qs0, qs1, (const bf16 *)k, ks0, ks1, (const bf16 *)v, vs0, vs1, cu_seqlens,
      (int)q_heads, (int)kv_heads, scale, causal, (bf16 *)out);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
