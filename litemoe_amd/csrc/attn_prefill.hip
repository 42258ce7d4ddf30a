// Packed variable-length (causal) attention on MFMA, head_dim 64.
//
// Workgroup (query block of 64, q head, sequence); wave w owns 16 queries.
// Keys stream in tiles of 32 staged through LDS (K row-major, V transposed).
// Scores are computed transposed, S^T = K . Q^T, so each lane's C fragment
// (keys 16h + 4*(l/16) + i, query l%16) is directly the A operand of P . V:
// the eight keys a lane holds become the eight k slots of one
// v_mfma_f32_16x16x32_bf16, and V^T in LDS supplies the matching B slots.
// Online softmax (fp32) per query; P is rounded to bf16 for the MFMA.
//
// Reference semantics: litemoe/packed.py:12-16 (aten varlen flash attention,
// causal, q and k share cu_seqlens).
#include "common.h"

namespace lm {
namespace {

constexpr int kD = 64;
constexpr int kThreads = 256;
constexpr int kBQ = 64;
constexpr int kBK = 32;
constexpr int kKPad = 8;
constexpr int kVPad = 8;

__device__ __forceinline__ float factor(float m, float mnew) {
  return m == -INFINITY ? 0.f : __expf(m - mnew);
}

__global__ void __launch_bounds__(kThreads)
prefill_kernel(const bf16 *__restrict__ q, int64_t qs0, int64_t qs1, const bf16 *__restrict__ k,
               int64_t ks0, int64_t ks1, const bf16 *__restrict__ v, int64_t vs0, int64_t vs1,
               const int32_t *__restrict__ cu, int q_heads, int kv_heads, float scale, int causal,
               bf16 *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) bf16 ks_lds[kBK][kD + kKPad];
  __shared__ __attribute__((aligned(16))) bf16 vt_lds[kD][kBK + kVPad];
  const int qb = blockIdx.x, hq = blockIdx.y, seq = blockIdx.z;
  const int start = cu[seq];
  const int len = cu[seq + 1] - start;
  const int q0 = qb * kBQ;
  if (q0 >= len) return;
  const int hk = hq / (q_heads / kv_heads);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  const int wq0 = q0 + wave * 16;
  const int qi = wq0 + col;  // this lane's query (softmax state owner)

  u32x4 qf0 = {0u, 0u, 0u, 0u}, qf1 = {0u, 0u, 0u, 0u};
  if (qi < len) {
    const bf16 *qp = q + (int64_t)(start + qi) * qs0 + (int64_t)hq * qs1 + grp * 8;
    qf0 = *reinterpret_cast<const u32x4 *>(qp);
    qf1 = *reinterpret_cast<const u32x4 *>(qp + 32);
  }
  float m = -INFINITY, l = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kend = causal ? min(len, q0 + kBQ) : len;
  const bool wave_live = wq0 < len;
  const int skey = threadIdx.x / 8, sdc = threadIdx.x % 8;
  for (int kt = 0; kt < kend; kt += kBK) {
    u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
    if (kt + skey < len) {
      const int64_t row = start + kt + skey;
      kv = *reinterpret_cast<const u32x4 *>(k + row * ks0 + (int64_t)hk * ks1 + sdc * 8);
      vv = *reinterpret_cast<const u32x4 *>(v + row * vs0 + (int64_t)hk * vs1 + sdc * 8);
    }
    __syncthreads();
    *reinterpret_cast<u32x4 *>(&ks_lds[skey][sdc * 8]) = kv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vt_lds[sdc * 8 + 2 * i][skey] = (bf16)(vv[i] & 0xffffu);
      vt_lds[sdc * 8 + 2 * i + 1][skey] = (bf16)(vv[i] >> 16);
    }
    __syncthreads();
    if (!wave_live || (causal && kt > wq0 + 15)) continue;
    f32x4 st[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 a0 = *reinterpret_cast<const u32x4 *>(&ks_lds[16 * h + col][grp * 8]);
      const u32x4 a1 = *reinterpret_cast<const u32x4 *>(&ks_lds[16 * h + col][32 + grp * 8]);
      st[h] = mfma16x16x32(a0, qf0, f32x4{0.f, 0.f, 0.f, 0.f});
      st[h] = mfma16x16x32(a1, qf1, st[h]);
    }
    float s[2][4];
    float mt = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = kt + 16 * h + grp * 4 + i;
        const bool masked = j >= len || (causal && j > qi);
        s[h][i] = masked ? -INFINITY : st[h][i] * scale;
        mt = fmaxf(mt, s[h][i]);
      }
    mt = fmaxf(mt, shfl_xor(mt, 16));
    mt = fmaxf(mt, shfl_xor(mt, 32));
    const float mn = fmaxf(m, mt);
    const float corr = factor(m, mn);
    float rs = 0.f;
    uint32_t pw[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = s[h][i] == -INFINITY ? 0.f : __expf(s[h][i] - mn);
        rs += p[i];
      }
      pw[2 * h] = pack_bf16(p[0], p[1]);
      pw[2 * h + 1] = pack_bf16(p[2], p[3]);
    }
    rs += shfl_xor(rs, 16);
    rs += shfl_xor(rs, 32);
    l = l * corr + rs;
    m = mn;
    const u32x4 pa = {pw[0], pw[1], pw[2], pw[3]};
    // O rows held by this lane are queries 4*grp + i of the wave.
    float rc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rc[i] = __shfl(corr, grp * 4 + i, kWave);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[d][i] *= rc[i];
      const bf16 *vr = &vt_lds[d * 16 + col][0];
      const uint2 lo = *reinterpret_cast<const uint2 *>(vr + grp * 4);
      const uint2 hi = *reinterpret_cast<const uint2 *>(vr + 16 + grp * 4);
      const u32x4 vb = {lo.x, lo.y, hi.x, hi.y};
      o[d] = mfma16x16x32(pa, vb, o[d]);
    }
  }
  if (!wave_live) return;
  float rl[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) rl[i] = __shfl(l, grp * 4 + i, kWave);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int qq = wq0 + grp * 4 + i;
    if (qq >= len) continue;
    bf16 *op = out + ((int64_t)(start + qq) * q_heads + hq) * kD;
#pragma unroll
    for (int d = 0; d < 4; ++d)
      op[d * 16 + col] = (bf16)f32_to_bf16(rl[i] > 0.f ? o[d][i] / rl[i] : 0.f);
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
  const dim3 grid((unsigned)cdiv(max_len, kBQ), (unsigned)q_heads, (unsigned)num_seqs);
  prefill_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(
      (const bf16 *)q, qs0, qs1, (const bf16 *)k, ks0, ks1, (const bf16 *)v, vs0, vs1, cu_seqlens,
      (int)q_heads, (int)kv_heads, scale, causal, (bf16 *)out);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
