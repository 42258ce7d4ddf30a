// Fused router (gate GEMV -> top-k -> softmax) and the deterministic
// expert-sorted route permutation.
//
// Selection rule: ids are the k largest bf16 logits in descending order,
// equal logits ordered by ascending expert id (a stable descending sort).
// Weights follow vLLM fused_topk / HF GraniteMoeTopKRouter: softmax over the
// k selected logits (renormalize) or over all E logits.
// References: litemoe/model.py:110-118, ops.py:7-12, ops.py:163-173.
#include "internal.h"

namespace lm {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / kWave;
constexpr int kMaxExperts = 256;  // one selecting thread per expert
constexpr int kMaxTopk = 16;
constexpr int kMaxNormVec = 2;    // hidden <= kMaxNormVec * 8 * kRouterThreads
constexpr int kExpertBatch = 5;   // experts whose weight loads one wave keeps in flight

// Monotone map float -> uint32 (NaN canonicalised above +inf, as torch.topk
// orders NaN first), combined with the inverted expert id so that a larger
// 64-bit key means a larger value or, for equal values, a lower id.
__device__ __forceinline__ uint64_t select_key(float v, int e) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) u = 0x7fc00000u;
  const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}

// logit[e] = bf16(z . W_r[e]) for all experts; z (nvec 16-byte words) is in
// LDS. Wave w takes experts w, w+4, ... in batches of kExpertBatch whose
// weight loads are issued together.
__device__ void router_gemv(const u32x4 *zs, const bf16 *__restrict__ wr, int nvec, int experts,
                            float *logit, bf16 *__restrict__ logits_row) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int per_wave = (experts - wave + kRouterWaves - 1) / kRouterWaves;
  for (int j0 = 0; j0 < per_wave; j0 += kExpertBatch) {
    float acc[kExpertBatch];
#pragma unroll
    for (int b = 0; b < kExpertBatch; ++b) acc[b] = 0.f;
    for (int i = lane; i < nvec; i += kWave) {
      const u32x4 zw = zs[i];
      u32x4 w[kExpertBatch];
#pragma unroll
      for (int b = 0; b < kExpertBatch; ++b) {
        const int e = wave + (j0 + b) * kRouterWaves;
        const int ee = e < experts ? e : wave;
        w[b] = reinterpret_cast<const u32x4 *>(wr + (int64_t)ee * nvec * 8)[i];
      }
#pragma unroll
      for (int b = 0; b < kExpertBatch; ++b) acc[b] = dot8_bf16_acc(zw, w[b], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < kExpertBatch; ++b) {
      const int e = wave + (j0 + b) * kRouterWaves;
      const float sum = wave_sum(acc[b]);
      if (lane == 0 && e < experts) {
        const uint32_t h = f32_to_bf16(sum);
        logit[e] = bf16_to_f32(h);
        if (logits_row) logits_row[e] = (bf16)h;
      }
    }
  }
}

// `renormalize` flags: bit 0, softmax over the selection (else over every
// logit); bit 1 (kIdOrder), each token's selection written in ascending
// expert id instead of descending logit (the same experts and weights; the
// denominator is summed in rank order either way).
constexpr int kIdOrder = 2;

// Top-k by rank: thread t (one per expert) counts the experts with a larger
// key; ranks are distinct, so rank < topk places expert t at that position.
// Weights: softmax over the selection (renormalize) or over all logits,
// with the denominator summed in a fixed order. Synchronises.
__device__ void select_topk(const float *logit, int experts, int topk, int renormalize,
                            float *sel_val, int *sel_id, float *__restrict__ tw,
                            int32_t *__restrict__ tid) {
  const int t = threadIdx.x;
  if (t < experts) {
    const uint64_t mine = select_key(logit[t], t);
    int rank = 0;
    for (int e = 0; e < experts; ++e) rank += select_key(logit[e], e) > mine;
    if (rank < topk) {
      sel_val[rank] = logit[t];
      sel_id[rank] = t;
    }
  }
  __syncthreads();
  if (t < topk) {
    const float m = sel_val[0];
    float denom = 0.f;
    if (renormalize & 1) {
      for (int j = 0; j < topk; ++j) denom += expf(sel_val[j] - m);
    } else {
      for (int e = 0; e < experts; ++e) denom += expf(logit[e] - m);
    }
    int pos = t;
    if (renormalize & kIdOrder) {
      pos = 0;
      for (int j = 0; j < topk; ++j) pos += sel_id[j] < sel_id[t];
    }
    tw[pos] = expf(sel_val[t] - m) / denom;
    tid[pos] = sel_id[t];
  }
}

// select_topk for experts <= 64, run by wave 0 alone with no barrier: logits
// are bf16, so (orderable bf16 bits, ~id) fits a 32-bit key, distinct per
// expert. Lane e holds expert e's key; rank r goes to the lane holding the
// wave's largest remaining key (a DPP maximum within rows of 16, then the
// four row maxima as scalars), which then drops out: topk rounds of register
// work, no LDS traffic. The softmax terms of the selection are summed in
// rank order through LDS. logit[kWave, 3*kWave) is scratch. The selection,
// the weights and the order of the softmax denominator's sum are those of
// select_topk. The caller synchronises before (logits in LDS).
// select_topk_lanes is the same selection for any one wave of the
// workgroup, with its own 2*kWave floats of LDS scratch.
__device__ __forceinline__ uint32_t select_key32(float v, int id) {
  uint32_t h = __float_as_uint(v) >> 16;  // exact: logits are bf16 values
  if ((h & 0x7fffu) > 0x7f80u) h = 0x7fc0u;
  const uint32_t ord = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
  return (ord << 16) | (0xffffu - (uint32_t)id);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));
  return max(max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16)),
             max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48)));
}

__device__ void select_topk_lanes(const float *logit, float *scratch, int t, int experts,
                                  int topk, int renormalize, float *__restrict__ tw,
                                  int32_t *__restrict__ tid) {
  const float v = logit[min(t, experts - 1)];
  uint32_t key = t < experts ? select_key32(v, t) : 0u;  // 0: below every real key
  float *terms = scratch + kWave;
  int rank = kWave;  // not selected
  for (int r = 0; r < topk; ++r) {
    const uint32_t top_key = wave_max_u32(key);
    if (key == top_key) {  // exactly one lane: keys are distinct
      rank = r;
      key = 0u;
    }
  }
  const int top = __builtin_ctzll(__ballot(rank == 0));
  const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), top));
  const float ex = expf(v - m);
  float denom = 0.f;
  if (renormalize & 1) {
    if (rank < topk) terms[rank] = ex;
#pragma unroll
    for (int r4 = 0; r4 < kMaxTopk / 4; ++r4) {
      const float4 t4 = *reinterpret_cast<const float4 *>(terms + 4 * r4);
      const float tv[4] = {t4.x, t4.y, t4.z, t4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) denom += 4 * r4 + i < topk ? tv[i] : 0.f;
    }
  } else {
    if (t < experts) terms[t] = ex;
#pragma unroll
    for (int e4 = 0; e4 < kWave / 4; ++e4) {
      const float4 t4 = *reinterpret_cast<const float4 *>(terms + 4 * e4);
      const float tv[4] = {t4.x, t4.y, t4.z, t4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) denom += 4 * e4 + i < experts ? tv[i] : 0.f;
    }
  }
  // kIdOrder: lane t's place among the selected lanes below it.
  const uint64_t chosen = __ballot(rank < topk);
  const int pos = (renormalize & kIdOrder) ? __popcll(chosen & ((1ull << t) - 1ull)) : rank;
  if (rank < topk) {
    tw[pos] = ex / denom;
    tid[pos] = t;
  }
}

__device__ __forceinline__ void select_topk_wave(float *logit, int experts, int topk,
                                                 int renormalize, float *__restrict__ tw,
                                                 int32_t *__restrict__ tid) {
  if (threadIdx.x >= kWave) return;
  select_topk_lanes(logit, logit + kWave, threadIdx.x, experts, topk, renormalize, tw, tid);
}

// Both selections end with the outputs written; neither needs a barrier
// after it.
__device__ __forceinline__ void select(float *logit, int experts, int topk, int renormalize,
                                       float *sel_val, int *sel_id, float *__restrict__ tw,
                                       int32_t *__restrict__ tid) {
  if (experts <= kWave)
    select_topk_wave(logit, experts, topk, renormalize, tw, tid);
  else
    select_topk(logit, experts, topk, renormalize, sel_val, sel_id, tw, tid);
}

// One workgroup per token: stage the row in LDS, GEMV, select.
__global__ void __launch_bounds__(kRouterThreads)
router_kernel(const bf16 *__restrict__ x, const bf16 *__restrict__ wr, int hidden, int experts,
              int topk, int renormalize, bf16 *__restrict__ logits_out, float *__restrict__ tw,
              int32_t *__restrict__ tid) {
  __shared__ u32x4 zs[kMaxNormVec * kRouterThreads];
  __shared__ __align__(16) float logit[kMaxExperts];
  __shared__ float sel_val[kMaxTopk];
  __shared__ int sel_id[kMaxTopk];
  const int64_t row = blockIdx.x;
  const int nvec = hidden / 8;
  for (int i = threadIdx.x; i < nvec; i += kRouterThreads)
    zs[i] = reinterpret_cast<const u32x4 *>(x + row * hidden)[i];
  __syncthreads();
  router_gemv(zs, wr, nvec, experts, logit, logits_out ? logits_out + row * experts : nullptr);
  __syncthreads();
  select(logit, experts, topk, renormalize, sel_val, sel_id, tw + row * topk, tid + row * topk);
}

__global__ void __launch_bounds__(kRouterThreads)
topk_from_logits_kernel(const bf16 *__restrict__ logits, int experts, int topk, int renormalize,
                        float *__restrict__ tw, int32_t *__restrict__ tid) {
  __shared__ __align__(16) float logit[kMaxExperts];
  __shared__ float sel_val[kMaxTopk];
  __shared__ int sel_id[kMaxTopk];
  const int64_t row = blockIdx.x;
  for (int e = threadIdx.x; e < experts; e += kRouterThreads)
    logit[e] = bf16_to_f32(logits[row * experts + e]);
  __syncthreads();
  select(logit, experts, topk, renormalize, sel_val, sel_id, tw + row * topk, tid + row * topk);
}

// Residual add + RMSNorm + router GEMV + top-k, one workgroup per token.
// The normalised row stays in LDS for the GEMV.
__global__ void __launch_bounds__(kRouterThreads)
add_norm_router_kernel(bf16 *__restrict__ x, const bf16 *__restrict__ a, float alpha,
                       const bf16 *__restrict__ nw, float eps, bf16 *__restrict__ z,
                       const bf16 *__restrict__ wr, int hidden, int experts, int topk,
                       int renormalize, bf16 *__restrict__ logits_out, float *__restrict__ tw,
                       int32_t *__restrict__ tid) {
  __shared__ u32x4 zs[kMaxNormVec * kRouterThreads];
  __shared__ __align__(16) float logit[kMaxExperts];
  __shared__ float red[kRouterWaves];
  __shared__ float sel_val[kMaxTopk];
  __shared__ int sel_id[kMaxTopk];
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int nvec = hidden / 8;
  u32x4 *xr = reinterpret_cast<u32x4 *>(x + row * hidden);
  float xn[kMaxNormVec][8];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < kMaxNormVec; ++v) {
    const int i = threadIdx.x + v * kRouterThreads;
    if (i >= nvec) continue;
    unpack8(xr[i], xn[v]);
    if (a) {
      float g[8];
      unpack8(reinterpret_cast<const u32x4 *>(a + row * hidden)[i], g);
      u32x4 o;
#pragma unroll
      for (int c = 0; c < 8; ++c) xn[v][c] = round_bf16(xn[v][c] + alpha * g[c]);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = pack_bf16(xn[v][2 * c], xn[v][2 * c + 1]);
      xr[i] = o;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) ss += xn[v][c] * xn[v][c];
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kRouterWaves; ++w) total += red[w];
  const float scale = 1.0f / sqrtf(total / (float)hidden + eps);
#pragma unroll
  for (int v = 0; v < kMaxNormVec; ++v) {
    const int i = threadIdx.x + v * kRouterThreads;
    if (i >= nvec) continue;
    float g[8];
    unpack8(reinterpret_cast<const u32x4 *>(nw)[i], g);
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = pack_bf16(round_bf16(xn[v][2 * c] * scale) * g[2 * c],
                       round_bf16(xn[v][2 * c + 1] * scale) * g[2 * c + 1]);
    zs[i] = o;
    reinterpret_cast<u32x4 *>(z + row * hidden)[i] = o;
  }
  __syncthreads();
  router_gemv(zs, wr, nvec, experts, logit, logits_out ? logits_out + row * experts : nullptr);
  __syncthreads();
  select(logit, experts, topk, renormalize, sel_val, sel_id, tw + row * topk, tid + row * topk);
}

// Latency-bound variant for hidden = 512 * NV: 1024 threads, and every load
// the row needs (the row, the residual, the norm weight and the first round
// of gate rows) is issued at entry, so the kernel waits on memory once.
// The norm runs on the first 256 threads with the reduction order of
// rmsnorm_kernel, and the dot products keep router_gemv's order, so logits
// and z are bitwise those of the unfused kernels.
constexpr int kFastThreads = 1024;
constexpr int kFastWaves = kFastThreads / kWave;

template <int NV>
struct FastRouter {
  static constexpr int kBatch = 12 / NV > 4 ? 4 : (12 / NV < 1 ? 1 : 12 / NV);  // gate rows per wave per round
  static constexpr int kRound = kBatch * kFastWaves;                        // experts per round
  static constexpr int kNvec = NV * kWave;                                  // 16-byte words per row
  static constexpr int kNorm = (kNvec + kRouterThreads - 1) / kRouterThreads;
};

template <int NV>
__device__ __forceinline__ void load_gate_round(const bf16 *__restrict__ wr, int experts, int round,
                                                u32x4 (&w)[FastRouter<NV>::kBatch][NV]) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
  for (int b = 0; b < FastRouter<NV>::kBatch; ++b) {
    const int e = round * FastRouter<NV>::kRound + wave + b * kFastWaves;
    const u32x4 *row = reinterpret_cast<const u32x4 *>(wr) +
                       (int64_t)(e < experts ? e : 0) * FastRouter<NV>::kNvec;
#pragma unroll
    for (int v = 0; v < NV; ++v) w[b][v] = row[lane + v * kWave];
  }
}

template <int NV>
__device__ __forceinline__ void gate_round(const u32x4 *zs, int experts, int round,
                                           const u32x4 (&w)[FastRouter<NV>::kBatch][NV],
                                           float *logit, bf16 *__restrict__ logits_row) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
  for (int b = 0; b < FastRouter<NV>::kBatch; ++b) {
    const int e = round * FastRouter<NV>::kRound + wave + b * kFastWaves;
    if (e >= experts) continue;  // uniform across the wave
    float acc = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v) acc = dot8_bf16_acc(zs[lane + v * kWave], w[b][v], acc);
    const float sum = wave_sum(acc);
    if (lane == 0) {
      const uint32_t h = f32_to_bf16(sum);
      logit[e] = bf16_to_f32(h);
      if (logits_row) logits_row[e] = (bf16)h;
    }
  }
}

constexpr int kMaxResidualSplits = 4;  // partial slices held in VGPRs (128 per lane at 1024 threads)

// kNorm: z = rmsnorm(x [+ alpha*a]) is routed (and x, z are written);
// otherwise x itself is routed. kPart: a is given as fp32 split-K partials
// [asplits][tokens][hidden] (lm_linear_splitk) and a = bf16(sum of slices).
template <int NV, bool kNorm, bool kAdd, bool kPart>
__global__ void __launch_bounds__(kFastThreads)
fast_router_kernel(bf16 *__restrict__ x, const bf16 *__restrict__ a, float alpha,
                   const bf16 *__restrict__ nw, float eps, bf16 *__restrict__ z,
                   const bf16 *__restrict__ wr, int experts, int topk, int renormalize,
                   bf16 *__restrict__ logits_out, float *__restrict__ tw,
                   int32_t *__restrict__ tid, const float *__restrict__ ap, int asplits) {
  typedef FastRouter<NV> F;
  constexpr int nvec = F::kNvec, NN = F::kNorm;
  __shared__ u32x4 zs[nvec];
  __shared__ __align__(16) float logit[kMaxExperts];
  __shared__ float red[kRouterWaves];
  __shared__ float sel_val[kMaxTopk];
  __shared__ int sel_id[kMaxTopk];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const bool norm_wave = t < kRouterThreads;
  u32x4 *xr = reinterpret_cast<u32x4 *>(x + row * nvec * 8);
  const u32x4 *ar = reinterpret_cast<const u32x4 *>(a + row * nvec * 8);
  const u32x4 *gr = reinterpret_cast<const u32x4 *>(nw);
  u32x4 xv[NN], av[NN], gv[NN];
  f32x4 pv[kPart ? NN : 1][kPart ? kMaxResidualSplits : 1][2];
  if (norm_wave) {
#pragma unroll
    for (int v = 0; v < NN; ++v) {
      const int i = min(t + v * kRouterThreads, nvec - 1);
      xv[v] = xr[i];
      if constexpr (kPart) {
        // Unconditional loads (slice index clamped): a load under a branch
        // would make the compiler wait for every load before the first use.
        const f32x4 *src = reinterpret_cast<const f32x4 *>(ap + row * nvec * 8) + 2 * i;
#pragma unroll
        for (int s = 0; s < kMaxResidualSplits; ++s) {
          const int64_t at = (int64_t)min(s, asplits - 1) * gridDim.x * nvec * 2;
          pv[v][s][0] = src[at];
          pv[v][s][1] = src[at + 1];
        }
      } else if constexpr (kAdd) {
        av[v] = ar[i];
      }
      if constexpr (kNorm) gv[v] = gr[i];
    }
  }
  u32x4 w[F::kBatch][NV];
  load_gate_round<NV>(wr, experts, 0, w);
  // Intermediate roundings below skip the NaN fix-up: x and z leave through
  // pack_bf16 (canonical NaN), and z reaches the logits only as those bits.
  float xn[NN][8];
  if (norm_wave) {
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < NN; ++v) {
      const int i = t + v * kRouterThreads;
      if (i >= nvec) continue;
      unpack8(xv[v], xn[v]);
      if constexpr (kAdd) {
        float g[8];
        if constexpr (kPart) {
          f32x4 lo = pv[v][0][0], hi = pv[v][0][1];
#pragma unroll
          for (int s = 1; s < kMaxResidualSplits; ++s) {
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            lo += s < asplits ? pv[v][s][0] : zero;  // + 0 leaves the sum unchanged
            hi += s < asplits ? pv[v][s][1] : zero;
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            g[c] = round_bf16_nc(lo[c]);
            g[4 + c] = round_bf16_nc(hi[c]);
          }
        } else {
          unpack8(av[v], g);
        }
        u32x4 o;
#pragma unroll
        for (int c = 0; c < 8; ++c) xn[v][c] = round_bf16_nc(xn[v][c] + alpha * g[c]);
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = pack_bf16(xn[v][2 * c], xn[v][2 * c + 1]);
        xr[i] = o;
      }
      if constexpr (kNorm) {
#pragma unroll
        for (int c = 0; c < 8; ++c) ss += xn[v][c] * xn[v][c];
      } else {
        zs[i] = xv[v];
      }
    }
    if constexpr (kNorm) {
      ss = wave_sum(ss);
      if (lane == 0) red[wave] = ss;
    }
  }
  if constexpr (kNorm) {
    __syncthreads();
    if (norm_wave) {
      float total = 0.f;
#pragma unroll
      for (int q = 0; q < kRouterWaves; ++q) total += red[q];
      const float scale = 1.0f / sqrtf(total / (float)(nvec * 8) + eps);
      u32x4 *zr = reinterpret_cast<u32x4 *>(z + row * nvec * 8);
#pragma unroll
      for (int v = 0; v < NN; ++v) {
        const int i = t + v * kRouterThreads;
        if (i >= nvec) continue;
        float g[8];
        unpack8(gv[v], g);
        u32x4 o;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          o[c] = pack_bf16(round_bf16_nc(xn[v][2 * c] * scale) * g[2 * c],
                           round_bf16_nc(xn[v][2 * c + 1] * scale) * g[2 * c + 1]);
        zs[i] = o;
        zr[i] = o;
      }
    }
  }
  __syncthreads();
  bf16 *lrow = logits_out ? logits_out + row * experts : nullptr;
  gate_round<NV>(zs, experts, 0, w, logit, lrow);
  for (int round = 1; round * F::kRound < experts; ++round) {
    load_gate_round<NV>(wr, experts, round, w);
    gate_round<NV>(zs, experts, round, w, logit, lrow);
  }
  __syncthreads();
  select(logit, experts, topk, renormalize, sel_val, sel_id, tw + row * topk, tid + row * topk);
}

// hidden = 512 * NV for an instantiated NV, else 0.
int fast_nv(int64_t hidden) {
  if (hidden % 512) return 0;
  const int64_t nv = hidden / 512;
  return (nv == 1 || nv == 2 || nv == 3 || nv == 4 || nv == 6 || nv == 8) ? (int)nv : 0;
}

template <bool kNorm, bool kAdd, bool kPart = false>
void launch_fast_router(int nv, int64_t tokens, bf16 *x, const bf16 *a, float alpha, const bf16 *nw,
                        float eps, bf16 *z, const bf16 *wr, int experts, int topk, int renormalize,
                        bf16 *logits_out, float *tw, int32_t *tid, hipStream_t s,
                        const float *ap = nullptr, int asplits = 0) {
  const dim3 grid((unsigned)tokens);
  switch (nv) {
#define LM_FAST_ROUTER(NV)                                                                     \
  case NV:                                                                                     \
    fast_router_kernel<NV, kNorm, kAdd, kPart><<<grid, kFastThreads, 0, s>>>(                 \
        x, a, alpha, nw, eps, z, wr, experts, topk, renormalize, logits_out, tw, tid, ap,      \
        asplits);                                                                              \
    break;
    LM_FAST_ROUTER(1) LM_FAST_ROUTER(2) LM_FAST_ROUTER(3) LM_FAST_ROUTER(4)
#undef LM_FAST_ROUTER
    // hidden 3072/4096 with fp32 partials would not fit 128 VGPRs per lane
    case 6:
      if constexpr (!kPart)
        fast_router_kernel<6, kNorm, kAdd, false><<<grid, kFastThreads, 0, s>>>(
            x, a, alpha, nw, eps, z, wr, experts, topk, renormalize, logits_out, tw, tid, ap,
            asplits);
      break;
    case 8:
      if constexpr (!kPart)
        fast_router_kernel<8, kNorm, kAdd, false><<<grid, kFastThreads, 0, s>>>(
            x, a, alpha, nw, eps, z, wr, experts, topk, renormalize, logits_out, tw, tid, ap,
            asplits);
      break;
  }
}

// Prefill-sized router: a workgroup of four waves routes kBatchRows = 32
// tokens, for experts <= 64 and hidden = 512 * NVL.
//  1. (kNorm) Wave w normalises tokens 8w..8w+7 in turn, with the next
//     token's loads in flight: lane l holds 16-byte words l + 64i (i < NVL),
//     the words threads l + 64j of rmsnorm_kernel hold (word (l + 64j) +
//     256v for i = j + 4v). The sum of squares is kept per j in that
//     thread's order and reduced by wave_sum per j, then over j in order, so
//     x and z are bitwise the unfused kernels'.
//  2. The 32 rows of z (x when !kNorm) are read back as MFMA A operands, two
//     16-row blocks, and the gate rows as B operands (both from L2), each
//     gate fragment feeding both blocks; wave w accumulates k-steps
//     [w K/4, (w+1) K/4) of the 32 x 16*NT logits with
//     v_mfma_f32_16x16x32_bf16, and the four partial tiles are summed in
//     wave order through LDS and rounded to bf16 (and to logits_out). Per
//     row the accumulation order is that of a 16-row workgroup; 32 rows halve
//     the gate-weight reads (147 KB from L2 per workgroup at the 3B shape):
//     178 -> 155 us per call at 46,990 tokens; 64 rows (two workgroups per
//     CU) 171 us.
//  3. Wave w selects the top-k of tokens 8w..8w+7 (select_topk_lanes).
// The logits accumulate in the matrix core's order rather than
// router_gemv's, so a logit can differ from the GEMV kernels' by one bf16
// ulp (as a BLAS GEMM's order can); the selection is exact given the
// logits. All 32 rows must exist (the caller routes a tail of fewer tokens
// with the per-token kernels).
constexpr int kBatchMB = 2;  // 16-row MFMA blocks per workgroup: each gate fragment feeds kBatchMB
constexpr int kBatchRows = 16 * kBatchMB;
constexpr int kBatchWaves = 4;
constexpr int kBatchThreads = kBatchWaves * kWave;
constexpr int kRowsPerWave = kBatchRows / kBatchWaves;
#ifndef LM_BATCH_ROUTER_MIN_TOKENS
#define LM_BATCH_ROUTER_MIN_TOKENS 1024
#endif
constexpr int64_t kBatchRouterMinTokens = LM_BATCH_ROUTER_MIN_TOKENS;
constexpr int kBatchSteps = 4 / kBatchMB;  // k-steps whose operand loads are issued together

template <int NVL, bool kAdd>
__device__ __forceinline__ void batch_load_row(const bf16 *__restrict__ x,
                                               const bf16 *__restrict__ a, int64_t row,
                                               u32x4 (&xv)[NVL], u32x4 (&av)[NVL]) {
  const int lane = threadIdx.x % kWave;
  const u32x4 *xr = reinterpret_cast<const u32x4 *>(x) + row * NVL * kWave;
  const u32x4 *ar = reinterpret_cast<const u32x4 *>(a) + row * NVL * kWave;
#pragma unroll
  for (int i = 0; i < NVL; ++i) {
    xv[i] = xr[lane + i * kWave];
    if constexpr (kAdd) av[i] = ar[lane + i * kWave];
  }
}

template <int NVL, bool kAdd>
__device__ __forceinline__ void batch_norm_row(bf16 *__restrict__ x, float alpha,
                                               const u32x4 (&gv)[NVL], float eps,
                                               bf16 *__restrict__ z, int64_t row,
                                               const u32x4 (&xv)[NVL], const u32x4 (&av)[NVL]) {
  constexpr int kJ = NVL < kRouterWaves ? NVL : kRouterWaves;
  const int lane = threadIdx.x % kWave;
  u32x4 *xr = reinterpret_cast<u32x4 *>(x) + row * NVL * kWave;
  u32x4 *zr = reinterpret_cast<u32x4 *>(z) + row * NVL * kWave;
  float xn[NVL][8];
  float ss[kJ];
#pragma unroll
  for (int j = 0; j < kJ; ++j) ss[j] = 0.f;
#pragma unroll
  for (int i = 0; i < NVL; ++i) {
    unpack8(xv[i], xn[i]);
    if constexpr (kAdd) {
      float g[8];
      unpack8(av[i], g);
      u32x4 o;
#pragma unroll
      for (int c = 0; c < 8; ++c) xn[i][c] = round_bf16(xn[i][c] + alpha * g[c]);
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = pack_bf16(xn[i][2 * c], xn[i][2 * c + 1]);
      xr[lane + i * kWave] = o;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) ss[i % kRouterWaves] += xn[i][c] * xn[i][c];
  }
  float total = 0.f;
#pragma unroll
  for (int j = 0; j < kJ; ++j) total += wave_sum(ss[j]);
  const float scale = 1.0f / sqrtf(total / (float)(NVL * 512) + eps);
#pragma unroll
  for (int i = 0; i < NVL; ++i) {
    float g[8];
    unpack8(gv[i], g);
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = pack_bf16(round_bf16(xn[i][2 * c] * scale) * g[2 * c],
                       round_bf16(xn[i][2 * c + 1] * scale) * g[2 * c + 1]);
    zr[lane + i * kWave] = o;
  }
}

// Occupancy target: four waves per SIMD up to hidden 1536 and 48 experts;
// the 49-64 expert tiles need more registers (three waves), wider rows two.
template <int NVL, int NT, bool kNorm, bool kAdd>
__global__ void __launch_bounds__(kBatchThreads, NVL <= 3 ? (NT <= 3 ? 4 : 3) : 2)
batched_router_kernel(bf16 *__restrict__ x, const bf16 *__restrict__ a, float alpha,
                      const bf16 *__restrict__ nw, float eps, bf16 *__restrict__ z,
                      const bf16 *__restrict__ wr, int experts, int topk, int renormalize,
                      bf16 *__restrict__ logits_out, float *__restrict__ tw,
                      int32_t *__restrict__ tid) {
  constexpr int kNvec = NVL * kWave, kSteps = NVL * 16, kCols = NT * 16;
  constexpr int kWaveSteps = kSteps / kBatchWaves;
  static_assert(kWaveSteps % kBatchSteps == 0, "k-steps per load batch");
  __shared__ __align__(16) float part[kBatchWaves][kBatchMB][NT][4][kWave];
  __shared__ __align__(16) float logit[kBatchRows][kCols];
  __shared__ __align__(16) float scratch[kBatchWaves][2 * kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t row0 = (int64_t)blockIdx.x * kBatchRows;
  if constexpr (kNorm) {
    u32x4 gv[NVL];
#pragma unroll
    for (int i = 0; i < NVL; ++i) gv[i] = reinterpret_cast<const u32x4 *>(nw)[lane + i * kWave];
    const int64_t r0 = row0 + wave * kRowsPerWave;
    u32x4 xa[NVL], aa[NVL], xb[NVL], ab[NVL];
    batch_load_row<NVL, kAdd>(x, a, r0, xa, aa);
#pragma unroll
    for (int r = 0; r < kRowsPerWave; r += 2) {
      batch_load_row<NVL, kAdd>(x, a, r0 + r + 1, xb, ab);
      batch_norm_row<NVL, kAdd>(x, alpha, gv, eps, z, r0 + r, xa, aa);
      if (r + 2 < kRowsPerWave) batch_load_row<NVL, kAdd>(x, a, r0 + r + 2, xa, aa);
      batch_norm_row<NVL, kAdd>(x, alpha, gv, eps, z, r0 + r + 1, xb, ab);
    }
    __syncthreads();  // every wave reads all 16 rows of z back below
  }
  const int tr = lane % 16, kg = lane / 16;
  const int64_t k0 = (int64_t)wave * kWaveSteps * 4 + kg;  // 16-byte word of the wave's first k-step
  const u32x4 *ap = reinterpret_cast<const u32x4 *>(kNorm ? z : x) + (row0 + tr) * kNvec + k0;
  constexpr int64_t kBlockStride = 16 * (int64_t)kNvec;  // the next 16-row block of A
  const u32x4 *bp[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n)
    bp[n] = reinterpret_cast<const u32x4 *>(wr) + (int64_t)min(16 * n + tr, experts - 1) * kNvec + k0;
  f32x4 acc[kBatchMB][NT];
#pragma unroll
  for (int mb = 0; mb < kBatchMB; ++mb)
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[mb][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < kWaveSteps; s0 += kBatchSteps) {
    u32x4 av[kBatchSteps][kBatchMB], bv[kBatchSteps][NT];
#pragma unroll
    for (int u = 0; u < kBatchSteps; ++u) {
#pragma unroll
      for (int mb = 0; mb < kBatchMB; ++mb) av[u][mb] = ap[mb * kBlockStride + 4 * (s0 + u)];
#pragma unroll
      for (int n = 0; n < NT; ++n) bv[u][n] = bp[n][4 * (s0 + u)];
    }
#pragma unroll
    for (int u = 0; u < kBatchSteps; ++u)
#pragma unroll
      for (int mb = 0; mb < kBatchMB; ++mb)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[mb][n] = mfma16x16x32(av[u][mb], bv[u][n], acc[mb][n]);
  }
#pragma unroll
  for (int mb = 0; mb < kBatchMB; ++mb)
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[wave][mb][n][i][lane] = acc[mb][n][i];
  __syncthreads();
  // C layout: lane l of a tile holds rows 4*(l/16) + i of column l % 16.
  for (int idx = threadIdx.x; idx < kBatchMB * NT * 4 * kWave; idx += kBatchThreads) {
    const int mb = idx / (NT * 4 * kWave), n = idx / (4 * kWave) % NT, i = idx / kWave % 4,
              l = idx % kWave;
    float sum = part[0][mb][n][i][l];
#pragma unroll
    for (int w = 1; w < kBatchWaves; ++w) sum += part[w][mb][n][i][l];
    const int e = 16 * n + l % 16, row = 16 * mb + 4 * (l / 16) + i;
    const uint32_t h = f32_to_bf16(sum);
    logit[row][e] = bf16_to_f32(h);
    if (logits_out && e < experts) logits_out[(row0 + row) * experts + e] = (bf16)h;
  }
  __syncthreads();
#pragma unroll
  for (int r = wave * kRowsPerWave; r < (wave + 1) * kRowsPerWave; ++r)
    select_topk_lanes(logit[r], scratch[wave], lane, experts, topk, renormalize,
                      tw + (row0 + r) * topk, tid + (row0 + r) * topk);
}

// Routes the first tokens - tokens % kBatchRows tokens with
// batched_router_kernel when the shape allows it; returns how many it routed
// (0: none, the per-token kernels route them all).
template <bool kNorm, bool kAdd>
int64_t launch_batched_router(int64_t tokens, int64_t hidden, bf16 *x, const bf16 *a,
                              float alpha, const bf16 *nw, float eps, bf16 *z, const bf16 *wr,
                              int experts, int topk, int renormalize, bf16 *logits_out,
                              float *tw, int32_t *tid, hipStream_t s) {
  const int nv = fast_nv(hidden);
  if (tokens < kBatchRouterMinTokens || !nv || experts > kWave || experts <= 16) return 0;
  const int64_t rows = tokens - tokens % kBatchRows;
  const int nt = (experts + 15) / 16;
  const dim3 grid((unsigned)(rows / kBatchRows));
#define LM_BATCH_ROUTER(NVL, NT)                                                                \
  if (nv == NVL && nt == NT) {                                                                  \
    batched_router_kernel<NVL, NT, kNorm, kAdd><<<grid, kBatchThreads, 0, s>>>(                         \
        x, a, alpha, nw, eps, z, wr, experts, topk, renormalize, logits_out, tw, tid);          \
    return rows;                                                                                \
  }
#define LM_BATCH_ROUTER_NT(NVL) LM_BATCH_ROUTER(NVL, 2) LM_BATCH_ROUTER(NVL, 3) LM_BATCH_ROUTER(NVL, 4)
  LM_BATCH_ROUTER_NT(1) LM_BATCH_ROUTER_NT(2) LM_BATCH_ROUTER_NT(3) LM_BATCH_ROUTER_NT(4)
  LM_BATCH_ROUTER_NT(6) LM_BATCH_ROUTER_NT(8)
#undef LM_BATCH_ROUTER_NT
#undef LM_BATCH_ROUTER
  return 0;
}

constexpr int kAlignThreads = 1024;
constexpr int kAlignWaves = kAlignThreads / kWave;
constexpr int kMaxAlignExperts = 511;

// Lanes of the wave whose key equals this lane's key (among `valid` lanes),
// from one ballot per key bit.
__device__ __forceinline__ uint64_t match_key(int key, bool valid, int nbits) {
  uint64_t eq = __ballot(valid);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (key >> b) & 1;
    const uint64_t m = __ballot(valid && bit);
    eq &= bit ? m : ~m;
  }
  return eq;
}

// Single workgroup. Wave w owns the contiguous route segment
// [w*seg, (w+1)*seg): pass 1 counts keys per segment, a scan turns the
// counts into per-(segment, key) bases, pass 2 scatters each route to
// base + its rank among equal keys earlier in the segment. No atomics: the
// permutation is the stable argsort of the key.
__global__ void __launch_bounds__(kAlignThreads)
align_kernel(const int32_t *__restrict__ ids, int routes, int first, int local,
             int32_t *__restrict__ offsets, int32_t *__restrict__ sorted,
             int32_t *__restrict__ inverse) {
  extern __shared__ int smem[];
  const int keys = local + 1;
  int *cnt = smem;                            // [kAlignWaves][keys]
  int *scan = smem + kAlignWaves * keys;      // [2][1024]
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  for (int i = threadIdx.x; i < kAlignWaves * keys; i += kAlignThreads) cnt[i] = 0;
  __syncthreads();
  const int seg = (int)(cdiv(cdiv(routes, kAlignWaves), kWave) * kWave);
  const int begin = wave * seg;
  const int end = min(routes, begin + seg);
  const int nbits = 32 - __clz(local);
  const uint64_t below = (1ull << lane) - 1ull;
  for (int base = begin; base < end; base += kWave) {
    const int r = base + lane;
    const bool valid = r < end;
    int key = local;
    if (valid) {
      const int e = ids[r] - first;
      key = (e >= 0 && e < local) ? e : local;
    }
    const uint64_t eq = match_key(key, valid, nbits);
    if (valid && (eq & below) == 0ull) cnt[wave * keys + key] += __popcll(eq);
  }
  __syncthreads();
  // Totals per key, then an inclusive Hillis-Steele scan over keys.
  int total = 0;
  if (threadIdx.x < keys)
    for (int w = 0; w < kAlignWaves; ++w) total += cnt[w * keys + threadIdx.x];
  scan[threadIdx.x] = threadIdx.x < keys ? total : 0;
  __syncthreads();
  int src = 0;
  for (int d = 1; d < kAlignThreads; d <<= 1) {
    const int v = scan[src * kAlignThreads + threadIdx.x] +
                  (threadIdx.x >= d ? scan[src * kAlignThreads + threadIdx.x - d] : 0);
    scan[(1 - src) * kAlignThreads + threadIdx.x] = v;
    src = 1 - src;
    __syncthreads();
  }
  if (threadIdx.x < keys) {
    int running = scan[src * kAlignThreads + threadIdx.x] - total;  // exclusive
    offsets[threadIdx.x] = running;
    for (int w = 0; w < kAlignWaves; ++w) {
      const int c = cnt[w * keys + threadIdx.x];
      cnt[w * keys + threadIdx.x] = running;
      running += c;
    }
  }
  __syncthreads();
  for (int base = begin; base < end; base += kWave) {
    const int r = base + lane;
    const bool valid = r < end;
    int key = local;
    if (valid) {
      const int e = ids[r] - first;
      key = (e >= 0 && e < local) ? e : local;
    }
    const uint64_t eq = match_key(key, valid, nbits);
    const int rank = __popcll(eq & below);
    int pos = 0;
    if (valid) pos = cnt[wave * keys + key] + rank;
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      sorted[pos] = r;
      if (inverse) inverse[r] = pos;
      if (rank == 0) cnt[wave * keys + key] += __popcll(eq);
    }
    __builtin_amdgcn_wave_barrier();
  }
}


// The same stable argsort for large route counts, over chunks of 1024 routes
// (16 waves x 64) in three launches: per-chunk key counts; one workgroup
// turning them into key offsets and per-(chunk, key) bases (key-major, then
// chunk order); and the scatter, each route to its chunk's base plus its rank
// among equal keys earlier in the chunk. Every lane loads one id (clamped,
// masked), so no wave waits on a chain of loads.
constexpr int kChunk = 1024;

template <bool kScatter>
__global__ void __launch_bounds__(kChunk)
align_chunk_kernel(const int32_t *__restrict__ ids, int routes, int first, int local,
                   int32_t *__restrict__ counts, const int32_t *__restrict__ bases,
                   int32_t *__restrict__ sorted, int32_t *__restrict__ inverse) {
  extern __shared__ int wave_cnt[];  // [kAlignWaves][keys]
  const int keys = local + 1;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  for (int i = threadIdx.x; i < kAlignWaves * keys; i += kChunk) wave_cnt[i] = 0;
  const int r = blockIdx.x * kChunk + threadIdx.x;
  const bool valid = r < routes;
  const int e = ids[min(r, routes - 1)] - first;
  const int key = valid && e >= 0 && e < local ? e : local;
  const uint64_t eq = match_key(key, valid, 32 - __clz(local));
  const uint64_t below = (1ull << lane) - 1ull;
  __syncthreads();
  if (valid && (eq & below) == 0ull) wave_cnt[wave * keys + key] = __popcll(eq);
  __syncthreads();
  if constexpr (!kScatter) {
    if (threadIdx.x < keys) {
      int total = 0;
#pragma unroll
      for (int w = 0; w < kAlignWaves; ++w) total += wave_cnt[w * keys + threadIdx.x];
      counts[(int64_t)blockIdx.x * keys + threadIdx.x] = total;
    }
  } else {
    if (threadIdx.x < keys) {
      int running = bases[(int64_t)blockIdx.x * keys + threadIdx.x];
#pragma unroll
      for (int w = 0; w < kAlignWaves; ++w) {
        const int c = wave_cnt[w * keys + threadIdx.x];
        wave_cnt[w * keys + threadIdx.x] = running;
        running += c;
      }
    }
    __syncthreads();
    if (valid) {
      const int pos = wave_cnt[wave * keys + key] + __popcll(eq & below);
      sorted[pos] = r;
      if (inverse) inverse[r] = pos;
    }
  }
}

// One workgroup: offsets[k] = routes with a smaller key; bases[c][k] =
// offsets[k] + routes of key k in chunks before c. Lane l takes key 64*g + l
// (key groups g of 64), wave w the chunks [w*per, (w+1)*per): a load reads
// one chunk's counts of 64 adjacent keys, and a wave's up to kScanRegs counts
// per key are held in LDS from the sum to the writes. (One thread per key
// walking every chunk waits on one load round trip per eight chunks.) With
// 24 counts per lane in flight at once, up to 384 chunks (393,216 routes) take
// one load round trip.
constexpr int kScanWaves = 16, kScanRegs = 24;
__global__ void __launch_bounds__(kScanWaves * kWave)
align_scan_kernel(const int32_t *__restrict__ counts, int chunks, int keys,
                  int32_t *__restrict__ bases, int32_t *__restrict__ offsets) {
  __shared__ int part[kScanWaves][kWave];  // per wave and key: sum, then exclusive prefix over waves
  __shared__ int key_base[kWave];
  __shared__ int held[kScanWaves * kScanRegs][kWave];  // the counts, from the sum to the writes
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int per = (chunks + kScanWaves - 1) / kScanWaves;
  const int c0 = wave * per, c1 = min(c0 + per, chunks);
  int carry = 0;  // wave 0: routes of the key groups before g
  for (int g = 0; g * kWave < keys; ++g) {
    const int k = g * kWave + lane, kc = min(k, keys - 1);
    const bool key_ok = k < keys;
    int sum = 0;
    if (per <= kScanRegs) {
      // one pointer stepped a chunk at a time, held at the last chunk of the range
      const int32_t *src = counts + (int64_t)min(c0, chunks - 1) * keys + kc;
      int v[kScanRegs];
#pragma unroll
      for (int i = 0; i < kScanRegs; ++i) {
        v[i] = *src;
        src += c0 + i + 1 < c1 ? keys : 0;
      }
#pragma unroll
      for (int i = 0; i < kScanRegs; ++i) {
        v[i] = c0 + i < c1 ? v[i] : 0;
        sum += v[i];
        held[wave * kScanRegs + i][lane] = v[i];
      }
    } else {
      for (int c = c0; c < c1; c += 8) {
        int w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = counts[(int64_t)min(c + i, c1 - 1) * keys + kc];
#pragma unroll
        for (int i = 0; i < 8; ++i) sum += c + i < c1 ? w[i] : 0;
      }
    }
    part[wave][lane] = key_ok ? sum : 0;
    __syncthreads();
    if (wave == 0) {
      int total = 0;
#pragma unroll
      for (int w = 0; w < kScanWaves; ++w) {
        const int x = part[w][lane];
        part[w][lane] = total;
        total += x;
      }
      int incl = total;
#pragma unroll
      for (int d = 1; d < kWave; d *= 2) {
        const int up = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += up;
      }
      const int excl = carry + incl - total;
      if (key_ok) offsets[k] = excl;
      key_base[lane] = excl;
      carry += __shfl(incl, kWave - 1, kWave);
    }
    __syncthreads();
    if (key_ok) {
      int running = key_base[lane] + part[wave][lane];
      if (per <= kScanRegs) {
        for (int c = c0; c < c1; ++c) {
          bases[(int64_t)c * keys + k] = running;
          running += held[wave * kScanRegs + c - c0][lane];
        }
      } else {
        for (int c = c0; c < c1; ++c) {
          bases[(int64_t)c * keys + k] = running;
          running += counts[(int64_t)c * keys + k];
        }
      }
    }
    __syncthreads();  // part and key_base are reused by the next key group
  }
}

}  // namespace
}  // namespace lm

using namespace lm;

extern "C" int lm_router(const void *x, const void *gate_weight, int64_t tokens, int64_t hidden,
                         int64_t experts, int64_t topk, int renormalize, void *logits_out,
                         float *topk_weights, int32_t *topk_ids, void *stream) {
  LM_REQUIRE(tokens >= 0 && hidden > 0 && experts > 0 && topk > 0);
  if (hidden % 8 || hidden > kMaxNormVec * 8 * kRouterThreads || experts > kMaxExperts ||
      topk > kMaxTopk || topk > experts)
    return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && gate_weight && topk_weights && topk_ids);
  if (const int nv = fast_nv(hidden)) {
    const int64_t done = launch_batched_router<false, false>(
        tokens, hidden, (bf16 *)x, nullptr, 0.f, nullptr, 0.f, nullptr, (const bf16 *)gate_weight,
        (int)experts, (int)topk, renormalize, (bf16 *)logits_out, topk_weights, topk_ids,
        (hipStream_t)stream);
    if (done < tokens)
      launch_fast_router<false, false>(
          nv, tokens - done, (bf16 *)x + done * hidden, nullptr, 0.f, nullptr, 0.f, nullptr,
          (const bf16 *)gate_weight, (int)experts, (int)topk, renormalize,
          logits_out ? (bf16 *)logits_out + done * experts : nullptr, topk_weights + done * topk,
          topk_ids + done * topk, (hipStream_t)stream);
    LM_CHECK_LAUNCH();
    return LM_OK;
  }
  router_kernel<<<dim3((unsigned)tokens), kRouterThreads, 0, (hipStream_t)stream>>>(
      (const bf16 *)x, (const bf16 *)gate_weight, (int)hidden, (int)experts, (int)topk,
      renormalize, (bf16 *)logits_out, topk_weights, topk_ids);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_add_rmsnorm_router(void *x, const void *a, float alpha, const void *norm_weight,
                                     float eps, void *z, const void *gate_weight, int64_t tokens,
                                     int64_t hidden, int64_t experts, int64_t topk, int renormalize,
                                     void *logits_out, float *topk_weights, int32_t *topk_ids,
                                     void *stream) {
  LM_REQUIRE(tokens >= 0 && hidden > 0 && experts > 0 && topk > 0);
  if (hidden % 8 || hidden > kMaxNormVec * 8 * kRouterThreads || experts > kMaxExperts ||
      topk > kMaxTopk || topk > experts)
    return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && norm_weight && z && gate_weight && topk_weights && topk_ids);
  if (const int nv = fast_nv(hidden)) {
    const hipStream_t s = (hipStream_t)stream;
    const int64_t done =
        a ? launch_batched_router<true, true>(tokens, hidden, (bf16 *)x, (const bf16 *)a, alpha,
                                              (const bf16 *)norm_weight, eps, (bf16 *)z,
                                              (const bf16 *)gate_weight, (int)experts, (int)topk,
                                              renormalize, (bf16 *)logits_out, topk_weights,
                                              topk_ids, s)
          : launch_batched_router<true, false>(tokens, hidden, (bf16 *)x, nullptr, 0.f,
                                               (const bf16 *)norm_weight, eps, (bf16 *)z,
                                               (const bf16 *)gate_weight, (int)experts,
                                               (int)topk, renormalize, (bf16 *)logits_out,
                                               topk_weights, topk_ids, s);
    if (done < tokens) {
      // The per-token kernels take the rows the batched kernel left.
      bf16 *xt = (bf16 *)x + done * hidden, *zt = (bf16 *)z + done * hidden;
      bf16 *lt = logits_out ? (bf16 *)logits_out + done * experts : nullptr;
      if (a)
        launch_fast_router<true, true>(nv, tokens - done, xt, (const bf16 *)a + done * hidden,
                                       alpha, (const bf16 *)norm_weight, eps, zt,
                                       (const bf16 *)gate_weight, (int)experts, (int)topk,
                                       renormalize, lt, topk_weights + done * topk,
                                       topk_ids + done * topk, s);
      else
        launch_fast_router<true, false>(nv, tokens - done, xt, nullptr, 0.f,
                                        (const bf16 *)norm_weight, eps, zt,
                                        (const bf16 *)gate_weight, (int)experts, (int)topk,
                                        renormalize, lt, topk_weights + done * topk,
                                        topk_ids + done * topk, s);
    }
    LM_CHECK_LAUNCH();
    return LM_OK;
  }
  add_norm_router_kernel<<<dim3((unsigned)tokens), kRouterThreads, 0, (hipStream_t)stream>>>(
      (bf16 *)x, (const bf16 *)a, alpha, (const bf16 *)norm_weight, eps, (bf16 *)z,
      (const bf16 *)gate_weight, (int)hidden, (int)experts, (int)topk, renormalize,
      (bf16 *)logits_out, topk_weights, topk_ids);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_add_rmsnorm_router_splitk(void *x, const float *a_partials, int64_t a_splits,
                                            float alpha, const void *norm_weight, float eps,
                                            void *z, const void *gate_weight, int64_t tokens,
                                            int64_t hidden, int64_t experts, int64_t topk,
                                            int renormalize, void *logits_out,
                                            float *topk_weights, int32_t *topk_ids,
                                            void *stream) {
  LM_REQUIRE(tokens >= 0 && hidden > 0 && experts > 0 && topk > 0 && a_splits > 0);
  const int nv = fast_nv(hidden);
  if (!nv || nv > 4 || experts > kMaxExperts || topk > kMaxTopk || topk > experts ||
      a_splits > kMaxResidualSplits)
    return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && a_partials && norm_weight && z && gate_weight && topk_weights && topk_ids);
  launch_fast_router<true, true, true>(nv, tokens, (bf16 *)x, nullptr, alpha,
                                       (const bf16 *)norm_weight, eps, (bf16 *)z,
                                       (const bf16 *)gate_weight, (int)experts, (int)topk,
                                       renormalize, (bf16 *)logits_out, topk_weights, topk_ids,
                                       (hipStream_t)stream, a_partials, (int)a_splits);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_topk_softmax(const void *logits, int64_t tokens, int64_t experts, int64_t topk,
                               int renormalize, float *topk_weights, int32_t *topk_ids,
                               void *stream) {
  LM_REQUIRE(tokens >= 0 && experts > 0 && topk > 0);
  if (experts > kMaxExperts || topk > kMaxTopk || topk > experts) return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(logits && topk_weights && topk_ids);
  topk_from_logits_kernel<<<dim3((unsigned)tokens), kRouterThreads, 0, (hipStream_t)stream>>>(
      (const bf16 *)logits, (int)experts, (int)topk, renormalize, topk_weights, topk_ids);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

namespace lm {

int64_t align_scratch_bytes(int64_t routes, int64_t local_experts) {
  return routes > kAlignChunkedMinRoutes ? 2 * 4 * cdiv(routes, kChunk) * (local_experts + 1) : 0;
}

int launch_align(const int32_t *ids, int64_t routes, int64_t first_expert, int64_t local_experts,
                 int32_t *offsets, int32_t *sorted, int32_t *inverse, int32_t *scratch,
                 int64_t scratch_bytes, hipStream_t stream) {
  const int keys = (int)local_experts + 1;
  const size_t wave_bytes = sizeof(int) * (size_t)kAlignWaves * keys;
  const int64_t need = align_scratch_bytes(routes, local_experts);
  if (need > 0 && scratch && scratch_bytes >= need) {
    const int chunks = (int)cdiv(routes, kChunk);
    int32_t *counts = scratch, *bases = scratch + (int64_t)chunks * keys;
    align_chunk_kernel<false><<<chunks, kChunk, wave_bytes, stream>>>(
        ids, (int)routes, (int)first_expert, (int)local_experts, counts, nullptr, nullptr, nullptr);
    align_scan_kernel<<<1, kScanWaves * kWave, 0, stream>>>(counts, chunks, keys, bases, offsets);
    align_chunk_kernel<true><<<chunks, kChunk, wave_bytes, stream>>>(
        ids, (int)routes, (int)first_expert, (int)local_experts, nullptr, bases, sorted, inverse);
  } else {
    align_kernel<<<1, kAlignThreads, wave_bytes + sizeof(int) * 2 * kAlignThreads, stream>>>(
        ids, (int)routes, (int)first_expert, (int)local_experts, offsets, sorted, inverse);
  }
  LM_CHECK_LAUNCH();
  return LM_OK;
}

}  // namespace lm

extern "C" int lm_moe_align(const int32_t *ids, int64_t routes, int64_t first_expert,
                            int64_t local_experts, int32_t *expert_offsets, int32_t *sorted_routes,
                            int32_t *inverse, void *stream) {
  LM_REQUIRE(routes >= 0 && routes < (int64_t)1 << 30 && local_experts > 0 && first_expert >= 0);
  if (local_experts > kMaxAlignExperts) return LM_EUNSUPPORTED;
  LM_REQUIRE(expert_offsets && (routes == 0 || (ids && sorted_routes)));
  return launch_align(ids, routes, first_expert, local_experts, expert_offsets, sorted_routes,
                      inverse, nullptr, 0, (hipStream_t)stream);
}
