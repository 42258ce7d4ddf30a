// Weighted combine of route outputs (the moe_finish contract):
//   out[t] = bf16( sum_{j in ascending logical(ids[t,j])*K + j}
//                  bf16(bf16(y[row(t,j)]) * bf16(scales[t,j])) )   (fp32 sum)
// Non-owned routes are skipped and their rows never read.
// Reference: litemoe/moe_finish.py:7-31 (`_finish`), :34-57 (`finish`).
#include "internal.h"

namespace lm {
namespace {

constexpr int kMaxK = 8;

// grid (tokens, column blocks); each thread owns kCols consecutive columns.
template <int kCols>
__global__ void __launch_bounds__(256)
finish_kernel(const bf16 *__restrict__ y, const int32_t *__restrict__ ids,
              const int32_t *__restrict__ inverse, const float *__restrict__ scales,
              const int64_t *__restrict__ logical, bf16 *__restrict__ out, int hidden, int topk,
              int64_t rank, int64_t count) {
  const int64_t t = blockIdx.x;
  const int c0 = (blockIdx.y * 256 + threadIdx.x) * kCols;
  if (c0 >= hidden) return;
  // Rank of each branch under the key logical*K + j (keys are distinct:
  // j differs). A route that is not owned adds nothing wherever it ranks, so
  // its key uses the raw id and the map is read for owned ids only (an id
  // outside every rank's range never indexes it). The workgroup's threads
  // share the token, so ids, keys and ranks are uniform (scalar registers)
  // and the ordered sum below branches uniformly.
  int64_t key[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; ++j) {
    if (j < topk) {
      const int64_t e = __builtin_amdgcn_readfirstlane(ids[t * topk + j]);
      const bool owned = e - rank * count >= 0 && e - rank * count < count;
      key[j] = (logical && owned ? logical[e] : e) * topk + j;
    } else {
      key[j] = INT64_MAX;
    }
  }
  int order[kMaxK];
#pragma unroll
  for (int j = 0; j < kMaxK; ++j) {
    int r = 0;
#pragma unroll
    for (int i = 0; i < kMaxK; ++i) r += key[i] < key[j];
    order[j] = r;
  }
  // All loads first (scales and the owned rows), then the ordered sum; the
  // order is the same for every thread of the token, so the branches are
  // uniform.
  float contrib[kMaxK][kCols];
#pragma unroll
  for (int j = 0; j < kMaxK; ++j) {
    const int64_t r = t * topk + j;
    const int64_t e = j < topk ? (int64_t)ids[r] - rank * count : -1;
    const bool use = j < topk && e >= 0 && e < count;
    const float s = use ? round_bf16(scales[r]) : 0.f;
    if (use) {
      const bf16 *yr = y + (inverse ? (int64_t)inverse[r] : r) * hidden + c0;
      if constexpr (kCols == 8) {
        float v[8];
        unpack8(*reinterpret_cast<const u32x4 *>(yr), v);
#pragma unroll
        for (int c = 0; c < 8; ++c) contrib[j][c] = round_bf16(v[c] * s);
      } else {
        contrib[j][0] = round_bf16(bf16_to_f32(yr[0]) * s);
      }
    } else {
#pragma unroll
      for (int c = 0; c < kCols; ++c) contrib[j][c] = 0.f;
    }
  }
  float total[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) total[c] = 0.f;
#pragma unroll
  for (int q = 0; q < kMaxK; ++q) {
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      if (order[j] == q) {
#pragma unroll
        for (int c = 0; c < kCols; ++c) total[c] += contrib[j][c];
      }
    }
  }
  bf16 *o = out + t * hidden + c0;
  if constexpr (kCols == 8) {
    u32x4 w;
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = pack_bf16(total[2 * c], total[2 * c + 1]);
    *reinterpret_cast<u32x4 *>(o) = w;
  } else {
    o[0] = (bf16)f32_to_bf16(total[0]);
  }
}

// Finish fused with the residual add and the next RMSNorm; one workgroup per
// token, 8 columns per thread, hidden <= kMaxVec * 8 * 256. Every load (ids,
// scales, the token's route rows, the residual row, the norm weight) is
// issued at entry with clamped indices, so the kernel waits on memory once;
// the arithmetic and the reduction order are those of finish_kernel followed
// by rmsnorm_kernel.
constexpr int kMaxVec = 2;

template <int NN>
__global__ void __launch_bounds__(256)
finish_add_norm_kernel(const bf16 *__restrict__ y, const int32_t *__restrict__ ids,
                       const float *__restrict__ scales, const int64_t *__restrict__ logical,
                       bf16 *__restrict__ x, float alpha, const bf16 *__restrict__ w,
                       float eps, bf16 *__restrict__ z, int hidden, int topk) {
  __shared__ float red[4];
  const int64_t t = blockIdx.x;
  const int nvec = hidden / 8;
  const int lane = threadIdx.x % kWave;
  // The token's route ids and scales, lane j holding route j (lanes past
  // topk repeat the last): lane-dependent addresses make these vector loads,
  // issued with the rows below and in flight together. (Uniform addresses
  // would become scalar loads, which wait one after another through the
  // scalar cache, each a round trip to memory the previous kernel wrote.)
  const int64_t rl = t * topk + min(lane, topk - 1);
  const int id_lane = ids[rl];
  const float sc_lane = scales[rl];
  u32x4 yv[NN][kMaxK], xv[NN], wv[NN];
#pragma unroll
  for (int v = 0; v < NN; ++v) {
    const int i = min((int)threadIdx.x + v * 256, nvec - 1);
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      const int64_t r = t * topk + (j < topk ? j : topk - 1);
      yv[v][j] = reinterpret_cast<const u32x4 *>(y + r * hidden)[i];
    }
    xv[v] = reinterpret_cast<const u32x4 *>(x + t * hidden)[i];
    wv[v] = reinterpret_cast<const u32x4 *>(w)[i];
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait
  // Intermediate roundings skip the NaN fix-up: a NaN term makes its sum, x
  // and z NaN whatever the payload, and x and z are stored through pack_bf16,
  // so the stored bits are those of the canonicalizing form.
  // Every thread of the workgroup combines the same token, so its route
  // keys (logical id, branch) are uniform: read from their lanes into scalar
  // registers, ranked with scalar work, and the ordered sum branches
  // uniformly on the ranks. Ids lie in [0, experts) (the caller's
  // contract), so the keys fit 32 bits.
  int order[kMaxK];
  float sc[kMaxK];
  {
    int key[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      const int id = __builtin_amdgcn_readlane(id_lane, j);
      sc[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc_lane), j));
      const int lid = logical ? (int)logical[id] : id;
      key[j] = j < topk ? lid * kMaxK + j : INT_MAX;
    }
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      int r = 0;
#pragma unroll
      for (int i = 0; i < kMaxK; ++i) r += key[i] < key[j];
      order[j] = r;
    }
  }
  float xn[NN][8];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < NN; ++v) {
    const int i = threadIdx.x + v * 256;
    if (i >= nvec) continue;
    float total[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < topk; ++q) {
#pragma unroll
      for (int j = 0; j < kMaxK; ++j) {
        if (order[j] == q) {  // uniform
          const float s = round_bf16_nc(sc[j]);
          float f[8];
          unpack8(yv[v][j], f);
          u32x4 p;
#pragma unroll
          for (int c = 0; c < 4; ++c) p[c] = pack_bf16_nc(f[2 * c] * s, f[2 * c + 1] * s);
          float term[8];
          unpack8(p, term);
#pragma unroll
          for (int c = 0; c < 8; ++c) total[c] += term[c];
        }
      }
    }
    if (topk < kMaxK) {
      // the unused branch slots rank last and add +0 (finish_kernel's sum)
#pragma unroll
      for (int c = 0; c < 8; ++c) total[c] += 0.f;
    }
    float xf[8];
    unpack8(xv[v], xf);
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      xn[v][c] = round_bf16_nc(xf[c] + alpha * round_bf16_nc(total[c]));
      ss += xn[v][c] * xn[v][c];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = pack_bf16(xn[v][2 * c], xn[v][2 * c + 1]);
    reinterpret_cast<u32x4 *>(x + t * hidden)[i] = o;
  }
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float scale = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)hidden + eps);
#pragma unroll
  for (int v = 0; v < NN; ++v) {
    const int i = threadIdx.x + v * 256;
    if (i >= nvec) continue;
    float g[8];
    unpack8(wv[v], g);
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = pack_bf16(round_bf16_nc(xn[v][2 * c] * scale) * g[2 * c],
                       round_bf16_nc(xn[v][2 * c + 1] * scale) * g[2 * c + 1]);
    reinterpret_cast<u32x4 *>(z + t * hidden)[i] = o;
  }
}

__global__ void __launch_bounds__(256)
invert_kernel(const int64_t *__restrict__ order, int64_t n, int32_t *__restrict__ inverse) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= n) return;
  const int64_t r = order[p];
  if (r >= 0 && r < n) inverse[r] = (int32_t)p;
}

}  // namespace

int launch_finish(const bf16 *y, const int32_t *ids, const int32_t *inverse, const float *scales,
                  const int64_t *logical, bf16 *out, int64_t tokens, int64_t hidden, int64_t topk,
                  int64_t rank, int64_t count, hipStream_t stream) {
  if (tokens == 0) return LM_OK;
  if (hidden % 8 == 0) {
    const dim3 grid((unsigned)tokens, (unsigned)cdiv(hidden, 256 * 8));
    finish_kernel<8><<<grid, 256, 0, stream>>>(y, ids, inverse, scales, logical, out, (int)hidden,
                                               (int)topk, rank, count);
  } else {
    const dim3 grid((unsigned)tokens, (unsigned)cdiv(hidden, 256));
    finish_kernel<1><<<grid, 256, 0, stream>>>(y, ids, inverse, scales, logical, out, (int)hidden,
                                               (int)topk, rank, count);
  }
  LM_CHECK_LAUNCH();
  return LM_OK;
}

}  // namespace lm

using namespace lm;

extern "C" int lm_moe_finish(const void *y, const int32_t *ids, const int64_t *order,
                             const float *scales, const int64_t *logical, void *out,
                             int64_t tokens, int64_t hidden, int64_t topk, int64_t rank,
                             int64_t count, void *workspace, int64_t workspace_bytes,
                             void *stream) {
  LM_REQUIRE(tokens >= 0 && hidden > 0 && topk >= 1 && topk <= kMaxK && count > 0 && rank >= 0);
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(y && ids && scales && out);
  hipStream_t s = (hipStream_t)stream;
  const int64_t routes = tokens * topk;
  int32_t *inverse = nullptr;
  if (order) {
    if (!workspace || workspace_bytes < 4 * routes) return LM_EWORKSPACE;
    inverse = static_cast<int32_t *>(workspace);
    invert_kernel<<<dim3((unsigned)cdiv(routes, 256)), 256, 0, s>>>(order, routes, inverse);
    LM_CHECK_LAUNCH();
  }
  return launch_finish((const bf16 *)y, ids, inverse, scales, logical, (bf16 *)out, tokens, hidden,
                       topk, rank, count, s);
}

extern "C" int lm_moe_finish_add_rmsnorm(const void *y, const int32_t *ids, const float *scales,
                                         const int64_t *logical, void *x, float alpha,
                                         const void *norm_weight, float eps, void *z,
                                         int64_t tokens, int64_t hidden, int64_t topk,
                                         void *stream) {
  LM_REQUIRE(tokens >= 0 && hidden > 0 && topk >= 1 && topk <= kMaxK);
  if (hidden % 8 || hidden > kMaxVec * 8 * 256) return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(y && ids && scales && x && norm_weight && z);
  if (hidden <= 8 * 256)
    finish_add_norm_kernel<1><<<dim3((unsigned)tokens), 256, 0, (hipStream_t)stream>>>(
        (const bf16 *)y, ids, scales, logical, (bf16 *)x, alpha, (const bf16 *)norm_weight, eps,
        (bf16 *)z, (int)hidden, (int)topk);
  else
    finish_add_norm_kernel<2><<<dim3((unsigned)tokens), 256, 0, (hipStream_t)stream>>>(
        (const bf16 *)y, ids, scales, logical, (bf16 *)x, alpha, (const bf16 *)norm_weight, eps,
        (bf16 *)z, (int)hidden, (int)topk);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
