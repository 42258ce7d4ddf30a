// Split-K dense projection for decode-sized row counts on MFMA:
//
//   partials[s][m][n] = sum_{k in slice s} A[m][k] * W[n][k]        (fp32)
//
// W is an nn.Linear weight [N, K] (row-major), A is bf16 [M, K] with row
// stride lda, M <= 128. F.linear's bf16 output is bf16(sum_s partials[s]),
// the slices summed in ascending order; lm_linear_splitk_reduce does that,
// and the decode consumers (lm_flash_decode_qkv, lm_add_rmsnorm_router_splitk)
// do it on their own loads, so the projection costs one launch and the
// reduction none.
//
// Why split K: with M = batch rows, every workgroup that covers the full K
// range must read all of A (M x K bf16), which bounds the workgroup by its
// CU's load rate rather than by HBM. Slicing K divides both A and W per
// workgroup; the price is S fp32 partial rows, read once by the consumer.
//
// Workgroup (column tile of 32, slice s), 4 waves; wave w takes KW 32-wide
// k steps of the slice. Each wave loads its B fragment (32 weight rows) and
// the A fragments of every 16-row block once, all before any MFMA; the four
// wave partials are summed through LDS in a fixed order.
//
// Reference: the projections of litemoe/model.py:47-49 (qkv) and :73 (o_proj),
// F.linear in the reference.
#include "internal.h"

namespace lm {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTileN = 32;
constexpr int kMaxRows = 128;

__device__ __forceinline__ u32x4 load16(const bf16 *p) { return *reinterpret_cast<const u32x4 *>(p); }

// kFragA: A is in the fragment order of frag_offset_rows (mb = MB), so each
// A load reads 1 KB contiguously; lda is unused. Measured on the QKV shape
// (64 rows, K 1536, 3 slices): 4.94 against 5.87 us per launch.
// kNorm: A is rmsnorm(x) (x row-major, lda = K), formed here from x, the
// norm weight and the per-64-column sums of squares of x that
// lm_moe_routes_combine wrote (sumsq [M, K/64]), in rmsnorm_kernel's order:
// the tiles' sums are the 8-lane DPP sums of that kernel, summed here in its
// tree (pairs of tiles, then four such pairs per wave, then the waves), so
// A is bitwise the lm_rmsnorm output it replaces.
struct NormIn {
  const float *sumsq;  // [M, K / 64]
  const bf16 *weight;  // [K]
  float eps;
};

constexpr int kMaxNormTiles = 32;  // K <= 2048

// kStreamW: the weight tile is read with non-temporal loads. The decode step
// streams the packed QKV weights this way (lm_linear_splitk, _rmsnorm) and
// leaves o_proj's (lm_linear_splitk_frag) to the caches: with every other
// stream-once read of the step non-temporal, o_proj's 4.7 MB per layer then
// stay in the 256 MB memory-side cache from one step to the next. cfg 3
// decode step, A/B on one box, three runs each: QKV only 2.784-2.785 ms,
// o_proj only 2.791-2.793, both 2.810, neither 2.796-2.801.
template <int KW, int MB, bool kFragA, bool kNorm = false, bool kStreamW = false>
__global__ void __launch_bounds__(kThreads)
splitk_kernel(const bf16 *__restrict__ a, int64_t lda, const bf16 *__restrict__ w, int M, int N,
              int K, float *__restrict__ part, NormIn norm) {
  __shared__ f32x4 red[kWaves][MB][2][kWave];
  __shared__ float row_scale[kNorm ? kMaxRows : 1];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  const int n0 = blockIdx.x * kTileN, s = blockIdx.y;
  const int k0 = (s * kWaves + wave) * KW * 32 + grp * 8;
  u32x4 b[2][KW], av[MB][KW];
  // kNorm: the row sums, x and the norm weight are requested before the
  // weights, so the norm is formed while the weights stream (vector loads
  // complete in issue order).
  const int ntiles = K / 64;
  f32x4 gs[kNorm ? kMaxNormTiles / 4 : 1];
  u32x4 nwv[kNorm ? KW : 1];
  if constexpr (kNorm) {
    const f32x4 *src = reinterpret_cast<const f32x4 *>(norm.sumsq + (int64_t)min((int)threadIdx.x, M - 1) * ntiles);
#pragma unroll
    for (int q = 0; q < kMaxNormTiles / 4; ++q) gs[q] = src[min(q, ntiles / 4 - 1)];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const bf16 *ar = a + (int64_t)min(m * 16 + col, M - 1) * lda + k0;
#pragma unroll
      for (int t = 0; t < KW; ++t) av[m][t] = load16(ar + t * 32);
    }
#pragma unroll
    for (int t = 0; t < KW; ++t) nwv[t] = load16(norm.weight + k0 + t * 32);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const bf16 *wr = w + (int64_t)(n0 + 16 * j + col) * K + k0;
#pragma unroll
    for (int t = 0; t < KW; ++t)
      b[j][t] = kStreamW ? __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wr + t * 32))
                         : load16(wr + t * 32);
  }
  if constexpr (kNorm) {
    __builtin_amdgcn_sched_barrier(0);
    if ((int)threadIdx.x < M) {
      float g[kMaxNormTiles];
#pragma unroll
      for (int q = 0; q < kMaxNormTiles / 4; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) g[4 * q + i] = 4 * q + i < ntiles ? gs[q][i] : 0.f;
      // rmsnorm_kernel: a 16-lane row adds its two 8-lane sums, a wave its
      // four rows in order, the workgroup its four waves in order.
      float waves[4];
#pragma unroll
      for (int wv = 0; wv < 4; ++wv) {
        float rows4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) rows4[r] = g[8 * wv + 2 * r] + g[8 * wv + 2 * r + 1];
        waves[wv] = ((rows4[0] + rows4[1]) + rows4[2]) + rows4[3];
      }
      const float total = ((waves[0] + waves[1]) + waves[2]) + waves[3];
      row_scale[threadIdx.x] = 1.0f / sqrtf(total / (float)K + norm.eps);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const float sc = row_scale[min(m * 16 + col, M - 1)];
#pragma unroll
      for (int t = 0; t < KW; ++t) {
        float f[8], g[8];
        unpack8(av[m][t], f);
        unpack8(nwv[t], g);
        u32x4 z;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t xs = pack_bf16_nc(f[2 * i] * sc, f[2 * i + 1] * sc);  // bf16(x * r), two at once
          z[i] = pack_bf16(lo_f32(xs) * g[2 * i], hi_f32(xs) * g[2 * i + 1]);
        }
        av[m][t] = z;
      }
    }
  }
  if constexpr (!kNorm) {
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      if constexpr (kFragA) {
        // k step c of this wave is (s*4 + wave)*KW + t; lane l's 8 values of
        // row m*16 + l%16, k group l/16 sit at ((c*MB + m)*64 + l)*8
        const bf16 *ab = a + ((int64_t)(s * kWaves + wave) * KW * MB + m) * 512 + lane * 8;
#pragma unroll
        for (int t = 0; t < KW; ++t) av[m][t] = load16(ab + (int64_t)t * MB * 512);
      } else {
        const bf16 *ar = a + (int64_t)min(m * 16 + col, M - 1) * lda + k0;
#pragma unroll
        for (int t = 0; t < KW; ++t) av[m][t] = load16(ar + t * 32);
      }
    }
  }
  f32x4 c[MB][2];
#pragma unroll
  for (int m = 0; m < MB; ++m) c[m][0] = c[m][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < KW; ++t)
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      c[m][0] = mfma16x16x32(av[m][t], b[0][t], c[m][0]);
      c[m][1] = mfma16x16x32(av[m][t], b[1][t], c[m][1]);
    }
  // The four waves' accumulators are summed through LDS in wave order, one
  // 16-byte LDS word per lane and MFMA tile (lane l of a 16x16 tile holds C
  // rows 4*(l/16) .. +3 of column l%16): thread -> (tile, lane) reads the
  // four waves' words and stores the four rows of its column.
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int j = 0; j < 2; ++j) red[wave][m][j][lane] = c[m][j];
  __syncthreads();
  constexpr int kGroups = MB * 2 * kWave;
#pragma unroll
  for (int g0 = 0; g0 < kGroups; g0 += kThreads) {
    const int g = g0 + threadIdx.x;
    if (kGroups % kThreads == 0 || g < kGroups) {
      const int l = g % kWave, j = (g / kWave) % 2, m = g / (2 * kWave);
      f32x4 v = red[0][m][j][l];
#pragma unroll
      for (int q = 1; q < kWaves; ++q) v += red[q][m][j][l];
      const int row0 = m * 16 + 4 * (l / 16), col = n0 + 16 * j + l % 16;
      float *dst = part + ((int64_t)s * M + row0) * N + col;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (row0 + i < M) dst[(int64_t)i * N] = v[i];
    }
  }
}

// out[m][n] = bf16(sum_s partials[s][m][n]), slices in ascending order.
__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float *__restrict__ part, int splits, int M, int N,
                     bf16 *__restrict__ out, int64_t ldo) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int64_t m = idx / N, n = idx % N;
  float v = 0.f;
  for (int s = 0; s < splits; ++s) v += part[(int64_t)s * M * N + idx];
  out[m * ldo + n] = (bf16)f32_to_bf16(v);
}

int row_blocks(int64_t M) { return frag_row_blocks(M); }

template <bool kFragA, bool kNorm = false, bool kStreamW = false>
int launch_splitk(const bf16 *a, int64_t lda, const bf16 *weight, int64_t rows,
                  int64_t out_features, int64_t in_features, int64_t splits, float *partials,
                  hipStream_t s, NormIn norm = NormIn{}) {
  const int kw = (int)(in_features / (splits * kWaves * 32));
  const dim3 grid((unsigned)(out_features / kTileN), (unsigned)splits);
  const int M = (int)rows, N = (int)out_features, K = (int)in_features;
  const int mb = row_blocks(rows);
#define LM_SPLITK(KW, MB)                                                                          \
  if (kw == KW && mb == MB) {                                                                      \
    splitk_kernel<KW, MB, kFragA, kNorm, kStreamW><<<grid, kThreads, 0, s>>>(a, lda, weight, M, N, K, partials, \
                                                                     norm);                       \
    LM_CHECK_LAUNCH();                                                                             \
    return LM_OK;                                                                                  \
  }
#define LM_SPLITK_MB(KW) LM_SPLITK(KW, 1) LM_SPLITK(KW, 2) LM_SPLITK(KW, 4) LM_SPLITK(KW, 8)
  LM_SPLITK_MB(1) LM_SPLITK_MB(2) LM_SPLITK_MB(3) LM_SPLITK_MB(4) LM_SPLITK_MB(6) LM_SPLITK_MB(8)
#undef LM_SPLITK_MB
#undef LM_SPLITK
  return LM_EUNSUPPORTED;
}

}  // namespace

bool splitk_shape_ok(int64_t M, int64_t N, int64_t K, int64_t splits) {
  if (M < 1 || M > kMaxRows || N % kTileN || splits < 1 || K % (splits * kWaves * 32)) return false;
  const int64_t kw = K / (splits * kWaves * 32);
  return kw == 1 || kw == 2 || kw == 3 || kw == 4 || kw == 6 || kw == 8;
}

}  // namespace lm

using namespace lm;

extern "C" int lm_linear_splitk(const void *a, int64_t lda, const void *weight, int64_t rows,
                                int64_t out_features, int64_t in_features, int64_t splits,
                                float *partials, void *stream) {
  LM_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && splits > 0 &&
             lda >= in_features && lda % 8 == 0);
  if (rows == 0) return LM_OK;
  if (!splitk_shape_ok(rows, out_features, in_features, splits)) return LM_EUNSUPPORTED;
  LM_REQUIRE(a && weight && partials);
  return launch_splitk<false, false, true>((const bf16 *)a, lda, (const bf16 *)weight, rows,
                                           out_features, in_features, splits, partials,
                                           (hipStream_t)stream);
}

extern "C" int lm_linear_splitk_frag(const void *a_frag, const void *weight, int64_t rows,
                                     int64_t out_features, int64_t in_features, int64_t splits,
                                     float *partials, void *stream) {
  LM_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && splits > 0 &&
             in_features % 32 == 0);
  if (rows == 0) return LM_OK;
  if (!splitk_shape_ok(rows, out_features, in_features, splits)) return LM_EUNSUPPORTED;
  LM_REQUIRE(a_frag && weight && partials);
  return launch_splitk<true>((const bf16 *)a_frag, 0, (const bf16 *)weight, rows, out_features,
                             in_features, splits, partials, (hipStream_t)stream);
}

extern "C" int lm_linear_splitk_rmsnorm(const void *x, const float *sumsq, const void *norm_weight,
                                        float eps, const void *weight, int64_t rows,
                                        int64_t out_features, int64_t in_features, int64_t splits,
                                        float *partials, void *stream) {
  LM_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && splits > 0);
  if (rows == 0) return LM_OK;
  if (!splitk_shape_ok(rows, out_features, in_features, splits) || in_features % 512 ||
      in_features / 64 > kMaxNormTiles)
    return LM_EUNSUPPORTED;
  LM_REQUIRE(x && sumsq && norm_weight && weight && partials);
  return launch_splitk<false, true, true>((const bf16 *)x, in_features, (const bf16 *)weight, rows,
                                    out_features, in_features, splits, partials,
                                    (hipStream_t)stream,
                                    NormIn{sumsq, (const bf16 *)norm_weight, eps});
}

extern "C" int lm_linear_splitk_reduce(const float *partials, int64_t splits, int64_t rows,
                                       int64_t out_features, void *out, int64_t ldo, void *stream) {
  LM_REQUIRE(splits > 0 && rows >= 0 && out_features > 0 && ldo >= out_features);
  if (rows == 0) return LM_OK;
  LM_REQUIRE(partials && out);
  const int64_t n = rows * out_features;
  splitk_reduce_kernel<<<dim3((unsigned)cdiv(n, 256)), 256, 0, (hipStream_t)stream>>>(
      partials, (int)splits, (int)rows, (int)out_features, (bf16 *)out, ldo);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
