// RMSNorm (plain and fused with the residual add), neox RoPE fused with the
// masked KV-cache store, and the bare KV store.
//
// Rounding follows the reference:
//   rmsnorm  litemoe/model.py:9-11, norm.py:15  bf16(x*rsqrt(mean x^2+eps)) * w
//   add      litemoe/model.py:108,122           bf16(x + alpha*a)
//   rope     litemoe/model.py:66-67             bf16(bf16(x1*c) - bf16(x2*s)), ...
//   kv store litemoe/kv_write.py:12-20          bit copy under the active mask
#include "common.h"

namespace lm {
namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) t += red[w];
  return t;
}

// One workgroup per row. When `a` is given, x <- bf16(x + alpha*a) first and
// the rounded sum is what gets normalised (the reference normalises the bf16
// residual stream).
template <bool kVec, bool kAdd>
__global__ void __launch_bounds__(kNormThreads)
rmsnorm_kernel(bf16 *__restrict__ x, const bf16 *__restrict__ a, float alpha,
               const bf16 *__restrict__ w, bf16 *__restrict__ y, int hidden, float eps) {
  __shared__ float red[kNormThreads / kWave];
  const int64_t row = blockIdx.x;
  bf16 *xr = x + row * hidden;
  bf16 *yr = y + row * hidden;
  float ss = 0.f;
  if constexpr (kVec) {
    const int nvec = hidden / 8;
    for (int i = threadIdx.x; i < nvec; i += kNormThreads) {
      u32x4 xv = reinterpret_cast<const u32x4 *>(xr)[i];
      float f[8];
      unpack8(xv, f);
      if constexpr (kAdd) {
        u32x4 av = reinterpret_cast<const u32x4 *>(a + row * hidden)[i];
        float g[8];
        unpack8(av, g);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = round_bf16(f[j] + alpha * g[j]);
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack_bf16(f[2 * j], f[2 * j + 1]);
        reinterpret_cast<u32x4 *>(xr)[i] = o;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += f[j] * f[j];
    }
  } else {
    for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
      float f = bf16_to_f32(xr[i]);
      if constexpr (kAdd) {
        f = round_bf16(f + alpha * bf16_to_f32(a[row * hidden + i]));
        xr[i] = (bf16)f32_to_bf16(f);
      }
      ss += f * f;
    }
  }
  const float total = block_sum(ss, red);
  const float scale = 1.0f / sqrtf(total / (float)hidden + eps);
  if constexpr (kVec) {
    const int nvec = hidden / 8;
    for (int i = threadIdx.x; i < nvec; i += kNormThreads) {
      float f[8], g[8];
      unpack8(reinterpret_cast<const u32x4 *>(xr)[i], f);
      unpack8(reinterpret_cast<const u32x4 *>(w)[i], g);
      u32x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = pack_bf16(round_bf16(f[2 * j] * scale) * g[2 * j],
                         round_bf16(f[2 * j + 1] * scale) * g[2 * j + 1]);
      reinterpret_cast<u32x4 *>(yr)[i] = o;
    }
  } else {
    for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
      const float f = bf16_to_f32(xr[i]);
      yr[i] = (bf16)f32_to_bf16(round_bf16(f * scale) * bf16_to_f32(w[i]));
    }
  }
}

template <int kElem>
struct Word;
template <>
struct Word<2> { typedef uint16_t T; };
template <>
struct Word<4> { typedef uint32_t T; };

// grid (rows, cdiv(heads*head_dim, 256)); one thread per (head, channel).
template <int kElem>
__global__ void __launch_bounds__(256)
kv_write_kernel(const void *__restrict__ k, int64_t ks0, int64_t ks1, int64_t ks3,
                const void *__restrict__ v, int64_t vs0, int64_t vs1, int64_t vs3,
                void *__restrict__ kc, void *__restrict__ vc, const int64_t *__restrict__ pos,
                const uint8_t *__restrict__ active, const int64_t *__restrict__ slots,
                int heads, int head_dim, int64_t capacity, int64_t cache_batch) {
  typedef typename Word<kElem>::T T;
  const int64_t row = blockIdx.x;
  const int x = blockIdx.y * 256 + threadIdx.x;
  if (x >= heads * head_dim || !active[row]) return;
  const int64_t p = pos[row];
  const int64_t slot = slots ? slots[row] : row;
  if (p < 0 || p >= capacity || slot < 0 || slot >= cache_batch) return;
  const int h = x / head_dim, c = x % head_dim;
  const int64_t target = ((slot * heads + h) * capacity + p) * head_dim + c;
  static_cast<T *>(kc)[target] = static_cast<const T *>(k)[row * ks0 + h * ks1 + c * ks3];
  static_cast<T *>(vc)[target] = static_cast<const T *>(v)[row * vs0 + h * vs1 + c * vs3];
}

// Neox rotation of one (x1, x2) pair with the reference's three roundings.
__device__ __forceinline__ void rotate(float x1, float x2, float c, float s, float &o1, float &o2) {
  o1 = round_bf16(round_bf16(x1 * c) - round_bf16(x2 * s));
  o2 = round_bf16(round_bf16(x2 * c) + round_bf16(x1 * s));
}

// One workgroup per row; head_dim 64. Work items are 16-byte channel units:
// a rotation item is the unit pair (channels 8u..8u+7, 32+8u..32+8u+7),
// u < 4, of one q or k head; a v item is one unit of a v head. Every load of
// an item is issued before any arithmetic.
__global__ void __launch_bounds__(256)
rope_kv_kernel(bf16 *__restrict__ q, int64_t qs0, int64_t qs1, bf16 *__restrict__ k, int64_t ks0,
               int64_t ks1, const bf16 *__restrict__ v, int64_t vs0, int64_t vs1,
               const bf16 *__restrict__ cos_sin, int64_t table_len, const int64_t *__restrict__ pos,
               const uint8_t *__restrict__ active, const int64_t *__restrict__ slots,
               bf16 *__restrict__ kc, bf16 *__restrict__ vc, int q_heads, int kv_heads,
               int64_t capacity, int64_t cache_batch, int write_k) {
  constexpr int D = 64, P = 32;
  const int64_t row = blockIdx.x;
  const int64_t p = pos[row];
  const int64_t slot = slots ? slots[row] : row;
  const bool store = kc != nullptr && active[row] && p >= 0 && p < capacity && slot >= 0 &&
                     slot < cache_batch;
  const bool in_table = p >= 0 && p < table_len;
  const bf16 *cs = cos_sin + (in_table ? p : 0) * D;
  const int nq = q_heads * 4, nk = kv_heads * 4, nv = kv_heads * 8;
  for (int item = threadIdx.x; item < nq + nk + nv; item += 256) {
    if (item < nq + nk) {
      const bool is_q = item < nq;
      const int j = is_q ? item : item - nq;
      const int h = j / 4, u = j % 4;
      bf16 *base = is_q ? q + row * qs0 + h * qs1 : k + row * ks0 + h * ks1;
      const u32x4 w1 = *reinterpret_cast<const u32x4 *>(base + 8 * u);
      const u32x4 w2 = *reinterpret_cast<const u32x4 *>(base + P + 8 * u);
      const u32x4 wc = *reinterpret_cast<const u32x4 *>(cs + 8 * u);
      const u32x4 ws = *reinterpret_cast<const u32x4 *>(cs + P + 8 * u);
      float x1[8], x2[8], c[8], sn[8];
      unpack8(w1, x1);
      unpack8(w2, x2);
      unpack8(wc, c);
      unpack8(ws, sn);
      u32x4 o1 = w1, o2 = w2;
      if (in_table) {
        float r1[8], r2[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) rotate(x1[i], x2[i], c[i], sn[i], r1[i], r2[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o1[i] = pack_bf16(r1[2 * i], r1[2 * i + 1]);
          o2[i] = pack_bf16(r2[2 * i], r2[2 * i + 1]);
        }
      }
      if (is_q || write_k) {
        *reinterpret_cast<u32x4 *>(base + 8 * u) = o1;
        *reinterpret_cast<u32x4 *>(base + P + 8 * u) = o2;
      }
      if (!is_q && store) {
        bf16 *dst = kc + ((slot * kv_heads + h) * capacity + p) * D;
        *reinterpret_cast<u32x4 *>(dst + 8 * u) = o1;
        *reinterpret_cast<u32x4 *>(dst + P + 8 * u) = o2;
      }
    } else if (store) {
      const int j = item - nq - nk;
      const int h = j / 8, u = j % 8;
      *reinterpret_cast<u32x4 *>(vc + ((slot * kv_heads + h) * capacity + p) * D + 8 * u) =
          *reinterpret_cast<const u32x4 *>(v + row * vs0 + h * vs1 + 8 * u);
    }
  }
}

}  // namespace
}  // namespace lm

using namespace lm;

extern "C" int lm_rmsnorm(const void *x, const void *weight, void *y, int64_t rows, int64_t hidden,
                          float eps, void *stream) {
  LM_REQUIRE(rows >= 0 && hidden > 0);
  if (rows == 0) return LM_OK;
  LM_REQUIRE(x && weight && y);
  hipStream_t s = (hipStream_t)stream;
  const bool vec = hidden % 8 == 0;
  if (vec)
    rmsnorm_kernel<true, false><<<dim3((unsigned)rows), kNormThreads, 0, s>>>(
        (bf16 *)x, nullptr, 0.f, (const bf16 *)weight, (bf16 *)y, (int)hidden, eps);
  else
    rmsnorm_kernel<false, false><<<dim3((unsigned)rows), kNormThreads, 0, s>>>(
        (bf16 *)x, nullptr, 0.f, (const bf16 *)weight, (bf16 *)y, (int)hidden, eps);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_add_rmsnorm(void *x, const void *a, float alpha, const void *weight, void *y,
                              int64_t rows, int64_t hidden, float eps, void *stream) {
  LM_REQUIRE(rows >= 0 && hidden > 0);
  if (rows == 0) return LM_OK;
  LM_REQUIRE(x && weight && y);
  if (!a) return lm_rmsnorm(x, weight, y, rows, hidden, eps, stream);
  hipStream_t s = (hipStream_t)stream;
  if (hidden % 8 == 0)
    rmsnorm_kernel<true, true><<<dim3((unsigned)rows), kNormThreads, 0, s>>>(
        (bf16 *)x, (const bf16 *)a, alpha, (const bf16 *)weight, (bf16 *)y, (int)hidden, eps);
  else
    rmsnorm_kernel<false, true><<<dim3((unsigned)rows), kNormThreads, 0, s>>>(
        (bf16 *)x, (const bf16 *)a, alpha, (const bf16 *)weight, (bf16 *)y, (int)hidden, eps);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_kv_write(const void *k, int64_t ks0, int64_t ks1, int64_t ks3, const void *v,
                           int64_t vs0, int64_t vs1, int64_t vs3, void *k_cache, void *v_cache,
                           const int64_t *positions, const uint8_t *active, const int64_t *slots,
                           int64_t rows, int64_t heads, int64_t head_dim, int64_t capacity,
                           int64_t cache_batch, int64_t elem_bytes, void *stream) {
  LM_REQUIRE(rows >= 0 && heads > 0 && head_dim > 0 && capacity > 0 && cache_batch > 0);
  LM_REQUIRE(elem_bytes == 2 || elem_bytes == 4);
  if (rows == 0) return LM_OK;
  LM_REQUIRE(k && v && k_cache && v_cache && positions && active);
  dim3 grid((unsigned)rows, (unsigned)cdiv(heads * head_dim, 256));
  hipStream_t s = (hipStream_t)stream;
  if (elem_bytes == 2)
    kv_write_kernel<2><<<grid, 256, 0, s>>>(k, ks0, ks1, ks3, v, vs0, vs1, vs3, k_cache, v_cache,
                                            positions, active, slots, (int)heads, (int)head_dim,
                                            capacity, cache_batch);
  else
    kv_write_kernel<4><<<grid, 256, 0, s>>>(k, ks0, ks1, ks3, v, vs0, vs1, vs3, k_cache, v_cache,
                                            positions, active, slots, (int)heads, (int)head_dim,
                                            capacity, cache_batch);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_rope_kv_write(void *q, int64_t qs0, int64_t qs1, void *k, int64_t ks0,
                                int64_t ks1, const void *v, int64_t vs0, int64_t vs1,
                                const void *cos_sin, int64_t table_len, const int64_t *positions,
                                const uint8_t *active, const int64_t *slots, void *k_cache,
                                void *v_cache, int64_t rows, int64_t q_heads, int64_t kv_heads,
                                int64_t head_dim, int64_t capacity, int64_t cache_batch,
                                int write_k, void *stream) {
  LM_REQUIRE(rows >= 0 && q_heads > 0 && kv_heads > 0 && capacity > 0 && cache_batch > 0 &&
             table_len > 0);
  if (head_dim != 64) return LM_EUNSUPPORTED;
  if (rows == 0) return LM_OK;
  LM_REQUIRE(q && k && cos_sin && positions);
  // Without caches this is the in-place rotation alone.
  LM_REQUIRE((k_cache == nullptr) == (v_cache == nullptr));
  LM_REQUIRE(!k_cache || (v && active));
  rope_kv_kernel<<<dim3((unsigned)rows), 256, 0, (hipStream_t)stream>>>(
      (bf16 *)q, qs0, qs1, (bf16 *)k, ks0, ks1, (const bf16 *)v, vs0, vs1, (const bf16 *)cos_sin,
      table_len, positions, active, slots, (bf16 *)k_cache, (bf16 *)v_cache, (int)q_heads,
      (int)kv_heads, capacity, cache_batch, write_k);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
