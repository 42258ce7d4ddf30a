// Shared device helpers for the gfx950 kernels: bf16 conversion, vector types,
// wavefront reductions and the launch-status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/litemoe_amd.h"

namespace lm {

typedef uint16_t bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
// Low / high halves of a packed pair of bf16 values.
__device__ __forceinline__ float lo_f32(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_f32(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even float -> bf16, NaN -> canonical quiet NaN 0x7fc0
// (c10::BFloat16's scalar conversion; torch's vectorised CPU conversion
// differs only in writing 0xffff for NaN). gfx950's v_cvt_pk_bf16_f32 rounds every
// non-NaN input (denormals included) exactly so; for NaN it keeps sign and
// payload, so NaN is replaced afterwards.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
  if (lo != lo) h = (h & 0xffff0000u) | 0x7fc0u;
  if (hi != hi) h = (h & 0xffffu) | 0x7fc00000u;
  return h;
}
// pack_bf16 for values known not to be NaN (e.g. exp2 of a finite or -inf
// argument): the conversion alone, the same bits.
__device__ __forceinline__ uint32_t pack_bf16_finite(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}
// pack_bf16 without the NaN canonicalization, for intermediates whose NaN (if
// any) reaches a canonicalizing conversion before anything is stored.
__device__ __forceinline__ uint32_t pack_bf16_nc(float lo, float hi) { return pack_bf16_finite(lo, hi); }
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t h = __builtin_bit_cast(uint16_t, (__bf16)f);
  return f != f ? 0x7fc0u : h;
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }
// round_bf16 without the NaN canonicalization, for an intermediate whose NaN
// (if any) reaches a canonicalizing conversion before anything is stored.
__device__ __forceinline__ float round_bf16_nc(float f) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f) << 16);
}

// Eight bf16 (one 16-byte word) to floats.
__device__ __forceinline__ void unpack8(const u32x4 &w, float *f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = lo_f32(w[i]);
    f[2 * i + 1] = hi_f32(w[i]);
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4 &w) {
  return __builtin_bit_cast(bf16x8, w);
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Sum over the 64 lanes of a wave: DPP lane moves within each row of 16
// lanes (quad_perm xor 1, xor 2, row_half_mirror, row_mirror), then the four
// row sums read as scalars. Every lane gets the same value, and every kernel
// that reduces a row this way rounds identically.
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
}

// The value of lane (lane ^ M) for M in {8, 16, 32}, with VALU lane moves
// instead of the LDS crossbar (ds_bpermute): DPP row_ror:8 swaps the two
// halves of each 16-lane row; gfx950's v_permlane16_swap / v_permlane32_swap
// exchange rows / wave halves between their two operands, and the lane's
// own half selects which result holds its partner (checked on the device).
template <int M>
__device__ __forceinline__ float xor_lanes(float v) {
  static_assert(M == 8 || M == 16 || M == 32, "lane distance");
  if constexpr (M == 8) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((__lane_id() & 16) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(__lane_id() < 32 ? r[1] : r[0]);
  }
}

// Sum over aligned groups of 8 lanes with DPP lane moves (no LDS crossbar):
// quad_perm xor 1, quad_perm xor 2, then row_half_mirror (lane i <- 7-i).
// Every lane of the group ends with the same, bitwise identical sum.
__device__ __forceinline__ float dpp_sum8(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
  return v;
}

// Direct global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's bytes at base + voff land at LDS byte lds + 16 * l (lds in M0,
// wave-uniform; base wave-uniform). Written as asm so that the compiler's
// wait-count pass does not take it for a load that every later LDS read must
// wait for (it cannot tell which LDS bytes the copy writes); the caller waits
// with lds_copy_wait() and then a barrier before the bytes are read.
__device__ __forceinline__ void lds_copy16(const void *base, uint32_t voff, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}
// Wait until every vector memory operation this wave issued has completed
// (s_waitcnt vmcnt(0)), LDS copies included.
__device__ __forceinline__ void lds_copy_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// The 32-bit LDS address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char *)p;
}

// acc + the dot product of the eight bf16 values of two 16-byte words: four
// v_dot2_f32_bf16 in channel-pair order (each adds two exact bf16 products).
// The pairs are taken with shufflevector from a bf16x8 view: bit-casting the
// indexed u32 elements inside an unrolled loop compiles to four dots of
// element 0.
__device__ __forceinline__ float dot8_bf16_acc(const u32x4 &a, const u32x4 &b, float acc) {
  const bf16x8 av = as_bf16x8(a), bv = as_bf16x8(b);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 0, 1),
                                        __builtin_shufflevector(bv, bv, 0, 1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 2, 3),
                                        __builtin_shufflevector(bv, bv, 2, 3), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 4, 5),
                                        __builtin_shufflevector(bv, bv, 4, 5), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 6, 7),
                                        __builtin_shufflevector(bv, bv, 6, 7), acc, false);
  return acc;
}

// x * sigmoid(x) from the hardware exp2 and reciprocal (each within one ulp;
// the product is within a few fp32 ulps of x / (1 + e^-x), far below the
// bf16 rounding every caller applies next). Large negative x gives -0 where
// e^-x overflows; +-inf and NaN behave as in x * sigmoid(x).
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// MFMA 16x16x32 bf16 (gfx950). Lane l supplies row l%16 of A and column l%16
// of B, each with the eight k values of k-group l/16; it receives C rows
// 4*(l/16) .. +3 of column l%16.
__device__ __forceinline__ f32x4 mfma16x16x32(const u32x4 &a, const u32x4 &b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__host__ __device__ constexpr inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Activation rows in MFMA A-fragment order (the "_frag" entry points): a
// [rows, K] bf16 matrix padded to 16*mb rows, mb = frag_row_blocks(rows), is
// stored as k steps of 32 outermost, then the mb 16-row blocks, then the 64
// lanes of a v_mfma_f32_16x16x32_bf16 A operand (lane = row%16 + 16*k group)
// with their 8 consecutive k values. One 64-lane load of 16 bytes then reads
// 1 KB contiguously instead of 16 rows x 64 bytes.
__host__ __device__ constexpr inline int frag_row_blocks(int64_t rows) {
  return rows <= 16 ? 1 : rows <= 32 ? 2 : rows <= 64 ? 4 : 8;
}
__host__ __device__ inline int64_t frag_offset_rows(int64_t row, int64_t k, int mb) {
  return ((k >> 5) * mb + (row >> 4)) * 512 + ((k >> 3) & 3) * 128 + (row & 15) * 8 + (k & 7);
}

}  // namespace lm

// Launch-status check for the C ABI wrappers.
#define LM_CHECK_LAUNCH()                                      \
  do {                                                         \
    if (hipGetLastError() != hipSuccess) return LM_ELAUNCH;    \
  } while (0)

#define LM_REQUIRE(cond)               \
  do {                                 \
    if (!(cond)) return LM_EINVAL;     \
  } while (0)
