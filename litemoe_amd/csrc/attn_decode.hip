// Split-K decode attention over the contiguous per-row KV cache
// [batch, kv_heads, capacity, 64] (one "page" per row, as the reference's
// paged call uses block_table = arange(batch), litemoe/flash_decode.py:10-12).
//
// Workgroup (split, kv head, row), 8 waves, covers keys
// [split*chunk, (split+1)*chunk) clipped to used[row]. A wave takes 16
// consecutive keys per iteration: lane l owns key slot l/8 of two 8-key
// groups and channels 8*(l%8) .. +7 (one 16-byte load per key for K and for
// V, 1 KB contiguous per wave load). The q.k dot product is summed over the 8
// lanes of a key with DPP lane moves; each lane keeps an online-softmax state
// (max, sum, 8-channel accumulator) per query head of the kv head, identical
// across the 8 lanes of a key slot. The next iteration's K/V loads are in
// flight while the current one is computed. States merge by log-sum-exp
// across key slots, waves, and (second kernel, only when split) splits.
//
// Reference semantics: softmax(scale * q.K^T) V over keys j < seqused_k,
// litemoe/flash_decode.py:16-22; masking litemoe/cache.py:42-47.
#include "internal.h"

namespace lm {
namespace {

constexpr int kD = 64;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kLanesPerKey = 8;
constexpr int kSlots = kWave / kLanesPerKey;  // key slots per wave
constexpr int kU = 2;                         // key groups per lane per iteration
static_assert(kU == 2, "P.V pairs the two keys of a lane's iteration");
constexpr int kKeysPerWave = kSlots * kU;     // 16
constexpr int kKeysPerIter = kKeysPerWave * kWaves;

struct Partial {
  float *o;  // [batch, q_heads, splits, 64]
  float *m;  // [batch, q_heads, splits]
  float *l;  // [batch, q_heads, splits]
};

// Scores and running maxima are kept in log2 units (scale * log2(e) folded
// into the q.k product), so every exponential is a bare v_exp_f32.
// Running max of a state that has seen no key: finite, so exp2(kEmpty - m)
// and exp2(-inf - kEmpty) are exactly 0 and the loop needs no special case.
constexpr float kEmpty = -1e30f;
// Slack of the running max: a state keeps its max until a score exceeds it
// by more than this (log2 units).
constexpr float kLazy = 8.f;

__device__ __forceinline__ float merge_factor(float m, float mnew) {
  return m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mnew);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Dot product of the 8 bf16 channels of two 16-byte words, four
// v_dot2_f32_bf16 in channel-pair order. The pairs are taken with
// shufflevector from a bf16x8 view (bit-casting indexed u32 lanes in an
// unrolled loop compiled to four dots of lane 0).
__device__ __forceinline__ float dot8_bf16(const u32x4 &a, const u32x4 &b) {
  const bf16x8 av = as_bf16x8(a), bv = as_bf16x8(b);
  float d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 0, 1),
                                            __builtin_shufflevector(bv, bv, 0, 1), 0.f, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 2, 3),
                                      __builtin_shufflevector(bv, bv, 2, 3), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 4, 5),
                                      __builtin_shufflevector(bv, bv, 4, 5), d, false);
  d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(av, av, 6, 7),
                                      __builtin_shufflevector(bv, bv, 6, 7), d, false);
  return d;
}

// The projection-fused form (lm_flash_decode_qkv): q, k and v of the row
// come from the split-K partials of the packed QKV projection instead of a
// rotated q and a cache that already holds the new key.
struct QkvIn {
  const float *part;      // [splits][batch][(q_heads + 2*kv_heads) * 64], NULL: unfused
  int splits;
  const bf16 *cos_sin;    // [table_len, 64]: cos | sin halves
  int64_t table_len;
  const int64_t *pos;     // [batch] position of the new key
  const uint8_t *active;  // [batch] or NULL (all rows write)
  const int32_t *order;   // [batch] row of workgroup z (longest first), or NULL: row z
};

constexpr int kMaxQkvSplits = 8;

// a and b summed over lane rows 0+1 and 2+3 (16-lane rows) with one
// v_permlane16_swap: the swap leaves rows [a0, b0, a2, b2] and [a1, b1, a3, b3],
// so the sum holds a's pair sums in rows 0 and 2 and b's in rows 1 and 3.
__device__ __forceinline__ float sum_lane_rows(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// c and d summed over wave halves with one v_permlane32_swap: the swap leaves
// rows [c0, c1, d0, d1] and [c2, c3, d2, d3]. Applied to two sum_lane_rows
// results it yields the four values' totals in rows 0, 1, 2, 3.
__device__ __forceinline__ float sum_row_pairs(float c, float d) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(d), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Neox rotation of one (x1, x2) pair with the reference's three roundings
// (the arithmetic of rope_kv_kernel).
__device__ __forceinline__ void rotate_pair(float x1, float x2, float c, float s, float &o1,
                                            float &o2) {
  o1 = round_bf16(round_bf16(x1 * c) - round_bf16(x2 * s));
  o2 = round_bf16(round_bf16(x2 * c) + round_bf16(x1 * s));
}

// G <= 3: four waves per SIMD (two workgroups per CU, <= 128 VGPRs); the KV stream
// needs both workgroups in flight.
// Output element (row b, q head hq, channel c): row-major [batch, q_heads*D],
// or with out_mb > 0 the fragment order of frag_offset_rows (the o_proj
// split-K projection's A operand).
__device__ __forceinline__ int64_t out_index(int64_t b, int hq, int c, int q_heads, int out_mb) {
  return out_mb ? frag_offset_rows(b, (int64_t)hq * kD + c, out_mb)
                : (b * q_heads + hq) * kD + c;
}

template <int G, bool kFused>
__global__ void __launch_bounds__(kThreads, G <= 3 ? 4 : 2)
decode_kernel(const bf16 *__restrict__ q, int64_t qs0, int64_t qs1, bf16 *__restrict__ kc,
              bf16 *__restrict__ vc, const int32_t *__restrict__ used, int q_heads,
              int kv_heads, int64_t capacity, float scale, int max_len, int chunk, int splits,
              Partial part, QkvIn in, bf16 *__restrict__ out, int out_mb) {
  __shared__ float sm_o[kWaves][G][kD];
  __shared__ float sm_m[kWaves][G];
  __shared__ float sm_l[kWaves][G];
  __shared__ float sm_qkv[kFused ? G + 2 : 1][kD];
  // Rotated q heads and new key as bf16, 16 bytes per lane group (dc).
  __shared__ u32x4 sm_rot[kFused ? G + 1 : 1][kLanesPerKey];
  const int split = blockIdx.x, h = blockIdx.y;
  // Workgroups are dispatched in z order; with a row order (rows by
  // descending length) the longest rows start first and a ragged batch ends
  // on short rows instead of a tail of long ones.
  const int64_t b = kFused && in.order ? in.order[blockIdx.z] : blockIdx.z;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int ks = lane / kLanesPerKey, dc = lane % kLanesPerKey;
  // Fused: this row's q|k|v slices of the packed projection, summed over the
  // K slices in ascending order and rounded to bf16 (F.linear's output);
  // the loads are issued before anything waits.
  f32x4 pv[kMaxQkvSplits];
  const int nstage = (G + 2) * (kD / 4);  // threads staging 4 channels each
  int64_t pnew = 0;
  if constexpr (kFused) {
    pnew = in.pos[b];
    if (threadIdx.x < nstage) {
      const int hs = threadIdx.x / (kD / 4), c4 = (threadIdx.x % (kD / 4)) * 4;
      const int head = hs < G ? h * G + hs : (hs == G ? q_heads + h : q_heads + kv_heads + h);
      const int64_t ncols = (int64_t)(q_heads + 2 * kv_heads) * kD;
      const float *src = in.part + b * ncols + (int64_t)head * kD + c4;
#pragma unroll
      for (int s = 0; s < kMaxQkvSplits; ++s)
        if (s < in.splits)
          pv[s] = *reinterpret_cast<const f32x4 *>(src + (int64_t)s * gridDim.z * ncols);
    }
  }
  int n = used[b];
  n = min(n, max_len);
  n = (int)min((int64_t)n, capacity);
  const int k0 = split * chunk;
  const int k1 = min(n, k0 + chunk);
  if (splits > 1 && k0 >= n && !kFused) return;  // the combine kernel skips empty splits
  // The new key is stored by the split whose key range holds its position
  // (split 0 when none does) and, when attended, taken from registers there:
  // its cache slot is loaded with the others but replaced.
  bool writer = false, own = false;
  if constexpr (kFused) {
    const bool writes = (!in.active || in.active[b]) && pnew >= 0 && pnew < capacity;
    const int64_t wsplit = pnew >= 0 && pnew < (int64_t)gridDim.x * chunk ? pnew / chunk : 0;
    writer = writes && split == wsplit;
    own = writer && pnew >= k0 && pnew < k1;
    if (splits > 1 && k0 >= n && !writer) return;
  }
  const int64_t head_base = ((int64_t)b * kv_heads + h) * capacity * kD + dc * 8;
  const bf16 *kbase = kc + head_base;
  const bf16 *vbase = vc + head_base;
  const int first = k0 + wave * kKeysPerWave + ks;  // key of group 0 in iteration 0
  const int niter = k1 > k0 ? (k1 - k0 + kKeysPerIter - 1) / kKeysPerIter : 0;

  // Every KV load is unconditional, its key clamped into [0, k1): a load
  // under a branch would make the compiler's wait counts fall back to
  // waiting for all loads, draining the prefetch. The loads are
  // non-temporal: each K/V word is read once per step by one workgroup, and
  // the whole cache streams through between two reads of it (cfg 3 decode
  // step 2.891-2.895 -> 2.824-2.825 ms, the attention 31.4 -> 27.7 us per
  // layer at context 1279; A/B on one box, two runs each).
  auto load = [&](u32x4 *kb, u32x4 *vb, int it) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = max(min(first + it * kKeysPerIter + u * kSlots, k1 - 1), 0);
      kb[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kbase + (int64_t)j * kD));
      vb[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vbase + (int64_t)j * kD));
    }
  };
  // Loads complete in issue order: the rotation table entries go first, then
  // the first two KV iterations, so nothing below waits on the KV stream.
  // Thread t < (G + 1) * 32 rotates pair t % 32 of head slot t / 32 (the G
  // q heads, then the new key): channels p and p + 32 of the neox halves.
  const bool in_table = kFused && pnew >= 0 && pnew < in.table_len;
  const int rot_pair = threadIdx.x % (kD / 2);
  const bool rot_thread = threadIdx.x < (G + 1) * (kD / 2);
  float cs_c = 0.f, cs_s = 0.f;
  if constexpr (kFused) {
    const bf16 *cs = in.cos_sin + (in_table ? pnew : 0) * kD;
    cs_c = bf16_to_f32(cs[rot_pair]);
    cs_s = bf16_to_f32(cs[kD / 2 + rot_pair]);
  }
  u32x4 ka[kU], va[kU], kb2[kU], vb2[kU];
  load(ka, va, 0);
  load(kb2, vb2, 1);

  // q stays bf16 (packed pairs); the softmax scale is applied to the dot.
  u32x4 qw[G];
  const float sl2 = scale * 1.4426950408889634f;
  if constexpr (kFused) {
    if (threadIdx.x < nstage) {
      const int hs = threadIdx.x / (kD / 4), c4 = (threadIdx.x % (kD / 4)) * 4;
      f32x4 acc4 = pv[0];
#pragma unroll
      for (int s = 1; s < kMaxQkvSplits; ++s)
        if (s < in.splits) acc4 += pv[s];
#pragma unroll
      for (int i = 0; i < 4; ++i) sm_qkv[hs][c4 + i] = round_bf16(acc4[i]);
    }
    __syncthreads();
    // Each (head slot, pair) is rotated once per workgroup, not once per wave.
    if (rot_thread) {
      const int hs = threadIdx.x / (kD / 2);
      const float x1 = sm_qkv[hs][rot_pair], x2 = sm_qkv[hs][kD / 2 + rot_pair];
      float o1 = x1, o2 = x2;
      if (in_table) rotate_pair(x1, x2, cs_c, cs_s, o1, o2);
      uint16_t *rot = reinterpret_cast<uint16_t *>(sm_rot[hs]);
      rot[rot_pair] = (uint16_t)f32_to_bf16(o1);
      rot[kD / 2 + rot_pair] = (uint16_t)f32_to_bf16(o2);
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) qw[g] = sm_rot[g][dc];
    // The rotated new key and the value go to the cache.
    if (writer && wave == 0 && ks == 0) {
      const int64_t at = (((int64_t)b * kv_heads + h) * capacity + pnew) * kD + dc * 8;
      u32x4 vo;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vo[i] = pack_bf16(sm_qkv[G + 1][dc * 8 + 2 * i], sm_qkv[G + 1][dc * 8 + 2 * i + 1]);
      *reinterpret_cast<u32x4 *>(kc + at) = sm_rot[G][dc];
      *reinterpret_cast<u32x4 *>(vc + at) = vo;
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g)
      qw[g] = *reinterpret_cast<const u32x4 *>(q + b * qs0 + (int64_t)(h * G + g) * qs1 + dc * 8);
  }
  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kEmpty;
    l[g] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  }

  auto compute = [&](const u32x4 *kb, const u32x4 *vb, int it) {
    float s[kU][G];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int j = first + it * kKeysPerIter + u * kSlots;
      const bool ok = j < k1;
      u32x4 kw = kb[u];
      if constexpr (kFused) {
        if (own && j == pnew) kw = sm_rot[G][dc];
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = dpp_sum8(dot8_bf16(qw[g], kw));
        s[u][g] = ok ? d * sl2 : -INFINITY;
      }
    }
    u32x4 vw[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      vw[u] = vb[u];
      if constexpr (kFused) {
        if (own && first + it * kKeysPerIter + u * kSlots == pnew) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            vw[u][i] = pack_bf16(sm_qkv[G + 1][dc * 8 + 2 * i], sm_qkv[G + 1][dc * 8 + 2 * i + 1]);
        }
      }
    }
    // Channel c's values of the two keys as one bf16 pair (v_perm_b32), so
    // P.V is one v_dot2_f32_bf16 per channel with P rounded to bf16 (as a
    // flash-attention P.V on matrix cores rounds it).
    uint32_t vp[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      vp[2 * i] = __builtin_amdgcn_perm(vw[1][i], vw[0][i], 0x05040100u);
      vp[2 * i + 1] = __builtin_amdgcn_perm(vw[1][i], vw[0][i], 0x07060302u);
    }
    // The state's reference m[g] moves only when a score exceeds it by more
    // than 8 (log2 units), so p = exp2(s - m[g]) <= 2^8 stays far inside the
    // fp32 and bf16 ranges, and after the first keys the accumulators are
    // seldom rescaled. Against rescaling at every new maximum: cfg 3 decode
    // step 2.779-2.782 -> 2.764-2.771 ms, the attention 27.8-28.2 -> 27.1-27.5
    // us per layer (A/B on one box, three runs each). One branch for the G
    // heads (taken when any lane of the wave needs a rescale; a head that
    // does not is multiplied by exactly 1): 2.762 -> 2.756 ms, the same bits.
    float mx[G];
    bool need = false;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      mx[g] = m[g];
#pragma unroll
      for (int u = 0; u < kU; ++u) mx[g] = fmaxf(mx[g], s[u][g]);
      need |= mx[g] > m[g] + kLazy;
    }
    if (need) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const bool r = mx[g] > m[g] + kLazy;
        const float corr = r ? merge_factor(m[g], mx[g]) : 1.f;
        m[g] = r ? mx[g] : m[g];
        l[g] *= corr;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] *= corr;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      // masked keys: exp2(-inf) = 0
      const float p0 = __builtin_amdgcn_exp2f(s[0][g] - m[g]);
      const float p1 = __builtin_amdgcn_exp2f(s[1][g] - m[g]);
      l[g] += p0;
      l[g] += p1;
      bf16x2 pp;
      pp[0] = (__bf16)p0;
      pp[1] = (__bf16)p1;
#pragma unroll
      for (int c = 0; c < 8; ++c)
        acc[g][c] = __builtin_amdgcn_fdot2_f32_bf16(pp, __builtin_bit_cast(bf16x2, vp[c]),
                                                    acc[g][c], false);
    }
  };

  // Two iterations in flight: iteration it+2 is issued once it is consumed
  // (past the end the loads repeat the last key and are not used).
  for (int it = 0; it < niter; it += 2) {
    compute(ka, va, it);
    load(ka, va, it + 2);
    if (it + 1 < niter) compute(kb2, vb2, it + 1);
    load(kb2, vb2, it + 3);
  }

  // Merge the 8 key slots of the wave (lanes with equal dc). Every slot is
  // rescaled to the wave's maximum once; the slot sums then pair values
  // across lane rows (v_permlane16_swap / v_permlane32_swap), so one swap
  // and one add reduce two values, and finish with one DPP add (lanes l and
  // l ^ 8). The 9G sums (acc g-major, then l) end in ceil(9G / 4) registers:
  // value 4k + r in row r (lanes 16r .. 16r + 7, channel group dc) of
  // register k.
  constexpr int kVals = 9 * G, kRegs = (kVals + 3) / 4;
  float vals[4 * kRegs];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = fmaxf(m[g], xor_lanes<8>(m[g]));
    mx = fmaxf(mx, xor_lanes<16>(mx));
    mx = fmaxf(mx, xor_lanes<32>(mx));
    // m is finite (kEmpty when the slot saw no key), so f is 0 or a real factor.
    const float f = __builtin_amdgcn_exp2f(m[g] - mx);
    m[g] = mx;
#pragma unroll
    for (int i = 0; i < 8; ++i) vals[8 * g + i] = acc[g][i] * f;
    vals[8 * G + g] = l[g] * f;
  }
#pragma unroll
  for (int v = kVals; v < 4 * kRegs; ++v) vals[v] = 0.f;
  float sums[kRegs];
#pragma unroll
  for (int k = 0; k < kRegs; ++k) {
    const float t = sum_row_pairs(sum_lane_rows(vals[4 * k], vals[4 * k + 1]),
                                  sum_lane_rows(vals[4 * k + 2], vals[4 * k + 3]));
    sums[k] = t + xor_lanes<8>(t);
  }
  if ((lane & 8) == 0) {  // ks even: one lane per (row, dc)
    const int r = lane / 16;
#pragma unroll
    for (int k = 0; k < kRegs; ++k) {
      if (k < 2 * G) {
        sm_o[wave][k / 2][dc * 8 + 4 * (k % 2) + r] = sums[k];
      } else {
        const int gl = 4 * (k - 2 * G) + r;
        if (dc == 0 && gl < G) sm_l[wave][gl] = sums[k];
      }
    }
  }
  if (lane < G) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (lane == g) sm_m[wave][g] = m[g];
  }
  __syncthreads();
  // Threads (g, channel) merge the waves.
  for (int t = threadIdx.x; t < G * kD; t += kThreads) {
    const int g = t / kD, c = t % kD;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sm_m[w][g]);
    float lsum = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = merge_factor(sm_m[w][g], mx);
      lsum += sm_l[w][g] * f;
      o += sm_o[w][g][c] * f;
    }
    const int hq = h * G + g;
    if (splits == 1) {
      out[out_index(b, hq, c, q_heads, out_mb)] = (bf16)f32_to_bf16(lsum > 0.f ? o / lsum : 0.f);
    } else {
      const int64_t slot = ((int64_t)b * q_heads + hq) * splits + split;
      part.o[slot * kD + c] = o;
      if (c == 0) {
        part.m[slot] = mx;
        part.l[slot] = lsum;
      }
    }
  }
}

// grid (q_heads, batch), one thread per channel.
__global__ void __launch_bounds__(kD)
decode_combine_kernel(const int32_t *__restrict__ used, int q_heads, int64_t capacity, int max_len,
                      int chunk, int splits, Partial part, bf16 *__restrict__ out, int out_mb) {
  const int hq = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int c = threadIdx.x;
  int n = used[b];
  n = min(n, max_len);
  n = (int)min((int64_t)n, capacity);
  const int valid = n > 0 ? min(splits, (n + chunk - 1) / chunk) : 0;
  const int64_t base = ((int64_t)b * q_heads + hq) * splits;
  float mx = -INFINITY;
  for (int s = 0; s < valid; ++s) mx = fmaxf(mx, part.m[base + s]);
  float lsum = 0.f, o = 0.f;
  for (int s = 0; s < valid; ++s) {
    const float f = merge_factor(part.m[base + s], mx);
    lsum += part.l[base + s] * f;
    o += part.o[(base + s) * kD + c] * f;
  }
  out[out_index(b, hq, c, q_heads, out_mb)] = (bf16)f32_to_bf16(lsum > 0.f ? o / lsum : 0.f);
}

int64_t workspace_bytes(int64_t batch, int64_t q_heads, int64_t splits) {
  if (splits <= 1) return 0;
  const int64_t n = batch * q_heads * splits;
  return n * kD * 4 + 2 * ((n * 4 + 255) / 256 * 256);
}

}  // namespace
}  // namespace lm

using namespace lm;

extern "C" int lm_flash_decode_workspace_size(int64_t batch, int64_t q_heads, int64_t head_dim,
                                              int64_t num_splits, int64_t *bytes) {
  LM_REQUIRE(bytes && batch >= 0 && q_heads > 0 && num_splits > 0);
  if (head_dim != kD) return LM_EUNSUPPORTED;
  *bytes = workspace_bytes(batch, q_heads, num_splits);
  return LM_OK;
}

namespace {

// Shared launcher of lm_flash_decode and lm_flash_decode_qkv.
int launch_decode(const void *q, int64_t qs0, int64_t qs1, void *k_cache, void *v_cache,
                  const int32_t *used, int64_t batch, int64_t q_heads, int64_t kv_heads,
                  int64_t capacity, float scale, int64_t max_len, int64_t num_splits,
                  const QkvIn &in, void *out, int out_mb, void *workspace,
                  int64_t workspace_bytes_, void *stream) {
  const int64_t need = workspace_bytes(batch, q_heads, num_splits);
  if (need > 0 && (!workspace || workspace_bytes_ < need)) return LM_EWORKSPACE;
  const int chunk = (int)align_up(cdiv(max_len, num_splits), 16);
  const int splits = (int)cdiv(max_len, chunk);
  Partial part{nullptr, nullptr, nullptr};
  if (splits > 1) {
    const int64_t n = batch * q_heads * num_splits;
    char *w = static_cast<char *>(workspace);
    part.o = reinterpret_cast<float *>(w);
    part.m = reinterpret_cast<float *>(w + n * kD * 4);
    part.l = reinterpret_cast<float *>(w + n * kD * 4 + (n * 4 + 255) / 256 * 256);
  }
  // Partials are indexed with the caller's split count as the stride.
  const int stride_splits = splits > 1 ? (int)num_splits : 1;
  const dim3 grid((unsigned)splits, (unsigned)kv_heads, (unsigned)batch);
  hipStream_t s = (hipStream_t)stream;
  const int G = (int)(q_heads / kv_heads);
  const bool fused = in.part != nullptr;
  switch (G) {
#define X(GG)                                                                                     \
  case GG:                                                                                        \
    if (fused)                                                                                    \
      decode_kernel<GG, true><<<grid, kThreads, 0, s>>>(                                          \
          (const bf16 *)q, qs0, qs1, (bf16 *)k_cache, (bf16 *)v_cache, used, (int)q_heads,        \
          (int)kv_heads, capacity, scale, (int)max_len, chunk, stride_splits, part, in,           \
          (bf16 *)out, out_mb);                                                                   \
    else                                                                                          \
      decode_kernel<GG, false><<<grid, kThreads, 0, s>>>(                                         \
          (const bf16 *)q, qs0, qs1, (bf16 *)k_cache, (bf16 *)v_cache, used, (int)q_heads,        \
          (int)kv_heads, capacity, scale, (int)max_len, chunk, stride_splits, part, in,           \
          (bf16 *)out, out_mb);                                                                   \
    break;
    X(1) X(2) X(3) X(4) X(6) X(8)
#undef X
    default:
      return LM_EUNSUPPORTED;
  }
  LM_CHECK_LAUNCH();
  if (splits > 1) {
    decode_combine_kernel<<<dim3((unsigned)q_heads, (unsigned)batch), kD, 0, s>>>(
        used, (int)q_heads, capacity, (int)max_len, chunk, stride_splits, part, (bf16 *)out,
        out_mb);
    LM_CHECK_LAUNCH();
  }
  return LM_OK;
}

bool decode_args_ok(int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity,
                    int64_t max_len, int64_t num_splits) {
  return batch >= 0 && q_heads > 0 && kv_heads > 0 && q_heads % kv_heads == 0 && capacity > 0 &&
         max_len > 0 && num_splits > 0 && num_splits <= 1024 && max_len < ((int64_t)1 << 30) &&
         batch <= 65535 && kv_heads <= 65535;
}

}  // namespace

extern "C" int lm_flash_decode(const void *q, int64_t qs0, int64_t qs1, const void *k_cache,
                               const void *v_cache, const int32_t *used, int64_t batch,
                               int64_t q_heads, int64_t kv_heads, int64_t capacity,
                               int64_t head_dim, float scale, int64_t max_len, int64_t num_splits,
                               void *out, void *workspace, int64_t workspace_bytes_, void *stream) {
  LM_REQUIRE(decode_args_ok(batch, q_heads, kv_heads, capacity, max_len, num_splits));
  if (head_dim != kD) return LM_EUNSUPPORTED;
  if (batch == 0) return LM_OK;
  LM_REQUIRE(q && k_cache && v_cache && used && out);
  const QkvIn in{nullptr, 0, nullptr, 0, nullptr, nullptr, nullptr};
  return launch_decode(q, qs0, qs1, const_cast<void *>(k_cache), const_cast<void *>(v_cache),
                       used, batch, q_heads, kv_heads, capacity, scale, max_len, num_splits, in,
                       out, 0, workspace, workspace_bytes_, stream);
}

namespace {

int flash_decode_qkv(const float *qkv_partials, int64_t qkv_splits, const void *cos_sin,
                     int64_t table_len, const int64_t *positions, const uint8_t *active,
                     void *k_cache, void *v_cache, const int32_t *used, const int32_t *row_order,
                     int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t capacity,
                     int64_t head_dim, float scale, int64_t max_len, int64_t num_splits, void *out,
                     bool frag_out, void *workspace, int64_t workspace_bytes_, void *stream) {
  LM_REQUIRE(decode_args_ok(batch, q_heads, kv_heads, capacity, max_len, num_splits));
  LM_REQUIRE(qkv_splits >= 1 && table_len > 0);
  if (head_dim != kD || qkv_splits > kMaxQkvSplits) return LM_EUNSUPPORTED;
  if (frag_out && batch > 128) return LM_EUNSUPPORTED;
  if (batch == 0) return LM_OK;
  LM_REQUIRE(qkv_partials && cos_sin && positions && k_cache && v_cache && used && out);
  const QkvIn in{qkv_partials, (int)qkv_splits, (const bf16 *)cos_sin, table_len, positions,
                 active, row_order};
  return launch_decode(nullptr, 0, 0, k_cache, v_cache, used, batch, q_heads, kv_heads, capacity,
                       scale, max_len, num_splits, in, out, frag_out ? frag_row_blocks(batch) : 0,
                       workspace, workspace_bytes_, stream);
}

}  // namespace

extern "C" int lm_flash_decode_qkv(const float *qkv_partials, int64_t qkv_splits,
                                   const void *cos_sin, int64_t table_len,
                                   const int64_t *positions, const uint8_t *active,
                                   void *k_cache, void *v_cache, const int32_t *used,
                                   const int32_t *row_order, int64_t batch, int64_t q_heads,
                                   int64_t kv_heads,
                                   int64_t capacity, int64_t head_dim, float scale,
                                   int64_t max_len, int64_t num_splits, void *out,
                                   void *workspace, int64_t workspace_bytes_, void *stream) {
  return flash_decode_qkv(qkv_partials, qkv_splits, cos_sin, table_len, positions, active,
                          k_cache, v_cache, used, row_order, batch, q_heads, kv_heads, capacity,
                          head_dim, scale, max_len, num_splits, out, false, workspace,
                          workspace_bytes_, stream);
}

extern "C" int lm_flash_decode_qkv_frag(const float *qkv_partials, int64_t qkv_splits,
                                        const void *cos_sin, int64_t table_len,
                                        const int64_t *positions, const uint8_t *active,
                                        void *k_cache, void *v_cache, const int32_t *used,
                                        const int32_t *row_order, int64_t batch, int64_t q_heads,
                                        int64_t kv_heads, int64_t capacity, int64_t head_dim,
                                        float scale, int64_t max_len, int64_t num_splits,
                                        void *out_frag, void *workspace, int64_t workspace_bytes_,
                                        void *stream) {
  return flash_decode_qkv(qkv_partials, qkv_splits, cos_sin, table_len, positions, active,
                          k_cache, v_cache, used, row_order, batch, q_heads, kv_heads, capacity,
                          head_dim, scale, max_len, num_splits, out_frag, true, workspace,
                          workspace_bytes_, stream);
}
