// The ends of a greedy decode step, each one launch:
//
//   prologue  valid = active; pos = valid ? length : 0; used = pos + 1;
//             x = bf16(embedding[next] * multiplier); z = rmsnorm(x)
//   epilogue  candidate = argmax_v bf16(logits[v] * (1 / logits_scaling))
//             (first index of the maximum, as torch.argmax); then the
//             engine's state update and the emit row. torch divides a bf16
//             tensor by a Python scalar as a product with the fp32
//             reciprocal, so the epilogue does the same.
//
// Emit ring: with a step counter the prologue counts the step (one thread
// adds 1) and the epilogue also stores each emit row into slot
// (counter - 1) % depth of a ring in pinned host memory, with system-scope
// stores that go straight to host memory. The decode step then publishes
// its emit rows itself, inside the captured graph: the host reads a slot
// after an event recorded behind the step, with no copy or stream of its
// own.
//
// Reference: litemoe/engine.py:87-102 (decode_step), litemoe/model.py:103
// (used), :104 (embedding * multiplier), :106 (first norm) and :127
// (logits / logits_scaling).
// The prologue's norm has rmsnorm_kernel's reduction order, so x and z are
// bitwise those of the unfused ops.
#include "internal.h"

namespace lm {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxVec = 2;  // hidden <= kMaxVec * 8 * kThreads

__global__ void __launch_bounds__(kThreads)
prologue_kernel(const uint8_t *__restrict__ active, const int64_t *__restrict__ length,
                const int64_t *__restrict__ next, const bf16 *__restrict__ table, float multiplier,
                const bf16 *__restrict__ nw, float eps, bf16 *__restrict__ x,
                bf16 *__restrict__ z, uint8_t *__restrict__ valid,
                int64_t *__restrict__ positions, int32_t *__restrict__ used,
                int32_t *__restrict__ order, int64_t *__restrict__ step_counter, int hidden,
                int64_t vocab) {
  __shared__ float red[kThreads / kWave];
  __shared__ float rank_red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const int nvec = hidden / 8;
  const int64_t tok = min(max(next[row], (int64_t)0), vocab - 1);
  const u32x4 *er = reinterpret_cast<const u32x4 *>(table + tok * hidden);
  u32x4 ev[kMaxVec], gv[kMaxVec];
#pragma unroll
  for (int v = 0; v < kMaxVec; ++v) {
    const int i = min((int)threadIdx.x + v * kThreads, nvec - 1);
    ev[v] = er[i];
    gv[v] = reinterpret_cast<const u32x4 *>(nw)[i];
  }
  if (threadIdx.x == 0) {
    const bool act = active[row] != 0;
    const int64_t pos = act ? length[row] : 0;
    valid[row] = act;
    positions[row] = pos;
    used[row] = (int32_t)(pos + 1);
    if (step_counter && row == 0) *step_counter += 1;  // no other thread of the grid touches it
  }
  if (order) {
    // This row's rank among all rows by descending used (equal used: lower
    // row first), i.e. order = the stable argsort of -used; the decode
    // attention runs its workgroups in that order.
    const int rows = (int)gridDim.x;
    const int64_t mine = active[row] ? length[row] + 1 : 1;
    float cnt = 0.f;  // exact below 2^24
    for (int j = threadIdx.x; j < rows; j += kThreads) {
      const int64_t u = active[j] ? length[j] + 1 : 1;
      cnt += (u > mine || (u == mine && j < row)) ? 1.f : 0.f;
    }
    cnt = wave_sum(cnt);
    if (threadIdx.x % kWave == 0) rank_red[threadIdx.x / kWave] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < kThreads / kWave; ++w) r += rank_red[w];
      order[(int)r] = (int32_t)row;
    }
  }
  float xn[kMaxVec][8];
  float ss = 0.f;
#pragma unroll
  for (int v = 0; v < kMaxVec; ++v) {
    const int i = threadIdx.x + v * kThreads;
    if (i >= nvec) continue;
    float f[8];
    unpack8(ev[v], f);
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      xn[v][c] = round_bf16(f[c] * multiplier);
      ss += xn[v][c] * xn[v][c];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = pack_bf16(xn[v][2 * c], xn[v][2 * c + 1]);
    reinterpret_cast<u32x4 *>(x + row * hidden)[i] = o;
  }
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / kWave; ++w) total += red[w];
  const float scale = 1.0f / sqrtf(total / (float)hidden + eps);
#pragma unroll
  for (int v = 0; v < kMaxVec; ++v) {
    const int i = threadIdx.x + v * kThreads;
    if (i >= nvec) continue;
    float g[8];
    unpack8(gv[v], g);
    u32x4 o;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      o[c] = pack_bf16(round_bf16(xn[v][2 * c] * scale) * g[2 * c],
                       round_bf16(xn[v][2 * c + 1] * scale) * g[2 * c + 1]);
    reinterpret_cast<u32x4 *>(z + row * hidden)[i] = o;
  }
}

// The argmax of a logits row is split over `parts` workgroups per row, each
// scanning a slice of the row's aligned 16-byte chunks, so the whole GPU
// takes part (one workgroup per row leaves most CUs idle and the scan's VALU
// work serial). A slice's result is one 64-bit word: (key + 1) << 32 |
// (0xffffffff - index), key the orderable bf16 of the scaled value (NaN
// above everything, -0 equal to +0). The largest word is the largest value
// at its lowest index (torch.argmax); 0 means an empty slice. The state
// update then reduces the row's words.
constexpr int kArgThreads = 256;
constexpr int kArgChunks = 2;  // 16-byte loads per lane per round (a slice is about two per lane)

__device__ __forceinline__ uint64_t pack_best(uint32_t key1, int index) {
  return ((uint64_t)key1 << 32) | (uint64_t)(0xffffffffu - (uint32_t)index);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, kWave);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, kWave);
    v = max_u64(v, ((uint64_t)hi << 32) | lo);
  }
  return v;
}

__global__ void __launch_bounds__(kArgThreads)
argmax_part_kernel(const bf16 *__restrict__ logits, int64_t ld, float inv_scaling, int vocab,
                   int parts, uint64_t *__restrict__ best_out) {
  __shared__ uint64_t sb[kArgThreads / kWave];
  const int64_t row = blockIdx.y;
  const int part = blockIdx.x;
  // The row is read in aligned 16-byte chunks (rows of an odd vocab start
  // anywhere): chunk c holds values 8c - lead .. 8c - lead + 7, and only
  // those in [0, vocab) count. An aligned chunk never leaves the page of the
  // row value it holds.
  const bf16 *lr = logits + row * ld;
  const int mis = (int)(reinterpret_cast<uintptr_t>(lr) & 15);
  const u32x4 *chunks = reinterpret_cast<const u32x4 *>(reinterpret_cast<const char *>(lr) - mis);
  const int lead = mis / 2;
  const int nchunks = (lead + vocab + 7) / 8;
  const int per = (nchunks + parts - 1) / parts;
  const int c0 = part * per, c1 = min(nchunks, c0 + per);
  // A lane visits its values in increasing index order, so a strict
  // comparison of orderable keys keeps the first index of its maximum.
  uint32_t bk = 0;  // key + 1 of the best so far (0: none)
  int bi = vocab;
  u32x4 raw[kArgChunks];
  for (int base = c0 + threadIdx.x; base < c1; base += kArgThreads * kArgChunks) {
    // every chunk load of the round before any arithmetic (clamped indices,
    // masked below)
#pragma unroll
    for (int u = 0; u < kArgChunks; ++u) raw[u] = chunks[min(base + u * kArgThreads, c1 - 1)];
#pragma unroll
    for (int u = 0; u < kArgChunks; ++u) {
      float f[8];
      unpack8(raw[u], f);
      const int c = base + u * kArgThreads;
      const int v0 = c * 8 - lead;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // two values per conversion (v_cvt_pk_bf16_f32, NaN made 0x7fc0)
        const uint32_t pair = pack_bf16(f[2 * j] * inv_scaling, f[2 * j + 1] * inv_scaling);
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          uint32_t h = h2 ? pair >> 16 : pair & 0xffffu;
          const int v = v0 + 2 * j + h2;
          h = h == 0x8000u ? 0u : h;  // -0 ties with +0, as in a float compare
          const uint32_t key = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);  // NaN 0x7fc0: top
          const bool in = c < c1 && v >= 0 && v < vocab;
          if (in && key + 1u > bk) {
            bk = key + 1u;
            bi = v;
          }
        }
      }
    }
  }
  uint64_t b = wave_max_u64(bk ? pack_best(bk, bi) : 0ull);
  if (threadIdx.x % kWave == 0) sb[threadIdx.x / kWave] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kArgThreads / kWave; ++w) b = max_u64(b, sb[w]);
    best_out[row * parts + part] = b;
  }
}

// The row's slice results reduced to the candidate token, then the emit row
// and the engine's state update (one wave per row).
__global__ void __launch_bounds__(kWave)
greedy_update_kernel(const uint64_t *__restrict__ best, int parts, const uint8_t *__restrict__ valid,
                     int64_t *__restrict__ next, int64_t *__restrict__ length,
                     int64_t *__restrict__ generated, const int64_t *__restrict__ budget,
                     uint8_t *__restrict__ active, int64_t *__restrict__ emit,
                     const int64_t *__restrict__ eos, int neos, int ignore_eos,
                     int64_t *__restrict__ ring, int64_t depth,
                     const int64_t *__restrict__ step_counter) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  uint64_t b = 0;
  for (int p = lane; p < parts; p += kWave) b = max_u64(b, best[row * parts + p]);
  b = wave_max_u64(b);
  if (lane == 0) {
    const int64_t candidate = (int64_t)(0xffffffffu - (uint32_t)b);
    const bool val = valid[row] != 0;
    const int64_t gen = generated[row];
    emit[row * 3 + 0] = candidate;
    emit[row * 3 + 1] = gen;
    emit[row * 3 + 2] = val;
    if (ring) {
      const int64_t slot = ((*step_counter - 1) % depth + depth) % depth;
      int64_t *dst = ring + (slot * (int64_t)gridDim.x + row) * 3;
      __hip_atomic_store(dst + 0, candidate, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(dst + 1, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      __hip_atomic_store(dst + 2, (int64_t)val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    const int64_t gen1 = gen + (val ? 1 : 0);
    length[row] += val ? 1 : 0;
    generated[row] = gen1;
    if (val) next[row] = candidate;
    bool done = gen1 >= budget[row];
    if (!ignore_eos)
      for (int e = 0; e < neos; ++e) done = done || candidate == eos[e];
    active[row] = val && !done;
  }
}

// Slices per row: about 4096 values each, at most 64.
int arg_parts(int64_t vocab) { return (int)max((int64_t)1, min((int64_t)64, cdiv(vocab, 4096))); }

}  // namespace
}  // namespace lm

using namespace lm;

extern "C" int lm_decode_prologue(const uint8_t *active, const int64_t *length, const int64_t *next,
                                  const void *embedding, float multiplier, const void *norm_weight,
                                  float eps, void *x, void *z, uint8_t *valid, int64_t *positions,
                                  int32_t *used, int32_t *row_order, int64_t *step_counter,
                                  int64_t rows, int64_t hidden, int64_t vocab, void *stream) {
  LM_REQUIRE(rows >= 0 && hidden > 0 && vocab > 0);
  if (hidden % 8 || hidden > kMaxVec * 8 * kThreads) return LM_EUNSUPPORTED;
  if (rows == 0) return LM_OK;
  LM_REQUIRE(active && length && next && embedding && norm_weight && x && z && valid &&
             positions && used);
  prologue_kernel<<<dim3((unsigned)rows), kThreads, 0, (hipStream_t)stream>>>(
      active, length, next, (const bf16 *)embedding, multiplier, (const bf16 *)norm_weight, eps,
      (bf16 *)x, (bf16 *)z, valid, positions, used, row_order, step_counter, (int)hidden, vocab);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_greedy_epilogue_workspace_size(int64_t rows, int64_t vocab, int64_t *bytes) {
  LM_REQUIRE(bytes && rows >= 0 && vocab > 0);
  *bytes = rows * arg_parts(vocab) * 8;
  return LM_OK;
}

extern "C" int lm_greedy_epilogue(const void *logits, int64_t ld, float logits_scaling,
                                  int64_t vocab, int64_t rows, const uint8_t *valid,
                                  int64_t *next, int64_t *length, int64_t *generated,
                                  const int64_t *budget, uint8_t *active, int64_t *emit,
                                  const int64_t *eos, int64_t neos, int ignore_eos,
                                  int64_t *emit_ring, int64_t ring_depth,
                                  const int64_t *step_counter, void *workspace,
                                  int64_t workspace_bytes, void *stream) {
  LM_REQUIRE(rows >= 0 && vocab > 0 && vocab < ((int64_t)1 << 31) && ld >= vocab && neos >= 0 &&
             logits_scaling > 0.f && (!emit_ring || (ring_depth > 0 && step_counter)) &&
             rows <= 65535);
  if (rows == 0) return LM_OK;
  LM_REQUIRE(logits && valid && next && length && generated && budget && active && emit &&
             (neos == 0 || eos) && workspace);
  const int parts = arg_parts(vocab);
  if (workspace_bytes < rows * parts * 8) return LM_EWORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  uint64_t *best = static_cast<uint64_t *>(workspace);
  argmax_part_kernel<<<dim3((unsigned)parts, (unsigned)rows), kArgThreads, 0, s>>>(
      (const bf16 *)logits, ld, 1.0f / logits_scaling, (int)vocab, parts, best);
  LM_CHECK_LAUNCH();
  greedy_update_kernel<<<dim3((unsigned)rows), kWave, 0, s>>>(
      best, parts, valid, next, length, generated, budget, active, emit, eos, (int)neos,
      ignore_eos, emit_ring, ring_depth, step_counter);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
