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

constexpr int kArgThreads = 1024;
constexpr int kArgChunks = 8;  // 16-byte loads per lane in flight

// (value, index) order of torch.argmax: larger value first, then lower index;
// NaN above everything (torch.argmax returns the first NaN).
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

__global__ void __launch_bounds__(kArgThreads)
epilogue_kernel(const bf16 *__restrict__ logits, int64_t ld, float inv_scaling, int vocab,
                const uint8_t *__restrict__ valid, int64_t *__restrict__ next,
                int64_t *__restrict__ length, int64_t *__restrict__ generated,
                const int64_t *__restrict__ budget, uint8_t *__restrict__ active,
                int64_t *__restrict__ emit, const int64_t *__restrict__ eos, int neos,
                int ignore_eos, int64_t *__restrict__ ring, int64_t depth,
                const int64_t *__restrict__ step_counter) {
  __shared__ float sv[kArgThreads / kWave];
  __shared__ int si[kArgThreads / kWave];
  const int64_t row = blockIdx.x;
  // The row is read in aligned 16-byte chunks (rows of an odd vocab start
  // anywhere): chunk c holds values 8c - lead .. 8c - lead + 7, and only
  // those in [0, vocab) count. An aligned chunk never leaves the page of the
  // row value it holds.
  const bf16 *lr = logits + row * ld;
  const int mis = (int)(reinterpret_cast<uintptr_t>(lr) & 15);  // bytes past the last 16-byte boundary
  const u32x4 *chunks = reinterpret_cast<const u32x4 *>(reinterpret_cast<const char *>(lr) - mis);
  const int lead = mis / 2;
  const int nchunks = (lead + vocab + 7) / 8;
  // A lane visits its values in increasing index order, so a strict
  // comparison of orderable keys (NaN above everything) keeps the first
  // index of its maximum; lanes and waves then merge with better().
  uint32_t bk = 0;  // below every real key
  int bi = vocab;   // none yet
  u32x4 raw[kArgChunks];
  auto load = [&](int base) {
#pragma unroll
    for (int u = 0; u < kArgChunks; ++u) raw[u] = chunks[min(base + u * kArgThreads, nchunks - 1)];
  };
  auto scan = [&](int base) {
#pragma unroll
    for (int u = 0; u < kArgChunks; ++u) {
      float f[8];
      unpack8(raw[u], f);
      const int v0 = (base + u * kArgThreads) * 8 - lead;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int v = v0 + j;
        uint32_t h = f32_to_bf16(f[j] * inv_scaling);
        h = h == 0x8000u ? 0u : h;  // -0 ties with +0, as in a float compare
        const uint32_t key = (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);  // NaN is 0x7fc0: top
        const bool in = base + u * kArgThreads < nchunks && v >= 0 && v < vocab;
        if (in && key + 1u > bk) {  // key + 1 > 0 for every real value
          bk = key + 1u;
          bi = v;
        }
      }
    }
  };
  // First round (rows up to 8 * kArgThreads * kArgChunks values): every
  // chunk load, then the row's state, are issued before anything waits; the
  // state is used only at the end. eos may be NULL when neos == 0: the row's
  // own counter is read instead.
  load(threadIdx.x);
  const bool val = valid[row] != 0;
  const int64_t gen = generated[row], len = length[row], bud = budget[row];
  const int64_t eos_read = *(neos > 0 ? eos : generated + row);
  __builtin_amdgcn_sched_barrier(0);
  scan(threadIdx.x);
  for (int base = threadIdx.x + kArgThreads * kArgChunks; base < nchunks;
       base += kArgThreads * kArgChunks) {
    load(base);
    scan(base);
  }
  const int64_t eos_first = neos > 0 ? eos_read : -1;
  float best = -INFINITY;
  if (bi < vocab) {
    const uint32_t key = bk - 1u;
    best = bf16_to_f32((key & 0x8000u) ? (key & 0x7fffu) : (~key & 0xffffu));
  }
  // Wave then workgroup reduction of (value, index).
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgThreads / kWave; ++w)
      if (better(sv[w], si[w], best, bi)) {
        best = sv[w];
        bi = si[w];
      }
    const int64_t candidate = bi;
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
    length[row] = len + (val ? 1 : 0);
    generated[row] = gen1;
    if (val) next[row] = candidate;
    bool done = gen1 >= bud;
    if (!ignore_eos && neos > 0) {
      done = done || candidate == eos_first;
      for (int e = 1; e < neos; ++e) done = done || candidate == eos[e];
    }
    active[row] = val && !done;
  }
}

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

extern "C" int lm_greedy_epilogue(const void *logits, int64_t ld, float logits_scaling,
                                  int64_t vocab, int64_t rows, const uint8_t *valid,
                                  int64_t *next, int64_t *length, int64_t *generated,
                                  const int64_t *budget, uint8_t *active, int64_t *emit,
                                  const int64_t *eos, int64_t neos, int ignore_eos,
                                  int64_t *emit_ring, int64_t ring_depth,
                                  const int64_t *step_counter, void *stream) {
  LM_REQUIRE(rows >= 0 && vocab > 0 && vocab < ((int64_t)1 << 31) && ld >= vocab && neos >= 0 &&
             logits_scaling > 0.f && (!emit_ring || (ring_depth > 0 && step_counter)));
  if (rows == 0) return LM_OK;
  LM_REQUIRE(logits && valid && next && length && generated && budget && active && emit &&
             (neos == 0 || eos));
  const float inv_scaling = 1.0f / logits_scaling;
  epilogue_kernel<<<dim3((unsigned)rows), kArgThreads, 0, (hipStream_t)stream>>>(
      (const bf16 *)logits, ld, inv_scaling, (int)vocab, valid, next, length, generated,
      budget, active, emit, eos, (int)neos, ignore_eos, emit_ring, ring_depth, step_counter);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
