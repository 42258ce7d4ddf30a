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

// Orderable key of a bf16 value: larger value, larger key; -0 equal to +0;
// the canonical NaN 0x7fc0 above every number.
__device__ __forceinline__ uint32_t order_key(uint32_t h) {
  h = h == 0x8000u ? 0u : h;
  return (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
}

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
          const uint32_t h = h2 ? pair >> 16 : pair & 0xffffu;
          const int v = v0 + 2 * j + h2;
          const uint32_t key = order_key(h);
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

// The LM head product with the greedy argmax in its epilogue: one launch
// streams the head weights [vocab, hidden] once and leaves, per row and
// workgroup, the best (key, index) word of the workgroup's vocabulary
// slice, in argmax_part_kernel's format; greedy_update_kernel then reduces
// the words and updates the state. The raw head output (F.linear's bf16
// logits) is never written unless the caller asks for it.
//
// Workgroup = 4 waves over a slice of 4*TW vocabulary tiles of 16 rows;
// every wave owns TW tiles and all M (<= 16*MB) rows, so no partial sums
// cross waves. The head rows are the MFMA B operand, read from the head in
// fragment order, k-step major (lm_head_pack: each wave load is 1 KB
// contiguous, a wave's TW tiles of one k-step are adjacent, and all the
// workgroups of a k-step read one contiguous block of vocab*64 bytes, so
// the DRAM sees a front sweeping through memory rather than 64 bytes of 48
// rows at a time) into a register ring kHeadDepth k-steps ahead. The rows
// z [M, hidden] are the A
// operand, read from LDS, where they are staged in phases of KP k-steps
// (at most 32 KB, two buffers; 16-byte chunk c of row r at c ^ (r & 15),
// conflict-free).
// Vector loads complete in issue order, so the loads of phase p+1 are
// issued right behind the head loads of k-step (p+1)*KP: waiting for them at
// the end of phase p then waits for no head load that is not due next, and
// the head stream never drains. Per lane: C rows 4*(l/16)+i of vocabulary
// column l%16 of a tile. logits = bf16(sum) (one rounding, as F.linear's
// output); the argmax key is that of bf16(logits * (1 / logits_scaling)),
// as in argmax_part_kernel, so the candidate equals lm_greedy_epilogue's
// over the same logits.
constexpr int kHeadWaves = 4;
constexpr int kHeadThreads = kHeadWaves * kWave;
// Tuning knobs (compile-time): k-steps of head loads in flight per wave,
// LDS bytes for one phase of z.
#ifndef LM_HEAD_DEPTH
#define LM_HEAD_DEPTH 4
#endif
#ifndef LM_HEAD_PHASE_KB
#define LM_HEAD_PHASE_KB 16
#endif
constexpr int kHeadDepth = LM_HEAD_DEPTH;
constexpr int kHeadPhaseBytes = LM_HEAD_PHASE_KB << 10;

__device__ __forceinline__ u32x4 load16(const bf16 *p) { return *reinterpret_cast<const u32x4 *>(p); }

// Vocabulary tiles per wave. With the head read non-temporal, 2 (385
// workgroups at the Granite vocabulary, about one and a half waves per SIMD)
// beats 3 (257 workgroups, one wave per SIMD): the cfg 3 decode step
// 2.777-2.780 -> 2.768-2.769 ms, 1 tile 2.770 ms (A/B on one box, three runs
// each). Before the head's loads were non-temporal the three were level.
template <int MB>
constexpr int head_tiles_per_wave() { return 2; }

// k-steps per phase: the largest divisor of KS whose phase fits the LDS
// budget (a k-step of z is MB*16 rows x 64 bytes).
// (at least 4, the k-steps of one swizzle row of 16 chunks)
template <int MB, int KS>
constexpr int head_phase_steps() {
  int kp = KS;
  while (kp > 4 && (KS % kp != 0 || MB * 16 * kp * 64 > kHeadPhaseBytes || kp % 4 != 0)) --kp;
  return kp;
}

template <int MB, int KS>
__global__ void __launch_bounds__(kHeadThreads)
head_argmax_kernel(const bf16 *__restrict__ z, int64_t ldz, const bf16 *__restrict__ head,
                   int M, int vocab, float inv_scaling, bf16 *__restrict__ logits, int64_t ldo,
                   uint64_t *__restrict__ best_out) {
  constexpr int TW = head_tiles_per_wave<MB>();
  constexpr int kRows = MB * 16;
  constexpr int KP = head_phase_steps<MB, KS>();
  constexpr int NP = KS / KP;
  constexpr int kChunksPerRow = KP * 4;                         // 16-byte chunks of a phase row
  constexpr int kPer = kRows * kChunksPerRow / kHeadThreads;    // chunks per thread and phase
  constexpr int D = kHeadDepth < KS ? kHeadDepth : KS;
  // phase p+1 is issued behind the head loads of k-step (p+1)*KP, i.e. after
  // computing k-step (p+1)*KP - D (at the start of phase p if KP <= D)
  constexpr int kIssueAt = KP > D ? KP - D : 0;
  static_assert(KS % KP == 0 && KP % 4 == 0 && kPer >= 1 &&
                kRows * kChunksPerRow % kHeadThreads == 0, "phase shape");
  __shared__ u32x4 abuf[2][kRows * kChunksPerRow];
  __shared__ uint64_t wbest[kHeadWaves][kRows];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  const int tile0 = ((int)blockIdx.x * kHeadWaves + wave) * TW;
  const int tiles = (vocab + 15) / 16;
  const bf16 *wp[TW];
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    // tiles past the vocabulary repeat the last one (loads stay in bounds;
    // those columns are masked below)
    const int tile = min(tile0 + t, tiles - 1);
    wp[t] = head + ((int64_t)tile * kWave + lane) * 8;
  }
  // D + 1 slots: the refill of k-step ks + D is issued before the MFMAs of
  // k-step ks, into a slot those MFMAs do not read.
  u32x4 ring[D + 1][TW];
  u32x4 ra[kPer];
  // The head is read once per step, so its loads are non-temporal (with the
  // attention's K/V loads also non-temporal, the decode step 2.825 -> 2.797
  // ms at cfg 3; A/B on one box, two runs each).
  auto load_b = [&](int ks) {
#pragma unroll
    for (int t = 0; t < TW; ++t)
      ring[ks % (D + 1)][t] =
          __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp[t] + (int64_t)ks * tiles * kWave * 8));
  };
  auto load_a = [&](int p) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int q = (int)threadIdx.x + i * kHeadThreads;
      const int row = q / kChunksPerRow, c = q % kChunksPerRow;
      ra[i] = load16(z + (int64_t)min(row, M - 1) * ldz + p * KP * 32 + c * 8);
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int q = (int)threadIdx.x + i * kHeadThreads;
      const int row = q / kChunksPerRow, c = q % kChunksPerRow;
      abuf[buf][row * kChunksPerRow + (c ^ (row & 15))] = ra[i];
    }
  };
  load_a(0);
#pragma unroll
  for (int ks = 0; ks < D; ++ks) load_b(ks);
  store_a(0);
  __syncthreads();
  f32x4 acc[TW][MB];
#pragma unroll
  for (int t = 0; t < TW; ++t)
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[t][m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int p = ks / KP, j = ks % KP;
    if (NP > 1 && p + 1 < NP && j == kIssueAt && kIssueAt == 0) load_a(p + 1);
    if (ks + D < KS) load_b(ks + D);
    if (NP > 1 && p + 1 < NP && j == kIssueAt && kIssueAt > 0) load_a(p + 1);
    // Keep the refill ahead of the MFMAs: left alone, the scheduler sinks
    // the loads below later k-steps' MFMAs and the ring drains.
    __builtin_amdgcn_sched_barrier(0);
    u32x4 a[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m)
      a[m] = abuf[p & 1][(m * 16 + col) * kChunksPerRow + ((4 * j + grp) ^ col)];
#pragma unroll
    for (int t = 0; t < TW; ++t)
#pragma unroll
      for (int m = 0; m < MB; ++m) acc[t][m] = mfma16x16x32(a[m], ring[ks % (D + 1)][t], acc[t][m]);
    // Phase p+1 goes into the other buffer, last read in phase p-1, which
    // every wave left at the previous barrier; one barrier per phase.
    if (NP > 1 && p + 1 < NP && j == KP - 1) {
      store_a((p + 1) & 1);
      __syncthreads();
    }
  }
  // Epilogue: bf16 logits, optional store, running best per row over this
  // lane's columns (ascending index, strict compare keeps the first).
  uint32_t bk[MB][4];
  int bi[MB][4];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      bk[m][i] = 0u;
      bi[m][i] = vocab;
    }
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    const int v = (tile0 + t) * 16 + col;
    const bool in = v < vocab;
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t h = f32_to_bf16(acc[t][m][i]);
        const int row = m * 16 + grp * 4 + i;
        if (logits && in && row < M) logits[(int64_t)row * ldo + v] = (bf16)h;
        const uint32_t key1 = order_key(f32_to_bf16(bf16_to_f32(h) * inv_scaling)) + 1u;
        if (in && key1 > bk[m][i]) {
          bk[m][i] = key1;
          bi[m][i] = v;
        }
      }
  }
  // Largest word over the 16 lanes of each row group, then over the waves.
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint64_t b = bk[m][i] ? pack_best(bk[m][i], bi[m][i]) : 0ull;
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) {
        const uint32_t lo = __shfl_xor((uint32_t)b, off, kWave);
        const uint32_t hi = __shfl_xor((uint32_t)(b >> 32), off, kWave);
        b = max_u64(b, ((uint64_t)hi << 32) | lo);
      }
      if (col == 0) wbest[wave][m * 16 + grp * 4 + i] = b;
    }
  __syncthreads();
  for (int row = threadIdx.x; row < M; row += kHeadThreads) {
    uint64_t b = wbest[0][row];
#pragma unroll
    for (int w = 1; w < kHeadWaves; ++w) b = max_u64(b, wbest[w][row]);
    best_out[(int64_t)row * gridDim.x + blockIdx.x] = b;
  }
}

int head_row_blocks(int64_t rows) { return rows <= 16 ? 1 : rows <= 32 ? 2 : rows <= 64 ? 4 : 8; }

// Workgroups of the fused head: one per slice of 4*TW vocabulary tiles.
int64_t head_parts(int64_t rows, int64_t vocab) {
  const int mb = head_row_blocks(rows);
  const int tw = mb <= 4 ? head_tiles_per_wave<4>() : head_tiles_per_wave<8>();
  return cdiv(cdiv(vocab, 16), (int64_t)kHeadWaves * tw);
}

// The head in MFMA fragment order, k-step major: 16-byte chunk (k-step,
// tile, lane) = head[16*tile + lane%16][32*k-step + 8*(lane/16) .. +8],
// zero past the vocabulary (one thread per chunk).
__global__ void __launch_bounds__(256)
head_pack_kernel(const bf16 *__restrict__ head, int vocab, int hidden, int64_t chunks,
                 bf16 *__restrict__ packed) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= chunks) return;
  const int64_t tiles = cdiv(vocab, 16);
  const int lane = (int)(q % kWave);
  const int64_t rest = q / kWave;
  const int64_t tile = rest % tiles;
  const int ks = (int)(rest / tiles);
  const int64_t row = tile * 16 + lane % 16;
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (row < vocab) v = load16(head + row * hidden + ks * 32 + (lane / 16) * 8);
  reinterpret_cast<u32x4 *>(packed)[q] = v;
}

bool head_shape_ok(int64_t rows, int64_t vocab, int64_t hidden) {
  if (rows < 1 || rows > 128 || vocab < 1 || vocab >= ((int64_t)1 << 31)) return false;
  return hidden == 512 || hidden == 1024 || hidden == 1536 || hidden == 2048;
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

extern "C" int lm_head_greedy_workspace_size(int64_t rows, int64_t vocab, int64_t hidden,
                                             int64_t *bytes) {
  LM_REQUIRE(bytes && rows >= 0 && vocab > 0 && hidden > 0);
  if (rows == 0) {
    *bytes = 0;
    return LM_OK;
  }
  if (!head_shape_ok(rows, vocab, hidden)) return LM_EUNSUPPORTED;
  *bytes = rows * head_parts(rows, vocab) * 8;
  return LM_OK;
}

extern "C" int lm_head_greedy(const void *z, int64_t ldz, const void *head, int64_t rows,
                              int64_t vocab, int64_t hidden, float logits_scaling, void *logits,
                              int64_t ldo, const uint8_t *valid, int64_t *next, int64_t *length,
                              int64_t *generated, const int64_t *budget, uint8_t *active,
                              int64_t *emit, const int64_t *eos, int64_t neos, int ignore_eos,
                              int64_t *emit_ring, int64_t ring_depth, const int64_t *step_counter,
                              void *workspace, int64_t workspace_bytes, void *stream) {
  LM_REQUIRE(rows >= 0 && vocab > 0 && hidden > 0 && ldz >= hidden && ldz % 8 == 0 &&
             (!logits || ldo >= vocab) && neos >= 0 && logits_scaling > 0.f &&
             (!emit_ring || (ring_depth > 0 && step_counter)));
  if (rows == 0) return LM_OK;
  if (!head_shape_ok(rows, vocab, hidden)) return LM_EUNSUPPORTED;
  LM_REQUIRE(z && head && valid && next && length && generated && budget && active && emit &&
             (neos == 0 || eos) && workspace);
  LM_REQUIRE((reinterpret_cast<uintptr_t>(z) & 15) == 0 && (reinterpret_cast<uintptr_t>(head) & 15) == 0);
  const int64_t parts = head_parts(rows, vocab);
  if (workspace_bytes < rows * parts * 8) return LM_EWORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  uint64_t *best = static_cast<uint64_t *>(workspace);
  const float inv = 1.0f / logits_scaling;
  const int mb = head_row_blocks(rows);
  const dim3 grid((unsigned)parts);
  bool launched = false;
#define LM_HEAD(MB, KS)                                                                          \
  if (!launched && mb == MB && hidden == KS * 32) {                                              \
    head_argmax_kernel<MB, KS><<<grid, kHeadThreads, 0, s>>>(                                    \
        (const bf16 *)z, ldz, (const bf16 *)head, (int)rows, (int)vocab, inv, (bf16 *)logits,   \
        ldo, best);                                                                              \
    launched = true;                                                                             \
  }
#define LM_HEAD_KS(MB) LM_HEAD(MB, 16) LM_HEAD(MB, 32) LM_HEAD(MB, 48) LM_HEAD(MB, 64)
  LM_HEAD_KS(1) LM_HEAD_KS(2) LM_HEAD_KS(4) LM_HEAD_KS(8)
#undef LM_HEAD_KS
#undef LM_HEAD
  if (!launched) return LM_EUNSUPPORTED;
  LM_CHECK_LAUNCH();
  greedy_update_kernel<<<dim3((unsigned)rows), kWave, 0, s>>>(
      best, (int)parts, valid, next, length, generated, budget, active, emit, eos, (int)neos,
      ignore_eos, emit_ring, ring_depth, step_counter);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

extern "C" int lm_head_pack_size(int64_t vocab, int64_t hidden, int64_t *bytes) {
  LM_REQUIRE(bytes && vocab > 0 && hidden > 0);
  if (hidden % 32) return LM_EUNSUPPORTED;
  *bytes = cdiv(vocab, 16) * 16 * hidden * 2;
  return LM_OK;
}

extern "C" int lm_head_pack(const void *head, int64_t vocab, int64_t hidden, void *packed,
                            void *stream) {
  LM_REQUIRE(head && packed && vocab > 0 && vocab < ((int64_t)1 << 31) && hidden > 0);
  if (hidden % 32) return LM_EUNSUPPORTED;
  LM_REQUIRE((reinterpret_cast<uintptr_t>(head) & 15) == 0 &&
             (reinterpret_cast<uintptr_t>(packed) & 15) == 0);
  const int64_t chunks = cdiv(vocab, 16) * 16 * hidden / 8;
  head_pack_kernel<<<dim3((unsigned)cdiv(chunks, 256)), 256, 0, (hipStream_t)stream>>>(
      (const bf16 *)head, (int)vocab, (int)hidden, chunks, (bf16 *)packed);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
