// Grouped SwiGLU expert GEMMs on MFMA (v_mfma_f32_16x16x32_bf16) for the
// decode-sized MoE, where the expert weights are the HBM traffic:
//
//   gate_up: act[r] = bf16(silu(bf16(x_t . W13[e, j])) * bf16(x_t . W13[e, I+j]))
//   down:    y[r]   = bf16(act[r] . W2[e, n])
//
// for route r = t*topk + branch of expert e; act and y are in route order.
// Workgroup = (column tile, route set of one expert). Its 4 waves split the
// reduction dimension K into quarters; each wave loads its slice of the
// workgroup's weight tile into registers once, then streams the route set
// through it in 16-row MFMA sub-blocks; the quarters are summed through LDS.
//
// Two ways to find a workgroup's routes:
//  * scan (decode, tokens <= kMaxScanRows): grid.y is the expert; the
//    workgroup collects the expert's routes from topk_ids itself with one
//    ballot per 64 routes, in ascending route order. No permutation pass.
//  * blocks (prefill): lm_moe_align sorts routes by expert; grid.y enumerates
//    blocks of at most block_rows routes of one expert, found on the device
//    from expert_offsets. Each expert's weights are read once per block.
// Both grids are fixed by the shapes alone (graph capture); an expert with
// no routes costs an early exit.
//
// Reference: the expert math of litemoe/ops.py:43-47 (reference_experts) and
// the vLLM fused_experts call at litemoe/ep.py:40-41.
#include <mutex>

#include "internal.h"

namespace lm {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxScanRows = 256;  // tokens of a call on the scan path

// How a workgroup finds its routes and when it loads its weight tile.
enum RouteMode : int {
  kBlocks = 0,        // lm_moe_align blocks; weights after the block lookup
  kScanLazy = 1,      // scan of topk_ids; weights only once routes are found
  kScanPrefetch = 2,  // scan of topk_ids; weights issued before the scan
};

// Block b of the per-expert blocks of block_rows routes.
__device__ __forceinline__ bool find_block(const int32_t *__restrict__ offsets, int experts, int bm,
                                           int b, int &e_out, int &r0, int &r1) {
  int o0 = offsets[0];
  for (int e = 0; e < experts; ++e) {
    const int o1 = offsets[e + 1];
    const int nb = (o1 - o0 + bm - 1) / bm;
    if (b < nb) {
      e_out = e;
      r0 = o0 + b * bm;
      r1 = min(o1, r0 + bm);
      return true;
    }
    b -= nb;
    o0 = o1;
  }
  return false;
}

// Route collection for the scan path, in two steps so that the ids loads
// are issued before the weight loads (vector loads complete in issue order:
// the scan then waits only for the ids, while the weights stream).
// Wave w owns routes [w*seg, (w+1)*seg), seg a multiple of 64, at most
// kScanIters loads of 64 ids per lane.
constexpr int kScanIters = 8;  // routes <= kWaves * kScanIters * 64 = 2048
// The LDS route list holds every route of the call, so an expert listed
// more than once by a token (more than `tokens` routes) still fits.
constexpr int kScanList = kWaves * kScanIters * kWave;

struct ScanIds {
  int id[kScanIters];  // ids[begin + it*64 + lane], valid below end
  int begin, end;
};

__device__ __forceinline__ ScanIds load_ids(const int32_t *__restrict__ ids, int routes) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int seg = (int)(cdiv(cdiv(routes, kWaves), kWave) * kWave);
  ScanIds s;
  s.begin = wave * seg;
  const int end = min(routes, s.begin + seg);
  // Unconditional loads at clamped indices, masked in scan_ids: a load
  // under a branch (or its mask computed here) would make the compiler wait
  // for these loads before the weight prefetch is issued, or for every load
  // in flight before the scan.
#pragma unroll
  for (int it = 0; it < kScanIters; ++it) s.id[it] = ids[min(s.begin + it * kWave + lane, routes - 1)];
  s.end = end;
  return s;
}

// Routes with id e, ascending, into list[]; returns the count. All threads
// of the workgroup must call it (it synchronises).
__device__ int scan_ids(const ScanIds &s, int e, int *list, int *wave_count) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint64_t below = (1ull << lane) - 1ull;
  int count = 0;
#pragma unroll
  for (int it = 0; it < kScanIters; ++it)
    count += __popcll(__ballot(s.id[it] == e && s.begin + it * kWave + lane < s.end));
  if (lane == 0) wave_count[wave] = count;
  __syncthreads();
  int offset = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    offset += w < wave ? wave_count[w] : 0;
    total += wave_count[w];
  }
#pragma unroll
  for (int it = 0; it < kScanIters; ++it) {
    const bool hit = s.id[it] == e && s.begin + it * kWave + lane < s.end;
    const uint64_t mask = __ballot(hit);
    const int slot = offset + __popcll(mask & below);
    if (hit) list[slot] = s.begin + it * kWave + lane;  // slot < total <= routes <= kScanList
    offset += __popcll(mask);
  }
  __syncthreads();
  return total;
}

constexpr int kXcdCount = 8;

// Expert e's column tiles all on XCD e % 8 (workgroups are dealt to the 8
// XCDs round-robin in dispatch order), so its activation rows are fetched
// into one L2 and the down kernel finds the act rows in the L2 that wrote
// them. Identity when the expert count is not a multiple of 8.
__device__ __forceinline__ void xcd_tile(int &e, int &tile) {
  const int tiles = gridDim.x, experts = gridDim.y;
  if (experts % kXcdCount) {
    e = blockIdx.y;
    tile = blockIdx.x;
    return;
  }
  const int lin = blockIdx.y * tiles + blockIdx.x;
  const int j = lin / kXcdCount;
  e = lin % kXcdCount + kXcdCount * (j / tiles);
  tile = j % tiles;
}

__device__ __forceinline__ u32x4 load16(const bf16 *p) { return *reinterpret_cast<const u32x4 *>(p); }
// Expert weight tiles of the decode scan kernels: each 16-byte word is read
// by one workgroup once per step, so the load is marked non-temporal (the
// weights need no room in L2 or the memory-side cache, which keep the
// activations and the partial results instead): the decode step at cfg 3
// 2.976 -> 2.903 ms, the MoE 45.8 -> 43.6-44.0 us per layer (A/B on one box,
// two runs each).
__device__ __forceinline__ u32x4 load16_stream(const bf16 *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

struct RouteSet {
  const int32_t *sorted;  // blocks mode: route of sorted position p
  const int *list;        // scan mode: LDS list of routes
  int r0, r1;
  __device__ __forceinline__ int route(int p) const { return list ? list[p] : sorted[p]; }
};

// KS: 32-wide k steps per wave, hidden = KS * 32 * kWaves. Column tile of 16
// gate rows and the matching 16 up rows.
template <int KS, int kMode, bool kPacked>
__global__ void __launch_bounds__(kThreads)
gate_up_kernel(const bf16 *__restrict__ x, const bf16 *__restrict__ w13,
               const int32_t *__restrict__ offsets, const int32_t *__restrict__ sorted,
               const int32_t *__restrict__ ids, int routes, int topk, int hidden, int inter,
               int experts, int bm, bf16 *__restrict__ act) {
  constexpr bool kScan = kMode != kBlocks;
  __shared__ float red[kWaves][2][4][kWave];
  __shared__ int list[kScan ? kScanList : 1];
  __shared__ int wave_count[kWaves];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  const int n0 = blockIdx.x * 16;
  const int kbase = wave * KS * 32 + grp * 8;
  u32x4 bg[KS], bu[KS];
  auto load_weights = [&](int e) {
    const int64_t rg = (int64_t)e * 2 * inter + n0 + col;
    const bf16 *wg = w13 + wofs<kPacked>(rg, kbase, hidden);
    const bf16 *wu = w13 + wofs<kPacked>(rg + inter, kbase, hidden);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bg[s] = load16(wg + s * wstep<kPacked>());
      bu[s] = load16(wu + s * wstep<kPacked>());
    }
  };
  RouteSet set{sorted, nullptr, 0, 0};
  if constexpr (kScan) {
    const int e = blockIdx.y;
    const ScanIds scan = load_ids(ids, routes);
    // The ids loads stay ahead of the weights, so the scan waits for them
    // only (vector loads complete in issue order). A compile-time choice: a
    // runtime branch around the prefetch would leave the scan's wait count
    // to the path without it, i.e. waiting for the weights too.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kMode == kScanPrefetch) load_weights(e);
    __builtin_amdgcn_sched_barrier(0);
    const int n = scan_ids(scan, e, list, wave_count);
    if (n == 0) return;
    if constexpr (kMode == kScanLazy) load_weights(e);
    set = RouteSet{nullptr, list, 0, n};
  } else {
    int e, r0, r1;
    if (!find_block(offsets, experts, bm, blockIdx.y, e, r0, r1)) return;
    load_weights(e);
    set.r0 = r0;
    set.r1 = r1;
  }
  for (int rb = set.r0; rb < set.r1; rb += 16) {
    const int p = rb + col;
    u32x4 a[KS];
    if (p < set.r1) {
      const bf16 *xr = x + (int64_t)(set.route(p) / topk) * hidden + kbase;
#pragma unroll
      for (int s = 0; s < KS; ++s) a[s] = load16(xr + s * 32);
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) a[s] = u32x4{0u, 0u, 0u, 0u};
    }
    f32x4 cg = {0.f, 0.f, 0.f, 0.f}, cu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      cg = mfma16x16x32(a[s], bg[s], cg);
      cu = mfma16x16x32(a[s], bu[s], cu);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[wave][0][i][lane] = cg[i];
      red[wave][1][i][lane] = cu[i];
    }
    __syncthreads();
    // Wave w finishes C row 4*grp + w of every lane group.
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      g += red[w][0][wave][lane];
      u += red[w][1][wave][lane];
    }
    const int row = rb + grp * 4 + wave;
    if (row < set.r1) {
      const float h = round_bf16(silu(round_bf16(g))) * round_bf16(u);
      act[(int64_t)set.route(row) * inter + n0 + col] = (bf16)f32_to_bf16(h);
    }
    __syncthreads();
  }
}


// The decode scan path with the weight tile prefetched (kScanPrefetch), as a
// kernel of its own: activation rows past the route set repeat its last
// route (unconditional loads; MFMA rows are independent and those outputs
// are never stored), and a set of at most 16 routes -- the common case --
// runs without the row-block loop. That keeps a wave within 128 registers up
// to hidden 1536, so four workgroups share a CU: 1024 of the decode step's
// 1280 weight tiles (Granite-3B shape) are in flight at once instead of 768.
template <int KS, bool kPacked>
__global__ void __launch_bounds__(kThreads, KS <= 12 ? 4 : 2)
gate_up_scan_kernel(const bf16 *__restrict__ x, const bf16 *__restrict__ w13,
                    const int32_t *__restrict__ ids, int routes, int topk, int hidden, int inter,
                    bf16 *__restrict__ act, int32_t *__restrict__ zero_counters, int counters) {
  // The arrival counters of the following down launch start at zero (they
  // are also left at zero by it): one workgroup clears them.
  if (zero_counters && blockIdx.x == 0 && blockIdx.y == 0 && (int)threadIdx.x < counters)
    zero_counters[threadIdx.x] = 0;
  __shared__ float red[kWaves][2][4][kWave];
  __shared__ int list[kScanList];
  __shared__ int wave_count[kWaves];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  int e, tile;
  xcd_tile(e, tile);
  const int n0 = tile * 16;
  const int kbase = wave * KS * 32 + grp * 8;
  const int64_t rg = (int64_t)e * 2 * inter + n0 + col;
  const bf16 *wg = w13 + wofs<kPacked>(rg, kbase, hidden);
  const bf16 *wu = w13 + wofs<kPacked>(rg + inter, kbase, hidden);
  u32x4 bg[KS], bu[KS], a[KS];
  const ScanIds scan = load_ids(ids, routes);
  __builtin_amdgcn_sched_barrier(0);  // ids first: the scan waits for them only
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    bg[s] = load16_stream(wg + s * wstep<kPacked>());
    bu[s] = load16_stream(wu + s * wstep<kPacked>());
  }
  __builtin_amdgcn_sched_barrier(0);
  const int n = scan_ids(scan, e, list, wave_count);
  if (n == 0) return;
  auto block = [&](int rb) {
    const bf16 *xr = x + (int64_t)(list[min(rb + col, n - 1)] / topk) * hidden + kbase;
#pragma unroll
    for (int s = 0; s < KS; ++s) a[s] = load16(xr + s * 32);
    f32x4 cg = {0.f, 0.f, 0.f, 0.f}, cu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      cg = mfma16x16x32(a[s], bg[s], cg);
      cu = mfma16x16x32(a[s], bu[s], cu);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[wave][0][i][lane] = cg[i];
      red[wave][1][i][lane] = cu[i];
    }
    __syncthreads();
    // Wave w finishes C row 4*grp + w of every lane group.
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      g += red[w][0][wave][lane];
      u += red[w][1][wave][lane];
    }
    const int row = rb + grp * 4 + wave;
    if (row < n) {
      const float h = round_bf16(silu(round_bf16(g))) * round_bf16(u);
      act[(int64_t)list[row] * inter + n0 + col] = (bf16)f32_to_bf16(h);
    }
    __syncthreads();
  };
  if (n <= 16) {
    block(0);
  } else if (kPacked && n <= 32) {
    // (fragment-order weights: the checkpoint-layout variant would spill)
    // Two row blocks in one pass over K: each weight fragment feeds both
    // blocks' MFMAs and is then dead, as in the one-block case, so the
    // second block's activations stream in behind the MFMAs instead of
    // waiting for the first block's reduction. Per row the same MFMAs in the
    // same order: the same bits as two passes.
    const bf16 *xr0 = x + (int64_t)(list[col] / topk) * hidden + kbase;
    const bf16 *xr1 = x + (int64_t)(list[min(16 + col, n - 1)] / topk) * hidden + kbase;
    f32x4 cg0 = {0.f, 0.f, 0.f, 0.f}, cu0 = cg0, cg1 = cg0, cu1 = cg0;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 a0 = load16(xr0 + s * 32), a1 = load16(xr1 + s * 32);
      cg0 = mfma16x16x32(a0, bg[s], cg0);
      cu0 = mfma16x16x32(a0, bu[s], cu0);
      cg1 = mfma16x16x32(a1, bg[s], cg1);
      cu1 = mfma16x16x32(a1, bu[s], cu1);
    }
    f32x4 cg[2] = {cg0, cg1}, cu[2] = {cu0, cu1};
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        red[wave][0][i][lane] = cg[hb][i];
        red[wave][1][i][lane] = cu[hb][i];
      }
      __syncthreads();
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        g += red[w][0][wave][lane];
        u += red[w][1][wave][lane];
      }
      const int row = 16 * hb + grp * 4 + wave;
      if (row < n) {
        const float h = round_bf16(silu(round_bf16(g))) * round_bf16(u);
        act[(int64_t)list[row] * inter + n0 + col] = (bf16)f32_to_bf16(h);
      }
      __syncthreads();
    }
  } else {
    for (int rb = 0; rb < n; rb += 16) block(rb);
  }
}

// KS: 32-wide k steps per wave, inter = KS * 32 * kWaves. Column tile of 32
// (two MFMA tiles).
template <int KS, int kMode, bool kPacked>
__global__ void __launch_bounds__(kThreads)
down_kernel(const bf16 *__restrict__ act, const bf16 *__restrict__ w2,
            const int32_t *__restrict__ offsets, const int32_t *__restrict__ sorted,
            const int32_t *__restrict__ ids, int routes, int hidden, int inter, int experts, int bm,
            bf16 *__restrict__ y) {
  constexpr bool kScan = kMode != kBlocks;
  __shared__ float red[kWaves][2][4][kWave];
  __shared__ int list[kScan ? kScanList : 1];
  __shared__ int wave_count[kWaves];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  const int n0 = blockIdx.x * 32;
  const int kbase = wave * KS * 32 + grp * 8;
  u32x4 b0[KS], b1[KS];
  auto load_weights = [&](int e) {
    const int64_t r0 = (int64_t)e * hidden + n0 + col;
    const bf16 *w0 = w2 + wofs<kPacked>(r0, kbase, inter);
    const bf16 *w1 = w2 + wofs<kPacked>(r0 + 16, kbase, inter);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      b0[s] = load16(w0 + s * wstep<kPacked>());
      b1[s] = load16(w1 + s * wstep<kPacked>());
    }
  };
  RouteSet set{sorted, nullptr, 0, 0};
  if constexpr (kScan) {
    const int e = blockIdx.y;
    const ScanIds scan = load_ids(ids, routes);
    // The ids loads stay ahead of the weights, so the scan waits for them
    // only (vector loads complete in issue order). A compile-time choice: a
    // runtime branch around the prefetch would leave the scan's wait count
    // to the path without it, i.e. waiting for the weights too.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kMode == kScanPrefetch) load_weights(e);
    __builtin_amdgcn_sched_barrier(0);
    const int n = scan_ids(scan, e, list, wave_count);
    if (n == 0) return;
    if constexpr (kMode == kScanLazy) load_weights(e);
    set = RouteSet{nullptr, list, 0, n};
  } else {
    int e, r0, r1;
    if (!find_block(offsets, experts, bm, blockIdx.y, e, r0, r1)) return;
    load_weights(e);
    set.r0 = r0;
    set.r1 = r1;
  }
  for (int rb = set.r0; rb < set.r1; rb += 16) {
    const int p = rb + col;
    u32x4 a[KS];
    if (p < set.r1) {
      const bf16 *ar = act + (int64_t)set.route(p) * inter + kbase;
#pragma unroll
      for (int s = 0; s < KS; ++s) a[s] = load16(ar + s * 32);
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) a[s] = u32x4{0u, 0u, 0u, 0u};
    }
    f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      c0 = mfma16x16x32(a[s], b0[s], c0);
      c1 = mfma16x16x32(a[s], b1[s], c1);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[wave][0][i][lane] = c0[i];
      red[wave][1][i][lane] = c1[i];
    }
    __syncthreads();
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      v0 += red[w][0][wave][lane];
      v1 += red[w][1][wave][lane];
    }
    const int row = rb + grp * 4 + wave;
    if (row < set.r1) {
      bf16 *yr = y + (int64_t)set.route(row) * hidden + n0 + col;
      yr[0] = (bf16)f32_to_bf16(v0);
      yr[16] = (bf16)f32_to_bf16(v1);
    }
    __syncthreads();
  }
}

// The combine fused into the down projection (kFin 1 and 2 of
// down_scan_kernel). Each workgroup writes, instead of its routes' y, the
// weighted terms bf16(y * bf16(scale)) of the moe_finish sum; the last
// workgroup to finish a column tile (counted with a device-scope atomic, one
// counter per tile) sums the tokens' terms in branch order j = 0..topk-1
// for that tile. A token's routes must be in ascending expert id (the
// router's id order), which makes j the moe_finish order (logical id*K + j,
// identity placement), so the sum is bitwise that of lm_moe_finish.
//   kFin 1: out[t] = bf16(sum);
//   kFin 2: x[t] <- bf16(x[t] + alpha * bf16(sum)) and sumsq[t][tile] = the
//           tile's sum of squares of the new x in rmsnorm_kernel's order (the
//           per-16-byte-word sums and the 8-lane DPP tree of wave_sum), from
//           which lm_linear_splitk_rmsnorm finishes the next RMSNorm.
// The terms cross XCDs (each XCD has its own L2): they are stored and loaded
// at device scope (write-through stores, loads that do not trust a possibly
// stale L2 line), each workgroup waits for its stores before it arrives, and
// the last arriver loads only after its arrival returned.
struct TileCombine {
  int32_t *counters;       // [column tiles]; zero on entry, left zero
  const float *scales;     // [tokens, topk]
  bf16 *out;               // kFin 1: out [tokens, hidden]; kFin 2: the residual x, updated
  float alpha;             // kFin 2
  float *sumsq;            // kFin 2: [tokens, hidden / 64]
  int tokens, topk;
};

__device__ __forceinline__ void store_dev32(bf16 *p, uint32_t v) {
  __hip_atomic_store(reinterpret_cast<uint32_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A buffer resource over `bytes` bytes from `base` (raw buffer: no stride,
// the gfx9 data-format word), for loads with explicit cache-policy bits.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes at `offset` with device scope (sc1: coherent across the XCDs' L2s).
__device__ __forceinline__ u32x4 load_dev16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
  constexpr int kDeviceScope = 16;  // cache-policy bit sc1
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)offset, 0, kDeviceScope);
}

// Wait until every vector memory operation of the wave has completed (the
// device-scope term stores are then visible to every XCD): s_waitcnt
// vmcnt(0) in gfx9's encoding (expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// The last arriver's sum for column tile `tile` (64 columns from n0): one
// task per (token, 16-byte word), 8 consecutive lanes per token, so that
// lanes 8g .. 8g+7 hold one token's 8 words as rmsnorm_kernel's lanes hold
// them and dpp_sum8 forms the same partial sum.
template <int kFin>
__device__ void combine_tile(const TileCombine &c, const bf16 *__restrict__ terms, int hidden,
                             int tile, int n0) {
  constexpr int kMaxK = 8;
  constexpr int kBatch = 2;  // tasks per thread whose loads are in flight together
  const int ntiles = hidden / 64;
  const __amdgpu_buffer_rsrc_t rsrc =
      buffer_over(terms, (uint32_t)((int64_t)c.tokens * c.topk * hidden * 2));
  const int tasks = c.tokens * 8;
  for (int base = 0; base < tasks; base += kBatch * kThreads) {
    u32x4 tv[kBatch][kMaxK], xv[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int task = min(base + b * kThreads + (int)threadIdx.x, tasks - 1);
      const int t = task >> 3, col = n0 + (task & 7) * 8;
#pragma unroll
      for (int j = 0; j < kMaxK; ++j)
        tv[b][j] = load_dev16(rsrc, (uint32_t)((((int64_t)t * c.topk + min(j, c.topk - 1)) * hidden + col) * 2));
      xv[b] = u32x4{0u, 0u, 0u, 0u};
      if constexpr (kFin == 2) xv[b] = *reinterpret_cast<const u32x4 *>(c.out + (int64_t)t * hidden + col);
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int task = base + b * kThreads + (int)threadIdx.x;
      const int t = min(task, tasks - 1) >> 3, wd = task & 7, col = n0 + wd * 8;
      // Intermediate roundings skip the NaN fix-up (the stores canonicalize).
      float total[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < kMaxK; ++j) {
        if (j < c.topk) {
          float f[8];
          unpack8(tv[b][j], f);
#pragma unroll
          for (int q = 0; q < 8; ++q) total[q] += f[q];
        }
      }
      u32x4 o;
      if constexpr (kFin == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = pack_bf16(total[2 * q], total[2 * q + 1]);
        if (task < tasks) *reinterpret_cast<u32x4 *>(c.out + (int64_t)t * hidden + col) = o;
      } else {
        float xf[8], xn[8];
        unpack8(xv[b], xf);
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          xn[q] = round_bf16_nc(xf[q] + c.alpha * round_bf16_nc(total[q]));
          ss += xn[q] * xn[q];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = pack_bf16(xn[2 * q], xn[2 * q + 1]);
        ss = dpp_sum8(ss);  // every lane of the group takes part (tasks come in whole groups)
        if (task < tasks) {
          *reinterpret_cast<u32x4 *>(c.out + (int64_t)t * hidden + col) = o;
          if (wd == 0) c.sumsq[(int64_t)t * ntiles + tile] = ss;
        }
      }
    }
  }
}

// The decode scan path of the down projection as a kernel of its own, as
// gate_up_scan_kernel is for gate/up: weights prefetched before the scan,
// activation rows past the route set repeating its last route (no
// divergent loads), no row-block loop for sets of at most 16 routes. A
// workgroup covers NT MFMA tiles of 16 output columns (KS: 32-wide k steps
// per wave, inter = KS * 32 * kWaves); its activation loads are issued back
// to back. Same MFMA order and wave-order sum as down_kernel, hence the same
// bits. kFin: the combine fused in (TileCombine; NT == 4, 64-column tiles).
template <int KS, int NT, bool kPacked, int kFin = 0>
__global__ void __launch_bounds__(kThreads)
down_scan_kernel(const bf16 *__restrict__ act, const bf16 *__restrict__ w2,
                 const int32_t *__restrict__ ids, int routes, int hidden, int inter,
                 bf16 *__restrict__ y, TileCombine fin) {
  static_assert(kFin == 0 || NT == 4, "the fused combine works on 64-column tiles");
  __shared__ float red[kWaves][NT][4][kWave];
  __shared__ int list[kScanList];
  __shared__ int wave_count[kWaves];
  __shared__ int last_flag;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int col = lane % 16, grp = lane / 16;
  int e, tile;
  xcd_tile(e, tile);
  const int n0 = tile * 16 * NT;
  const int kbase = wave * KS * 32 + grp * 8;
  const int64_t r0 = (int64_t)e * hidden + n0 + col;
  u32x4 b[NT][KS], a[KS];
  const ScanIds scan = load_ids(ids, routes);
  __builtin_amdgcn_sched_barrier(0);  // ids first: the scan waits for them only
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const bf16 *wt = w2 + wofs<kPacked>(r0 + 16 * t, kbase, inter);
#pragma unroll
    for (int s = 0; s < KS; ++s) b[t][s] = load16_stream(wt + s * wstep<kPacked>());
  }
  __builtin_amdgcn_sched_barrier(0);
  const int n = scan_ids(scan, e, list, wave_count);
  auto block = [&](int rb) {
    const bf16 *ar = act + (int64_t)list[min(rb + col, n - 1)] * inter + kbase;
#pragma unroll
    for (int s = 0; s < KS; ++s) a[s] = load16(ar + s * 32);
    // Wave w finishes C row 4*grp + w of every lane group (below); its
    // route's scale is requested behind the activations.
    const int row = rb + grp * 4 + wave;
    const int route = list[min(row, n - 1)];
    float sc = 0.f;
    if constexpr (kFin != 0) sc = fin.scales[route];
    __builtin_amdgcn_sched_barrier(0);  // all activation loads in flight before the MFMAs
    f32x4 c[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) c[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int t = 0; t < NT; ++t) c[t] = mfma16x16x32(a[s], b[t][s], c[t]);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][t][i][lane] = c[t][i];
    __syncthreads();
    bf16 *yr = y + (int64_t)route * hidden + n0 + col;
    sc = round_bf16_nc(sc);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) v += red[w][t][wave][lane];
      if constexpr (kFin == 0) {
        if (row < n) yr[16 * t] = (bf16)f32_to_bf16(v);
      } else {
        // the moe_finish term bf16(bf16(y) * bf16(scale)); lanes col and
        // col + 1 (DPP quad_perm [1,0,3,2]) store as one 4-byte word
        const float term = round_bf16_nc(round_bf16_nc(v) * sc);
        const float next = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(term), 0xB1, 0xF, 0xF, true));
        if (row < n && (col & 1) == 0) store_dev32(yr + 16 * t, pack_bf16(term, next));
      }
    }
    __syncthreads();
  };
  if (n > 0) {
    if (n <= 16) {
      block(0);
    } else {
      for (int rb = 0; rb < n; rb += 16) block(rb);
    }
  }
  if constexpr (kFin != 0) {
    // Every workgroup of the tile arrives once (an expert without routes
    // too), after its term stores have completed.
    wait_vector_memory();
    __syncthreads();
    if (threadIdx.x == 0) {
      const int before = __hip_atomic_fetch_add(fin.counters + tile, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      last_flag = before == (int)gridDim.y - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    if (threadIdx.x == 0)
      __hip_atomic_store(fin.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    combine_tile<kFin>(fin, y, hidden, tile, n0);
  }
}

// Supported k steps per wave (reduction length / 128).
#define LM_KS_LIST(X) X(1) X(2) X(3) X(4) X(6) X(8) X(12) X(16)

bool ks_ok(int64_t n) {
  if (n % 128) return false;
  switch (n / 128) {
#define X(KS) case KS:
    LM_KS_LIST(X)
#undef X
    return true;
    default:
      return false;
  }
}

// Weight tiles are prefetched before the route scan when an empty expert is
// unlikely (>= 4 routes per expert on average).
int route_mode(bool scan, int64_t routes, int64_t experts) {
  return !scan ? kBlocks : (routes >= 4 * experts ? kScanPrefetch : kScanLazy);
}

}  // namespace

bool expert_shapes_ok(int64_t hidden, int64_t inter) { return ks_ok(hidden) && ks_ok(inter); }

int pick_block_rows(int64_t block_rows, int64_t tokens) {
  if (block_rows > 0) return (int)block_rows;
  // Every token picks an expert at most once, so a block of >= tokens rows
  // holds a whole expert; larger batches trade weight re-reads for blocks.
  const int64_t bm = align_up(tokens, 16);
  return (int)(bm > 256 ? 256 : (bm < 16 ? 16 : bm));
}

bool scan_path(int64_t tokens, int64_t topk) {
  return tokens <= kMaxScanRows && tokens * topk <= kWaves * kScanIters * kWave;
}

namespace {
template <bool kPacked>
int launch_gate_up_t(const bf16 *x, const bf16 *w13, const int32_t *offsets, const int32_t *sorted,
                     const int32_t *ids, int64_t routes, int64_t topk, int64_t hidden, int64_t inter,
                     int64_t experts, int64_t block_rows, bf16 *act, hipStream_t stream) {
  if (routes == 0) return LM_OK;
  const bool scan = ids != nullptr;
  const int bm = (int)block_rows;
  const int64_t gy = scan ? experts : cdiv(routes, bm) + experts;
  if (gy > 65535) return LM_EUNSUPPORTED;
  const dim3 grid((unsigned)(inter / 16), (unsigned)gy);
  const int mode = route_mode(scan, routes, experts);
  switch (hidden / 128) {
#define X(KS)                                                                                   \
  case KS:                                                                                      \
    if (mode == kScanPrefetch)                                                                  \
      gate_up_scan_kernel<KS, kPacked><<<grid, kThreads, 0, stream>>>(x, w13, ids, (int)routes,          \
          (int)topk, (int)hidden, (int)inter, act, nullptr, 0);                                 \
    else if (mode == kScanLazy)                                                                 \
      gate_up_kernel<KS, kScanLazy, kPacked><<<grid, kThreads, 0, stream>>>(x, w13, offsets, sorted,     \
          ids, (int)routes, (int)topk, (int)hidden, (int)inter, (int)experts, bm, act);         \
    else                                                                                        \
      gate_up_kernel<KS, kBlocks, kPacked><<<grid, kThreads, 0, stream>>>(x, w13, offsets, sorted, ids,  \
          (int)routes, (int)topk, (int)hidden, (int)inter, (int)experts, bm, act);              \
    break;
    LM_KS_LIST(X)
#undef X
    default:
      return LM_EUNSUPPORTED;
  }
  LM_CHECK_LAUNCH();
  return LM_OK;
}

template <bool kPacked>
int launch_down_t(const bf16 *act, const bf16 *w2, const int32_t *offsets, const int32_t *sorted,
                  const int32_t *ids, int64_t routes, int64_t hidden, int64_t inter, int64_t experts,
                  int64_t block_rows, bf16 *y, hipStream_t stream) {
  if (routes == 0) return LM_OK;
  const bool scan = ids != nullptr;
  const int bm = (int)block_rows;
  const int64_t gy = scan ? experts : cdiv(routes, bm) + experts;
  if (gy > 65535) return LM_EUNSUPPORTED;
  const dim3 grid((unsigned)(hidden / 32), (unsigned)gy);
  const int mode = route_mode(scan, routes, experts);
#ifndef LM_DOWN_SCAN_TILES
#define LM_DOWN_SCAN_TILES 4
#endif
  constexpr int kNT = LM_DOWN_SCAN_TILES;
  if (kNT > 0 && mode == kScanPrefetch && hidden % (16 * kNT) == 0 && inter <= 8 * 128) {
    const dim3 sgrid((unsigned)(hidden / (16 * kNT)), (unsigned)experts);
    switch (inter / 128) {
#define X(KS)                                                                                  \
  case KS:                                                                                     \
    down_scan_kernel<KS, (kNT > 0 ? kNT : 1), kPacked><<<sgrid, kThreads, 0, stream>>>(                 \
        act, w2, ids, (int)routes, (int)hidden, (int)inter, y, TileCombine{});                 \
    LM_CHECK_LAUNCH();                                                                         \
    return LM_OK;
      X(1) X(2) X(3) X(4) X(6) X(8)
#undef X
      default:
        break;
    }
  }
  switch (inter / 128) {
#define X(KS)                                                                                  \
  case KS:                                                                                     \
    if (mode == kScanPrefetch)                                                                 \
      down_kernel<KS, kScanPrefetch, kPacked><<<grid, kThreads, 0, stream>>>(act, w2, offsets, sorted,  \
          ids, (int)routes, (int)hidden, (int)inter, (int)experts, bm, y);                     \
    else if (mode == kScanLazy)                                                                \
      down_kernel<KS, kScanLazy, kPacked><<<grid, kThreads, 0, stream>>>(act, w2, offsets, sorted, ids, \
          (int)routes, (int)hidden, (int)inter, (int)experts, bm, y);                          \
    else                                                                                       \
      down_kernel<KS, kBlocks, kPacked><<<grid, kThreads, 0, stream>>>(act, w2, offsets, sorted, ids,   \
          (int)routes, (int)hidden, (int)inter, (int)experts, bm, y);                          \
    break;
    LM_KS_LIST(X)
#undef X
    default:
      return LM_EUNSUPPORTED;
  }
  LM_CHECK_LAUNCH();
  return LM_OK;
}

// gate/up then down with the combine fused in, on the scan kernels (weights
// prefetched before the route scan at every route count): LM_EUNSUPPORTED
// where those kernels do not apply.
template <bool kPacked>
int launch_routes_combine_t(const bf16 *x, const bf16 *w13, const bf16 *w2, const int32_t *ids,
                            int64_t tokens, int64_t topk, int64_t hidden, int64_t inter,
                            int64_t experts, bf16 *act, bf16 *terms, const TileCombine &fin,
                            bool residual, hipStream_t stream) {
  const int64_t routes = tokens * topk;
  if (hidden % 64 || hidden / 64 > kThreads || inter > 8 * 128 || experts > 65535)
    return LM_EUNSUPPORTED;
  const dim3 ggrid((unsigned)(inter / 16), (unsigned)experts);
  const dim3 dgrid((unsigned)(hidden / 64), (unsigned)experts);
  switch (hidden / 128) {
#define X(KS)                                                                                      \
  case KS:                                                                                         \
    gate_up_scan_kernel<KS, kPacked><<<ggrid, kThreads, 0, stream>>>(                              \
        x, w13, ids, (int)routes, (int)topk, (int)hidden, (int)inter, act, fin.counters,           \
        (int)(hidden / 64));                                                                       \
    break;
    LM_KS_LIST(X)
#undef X
    default:
      return LM_EUNSUPPORTED;
  }
  LM_CHECK_LAUNCH();
  switch (inter / 128) {
#define X(KS)                                                                                      \
  case KS:                                                                                         \
    if (residual)                                                                                  \
      down_scan_kernel<KS, 4, kPacked, 2><<<dgrid, kThreads, 0, stream>>>(                         \
          act, w2, ids, (int)routes, (int)hidden, (int)inter, terms, fin);                         \
    else                                                                                           \
      down_scan_kernel<KS, 4, kPacked, 1><<<dgrid, kThreads, 0, stream>>>(                         \
          act, w2, ids, (int)routes, (int)hidden, (int)inter, terms, fin);                         \
    break;
    X(1) X(2) X(3) X(4) X(6) X(8)
#undef X
    default:
      return LM_EUNSUPPORTED;
  }
  LM_CHECK_LAUNCH();
  return LM_OK;
}

}  // namespace

int launch_gate_up(const bf16 *x, const bf16 *w13, const int32_t *offsets, const int32_t *sorted,
                   const int32_t *ids, int64_t routes, int64_t topk, int64_t hidden, int64_t inter,
                   int64_t experts, int64_t block_rows, bf16 *act, bool packed, hipStream_t stream) {
  return packed ? launch_gate_up_t<true>(x, w13, offsets, sorted, ids, routes, topk, hidden, inter,
                                         experts, block_rows, act, stream)
                : launch_gate_up_t<false>(x, w13, offsets, sorted, ids, routes, topk, hidden, inter,
                                          experts, block_rows, act, stream);
}

int launch_down(const bf16 *act, const bf16 *w2, const int32_t *offsets, const int32_t *sorted,
                const int32_t *ids, int64_t routes, int64_t hidden, int64_t inter, int64_t experts,
                int64_t block_rows, bf16 *y, bool packed, hipStream_t stream) {
  return packed ? launch_down_t<true>(act, w2, offsets, sorted, ids, routes, hidden, inter, experts,
                                      block_rows, y, stream)
                : launch_down_t<false>(act, w2, offsets, sorted, ids, routes, hidden, inter, experts,
                                       block_rows, y, stream);
}

}  // namespace lm

using namespace lm;

namespace {
struct ExpertWorkspace {
  int32_t *offsets, *sorted, *align_scratch;
  int64_t align_bytes;
  bf16 *act, *y;
  int32_t *counters;
  int64_t bytes;
};

// Layout: offsets [E+1], sorted [R] (block path only), the chunked align's
// counts and bases (large R only), act [R, I], (for lm_fused_experts and the
// combine entry points) y [R, H], and (combine entry points) the arrival
// counters of the column tiles [H / 64].
ExpertWorkspace carve(void *base, int64_t tokens, int64_t topk, int64_t hidden, int64_t inter,
                      int64_t experts, bool with_y, bool with_counters = false) {
  const int64_t routes = tokens * topk;
  char *p = static_cast<char *>(base);
  ExpertWorkspace w;
  int64_t off = 0;
  w.offsets = reinterpret_cast<int32_t *>(p + off);
  off += align_up(4 * (experts + 1), 256);
  w.sorted = reinterpret_cast<int32_t *>(p + off);
  off += align_up(4 * routes, 256);
  w.align_scratch = reinterpret_cast<int32_t *>(p + off);
  w.align_bytes = align_scratch_bytes(routes, experts);
  off += align_up(w.align_bytes, 256);
  w.act = reinterpret_cast<bf16 *>(p + off);
  off += align_up(2 * routes * inter, 256);
  w.y = with_y ? reinterpret_cast<bf16 *>(p + off) : nullptr;
  if (with_y) off += align_up(2 * routes * hidden, 256);
  w.counters = with_counters ? reinterpret_cast<int32_t *>(p + off) : nullptr;
  if (with_counters) off += align_up(4 * cdiv(hidden, 64), 256);
  w.bytes = off;
  return w;
}

// y in route order; act in route order on the scan and block paths, in
// sorted order between the two expert GEMMs.
int run_routes(const void *x, const void *w13, const void *w2, const int32_t *topk_ids,
               int64_t tokens, int64_t hidden, int64_t inter, int64_t experts, int64_t topk,
               int64_t block_rows, bf16 *y, const ExpertWorkspace &w, bool packed, void *stream) {
  hipStream_t s = (hipStream_t)stream;
  const int64_t routes = tokens * topk;
  if (scan_path(tokens, topk) && block_rows == 0) {
    int rc = launch_gate_up((const bf16 *)x, (const bf16 *)w13, nullptr, nullptr, topk_ids, routes,
                            topk, hidden, inter, experts, 0, w.act, packed, s);
    if (rc) return rc;
    return launch_down(w.act, (const bf16 *)w2, nullptr, nullptr, topk_ids, routes, hidden, inter,
                       experts, 0, y, packed, s);
  }
  const int bm = pick_block_rows(block_rows, tokens);
  int rc = launch_align(topk_ids, routes, 0, experts, w.offsets, w.sorted, nullptr,
                        w.align_scratch, w.align_bytes, s);
  if (rc) return rc;
  if (block_rows == 0 && expert_gemm_ok(routes, hidden, inter, experts)) {
    // act stays internal here: sorted order, read contiguously by down.
    rc = launch_expert_gemm_gate_up((const bf16 *)x, (const bf16 *)w13, w.offsets, w.sorted, routes,
                                    topk, hidden, inter, experts, w.act, packed, true, s);
    if (rc) return rc;
    return launch_expert_gemm_down(w.act, (const bf16 *)w2, w.offsets, w.sorted, routes, hidden,
                                   inter, experts, y, packed, true, s);
  }
  rc = launch_gate_up((const bf16 *)x, (const bf16 *)w13, w.offsets, w.sorted, nullptr, routes,
                      topk, hidden, inter, experts, bm, w.act, packed, s);
  if (rc) return rc;
  return launch_down(w.act, (const bf16 *)w2, w.offsets, w.sorted, nullptr, routes, hidden, inter,
                     experts, bm, y, packed, s);
}
}  // namespace

extern "C" int lm_fused_experts_workspace_size(int64_t tokens, int64_t topk, int64_t hidden,
                                               int64_t inter, int64_t experts, int64_t *bytes) {
  LM_REQUIRE(bytes && tokens >= 0 && topk > 0 && hidden > 0 && inter > 0 && experts > 0);
  *bytes = carve(nullptr, tokens, topk, hidden, inter, experts, true).bytes;
  return LM_OK;
}

extern "C" int lm_moe_routes_workspace_size(int64_t tokens, int64_t topk, int64_t hidden,
                                            int64_t inter, int64_t experts, int64_t *bytes) {
  LM_REQUIRE(bytes && tokens >= 0 && topk > 0 && hidden > 0 && inter > 0 && experts > 0);
  *bytes = carve(nullptr, tokens, topk, hidden, inter, experts, false).bytes;
  return LM_OK;
}

namespace {
int moe_gate_up(const void *x, const void *w13, const int32_t *expert_offsets,
                const int32_t *sorted_routes, const int32_t *topk_ids, int64_t routes,
                int64_t topk, int64_t hidden, int64_t inter, int64_t experts, int64_t block_rows,
                void *act, bool packed, void *stream) {
  LM_REQUIRE(routes >= 0 && topk > 0 && experts > 0 && block_rows >= 0 && block_rows % 16 == 0);
  if (!expert_shapes_ok(hidden, inter)) return LM_EUNSUPPORTED;
  if (topk_ids && !scan_path(routes / topk, topk)) return LM_EUNSUPPORTED;
  if (routes == 0) return LM_OK;
  LM_REQUIRE(x && w13 && act && (topk_ids || (expert_offsets && sorted_routes)));
  if (!topk_ids && block_rows == 0 && expert_gemm_ok(routes, hidden, inter, experts))
    return launch_expert_gemm_gate_up((const bf16 *)x, (const bf16 *)w13, expert_offsets,
                                      sorted_routes, routes, topk, hidden, inter, experts,
                                      (bf16 *)act, packed, false, (hipStream_t)stream);
  return launch_gate_up((const bf16 *)x, (const bf16 *)w13, expert_offsets, sorted_routes, topk_ids,
                        routes, topk, hidden, inter, experts, pick_block_rows(block_rows, routes),
                        (bf16 *)act, packed, (hipStream_t)stream);
}

int moe_down(const void *act, const void *w2, const int32_t *expert_offsets,
             const int32_t *sorted_routes, const int32_t *topk_ids, int64_t routes, int64_t hidden,
             int64_t inter, int64_t experts, int64_t block_rows, void *y, bool packed,
             void *stream) {
  LM_REQUIRE(routes >= 0 && experts > 0 && block_rows >= 0 && block_rows % 16 == 0);
  if (!expert_shapes_ok(hidden, inter)) return LM_EUNSUPPORTED;
  if (topk_ids && routes > kWaves * kScanIters * kWave) return LM_EUNSUPPORTED;
  if (routes == 0) return LM_OK;
  LM_REQUIRE(act && w2 && y && (topk_ids || (expert_offsets && sorted_routes)));
  if (!topk_ids && block_rows == 0 && expert_gemm_ok(routes, hidden, inter, experts))
    return launch_expert_gemm_down((const bf16 *)act, (const bf16 *)w2, expert_offsets,
                                   sorted_routes, routes, hidden, inter, experts, (bf16 *)y, packed,
                                   false, (hipStream_t)stream);
  return launch_down((const bf16 *)act, (const bf16 *)w2, expert_offsets, sorted_routes, topk_ids,
                     routes, hidden, inter, experts, pick_block_rows(block_rows, routes), (bf16 *)y,
                     packed, (hipStream_t)stream);
}
}  // namespace

extern "C" int lm_moe_gate_up(const void *x, const void *w13, const int32_t *expert_offsets,
                              const int32_t *sorted_routes, const int32_t *topk_ids, int64_t routes,
                              int64_t topk, int64_t hidden, int64_t inter, int64_t experts,
                              int64_t block_rows, void *act, void *stream) {
  return moe_gate_up(x, w13, expert_offsets, sorted_routes, topk_ids, routes, topk, hidden, inter,
                     experts, block_rows, act, false, stream);
}

extern "C" int lm_moe_gate_up_packed(const void *x, const void *w13, const int32_t *expert_offsets,
                                     const int32_t *sorted_routes, const int32_t *topk_ids,
                                     int64_t routes, int64_t topk, int64_t hidden, int64_t inter,
                                     int64_t experts, int64_t block_rows, void *act, void *stream) {
  return moe_gate_up(x, w13, expert_offsets, sorted_routes, topk_ids, routes, topk, hidden, inter,
                     experts, block_rows, act, true, stream);
}

extern "C" int lm_moe_down(const void *act, const void *w2, const int32_t *expert_offsets,
                           const int32_t *sorted_routes, const int32_t *topk_ids, int64_t routes,
                           int64_t hidden, int64_t inter, int64_t experts, int64_t block_rows,
                           void *y, void *stream) {
  return moe_down(act, w2, expert_offsets, sorted_routes, topk_ids, routes, hidden, inter, experts,
                  block_rows, y, false, stream);
}

extern "C" int lm_moe_down_packed(const void *act, const void *w2, const int32_t *expert_offsets,
                                  const int32_t *sorted_routes, const int32_t *topk_ids,
                                  int64_t routes, int64_t hidden, int64_t inter, int64_t experts,
                                  int64_t block_rows, void *y, void *stream) {
  return moe_down(act, w2, expert_offsets, sorted_routes, topk_ids, routes, hidden, inter, experts,
                  block_rows, y, true, stream);
}

namespace {
int moe_routes(const void *x, const void *w13, const void *w2, const int32_t *topk_ids,
               int64_t tokens, int64_t hidden, int64_t inter, int64_t experts, int64_t topk,
               int64_t block_rows, void *y, void *workspace, int64_t workspace_bytes, bool packed,
               void *stream) {
  LM_REQUIRE(tokens >= 0 && topk > 0 && topk <= experts && block_rows >= 0 &&
             block_rows % 16 == 0 && experts <= 511);
  if (!expert_shapes_ok(hidden, inter)) return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && w13 && w2 && topk_ids && y && workspace);
  ExpertWorkspace w = carve(workspace, tokens, topk, hidden, inter, experts, false);
  if (workspace_bytes < w.bytes) return LM_EWORKSPACE;
  return run_routes(x, w13, w2, topk_ids, tokens, hidden, inter, experts, topk, block_rows,
                    (bf16 *)y, w, packed, stream);
}

int fused_experts(const void *x, const void *w13, const void *w2, const float *topk_weights,
                  const int32_t *topk_ids, const int64_t *logical, int64_t tokens, int64_t hidden,
                  int64_t inter, int64_t experts, int64_t topk, int64_t block_rows, void *out,
                  void *workspace, int64_t workspace_bytes, bool packed, void *stream) {
  LM_REQUIRE(tokens >= 0 && topk > 0 && topk <= 8 && topk <= experts && block_rows >= 0 &&
             block_rows % 16 == 0 && experts <= 511);
  if (!expert_shapes_ok(hidden, inter)) return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && w13 && w2 && topk_weights && topk_ids && out && workspace);
  ExpertWorkspace w = carve(workspace, tokens, topk, hidden, inter, experts, true);
  if (workspace_bytes < w.bytes) return LM_EWORKSPACE;
  int rc = run_routes(x, w13, w2, topk_ids, tokens, hidden, inter, experts, topk, block_rows, w.y,
                      w, packed, stream);
  if (rc) return rc;
  return launch_finish(w.y, topk_ids, nullptr, topk_weights, logical, (bf16 *)out, tokens, hidden,
                       topk, 0, experts, (hipStream_t)stream);
}

// One thread per 16-byte chunk (tile, k-step, lane) of the fragment layout.
__global__ void __launch_bounds__(256)
expert_pack_kernel(const bf16 *__restrict__ src, int K, int64_t chunks, bf16 *__restrict__ dst) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= chunks) return;
  const int lane = (int)(q % kWave);
  const int64_t rest = q / kWave;
  const int steps = K / 32;
  const int ks = (int)(rest % steps);
  const int64_t row = (rest / steps) * 16 + lane % 16;
  reinterpret_cast<u32x4 *>(dst)[q] = load16(src + row * K + ks * 32 + (lane / 16) * 8);
}

int expert_pack(const void *src, int64_t rows, int64_t K, void *dst, hipStream_t stream) {
  const int64_t chunks = rows * K / 8;
  expert_pack_kernel<<<dim3((unsigned)cdiv(chunks, 256)), 256, 0, stream>>>(
      (const bf16 *)src, (int)K, chunks, (bf16 *)dst);
  LM_CHECK_LAUNCH();
  return LM_OK;
}
}  // namespace

extern "C" int lm_moe_routes(const void *x, const void *w13, const void *w2,
                             const int32_t *topk_ids, int64_t tokens, int64_t hidden,
                             int64_t inter, int64_t experts, int64_t topk, int64_t block_rows,
                             void *y, void *workspace, int64_t workspace_bytes, void *stream) {
  return moe_routes(x, w13, w2, topk_ids, tokens, hidden, inter, experts, topk, block_rows, y,
                    workspace, workspace_bytes, false, stream);
}

extern "C" int lm_moe_routes_packed(const void *x, const void *w13, const void *w2,
                                    const int32_t *topk_ids, int64_t tokens, int64_t hidden,
                                    int64_t inter, int64_t experts, int64_t topk,
                                    int64_t block_rows, void *y, void *workspace,
                                    int64_t workspace_bytes, void *stream) {
  return moe_routes(x, w13, w2, topk_ids, tokens, hidden, inter, experts, topk, block_rows, y,
                    workspace, workspace_bytes, true, stream);
}

extern "C" int lm_moe_routes_combine_workspace_size(int64_t tokens, int64_t topk, int64_t hidden,
                                                    int64_t inter, int64_t experts, int64_t *bytes) {
  LM_REQUIRE(bytes && tokens >= 0 && topk > 0 && hidden > 0 && inter > 0 && experts > 0);
  *bytes = carve(nullptr, tokens, topk, hidden, inter, experts, true, true).bytes;
  return LM_OK;
}

namespace {
int moe_routes_combine(const void *x, const void *w13, const void *w2, const int32_t *topk_ids,
                       const float *topk_weights, int64_t tokens, int64_t hidden, int64_t inter,
                       int64_t experts, int64_t topk, void *residual, float alpha, float *sumsq,
                       void *out, void *workspace, int64_t workspace_bytes, bool packed,
                       void *stream) {
  LM_REQUIRE(tokens >= 0 && topk > 0 && topk <= 8 && topk <= experts && experts <= 511);
  if (!expert_shapes_ok(hidden, inter) || !scan_path(tokens, topk)) return LM_EUNSUPPORTED;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && w13 && w2 && topk_ids && topk_weights && workspace);
  LM_REQUIRE(residual ? (sumsq != nullptr && out == nullptr) : (out != nullptr && sumsq == nullptr));
  ExpertWorkspace w = carve(workspace, tokens, topk, hidden, inter, experts, true, true);
  if (workspace_bytes < w.bytes) return LM_EWORKSPACE;
  TileCombine fin;
  fin.counters = w.counters;
  fin.scales = topk_weights;
  fin.out = (bf16 *)(residual ? residual : out);
  fin.alpha = alpha;
  fin.sumsq = sumsq;
  fin.tokens = (int)tokens;
  fin.topk = (int)topk;
  auto launch = packed ? launch_routes_combine_t<true> : launch_routes_combine_t<false>;
  return launch((const bf16 *)x, (const bf16 *)w13, (const bf16 *)w2, topk_ids, tokens, topk, hidden,
                inter, experts, w.act, w.y, fin, residual != nullptr, (hipStream_t)stream);
}
}  // namespace

extern "C" int lm_moe_routes_combine(const void *x, const void *w13, const void *w2,
                                     const int32_t *topk_ids, const float *topk_weights,
                                     int64_t tokens, int64_t hidden, int64_t inter,
                                     int64_t experts, int64_t topk, void *residual, float alpha,
                                     float *sumsq, void *out, void *workspace,
                                     int64_t workspace_bytes, void *stream) {
  return moe_routes_combine(x, w13, w2, topk_ids, topk_weights, tokens, hidden, inter, experts, topk,
                            residual, alpha, sumsq, out, workspace, workspace_bytes, false, stream);
}

extern "C" int lm_moe_routes_combine_packed(const void *x, const void *w13, const void *w2,
                                            const int32_t *topk_ids, const float *topk_weights,
                                            int64_t tokens, int64_t hidden, int64_t inter,
                                            int64_t experts, int64_t topk, void *residual,
                                            float alpha, float *sumsq, void *out, void *workspace,
                                            int64_t workspace_bytes, void *stream) {
  return moe_routes_combine(x, w13, w2, topk_ids, topk_weights, tokens, hidden, inter, experts, topk,
                            residual, alpha, sumsq, out, workspace, workspace_bytes, true, stream);
}

extern "C" int lm_expert_pack(const void *w13, const void *w2, int64_t experts, int64_t hidden,
                              int64_t inter, void *w13_packed, void *w2_packed, void *stream) {
  LM_REQUIRE(experts > 0 && hidden > 0 && inter > 0 && w13 && w2 && w13_packed && w2_packed &&
             w13 != w13_packed && w2 != w2_packed);
  if (!expert_shapes_ok(hidden, inter)) return LM_EUNSUPPORTED;
  LM_REQUIRE(((reinterpret_cast<uintptr_t>(w13) | reinterpret_cast<uintptr_t>(w2) |
               reinterpret_cast<uintptr_t>(w13_packed) | reinterpret_cast<uintptr_t>(w2_packed)) &
              15) == 0);
  hipStream_t s = (hipStream_t)stream;
  const int rc = expert_pack(w13, experts * 2 * inter, hidden, w13_packed, s);
  if (rc) return rc;
  return expert_pack(w2, experts * hidden, inter, w2_packed, s);
}

extern "C" int lm_fused_experts(const void *x, const void *w13, const void *w2,
                                const float *topk_weights, const int32_t *topk_ids,
                                const int64_t *logical, int64_t tokens, int64_t hidden,
                                int64_t inter, int64_t experts, int64_t topk, int64_t block_rows,
                                void *out, void *workspace, int64_t workspace_bytes, void *stream) {
  return fused_experts(x, w13, w2, topk_weights, topk_ids, logical, tokens, hidden, inter, experts,
                       topk, block_rows, out, workspace, workspace_bytes, false, stream);
}

extern "C" int lm_fused_experts_packed(const void *x, const void *w13, const void *w2,
                                       const float *topk_weights, const int32_t *topk_ids,
                                       const int64_t *logical, int64_t tokens, int64_t hidden,
                                       int64_t inter, int64_t experts, int64_t topk,
                                       int64_t block_rows, void *out, void *workspace,
                                       int64_t workspace_bytes, void *stream) {
  return fused_experts(x, w13, w2, topk_weights, topk_ids, logical, tokens, hidden, inter, experts,
                       topk, block_rows, out, workspace, workspace_bytes, true, stream);
}

// ---------------------------------------------------------------------------
// lm_fused_experts_noalloc: the same call with its workspace carved from a
// static device array instead of a caller buffer, for callers that cannot
// allocate. Each GPU holds its own copy of the array (at its own address)
// from the module's load to the end of the process. Nothing in the
// workspace needs to start at zero: every offset, route list, act and y
// row a kernel reads is written earlier in the same call, so the previous
// call's contents never leak into a result. Calls that overlap on one GPU
// (two streams, or two host threads) share the array and race.
namespace {
constexpr int64_t kNoAllocScratchBytes = int64_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void *scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once looked up

// The array's device address on the current device. In host code the name
// `scratch` is only a host-side stand-in: it must never reach a kernel or
// a copy, so every use goes through the looked-up address.
int scratch_address(int device, void **out) {
  if (device < 0 || device >= kMaxDevices) return LM_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[device]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LM_ELAUNCH;
    scratch_ptr[device] = p;
  }
  *out = scratch_ptr[device];
  return LM_OK;
}
}  // namespace

extern "C" int lm_fused_experts_noalloc(const void *x, const void *w13, const void *w2,
                                        const float *topk_weights, const int32_t *topk_ids,
                                        const int64_t *logical, int64_t tokens, int64_t hidden,
                                        int64_t inter, int64_t experts, int64_t topk,
                                        int64_t block_rows, void *out, void *stream) {
  LM_REQUIRE(tokens >= 0 && topk > 0 && topk <= 8 && topk <= experts && block_rows >= 0 &&
             block_rows % 16 == 0 && experts <= 511);
  if (!expert_shapes_ok(hidden, inter)) return LM_EUNSUPPORTED;
  if (carve(nullptr, tokens, topk, hidden, inter, experts, true).bytes > kNoAllocScratchBytes)
    return LM_ETOOLARGE;
  if (tokens == 0) return LM_OK;
  LM_REQUIRE(x && w13 && w2 && topk_weights && topk_ids && out);
  // The array is looked up with the stream's device current (the caller's
  // current device must be the stream's).
  int device = -1, current = -1;
  if (hipGetDevice(&current) != hipSuccess) return LM_ELAUNCH;
  if (stream) {
    if (hipStreamGetDevice((hipStream_t)stream, &device) != hipSuccess) return LM_EINVAL;
    if (device != current) return LM_EINVAL;
  } else {
    device = current;
  }
  void *base = nullptr;
  const int rc = scratch_address(device, &base);
  if (rc) return rc;
  ExpertWorkspace w = carve(base, tokens, topk, hidden, inter, experts, true);
  const int rr = run_routes(x, w13, w2, topk_ids, tokens, hidden, inter, experts, topk, block_rows,
                            w.y, w, false, stream);
  if (rr) return rr;
  return launch_finish(w.y, topk_ids, nullptr, topk_weights, logical, (bf16 *)out, tokens, hidden,
                       topk, 0, experts, (hipStream_t)stream);
}
