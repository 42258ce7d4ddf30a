// Grouped expert GEMMs for prefill-sized route counts, on MFMA with LDS tiles:
//
//   gate_up: act[r, j] = bf16(silu(bf16(x_t . W13[e, j])) * bf16(x_t . W13[e, I + j]))
//   down:    y[r, n]   = bf16(act[r] . W2[e, n])
//
// over the route blocks of lm_moe_align (routes sorted by expert; a block is
// at most kTM routes of one expert, found on the device from the offsets).
// y is in route order r = t*topk + branch, as on the decode path; act is in
// route order for the public gate_up / down entry points and in sorted order
// (row = position in the expert-sorted route list) between the two GEMMs of
// one fused call, so that down reads each route block's act rows as one
// contiguous run instead of gathering 128-byte pieces of rows spread over
// the whole buffer.
//
// Workgroup = (output column tile, route block). It computes a kTM x kTN
// fp32 tile (256 x 256 on 8 waves, or 128 x 128 on 4, see LargeTile /
// SmallTile): for gate_up the B tile is kTN/2 gate rows and the kTN/2 up rows
// of the same j, so silu(g)*u is formed in registers. The waves sit in
// kWM x kWN, each (kTM/kWM) x (kTN/kWN) as 16 x 16 tiles of
// v_mfma_f32_16x16x32_bf16.
//
// K runs in steps of 64. With two LDS stages (the large tile) the next
// step's A rows (gathered through the route list: each lane's copy has its
// own address) and B rows are copied from global memory straight into the
// other stage (global_load_lds_dwordx4, lds_copy16) while the MFMAs run on
// the current one; with one stage (the small tile) they are loaded into
// registers meanwhile and stored to LDS after a barrier. An LDS row is 64
// bf16 = 8 chunks of 16 bytes; chunk c of tile row r sits at position
// c ^ (r & 7), so the 16 rows read by one MFMA fragment load spread over the
// banks, and each wave instruction fills 1 KB contiguously.
//
// Reference: the expert math of litemoe/ops.py:43-47 (reference_experts) and
// vLLM fused_experts at litemoe/ep.py:40-41.
#include <algorithm>
#include <type_traits>

#include "internal.h"

namespace lm {
namespace {

constexpr int kBK = 64;   // K per stage
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2
constexpr int kRowBytes = kBK * 2;  // 128

// Two workgroup tiles, chosen per call by the routes per expert:
// - Large: 256 route rows x 256 B rows on 8 waves of 64 x 128 (4 x 2), two
//   LDS stages (128 KB, one workgroup per CU): a wave's fragments feed 32
//   MFMAs per 32-wide k step, half the LDS reads per MFMA of a 64 x 64 wave
//   tile. At cfg 4's 46,990 tokens (uniform routes, one box, register
//   staging): gate/up 1230 against 1561 us, down 912 against 1063 us for the
//   small tile; 16 waves of 64 x 64 1339 / 936 us, 128 x 256 on 8 waves
//   1412 / 1071 us. With the direct copies the MoE takes 2.13 against 2.34
//   ms; 16 waves of 64 x 64 (LM_EXPERT_LARGE_WN=4) are within 1% of 8.
// - Small: 128 x 128 on 4 waves of 64 x 64, one LDS stage (33 KB, several
//   workgroups per CU), for fewer than 1024 routes per expert, where a
//   256-route block would be mostly padding.
// (Earlier measurements of this kernel at 65k tokens: 128 x 128 with two
// stages 3.83 against 3.34 ms for the MoE; 256 x 256 on 4 waves with the
// accumulators in AGPRs 4.16 ms.)
template <int TM, int TN, int WMv, int WNv, int StagesV>
struct TileCfg {
  static constexpr int M = TM, N = TN, WM = WMv, WN = WNv, Stages = StagesV;
};
#ifndef LM_EXPERT_LARGE_WN
#define LM_EXPERT_LARGE_WN 2
#endif
using LargeTile = TileCfg<256, 256, 4, LM_EXPERT_LARGE_WN, 2>;
using SmallTile = TileCfg<128, 128, 2, 2, 1>;
constexpr int64_t kLargeTileRoutesPerExpert = 1024;

// Block b of the per-expert blocks of bm routes (offsets: exclusive prefix
// of per-expert counts, as lm_moe_align writes it), found by each wave with
// one vector load per 64 experts: lane l takes expert e0 + l's block count,
// an inclusive prefix sum over the lanes gives each expert's first block, and
// the expert holding b is the one lane whose block range contains it. (A
// scalar walk over the experts waits on one load per expert.)
__device__ __forceinline__ bool block_of(const int32_t *__restrict__ offsets, int experts, int bm,
                                         int b, int &e_out, int &r0, int &r1) {
  const int lane = threadIdx.x % kWave;
  int before = 0;  // blocks of the experts below e0
  for (int e0 = 0; e0 < experts; e0 += kWave) {
    const int e = e0 + lane;
    const int o0 = e < experts ? offsets[e] : 0;
    const int o1 = e < experts ? offsets[e + 1] : 0;
    const int nb = (o1 - o0 + bm - 1) / bm;
    int incl = nb;
#pragma unroll
    for (int d = 1; d < kWave; d *= 2) {
      const int up = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += up;
    }
    const int first = before + incl - nb;
    const uint64_t hit = __ballot(b >= first && b < first + nb);
    if (hit) {
      const int l = __ffsll((unsigned long long)hit) - 1;
      e_out = e0 + l;
      r0 = __shfl(o0, l, kWave) + (b - __shfl(first, l, kWave)) * bm;
      r1 = min(__shfl(o1, l, kWave), r0 + bm);
      return true;
    }
    before += __shfl(incl, kWave - 1, kWave);
  }
  return false;
}

// Byte offset in an operand tile of (row, 16-byte chunk).
__device__ __forceinline__ int frag_offset(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ (row & 7)) << 4);
}

// kGateUp: B rows [0, kTN/2) are W13[e, j0 + r], [kTN/2, kTN) are
// W13[e, I + j0 + r - kTN/2], output act; otherwise B rows are W2[e, n0 + r],
// output y. Waves sit in kWM x kWN; wave (wr, wc) owns rows wr*kTM/kWM .. and,
// for gate_up, the gate and up rows of the same kTN/(2*kWN) columns j.
// kPacked: weights in the fragment layout of lm_expert_pack (a load
// instruction then reads eight whole 128-byte runs: the 8 rows of one
// (k-step, k-group) are adjacent there).
// kSortedAct: act row of sorted position p is p (gate_up writes, down reads).
template <bool kGateUp, int kTM, int kTN, int kWM, int kWN, int kStages, bool kPacked,
          bool kSortedAct>
__global__ void __launch_bounds__(64 * kWM * kWN)
expert_gemm_kernel(const bf16 *__restrict__ a_src, const bf16 *__restrict__ w,
                   const int32_t *__restrict__ offsets, const int32_t *__restrict__ sorted,
                   int topk, int K, int out_cols, int inter, int experts,
                   bf16 *__restrict__ out) {
  constexpr int kWaves = kWM * kWN, kThreadsT = 64 * kWaves;
  constexpr int kWaveRows = kTM / kWM, kWaveCols = kTN / kWN;
  constexpr int kRB = kWaveRows / 16, kCB = kWaveCols / 16;  // 16-row / 16-column blocks per wave
  constexpr int kLA = kTM / (8 * kWaves), kLB = kTN / (8 * kWaves);  // 16-byte loads per lane
  static_assert(kLA * 8 * kWaves == kTM && kLB * 8 * kWaves == kTN, "tile rows per load round");
  static_assert(!kGateUp || kCB % 2 == 0, "gate/up waves hold gate and up blocks in pairs");
  constexpr int kABytes = kTM * kRowBytes, kStageBytes = (kTM + kTN) * kRowBytes;
  // kStages == 2: two LDS stages filled by direct copies; kStages == 1: one,
  // filled from registers.
  __shared__ __align__(16) char smem[kStageBytes];
  __shared__ __align__(16) char smem1[kStages == 2 ? kStageBytes : 16];
  __shared__ int route_of[kTM];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  // Workgroups are dealt to the 8 XCDs round-robin in launch order. Remap so
  // that each XCD takes a contiguous range of route blocks with all their
  // column tiles: a block's gathered A rows are then fetched into one L2, and
  // an expert's weight rows mostly into one or two.
  const int cols = gridDim.x;
  const int lin = blockIdx.y * cols + blockIdx.x;
  const int j = lin / kXcds;  // gridDim.y is a multiple of kXcds
  const int tile_y = (lin % kXcds) * (gridDim.y / kXcds) + j / cols;
  const int tile_x = j % cols;
  int e, r0, r1;
  if (!block_of(offsets, experts, kTM, tile_y, e, r0, r1)) return;
  const int n = r1 - r0;
  const int c0 = tile_x * (kGateUp ? kTN / 2 : kTN);  // first output column
  // The route list in LDS serves the A row offsets of gate_up and of down on
  // route-order act, and y's rows in down's epilogue. gate_up on sorted act
  // reads each row's route directly (no LDS round, no barrier); down on
  // sorted act fills the list only after its first k step's copies are out
  // (its rows are the block's own), so the two load round trips overlap.
  constexpr bool kRouteList = !(kGateUp && kSortedAct), kListFirst = !kSortedAct;
  auto fill_routes = [&]() {
    for (int t = threadIdx.x; t < kTM; t += kThreadsT) route_of[t] = sorted[r0 + min(t, n - 1)];
  };
  if constexpr (kListFirst) {
    fill_routes();
    __syncthreads();
  }

  // Load instruction i of wave w fills LDS rows 8*(w*L+i) .. +7 of an
  // operand (1 KB, lane l at byte 16*l): row 8*(w*L+i) + l/8, position l%8,
  // holding chunk (l%8) ^ (l/8), which is frag_offset's swizzle.
  const int chunk = (lane & 7) ^ (lane >> 3);
  int oa[kLA], ob[kLB];  // element offsets (< 2^31 at the supported sizes)
#pragma unroll
  for (int i = 0; i < kLA; ++i) {
    const int t = 8 * (wave * kLA + i) + lane / 8;
    if constexpr (!kGateUp && kSortedAct) {
      oa[i] = (r0 + min(t, n - 1)) * K + chunk * 8;
    } else {
      const int route = kListFirst ? route_of[t] : sorted[r0 + min(t, n - 1)];
      oa[i] = (kGateUp ? route / topk : route) * K + chunk * 8;
    }
  }
#pragma unroll
  for (int i = 0; i < kLB; ++i) {
    const int row = 8 * (wave * kLB + i) + lane / 8;
    const int wrow = kGateUp ? e * 2 * inter + (row < kTN / 2 ? c0 + row : inter + c0 + row - kTN / 2)
                             : e * out_cols + c0 + row;
    ob[i] = (int)wofs<kPacked>(wrow, chunk * 8, K);
  }
  // element advance of one kBK step of B (two 32-wide k-steps when packed)
  constexpr int kBStep = kPacked ? (int)(kBK / 32 * wstep<true>()) : kBK;
  // One stage: step k+1 is loaded into registers while step k is computed
  // from LDS, then stored to LDS after a barrier.
  u32x4 ra[kLA], rbv[kLB];
  auto load = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < kLA; ++i) ra[i] = *reinterpret_cast<const u32x4 *>(a_src + oa[i] + k0);
#pragma unroll
    for (int i = 0; i < kLB; ++i) rbv[i] = *reinterpret_cast<const u32x4 *>(w + ob[i] + kt * kBStep);
  };
  auto store = [&]() {
    char *base = smem + lane * 16;
#pragma unroll
    for (int i = 0; i < kLA; ++i) *reinterpret_cast<u32x4 *>(base + (wave * kLA + i) * 1024) = ra[i];
#pragma unroll
    for (int i = 0; i < kLB; ++i)
      *reinterpret_cast<u32x4 *>(base + kABytes + (wave * kLB + i) * 1024) = rbv[i];
  };
  // Two stages: step k+1 is copied from global memory straight into the
  // other stage while step k is computed (byte offsets: the element offsets
  // are below 2^31).
  const uint32_t uw = __builtin_amdgcn_readfirstlane(wave);
  auto issue_a = [&](int kt, const char *stage) {
    const bf16 *ak = a_src + kt * kBK;
    const uint32_t la = lds_address(stage) + uw * kLA * 1024;
#pragma unroll
    for (int i = 0; i < kLA; ++i) lds_copy16(ak, (uint32_t)oa[i] * 2, la + i * 1024);
  };
  auto issue_b = [&](int kt, const char *stage) {
    const bf16 *wk = w + kt * kBStep;
    const uint32_t lb = lds_address(stage) + kABytes + uw * kLB * 1024;
#pragma unroll
    for (int i = 0; i < kLB; ++i) lds_copy16(wk, (uint32_t)ob[i] * 2, lb + i * 1024);
  };

  const int wr = wave / kWN, wc = wave % kWN;
  const int fr = lane % 16, fk = lane / 16;
  constexpr int kGateCols = kWaveCols / 2;  // gate/up: gate (and up) columns of a wave
  int brow[kCB];
#pragma unroll
  for (int cb = 0; cb < kCB; ++cb)
    brow[cb] = kGateUp ? (cb < kCB / 2 ? wc * kGateCols + cb * 16
                                       : kTN / 2 + wc * kGateCols + (cb - kCB / 2) * 16)
                       : wc * kWaveCols + cb * 16;
  f32x4 acc[kRB][kCB];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int jj = 0; jj < kCB; ++jj) acc[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One 32-wide half of a k step.
  auto compute_kk = [&](const char *as, int kk) {
    const char *bs = as + kABytes;
    {
      // B fragments stay in registers for the whole k step; A fragments are
      // read one row block at a time.
      u32x4 bfr[kCB];
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
        bfr[cb] = *reinterpret_cast<const u32x4 *>(bs + frag_offset(brow[cb] + fr, kk * 4 + fk));
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        const u32x4 af =
            *reinterpret_cast<const u32x4 *>(as + frag_offset(wr * kWaveRows + rb * 16 + fr, kk * 4 + fk));
        // weights as the first operand: the tile is computed transposed
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) acc[rb][cb] = mfma16x16x32(bfr[cb], af, acc[rb][cb]);
      }
    }
  };
  auto compute = [&](const char *as) {
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) compute_kk(as, kk);
  };

  const int nk = K / kBK;
  if constexpr (kStages == 2) {
    // Before a stage is read: this wave's copies have landed (vmcnt) and the
    // barrier has seen every wave's, and every wave has left the step that
    // last read the stage the next copy goes into.
    // The next step's copies go out in two groups, one before each 32-wide
    // half of the current step's MFMAs, instead of all eight before the
    // first: gate/up issues its weight rows first, down its activation rows
    // (the cfg 4 prefill 99.0-99.6 -> 98.8-98.9 ms, the MoE 1.95-1.97 ->
    // 1.945-1.949 ms per layer with uniform routes; A/B on one box, three
    // runs each; the other orders and an even split of both within 1%).
    static_assert(kBK / 32 == 2, "two halves per k step");
    auto issue_first = [&](int kt, const char *stage) {
      if constexpr (kGateUp) issue_b(kt, stage); else issue_a(kt, stage);
    };
    auto issue_second = [&](int kt, const char *stage) {
      if constexpr (kGateUp) issue_a(kt, stage); else issue_b(kt, stage);
    };
    issue_a(0, smem);
    issue_b(0, smem);
    // published by the first barrier below; read only in the epilogue
    if constexpr (kRouteList && !kListFirst) fill_routes();
    for (int kt = 0; kt < nk; kt += 2) {
      lds_copy_wait();
      __syncthreads();
      if (kt + 1 < nk) issue_first(kt + 1, smem1);
      __builtin_amdgcn_sched_barrier(0);
      compute_kk(smem, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 1 < nk) issue_second(kt + 1, smem1);
      __builtin_amdgcn_sched_barrier(0);
      compute_kk(smem, 1);
      if (kt + 1 < nk) {
        lds_copy_wait();
        __syncthreads();
        if (kt + 2 < nk) issue_first(kt + 2, smem);
        __builtin_amdgcn_sched_barrier(0);
        compute_kk(smem1, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 2 < nk) issue_second(kt + 2, smem);
        __builtin_amdgcn_sched_barrier(0);
        compute_kk(smem1, 1);
      }
    }
  } else {
    load(0);
    if constexpr (kRouteList && !kListFirst) fill_routes();
    store();
    __syncthreads();
    for (int kt = 0; kt + 1 < nk; ++kt) {
      load(kt + 1);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before the MFMAs
      compute(smem);
      __syncthreads();  // every wave is done with the buffer
      store();
      __syncthreads();
    }
    compute(smem);
  }

  // Transposed C fragment: lane holds output row lane%16 of each 16-row block
  // and its output columns 4*(lane/16) .. +3 of each 16-column block, one
  // 8-byte word. Intermediate roundings skip the NaN canonicalization (a NaN
  // stays NaN through silu and the product, and the stored value is
  // canonicalized). The bf16 tile is staged in the (now idle) LDS stages and
  // written out row by row in 16-byte words, so that a store instruction
  // covers whole output rows (512 or 256 bytes each) instead of 32-byte
  // pieces of 16 rows. Staged row r's 16-byte chunk c sits at c ^ (r & kSw):
  // the 16 rows of one fragment store fall on different bank groups.
  constexpr int kOutCols = kGateUp ? kTN / 2 : kTN, kOB = kOutCols * 2;  // output row bytes
  constexpr int kChunks = kOB / 16, kSw = (kChunks < 16 ? kChunks : 16) - 1;
  constexpr int kHalfRows = kStageBytes / kOB;  // rows held by the first stage
  static_assert(kTM * kOB <= (kStages == 2 ? 2 : 1) * kStageBytes, "output tile fits the LDS stages");
  auto staged = [&](int row) -> char * {
    if constexpr (kTM <= kHalfRows) return smem + row * kOB;
    else return row < kHalfRows ? smem + row * kOB : smem1 + (row - kHalfRows) * kOB;
  };
  __syncthreads();  // every wave has finished reading the stages
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int row = wr * kWaveRows + rb * 16 + fr;
    char *srow = staged(row);
    if constexpr (kGateUp) {
#pragma unroll
      for (int cb = 0; cb < kCB / 2; ++cb) {
        float h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          h[i] = round_bf16_nc(silu(round_bf16_nc(acc[rb][cb][i]))) * round_bf16_nc(acc[rb][cb + kCB / 2][i]);
        const int byte = 2 * (wc * kGateCols + cb * 16 + 4 * fk);
        *reinterpret_cast<uint2 *>(srow + (((byte >> 4) ^ (row & kSw)) << 4) + (byte & 8)) =
            make_uint2(pack_bf16(h[0], h[1]), pack_bf16(h[2], h[3]));
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const int byte = 2 * (wc * kWaveCols + cb * 16 + 4 * fk);
        *reinterpret_cast<uint2 *>(srow + (((byte >> 4) ^ (row & kSw)) << 4) + (byte & 8)) =
            make_uint2(pack_bf16(acc[rb][cb][0], acc[rb][cb][1]), pack_bf16(acc[rb][cb][2], acc[rb][cb][3]));
      }
    }
  }
  __syncthreads();
  static_assert((kTM * kChunks) % kThreadsT == 0, "whole store rounds");
#pragma unroll
  for (int i = 0; i < kTM * kChunks / kThreadsT; ++i) {
    const int idx = i * kThreadsT + threadIdx.x;
    const int row = idx / kChunks, c = idx % kChunks;
    if (row >= n) continue;
    const int64_t orow = kGateUp && kSortedAct ? r0 + row : route_of[row];
    // Non-temporal: act and y are written once and read once by the next
    // launch, far more bytes (0.4 and 1.2 GB at cfg 4) than the caches hold
    // (the cfg 4 prefill 102.8 -> 100.1-100.5 ms, A/B on one box, three runs
    // each).
    __builtin_nontemporal_store(*reinterpret_cast<const u32x4 *>(staged(row) + ((c ^ (row & kSw)) << 4)),
                                reinterpret_cast<u32x4 *>(out + orow * out_cols + c0 + c * 8));
  }
}

}  // namespace

bool expert_gemm_ok(int64_t routes, int64_t hidden, int64_t inter, int64_t experts) {
  // 32-bit element offsets: the gathered rows and the weights stay below 2^31.
  const int64_t rows = std::max(routes, experts * std::max(2 * inter, hidden));
  return routes >= kExpertGemmMinRoutes && hidden % kBK == 0 && inter % kBK == 0 &&
         (2 * inter) % SmallTile::N == 0 && hidden % SmallTile::N == 0 &&
         rows * std::max(hidden, inter) < ((int64_t)1 << 31);
}

namespace {

template <class T>
int launch_tile(bool gate_up, const bf16 *a, const bf16 *w, const int32_t *offsets,
                const int32_t *sorted, int64_t routes, int64_t topk, int64_t K, int64_t out_cols,
                int64_t inter, int64_t experts, bf16 *out, bool packed, bool sorted_act,
                hipStream_t stream) {
  const int64_t blocks = align_up(cdiv(routes, T::M) + experts, kXcds);
  if (blocks > 65535) return LM_EUNSUPPORTED;
  const int64_t cols = gate_up ? 2 * inter : out_cols;
  const dim3 grid((unsigned)(cols / T::N), (unsigned)blocks);
  const int threads = 64 * T::WM * T::WN;
  auto go = [&](auto gate_c, auto packed_c, auto sorted_c) {
    expert_gemm_kernel<decltype(gate_c)::value, T::M, T::N, T::WM, T::WN, T::Stages,
                       decltype(packed_c)::value, decltype(sorted_c)::value>
        <<<grid, threads, 0, stream>>>(a, w, offsets, sorted, (int)topk, (int)K, (int)out_cols,
                                       (int)inter, (int)experts, out);
  };
  using Y = std::true_type;
  using F = std::false_type;
  auto by_layout = [&](auto gate_c) {
    if (packed) {
      if (sorted_act) go(gate_c, Y{}, Y{}); else go(gate_c, Y{}, F{});
    } else {
      if (sorted_act) go(gate_c, F{}, Y{}); else go(gate_c, F{}, F{});
    }
  };
  if (gate_up) by_layout(Y{}); else by_layout(F{});
  LM_CHECK_LAUNCH();
  return LM_OK;
}

bool large_tile(int64_t routes, int64_t hidden, int64_t inter, int64_t experts) {
  return routes >= kLargeTileRoutesPerExpert * experts && (2 * inter) % LargeTile::N == 0 &&
         hidden % LargeTile::N == 0;
}

}  // namespace

int launch_expert_gemm_gate_up(const bf16 *x, const bf16 *w13, const int32_t *offsets,
                               const int32_t *sorted, int64_t routes, int64_t topk, int64_t hidden,
                               int64_t inter, int64_t experts, bf16 *act, bool packed,
                               bool sorted_act, hipStream_t stream) {
  auto launch = large_tile(routes, hidden, inter, experts) ? launch_tile<LargeTile> : launch_tile<SmallTile>;
  return launch(true, x, w13, offsets, sorted, routes, topk, hidden, inter, inter, experts, act,
                packed, sorted_act, stream);
}

int launch_expert_gemm_down(const bf16 *act, const bf16 *w2, const int32_t *offsets,
                            const int32_t *sorted, int64_t routes, int64_t hidden, int64_t inter,
                            int64_t experts, bf16 *y, bool packed, bool sorted_act,
                            hipStream_t stream) {
  auto launch = large_tile(routes, hidden, inter, experts) ? launch_tile<LargeTile> : launch_tile<SmallTile>;
  return launch(false, act, w2, offsets, sorted, routes, 1, inter, hidden, inter, experts, y, packed,
                sorted_act, stream);
}

}  // namespace lm
