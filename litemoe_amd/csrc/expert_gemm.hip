// Grouped expert GEMMs for prefill-sized route counts, on MFMA with LDS tiles:
//
//   gate_up: act[r, j] = bf16(silu(bf16(x_t . W13[e, j])) * bf16(x_t . W13[e, I + j]))
//   down:    y[r, n]   = bf16(act[r] . W2[e, n])
//
// over the route blocks of lm_moe_align (routes sorted by expert; a block is
// at most 128 routes of one expert, found on the device from the offsets).
// act and y are in route order r = t*topk + branch, as on the decode path.
//
// Workgroup = (output column tile, route block), 4 waves. It computes a
// 128 x 128 fp32 tile: for gate_up the B tile is 64 gate rows and the 64 up
// rows of the same j, so silu(g)*u is formed in registers. The waves sit in
// 2 x 2, each 64 x 64 as 4 x 4 tiles of v_mfma_f32_16x16x32_bf16.
//
// K runs in steps of 64, double-buffered: the next step's A rows (gathered
// through the route list) and B rows are loaded into registers while the
// MFMAs run on the current step's LDS tiles, then stored to the other LDS
// buffer. (Direct global-to-LDS loads would save the registers, but the
// compiler then waits for every load in flight before each LDS read.) An LDS
// row is 64 bf16 = 8 chunks of 16 bytes; chunk c of tile row r sits at
// position c ^ (r & 7), so the 16 rows read by one MFMA fragment load spread
// over the banks, and each wave's stores fill 1 KB contiguously.
//
// Reference: the expert math of litemoe/ops.py:43-47 (reference_experts) and
// vLLM fused_experts at litemoe/ep.py:40-41.
#include "internal.h"

namespace lm {
namespace {

constexpr int kBM = 128;  // route rows per tile
constexpr int kBN = 128;  // B rows (output columns) per tile
constexpr int kBK = 64;   // K per stage
constexpr int kThreads = 256;
constexpr int kXcds = 8;  // MI355X: 8 XCDs, each with its own L2
constexpr int kRowBytes = kBK * 2;                // 128
constexpr int kOperandBytes = kBM * kRowBytes;    // 16 KB
constexpr int kStageBytes = 2 * kOperandBytes;    // A then B
constexpr int kLoadsPerOperand = kOperandBytes / (kThreads * 16);  // 4

// Block b of the per-expert blocks of bm routes (offsets: exclusive prefix
// of per-expert counts, as lm_moe_align writes it).
__device__ __forceinline__ bool block_of(const int32_t *__restrict__ offsets, int experts, int bm,
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

// Tile row and chunk each lane of a wave moves per load instruction: wave w,
// instruction i fills LDS rows 8*(4w+i) .. +7 (1 KB, lane l at byte 16*l),
// i.e. row 8*(4w+i) + l/8, position l%8, holding chunk (l%8) ^ (l/8).
__device__ __forceinline__ int load_row(int wave, int i, int lane) { return 8 * (4 * wave + i) + lane / 8; }
__device__ __forceinline__ int load_chunk(int lane) { return (lane & 7) ^ (lane >> 3); }

// Byte offset in an operand tile of (row, 16-byte chunk).
__device__ __forceinline__ int frag_offset(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ (row & 7)) << 4);
}

// kGateUp: B rows 0..63 are W13[e, j0 + r], 64..127 are W13[e, I + j0 + r - 64],
// output act; otherwise B rows are W2[e, n0 + r], output y.
template <bool kGateUp>
__global__ void __launch_bounds__(kThreads, 2)
expert_gemm_kernel(const bf16 *__restrict__ a_src, const bf16 *__restrict__ w,
                   const int32_t *__restrict__ offsets, const int32_t *__restrict__ sorted,
                   int topk, int K, int out_cols, int inter, int experts,
                   bf16 *__restrict__ out) {
  __shared__ __align__(16) char smem[2 * kStageBytes];
  __shared__ int route_of[kBM];
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
  if (!block_of(offsets, experts, kBM, tile_y, e, r0, r1)) return;
  const int n = r1 - r0;
  const int c0 = tile_x * (kGateUp ? kBN / 2 : kBN);  // first output column
  if (threadIdx.x < kBM) route_of[threadIdx.x] = sorted[r0 + min((int)threadIdx.x, n - 1)];
  __syncthreads();

  // Global row pointers of the 4 A rows and 4 B rows this lane loads.
  const int chunk = load_chunk(lane);
  const bf16 *ga[kLoadsPerOperand], *gb[kLoadsPerOperand];
#pragma unroll
  for (int i = 0; i < kLoadsPerOperand; ++i) {
    const int row = load_row(wave, i, lane);
    const int route = route_of[row];
    ga[i] = a_src + (int64_t)(kGateUp ? route / topk : route) * K + chunk * 8;
    int64_t wrow;
    if constexpr (kGateUp)
      wrow = (int64_t)e * 2 * inter + (row < kBN / 2 ? c0 + row : inter + c0 + row - kBN / 2);
    else
      wrow = (int64_t)e * out_cols + c0 + row;
    gb[i] = w + wrow * K + chunk * 8;
  }
  // Two register stages: the loads for step k+2 are issued while step k is
  // computed from LDS and step k+1 waits in registers for its LDS store.
  u32x4 ra[2][kLoadsPerOperand], rb_[2][kLoadsPerOperand];
  auto load = [&](int set, int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < kLoadsPerOperand; ++i) {
      ra[set][i] = *reinterpret_cast<const u32x4 *>(ga[i] + k0);
      rb_[set][i] = *reinterpret_cast<const u32x4 *>(gb[i] + k0);
    }
  };
  auto store = [&](int set, int buf) {
    char *base = smem + buf * kStageBytes + lane * 16;
#pragma unroll
    for (int i = 0; i < kLoadsPerOperand; ++i) {
      *reinterpret_cast<u32x4 *>(base + (4 * wave + i) * 1024) = ra[set][i];
      *reinterpret_cast<u32x4 *>(base + kOperandBytes + (4 * wave + i) * 1024) = rb_[set][i];
    }
  };

  const int wr = wave / 2, wc = wave % 2;
  const int fr = lane % 16, fk = lane / 16;
  // B tile rows of this wave's four 16-column blocks.
  int brow[4];
#pragma unroll
  for (int cb = 0; cb < 4; ++cb)
    brow[cb] = kGateUp ? (cb < 2 ? wc * 32 + cb * 16 : kBN / 2 + wc * 32 + (cb - 2) * 16)
                       : wc * 64 + cb * 16;
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int stage) {
    const char *as = smem + stage * kStageBytes;
    const char *bs = as + kOperandBytes;
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      u32x4 af[4], bfr[4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
        af[rb] = *reinterpret_cast<const u32x4 *>(as + frag_offset(wr * 64 + rb * 16 + fr, kk * 4 + fk));
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        bfr[cb] = *reinterpret_cast<const u32x4 *>(bs + frag_offset(brow[cb] + fr, kk * 4 + fk));
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = mfma16x16x32(af[rb], bfr[cb], acc[rb][cb]);
    }
  };

  // K is a multiple of 2 * kBK: the loop runs pairs of steps so that the
  // register sets alternate without copies.
  const int nk = K / kBK;
  load(0, 0);
  store(0, 0);
  load(0, 1);
  __syncthreads();
  for (int kt = 0; kt + 2 < nk; kt += 2) {
    // LDS buffer 0: step kt; registers 0: step kt+1 (in flight).
    load(1, kt + 2);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out before the MFMAs
    compute(0);
    store(0, 1);
    __syncthreads();
    // LDS buffer 1: step kt+1; registers 1: step kt+2 (in flight).
    load(0, kt + 3);
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
    store(1, 0);
    __syncthreads();
  }
  compute(0);
  store(0, 1);
  __syncthreads();
  compute(1);

  // C fragment: lane holds rows 4*(lane/16) + i of column lane%16.
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = wr * 64 + rb * 16 + 4 * fk + i;
      if (row >= n) continue;
      bf16 *o = out + (int64_t)route_of[row] * out_cols + c0;
      if constexpr (kGateUp) {
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const float h = round_bf16(silu(round_bf16(acc[rb][cb][i]))) * round_bf16(acc[rb][cb + 2][i]);
          o[wc * 32 + cb * 16 + fr] = (bf16)f32_to_bf16(h);
        }
      } else {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) o[wc * 64 + cb * 16 + fr] = (bf16)f32_to_bf16(acc[rb][cb][i]);
      }
    }
  }
}

}  // namespace

bool expert_gemm_ok(int64_t routes, int64_t hidden, int64_t inter) {
  return routes >= kExpertGemmMinRoutes && hidden % (2 * kBK) == 0 && inter % (2 * kBK) == 0 &&
         inter % (kBN / 2) == 0 && hidden % kBN == 0;
}

int launch_expert_gemm_gate_up(const bf16 *x, const bf16 *w13, const int32_t *offsets,
                               const int32_t *sorted, int64_t routes, int64_t topk, int64_t hidden,
                               int64_t inter, int64_t experts, bf16 *act, hipStream_t stream) {
  const int64_t blocks = align_up(cdiv(routes, kBM) + experts, kXcds);
  if (blocks > 65535) return LM_EUNSUPPORTED;
  const dim3 grid((unsigned)(inter / (kBN / 2)), (unsigned)blocks);
  expert_gemm_kernel<true><<<grid, kThreads, 0, stream>>>(
      x, w13, offsets, sorted, (int)topk, (int)hidden, (int)inter, (int)inter, (int)experts, act);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

int launch_expert_gemm_down(const bf16 *act, const bf16 *w2, const int32_t *offsets,
                            const int32_t *sorted, int64_t routes, int64_t hidden, int64_t inter,
                            int64_t experts, bf16 *y, hipStream_t stream) {
  const int64_t blocks = align_up(cdiv(routes, kBM) + experts, kXcds);
  if (blocks > 65535) return LM_EUNSUPPORTED;
  const dim3 grid((unsigned)(hidden / kBN), (unsigned)blocks);
  expert_gemm_kernel<false><<<grid, kThreads, 0, stream>>>(
      act, w2, offsets, sorted, 1, (int)inter, (int)hidden, (int)inter, (int)experts, y);
  LM_CHECK_LAUNCH();
  return LM_OK;
}

}  // namespace lm
