// Dense projection for prefill-sized (and above-128-row decode) row counts on
// MFMA with LDS tiles:
//
//   out[m, n] = bf16( sum_k a[m, k] * w[n, k] )          (fp32 accumulation)
//
// w is an nn.Linear weight [N, K] (row-major, row stride ldw), a is bf16
// [M, K] with row stride lda, out is bf16 [M, N] with row stride ldo.
//
// Each output element is reduced by one workgroup over all of K, in k steps
// of 32 taken in ascending order (one v_mfma_f32_16x16x32_bf16 per step and
// 16x16 block). The order depends neither on M nor on the row's or tile's
// position, so a row's result is the same bits in any batch, in any launch,
// eager or replayed from a graph (no split-K partials, no atomics, no stream-K
// fix-up whose summation order the caller cannot see).
//
// Workgroup = kTM x kTN output tile (256 x 256 on 16 waves, or 128 x 128 on
// 4), kWM x kWN waves, each wave a (kTM/kWM) x (kTN/kWN) block of 16 x 16
// MFMA tiles; K runs in steps of 64.
// The next step's A and B rows are copied from global memory straight into
// the other of two LDS stages (global_load_lds_dwordx4, no register staging)
// while the MFMAs run on the current step's stage; one barrier per step. An
// LDS row is 64 bf16 = 8 chunks of 16 bytes; chunk c of tile row r sits at
// position c ^ (r & 7), so the 16 rows of one fragment read spread over the
// banks, and each copy instruction fills 1 KB contiguously. At the cfg 4 QKV
// shape (46,990 x 1536 -> 2560, one box) the copies take the projection from
// 472 to 365 us against register staging; at the o_proj shape 261 -> 220 us.
// The weights are the MFMA's first operand, so a lane ends with four
// consecutive output columns of one row. When the output rows allow 16-byte
// stores, the bf16 tile is staged in the idle LDS stages and each store
// instruction writes whole row segments (the cfg 4 prefill 104.0 ->
// 103.0-103.3 ms, A/B on one box); otherwise each lane stores its four
// columns as one 8-byte word (or 2-byte stores for odd widths).
//
// Workgroups are dealt to the 8 XCDs round-robin in launch order; they are
// remapped so each XCD takes a contiguous range of row tiles with all their
// column tiles: a row tile's A rows are fetched into one L2 and reused there
// by every column tile.
//
// Reference: the packed QKV and output projections of litemoe/model.py:47-49
// and :60 (F.linear over the packed prefill rows), and the LM head :127.
#include <type_traits>

#include "internal.h"

namespace lm {
namespace {

constexpr int kBK = 64;
constexpr int kXcds = 8;
constexpr int kRowBytes = kBK * 2;  // 128

__device__ __forceinline__ int frag_offset(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ (row & 7)) << 4);
}

// The packed QKV projection's epilogue (lm_linear_rope_kv): each 64-column
// block is one head (q heads, then k, then v); q and k are rotated (neox,
// the three roundings of rope_kv_kernel) and written back rotated, k and v
// are stored into the KV cache layer under lm_kv_write's mask.
struct RopeKV {
  const int64_t *pos;      // [M] RoPE table row and cache position of each row
  const int64_t *slots;    // [M] cache row of each row, or NULL (the row index)
  const uint8_t *active;   // [M], or NULL: every row stores
  const bf16 *cos_sin;     // [table_len, 64]: cos | sin halves
  int64_t table_len;
  bf16 *kc, *vc;           // [cache_batch, kv_heads, capacity, 64]
  int64_t capacity, cache_batch;
  int q_heads, kv_heads;
};

__device__ __forceinline__ void rotate3(float x1, float x2, float c, float s, float &o1, float &o2) {
  o1 = round_bf16(round_bf16(x1 * c) - round_bf16(x2 * s));
  o2 = round_bf16(round_bf16(x2 * c) + round_bf16(x1 * s));
}

// kStore: 2 = whole rows in 16-byte words through LDS (N % 8 == 0, ldo % 8 == 0,
// out 16-byte aligned), 1 = 8-byte fragment words (N % 4 == 0, ldo % 4 == 0,
// out 8-byte aligned), 0 = 2-byte stores.
// kRope: the RopeKV epilogue (64-column wave blocks, kStore >= 1).
template <int kTM, int kTN, int kWM, int kWN, int kStore, bool kRope = false>
__global__ void __launch_bounds__(64 * kWM * kWN)
gemm_kernel(const bf16 *__restrict__ a, int64_t lda, const bf16 *__restrict__ w, int64_t ldw,
            bf16 *__restrict__ out, int64_t ldo, int M, int N, int K, int tiles_m, int tiles_n,
            int xcd_remap, RopeKV rk) {
  constexpr int kWaves = kWM * kWN;
  constexpr int kWaveRows = kTM / kWM, kWaveCols = kTN / kWN;
  constexpr int kRB = kWaveRows / 16, kCB = kWaveCols / 16;
  constexpr int kLA = kTM / (8 * kWaves), kLB = kTN / (8 * kWaves);  // 16-byte loads per lane
  static_assert(kLA * 8 * kWaves == kTM && kLB * 8 * kWaves == kTN, "tile rows per load round");
  constexpr int kABytes = kTM * kRowBytes, kStage = (kTM + kTN) * kRowBytes;
  __shared__ __align__(16) char s0[kStage];  // two LDS stages
  __shared__ __align__(16) char s1[kStage];
  __shared__ int64_t st_pos[kRope ? kTM : 1];  // kRope, kStore == 2: cache position per row
  __shared__ int st_slot[kRope ? kTM : 1];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lin = blockIdx.x;
  int tile_m = lin / tiles_n, tile_n = lin % tiles_n;
  if (xcd_remap) {  // grid = tiles_n * (tiles_m rounded up to a multiple of 8)
    const int per_xcd = (int)(gridDim.x / kXcds) / tiles_n;  // row tiles per XCD
    const int j = lin / kXcds;
    tile_m = (lin % kXcds) * per_xcd + j / tiles_n;
    tile_n = j % tiles_n;
  }
  if (tile_m >= tiles_m) return;
  const int m0 = tile_m * kTM, n0 = tile_n * kTN;

  // Copy instruction i of wave w fills LDS rows 8*(w*L+i) .. +7 of an
  // operand (1 KB; lane l at byte 16*l): row 8*(w*L+i) + l/8, position l%8,
  // holding chunk (l%8) ^ (l/8), which is frag_offset's swizzle. Rows past M
  // or N repeat the last row (finite values; their outputs are not stored).
  // Byte offsets from the k step's base fit 32 bits (the host checks that
  // every row start's element offset is below 2^31).
  const int chunk = (lane & 7) ^ (lane >> 3);
  uint32_t oa[kLA], ob[kLB];
#pragma unroll
  for (int i = 0; i < kLA; ++i) {
    const int r = min(m0 + 8 * (wave * kLA + i) + lane / 8, M - 1);
    oa[i] = ((uint32_t)r * (uint32_t)lda + chunk * 8) * 2;
  }
#pragma unroll
  for (int i = 0; i < kLB; ++i) {
    const int r = min(n0 + 8 * (wave * kLB + i) + lane / 8, N - 1);
    ob[i] = ((uint32_t)r * (uint32_t)ldw + chunk * 8) * 2;
  }
  const uint32_t uw = __builtin_amdgcn_readfirstlane(wave);
  // Step kt's A and B rows straight into an LDS stage (no register staging).
  auto issue = [&](int kt, const char *stage) {
    const bf16 *ak = a + kt * kBK, *wk = w + kt * kBK;
    const uint32_t la = lds_address(stage) + uw * kLA * 1024, lb = lds_address(stage) + kABytes + uw * kLB * 1024;
#pragma unroll
    for (int i = 0; i < kLA; ++i) lds_copy16(ak, oa[i], la + i * 1024);
#pragma unroll
    for (int i = 0; i < kLB; ++i) lds_copy16(wk, ob[i], lb + i * 1024);
  };

  const int wr = wave / kWN, wc = wave % kWN;
  const int fr = lane % 16, fk = lane / 16;
  f32x4 acc[kRB][kCB];
#pragma unroll
  for (int i = 0; i < kRB; ++i)
#pragma unroll
    for (int jj = 0; jj < kCB; ++jj) acc[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const char *as) {
    const char *bs = as + kABytes;
#pragma unroll
    for (int kk = 0; kk < kBK / 32; ++kk) {
      u32x4 bfr[kCB];
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
        bfr[cb] = *reinterpret_cast<const u32x4 *>(bs + frag_offset(wc * kWaveCols + cb * 16 + fr, kk * 4 + fk));
#pragma unroll
      for (int rb2 = 0; rb2 < kRB; ++rb2) {
        const u32x4 af = *reinterpret_cast<const u32x4 *>(
            as + frag_offset(wr * kWaveRows + rb2 * 16 + fr, kk * 4 + fk));
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) acc[rb2][cb] = mfma16x16x32(bfr[cb], af, acc[rb2][cb]);
      }
    }
  };

  // Step kt + 1 is copied into the other stage while step kt is computed.
  // Before a stage is read: this wave's copies have landed (vmcnt) and the
  // barrier has seen every wave's, and every wave has left the step that
  // last read the stage the next copy goes into.
  // kRope with staged stores: the positions of this lane's fragment rows and
  // the cache position of tile row threadIdx.x % kTM are requested before the
  // K loop (unconditional loads, rows clamped into [0, M)), so the epilogue
  // does not wait on them.
  constexpr bool kPre = kRope && kStore == 2;
  [[maybe_unused]] int64_t frag_pos[kPre ? kRB : 1];
  [[maybe_unused]] int64_t pre_pos = -1;
  [[maybe_unused]] int pre_slot = 0;
  if constexpr (kPre) {
#pragma unroll
    for (int rb2 = 0; rb2 < kRB; ++rb2) frag_pos[rb2] = rk.pos[min(m0 + wr * kWaveRows + rb2 * 16 + fr, M - 1)];
    const int row = m0 + (int)(threadIdx.x % kTM), rc = min(row, M - 1);
    const int64_t p = rk.pos[rc];
    const int64_t slot = rk.slots ? rk.slots[rc] : rc;
    const bool act = rk.active ? rk.active[rc] != 0 : true;
    if (row < M && rk.kc && act && p >= 0 && p < rk.capacity && slot >= 0 && slot < rk.cache_batch) {
      pre_pos = p;
      pre_slot = (int)slot;
    }
  }

  const int nk = K / kBK;
  issue(0, s0);
  for (int kt = 0; kt < nk; kt += 2) {
    lds_copy_wait();
    __syncthreads();
    if (kt + 1 < nk) issue(kt + 1, s1);
    __builtin_amdgcn_sched_barrier(0);
    compute(s0);
    if (kt + 1 < nk) {
      lds_copy_wait();
      __syncthreads();
      if (kt + 2 < nk) issue(kt + 2, s0);
      __builtin_amdgcn_sched_barrier(0);
      compute(s1);
    }
  }

  // Transposed C fragment: lane holds output row m0 + wr*kWaveRows + rb*16 +
  // lane%16 and its columns 4*(lane/16) .. +3 of each 16-column block.
  // kRope: channel 16*cb + 4*fk + i and its neox partner (+32) sit in the
  // same lane, blocks cb and cb + 2.
  static_assert(!kRope || (kWaveCols == 64 && kStore >= 1), "one head per wave column block");
  [[maybe_unused]] const int head = (n0 + wc * kWaveCols) / 64;  // kRope: uniform per wave
  [[maybe_unused]] const bool rot = head < rk.q_heads + rk.kv_heads;
  // Row block rb2's fragments for output row `row`: bf16-rounded and, for
  // kRope, q and k rotated (values of rows past M are never stored).
  auto values = [&](int rb2, int row, float (&v)[kCB][4]) {
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[cb][i] = kRope ? round_bf16(acc[rb2][cb][i]) : acc[rb2][cb][i];
    if constexpr (kRope) {
      if (!rot || row >= M) return;
      const int64_t p = rk.pos[row];
      if (p < 0 || p >= rk.table_len) return;
      const bf16 *cs = rk.cos_sin + p * 64;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const uint2 cw = *reinterpret_cast<const uint2 *>(cs + cb * 16 + 4 * fk);
        const uint2 sw = *reinterpret_cast<const uint2 *>(cs + 32 + cb * 16 + 4 * fk);
        const float c[4] = {lo_f32(cw.x), hi_f32(cw.x), lo_f32(cw.y), hi_f32(cw.y)};
        const float sn[4] = {lo_f32(sw.x), hi_f32(sw.x), lo_f32(sw.y), hi_f32(sw.y)};
#pragma unroll
        for (int i = 0; i < 4; ++i) rotate3(v[cb][i], v[cb + 2][i], c[i], sn[i], v[cb][i], v[cb + 2][i]);
      }
    }
  };

  if constexpr (kStore == 2) {
    // The bf16 tile is staged in the (now idle) LDS stages and written out
    // row by row in 16-byte words, so that a store instruction covers whole
    // 512- or 256-byte row segments instead of 32-byte pieces of 16 rows.
    // Staged row r's 16-byte chunk c sits at c ^ (r & kSw): the 16 rows of
    // one fragment store fall on different bank groups.
    constexpr int kOB = kTN * 2, kChunks = kOB / 16, kSw = (kChunks < 16 ? kChunks : 16) - 1;
    constexpr int kHalfRows = kStage / kOB;  // rows held by the first stage
    static_assert(kTM * kOB <= 2 * kStage, "output tile fits the LDS stages");
    auto staged = [&](int r) -> char * {
      if constexpr (kTM <= kHalfRows) return s0 + r * kOB;
      else return r < kHalfRows ? s0 + r * kOB : s1 + (r - kHalfRows) * kOB;
    };
    __syncthreads();  // every wave has finished reading the stages
    [[maybe_unused]] uint2 csw[kPre ? kRB : 1][4];
    if constexpr (kRope) {
      // Each row's cache position, or -1 where lm_kv_write's mask skips it.
      if (threadIdx.x < kTM) {
        st_pos[threadIdx.x] = pre_pos;
        st_slot[threadIdx.x] = pre_slot;
      }
      // cos | sin of every fragment row's channels, requested together (the
      // position clamped into the table; rows outside it are not rotated).
#pragma unroll
      for (int rb2 = 0; rb2 < kRB; ++rb2) {
        const bf16 *cs = rk.cos_sin + min(max(frag_pos[rb2], (int64_t)0), rk.table_len - 1) * 64 + 4 * fk;
#pragma unroll
        for (int i = 0; i < 4; ++i) csw[rb2][i] = *reinterpret_cast<const uint2 *>(cs + 16 * i);
      }
    }
#pragma unroll
    for (int rb2 = 0; rb2 < kRB; ++rb2) {
      const int rl = wr * kWaveRows + rb2 * 16 + fr;
      float v[kCB][4];
      if constexpr (kRope) {
        // The rotation's roundings skip the NaN canonicalization: every value
        // is canonicalized by the packing below.
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
          for (int i = 0; i < 4; ++i) v[cb][i] = round_bf16_nc(acc[rb2][cb][i]);
        // Rotated unconditionally and selected, so that no load or wait
        // moves under a branch.
        const int64_t p = frag_pos[rb2];
        const bool ok = rot && p >= 0 && p < rk.table_len;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const uint2 cw = csw[rb2][cb], sw = csw[rb2][cb + 2];
          const float c[4] = {lo_f32(cw.x), hi_f32(cw.x), lo_f32(cw.y), hi_f32(cw.y)};
          const float sn[4] = {lo_f32(sw.x), hi_f32(sw.x), lo_f32(sw.y), hi_f32(sw.y)};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x1 = v[cb][i], x2 = v[cb + 2][i];
            const float o1 = round_bf16_nc(round_bf16_nc(x1 * c[i]) - round_bf16_nc(x2 * sn[i]));
            const float o2 = round_bf16_nc(round_bf16_nc(x2 * c[i]) + round_bf16_nc(x1 * sn[i]));
            v[cb][i] = ok ? o1 : x1;
            v[cb + 2][i] = ok ? o2 : x2;
          }
        }
      } else {
        values(rb2, m0 + rl, v);
      }
      char *srow = staged(rl);
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const int byte = 2 * (wc * kWaveCols + cb * 16 + 4 * fk);
        *reinterpret_cast<uint2 *>(srow + (((byte >> 4) ^ (rl & kSw)) << 4) + (byte & 8)) =
            make_uint2(pack_bf16(v[cb][0], v[cb][1]), pack_bf16(v[cb][2], v[cb][3]));
      }
    }
    __syncthreads();
    static_assert((kTM * kChunks) % (64 * kWaves) == 0, "whole store rounds");
#pragma unroll
    for (int i = 0; i < kTM * kChunks / (64 * kWaves); ++i) {
      const int idx = i * 64 * kWaves + threadIdx.x;
      const int rl = idx / kChunks, c = idx % kChunks;
      const int row = m0 + rl, col = n0 + c * 8;
      if (row >= M || col >= N) continue;
      const u32x4 word = *reinterpret_cast<const u32x4 *>(staged(rl) + ((c ^ (rl & kSw)) << 4));
      *reinterpret_cast<u32x4 *>(out + (int64_t)row * ldo + col) = word;
      if constexpr (kRope) {
        const int h = col / 64 - rk.q_heads;  // k heads, then v heads
        const int64_t sp = st_pos[rl];
        if (h >= 0 && h < 2 * rk.kv_heads && sp >= 0) {
          const bool is_k = h < rk.kv_heads;
          const int kvh = is_k ? h : h - rk.kv_heads;
          bf16 *dst = (is_k ? rk.kc : rk.vc) + (((int64_t)st_slot[rl] * rk.kv_heads + kvh) * rk.capacity + sp) * 64;
          *reinterpret_cast<u32x4 *>(dst + col % 64) = word;
        }
      }
    }
    return;
  }
  if constexpr (kRope) {
    const bool is_k = rot && head >= rk.q_heads;
    const int kvh = rot ? head - rk.q_heads : head - rk.q_heads - rk.kv_heads;
    bf16 *cache = is_k ? rk.kc : rk.vc;
#pragma unroll
    for (int rb2 = 0; rb2 < kRB; ++rb2) {
      const int row = m0 + wr * kWaveRows + rb2 * 16 + fr;
      if (row >= M || head >= rk.q_heads + 2 * rk.kv_heads) continue;
      const int64_t p = rk.pos[row];
      const int64_t slot = rk.slots ? rk.slots[row] : row;
      const bool store = (is_k || !rot) && cache && (!rk.active || rk.active[row]) && p >= 0 &&
                         p < rk.capacity && slot >= 0 && slot < rk.cache_batch;
      float v[kCB][4];
      values(rb2, row, v);
      bf16 *o = out + (int64_t)row * ldo + n0 + wc * kWaveCols + 4 * fk;
      bf16 *dst = store ? cache + ((slot * rk.kv_heads + kvh) * rk.capacity + p) * 64 + 4 * fk : nullptr;
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const uint2 word = make_uint2(pack_bf16(v[cb][0], v[cb][1]), pack_bf16(v[cb][2], v[cb][3]));
        *reinterpret_cast<uint2 *>(o + cb * 16) = word;
        if (store) *reinterpret_cast<uint2 *>(dst + cb * 16) = word;
      }
    }
    return;
  }
#pragma unroll
  for (int rb2 = 0; rb2 < kRB; ++rb2) {
    const int row = m0 + wr * kWaveRows + rb2 * 16 + fr;
    if (row >= M) continue;
    bf16 *o = out + (int64_t)row * ldo;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
      const int col = n0 + wc * kWaveCols + cb * 16 + 4 * fk;
      const f32x4 v = acc[rb2][cb];
      if constexpr (kStore == 1) {
        if (col < N)
          *reinterpret_cast<uint2 *>(o + col) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < N) o[col + i] = (bf16)f32_to_bf16(v[i]);
      }
    }
  }
}

template <int TM, int TN, int WM, int WN>
int launch_gemm_cfg(const bf16 *a, int64_t lda, const bf16 *w, int64_t ldw, bf16 *out, int64_t ldo,
                    int64_t M, int64_t N, int64_t K, hipStream_t stream, const RopeKV *rope = nullptr) {
  const int64_t tiles_m = cdiv(M, TM), tiles_n = cdiv(N, TN);
  // With fewer row tiles than XCDs the remap would put every tile on a few
  // XCDs; the plain order spreads the column tiles instead.
  const bool remap = tiles_m >= kXcds;
  const int64_t blocks = (remap ? align_up(tiles_m, kXcds) : tiles_m) * tiles_n;
  const bool vec = N % 4 == 0 && ldo % 4 == 0 && ((uintptr_t)out & 7) == 0;
  const bool vec16 = N % 8 == 0 && ldo % 8 == 0 && ((uintptr_t)out & 15) == 0;
  const dim3 grid((unsigned)blocks);
  auto go = [&](auto store_c, auto rope_c) {
    gemm_kernel<TM, TN, WM, WN, decltype(store_c)::value, decltype(rope_c)::value>
        <<<grid, 64 * WM * WN, 0, stream>>>(a, lda, w, ldw, out, ldo, (int)M, (int)N, (int)K,
                                            (int)tiles_m, (int)tiles_n, (int)remap,
                                            rope ? *rope : RopeKV{});
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  if (rope) {
    if (!vec) return LM_EINVAL;
    if (vec16 && rope->table_len > 0) go(S2{}, std::true_type{});
    else go(S1{}, std::true_type{});
  } else if (vec16) {
    go(S2{}, std::false_type{});
  } else if (vec) {
    go(S1{}, std::false_type{});
  } else {
    go(S0{}, std::false_type{});
  }
  LM_CHECK_LAUNCH();
  return LM_OK;
}

// Prefill-sized row counts take 256 x 256 tiles on 16 waves of 64 x 64 (four
// waves per SIMD). On one box at the cfg 4 QKV shape (46,990 x 1536 x 2560):
// 443 us against 509 us for 8 waves of 64 x 128 (two per SIMD), 539-587 us
// for 128 x 256 / 256 x 128 on 16 waves; at the o_proj shape 280 against
// 326 us. Fewer rows keep 128 x 128 tiles, whose grid spreads over more CUs.
int launch_gemm_rope(const bf16 *a, int64_t lda, const bf16 *w, int64_t ldw, bf16 *out, int64_t ldo,
                     int64_t M, int64_t N, int64_t K, hipStream_t stream, const RopeKV *rope) {
  if (M >= 2048)
    return launch_gemm_cfg<256, 256, 4, 4>(a, lda, w, ldw, out, ldo, M, N, K, stream, rope);
  return launch_gemm_cfg<128, 128, 2, 2>(a, lda, w, ldw, out, ldo, M, N, K, stream, rope);
}

}  // namespace

bool gemm_shape_ok(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  const int64_t tiles = align_up(cdiv(M, 128), kXcds) * cdiv(N, 128);
  const int64_t lim = (int64_t)1 << 31;
  return M > 0 && N > 0 && K > 0 && K % kBK == 0 && (M - 1) * lda + K < lim &&
         (N - 1) * ldw + K < lim && tiles < lim;
}

int launch_gemm(const bf16 *a, int64_t lda, const bf16 *w, int64_t ldw, bf16 *out, int64_t ldo,
                int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  return launch_gemm_rope(a, lda, w, ldw, out, ldo, M, N, K, stream, nullptr);
}

}  // namespace lm

using namespace lm;

extern "C" int lm_linear_rope_kv(const void *a, int64_t lda, const void *weight, int64_t rows,
                                 int64_t q_heads, int64_t kv_heads, int64_t in_features, void *qkv,
                                 int64_t ldo, const int64_t *positions, const uint8_t *active,
                                 const int64_t *slots, const void *cos_sin, int64_t table_len,
                                 void *k_cache, void *v_cache, int64_t capacity,
                                 int64_t cache_batch, void *stream) {
  const int64_t n = (q_heads + 2 * kv_heads) * 64;
  LM_REQUIRE(rows >= 0 && q_heads > 0 && kv_heads > 0 && in_features > 0 && lda >= in_features &&
             lda % 8 == 0 && ldo >= n && ldo % 4 == 0 && capacity >= 0 && cache_batch >= 0 &&
             table_len >= 0);
  if (rows == 0) return LM_OK;
  if (!gemm_shape_ok(rows, n, in_features, lda, in_features)) return LM_EUNSUPPORTED;
  LM_REQUIRE(a && weight && qkv && positions && cos_sin);
  LM_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)weight & 15) == 0 && ((uintptr_t)qkv & 7) == 0 &&
             ((uintptr_t)cos_sin & 7) == 0);
  LM_REQUIRE((k_cache == nullptr) == (v_cache == nullptr));
  const RopeKV rope{positions, slots, active, (const bf16 *)cos_sin, table_len, (bf16 *)k_cache,
                    (bf16 *)v_cache, capacity, cache_batch, (int)q_heads, (int)kv_heads};
  return launch_gemm_rope((const bf16 *)a, lda, (const bf16 *)weight, in_features, (bf16 *)qkv, ldo, rows,
                          n, in_features, (hipStream_t)stream, &rope);
}

extern "C" int lm_linear(const void *a, int64_t lda, const void *weight, int64_t ldw, int64_t rows,
                         int64_t out_features, int64_t in_features, void *out, int64_t ldo,
                         void *stream) {
  LM_REQUIRE(rows >= 0 && out_features > 0 && in_features > 0 && lda >= in_features &&
             ldw >= in_features && ldo >= out_features && lda % 8 == 0 && ldw % 8 == 0);
  if (rows == 0) return LM_OK;
  if (!gemm_shape_ok(rows, out_features, in_features, lda, ldw)) return LM_EUNSUPPORTED;
  LM_REQUIRE(a && weight && out);
  LM_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)weight & 15) == 0 && ((uintptr_t)out & 1) == 0);
  return launch_gemm((const bf16 *)a, lda, (const bf16 *)weight, ldw, (bf16 *)out, ldo, rows,
                     out_features, in_features, (hipStream_t)stream);
}
