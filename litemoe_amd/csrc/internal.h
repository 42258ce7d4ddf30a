// Launchers shared between translation units of the library (not exported).
#pragma once

#include "common.h"

namespace lm {

// Expert weights [rows, K] (rows = experts * rows per expert) in one of two
// layouts: the checkpoint's row-major one, or the fragment order of
// lm_expert_pack, where 16-byte chunk (tile, k-step, lane) holds
// M[16*tile + lane%16][32*k-step + 8*(lane/16) .. +8], so a wave's MFMA B
// fragment of 16 rows x 32 k is 1 KB contiguous. wofs: element offset of
// the eight values at (row, k), k a multiple of 8.
template <bool kPacked>
__device__ __forceinline__ int64_t wofs(int64_t row, int k, int K) {
  if constexpr (!kPacked) {
    return row * K + k;
  } else {
    return (((row >> 4) * (K >> 5) + (k >> 5)) * 64 + ((k >> 3) & 3) * 16 + (row & 15)) * 8;
  }
}
// Element advance of one 32-wide k-step at a fixed (row, k % 32).
template <bool kPacked>
constexpr int64_t wstep() { return kPacked ? 64 * 8 : 32; }

// moe_finish.hip: combine of route outputs (see lm_moe_finish).
// inverse: sorted position of each route, or nullptr when y is in route order.
int launch_finish(const bf16 *y, const int32_t *ids, const int32_t *inverse, const float *scales,
                  const int64_t *logical, bf16 *out, int64_t tokens, int64_t hidden, int64_t topk,
                  int64_t rank, int64_t count, hipStream_t stream);

// moe_gemm.hip. With ids != nullptr a launch takes the scan path (grid.y =
// expert, routes collected from ids); otherwise offsets/sorted blocks.
// packed: weights in the lm_expert_pack layout.
int launch_gate_up(const bf16 *x, const bf16 *w13, const int32_t *offsets, const int32_t *sorted,
                   const int32_t *ids, int64_t routes, int64_t topk, int64_t hidden, int64_t inter,
                   int64_t experts, int64_t block_rows, bf16 *act, bool packed, hipStream_t stream);
int launch_down(const bf16 *act, const bf16 *w2, const int32_t *offsets, const int32_t *sorted,
                const int32_t *ids, int64_t routes, int64_t hidden, int64_t inter, int64_t experts,
                int64_t block_rows, bf16 *y, bool packed, hipStream_t stream);
bool expert_shapes_ok(int64_t hidden, int64_t inter);
bool scan_path(int64_t tokens, int64_t topk);

// Rows of one weight-tile block; 0 picks min(align16(tokens), 256).
int pick_block_rows(int64_t block_rows, int64_t tokens);

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// router.hip: the stable argsort of lm_moe_align. Above kAlignChunkedMinRoutes
// routes it runs over 1024-route chunks in three launches, given a scratch
// of align_scratch_bytes (else one workgroup).
constexpr int64_t kAlignChunkedMinRoutes = 8192;
int64_t align_scratch_bytes(int64_t routes, int64_t local_experts);
int launch_align(const int32_t *ids, int64_t routes, int64_t first_expert, int64_t local_experts,
                 int32_t *offsets, int32_t *sorted, int32_t *inverse, int32_t *scratch,
                 int64_t scratch_bytes, hipStream_t stream);

// expert_gemm.hip: LDS-tiled MFMA GEMMs over lm_moe_align's 128-route
// blocks, for prefill-sized route counts (act and y in route order).
constexpr int64_t kExpertGemmMinRoutes = 4096;
bool expert_gemm_ok(int64_t routes, int64_t hidden, int64_t inter, int64_t experts);
int launch_expert_gemm_gate_up(const bf16 *x, const bf16 *w13, const int32_t *offsets,
                               const int32_t *sorted, int64_t routes, int64_t topk, int64_t hidden,
                               int64_t inter, int64_t experts, bf16 *act, bool packed,
                               bool sorted_act, hipStream_t stream);
// sorted_act: act rows in expert-sorted route order (gate_up writes row p for
// sorted position p, down reads it there) instead of route order.
int launch_expert_gemm_down(const bf16 *act, const bf16 *w2, const int32_t *offsets,
                            const int32_t *sorted, int64_t routes, int64_t hidden, int64_t inter,
                            int64_t experts, bf16 *y, bool packed, bool sorted_act,
                            hipStream_t stream);

}  // namespace lm

namespace lm {

// gemm.hip: dense out = bf16(a . w^T), one workgroup per 128 x 128 output tile
// reducing all of K in ascending order.
bool gemm_shape_ok(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw);
int launch_gemm(const bf16 *a, int64_t lda, const bf16 *w, int64_t ldw, bf16 *out, int64_t ldo,
                int64_t M, int64_t N, int64_t K, hipStream_t stream);

}  // namespace lm
