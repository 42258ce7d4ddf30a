/*
 * litemoe_amd — C ABI of the MI355X (gfx950) MoE decode/prefill hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, plain integer sizes and a HIP stream passed as
 *     `void *` (a hipStream_t; NULL is the legacy default stream);
 *   - launches its kernels on that stream and returns at once: no allocation,
 *     no host<->device copy and no synchronisation, so every call can be
 *     recorded into a HIP graph by stream capture;
 *   - returns LM_OK (0) or a nonzero status (see lm_status_string).
 * Scratch memory ("workspace") is supplied by the caller; its size comes from
 * the matching *_workspace_size query.
 *
 * Element types: "bf16" is IEEE bfloat16 stored as uint16, round-to-nearest-
 * even wherever a float result is stored. Matrices are row-major; strides are
 * in elements.
 *
 * Each declaration names the reference interface it replaces
 * (ZhuLinsen/LiteMoE, path:line).
 */
#ifndef LITEMOE_AMD_H
#define LITEMOE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LM_OK = 0,
  LM_EINVAL = 1,        /* invalid argument (null pointer, negative size, bad shape) */
  LM_EUNSUPPORTED = 2,  /* shape this build has no kernel for (e.g. head_dim != 64) */
  LM_ELAUNCH = 3,       /* the HIP runtime rejected a kernel launch */
  LM_EWORKSPACE = 4,    /* workspace smaller than the size query returned */
  LM_ETOOLARGE = 5      /* problem larger than lm_fused_experts_noalloc's static scratch */
};

/* Library version string and a message for a status code. */
const char *lm_version(void);
const char *lm_status_string(int status);

/* The device address of pinned host memory (hipHostMalloc'd, e.g. a torch
 * tensor with pin_memory=True) for a kernel to write into: the emit ring of
 * lm_greedy_epilogue. LM_EINVAL if the runtime does not know the pointer.
 * Host-side helper of the output ring that replaces the reference's
 * side-stream copies (litemoe/execution.py:25-41); it launches nothing. */
int lm_host_device_pointer(void *host, void **device);

/* ---------------------------------------------------------------- norms -- */

/* y[r,:] = bf16( bf16(x[r,:] * rsqrt(mean(x[r,:]^2) + eps)) * w ), fp32 math.
 * Replaces litemoe/norm.py:19-29 (`norm.rmsnorm` -> Triton `_rms`,
 * norm.py:7-16), which restates model.py:9-11. x, y: [rows, hidden] bf16,
 * contiguous; w: [hidden] bf16. y may not alias x. */
int lm_rmsnorm(const void *x, const void *weight, void *y, int64_t rows,
               int64_t hidden, float eps, void *stream);

/* Residual add fused with the next RMSNorm:
 *   x[r,:] <- bf16(x[r,:] + alpha * a[r,:]);  y[r,:] = rmsnorm(x[r,:]).
 * Replaces the pair litemoe/model.py:108-109 (and :122 + :106 of the next
 * layer): `x.add(a, alpha=residual_multiplier)` then `norm.rmsnorm`. a may be
 * NULL (then x is only normalised). x is updated in place. */
int lm_add_rmsnorm(void *x, const void *a, float alpha, const void *weight,
                   void *y, int64_t rows, int64_t hidden, float eps,
                   void *stream);

/* ------------------------------------------------------- rope + kv cache -- */

/* Masked KV store, one writer per (row, head, channel):
 *   if active[r] and 0 <= pos[r] < capacity and 0 <= slot[r] < cache_batch:
 *     kc[slot[r], h, pos[r], c] = k[r*ks0 + h*ks1 + c*ks3]   (same for v)
 * Replaces litemoe/kv_write.py:23-29 (Triton `_store`, kv_write.py:6-20;
 * target index kv_write.py:16). The cache layer is [cache_batch, heads,
 * capacity, head_dim] contiguous. elem_bytes is 2 (bf16) or 4 (fp32): the
 * store is a bit copy. positions and slots are int64; slots may be NULL
 * (identity: slot = row); active is bool (one byte per row). Rows whose
 * position or slot is out of range are skipped (the reference leaves them
 * undefined). */
int lm_kv_write(const void *k, int64_t ks0, int64_t ks1, int64_t ks3,
                const void *v, int64_t vs0, int64_t vs1, int64_t vs3,
                void *k_cache, void *v_cache, const int64_t *positions,
                const uint8_t *active, const int64_t *slots, int64_t rows,
                int64_t heads, int64_t head_dim, int64_t capacity,
                int64_t cache_batch, int64_t elem_bytes, void *stream);

/* Neox rotary embedding on q and k fused with the masked KV store.
 * For every row r (positions[r] indexes cos_sin, [table_len, head_dim] bf16
 * holding cat(cos[:, :D/2], sin[:, :D/2]) as built at litemoe/model.py:31-35):
 *   q[r,h,i]     <- bf16( bf16(x1*c) - bf16(x2*s) )
 *   q[r,h,i+D/2] <- bf16( bf16(x2*c) + bf16(x1*s) )
 * with x1 = q[r,h,i], x2 = q[r,h,i+D/2], c/s the bf16 table entries, i < D/2:
 * the three roundings of the reference's bf16 torch formula
 * `q*cos + rotate_half(q)*sin` (model.py:13-15,66-67; each product and the
 * sum rounded to bf16, products formed in fp32),
 * and the same rotation of k, which is stored into k_cache at
 * (slot[r], h, pos[r]) under the lm_kv_write mask, v stored unrotated.
 * write_k (nonzero) also writes rotated k back in place (prefill needs it).
 * Replaces vLLM `_custom_ops.rotary_embedding(positions, q, k, D, cos_sin,
 * is_neox=True)` at litemoe/model.py:58,63-64 followed by `cache.write`
 * (model.py:59,70 -> kv_write.py:23-29). q, k, v rows have a row stride and a
 * head stride (multiples of 8 elements, 16-byte aligned rows); channels are
 * contiguous. head_dim must be 64. With k_cache and
 * v_cache both NULL nothing is stored (v and active may then be NULL): the
 * call is vLLM's in-place rotary_embedding alone. */
int lm_rope_kv_write(void *q, int64_t qs0, int64_t qs1, void *k, int64_t ks0,
                     int64_t ks1, const void *v, int64_t vs0, int64_t vs1,
                     const void *cos_sin, int64_t table_len,
                     const int64_t *positions, const uint8_t *active,
                     const int64_t *slots, void *k_cache, void *v_cache,
                     int64_t rows, int64_t q_heads, int64_t kv_heads,
                     int64_t head_dim, int64_t capacity, int64_t cache_batch,
                     int write_k, void *stream);

/* ------------------------------------------------------------ attention -- */

/* Workspace for lm_flash_decode with the given split count. */
int lm_flash_decode_workspace_size(int64_t batch, int64_t q_heads,
                                   int64_t head_dim, int64_t num_splits,
                                   int64_t *bytes);

/* Split-K decode attention over each row's contiguous KV sequence:
 *   out[b,h,:] = softmax(scale * q[b,h,:] . K[b,h/G,j,:], j < used[b]) V
 * K/V layer caches are [batch, kv_heads, capacity, head_dim] bf16 (row b is
 * cache page b), G = q_heads / kv_heads. used[b] (int32) is clamped to
 * [0, max_len] and to capacity; a row with used 0 gives zeros. The key range
 * [0, max_len) is cut into num_splits chunks, combined by log-sum-exp.
 * Replaces litemoe/flash_decode.py:16-34 (`FlashDecode.__call__` ->
 * vLLM `flash_attn_varlen_func(..., seqused_k, block_table=arange(B),
 * num_splits=0)`, flash_decode.py:19-22; aten varlen FA, :30-34). q: row
 * stride qs0, head stride qs1, channels contiguous; out: [batch, q_heads,
 * head_dim] contiguous bf16. head_dim must be 64. */
int lm_flash_decode(const void *q, int64_t qs0, int64_t qs1,
                    const void *k_cache, const void *v_cache,
                    const int32_t *used, int64_t batch, int64_t q_heads,
                    int64_t kv_heads, int64_t capacity, int64_t head_dim,
                    float scale, int64_t max_len, int64_t num_splits, void *out,
                    void *workspace, int64_t workspace_bytes, void *stream);

/* Decode attention fused with the packed QKV projection's reduction, RoPE and
 * the KV-cache store, for one new token per row:
 *   qkv[b] = bf16(sum_s qkv_partials[s][b])   (slices s ascending; the bf16
 *            output of F.linear, partials from lm_linear_splitk)
 *   q, k   = rope(qkv[b] q|k heads, positions[b])       (lm_rope_kv_write)
 *   k_cache[b,h,p], v_cache[b,h,p] = k, v  if active[b] and 0 <= p < capacity
 *   out    = lm_flash_decode over keys j < used[b] of the updated cache
 * with p = positions[b]. Results are bitwise those of lm_rope_kv_write
 * followed by lm_flash_decode; the new key is taken from registers rather
 * than re-read. Fuses litemoe/model.py:47-71 after the projection (qkv split,
 * `_rope`, `cache.write` -> kv_write.py:12-20, and the decode attention of
 * flash_decode.py:16-22). qkv_partials: fp32 [qkv_splits][batch][(q_heads +
 * 2*kv_heads) * 64] (q heads, then k, then v); 1 <= qkv_splits <= 8;
 * cos_sin, table_len, positions, active as lm_rope_kv_write (active may be
 * NULL: every row writes). row_order (int32 [batch], may be NULL): a
 * permutation of the rows, the order in which their workgroups are
 * dispatched (lm_decode_prologue writes rows by descending used, so that a
 * ragged batch does not end on a tail of long rows); results do not depend
 * on it. Other arguments and the workspace as lm_flash_decode. */
int lm_flash_decode_qkv(const float *qkv_partials, int64_t qkv_splits,
                        const void *cos_sin, int64_t table_len,
                        const int64_t *positions, const uint8_t *active,
                        void *k_cache, void *v_cache, const int32_t *used,
                        const int32_t *row_order,
                        int64_t batch, int64_t q_heads, int64_t kv_heads,
                        int64_t capacity, int64_t head_dim, float scale,
                        int64_t max_len, int64_t num_splits, void *out,
                        void *workspace, int64_t workspace_bytes, void *stream);

/* lm_flash_decode_qkv with out written in the fragment order that
 * lm_linear_splitk_frag reads (the o_proj input, litemoe/model.py:73): the
 * [batch, q_heads*64] output padded to 16*mb rows, mb = the smallest of
 * 1, 2, 4, 8 with 16*mb >= batch; element (b, k) at
 *   ((k/32)*mb + b/16)*512 + ((k%32)/8)*128 + (b%16)*8 + k%8.
 * Padding rows are never written. batch <= 128 (else LM_EUNSUPPORTED); the
 * same values as lm_flash_decode_qkv. No counterpart in the reference: a
 * layout of this build's decode step. */
int lm_flash_decode_qkv_frag(const float *qkv_partials, int64_t qkv_splits,
                             const void *cos_sin, int64_t table_len,
                             const int64_t *positions, const uint8_t *active,
                             void *k_cache, void *v_cache, const int32_t *used,
                             const int32_t *row_order,
                             int64_t batch, int64_t q_heads, int64_t kv_heads,
                             int64_t capacity, int64_t head_dim, float scale,
                             int64_t max_len, int64_t num_splits, void *out_frag,
                             void *workspace, int64_t workspace_bytes,
                             void *stream);

/* Variable-length attention over a packed batch (one row per token):
 * sequence s owns tokens [cu[s], cu[s+1]); token i of it attends keys
 * [0, i] of the same sequence when causal, all of them otherwise.
 * Replaces litemoe/packed.py:12-16 (`PackedPrefill.attention` ->
 * `aten._flash_attention_forward(q, k, v, cu, cu, max, max, 0.0, causal=True,
 * False, scale)`). q: [tokens, q_heads, 64], k/v: [tokens, kv_heads, 64] with
 * row/head strides (multiples of 8 elements), channels contiguous; out:
 * [tokens, q_heads, 64] contiguous bf16; q, k, v and out 16-byte aligned
 * (LM_EINVAL otherwise); cu: int32 [num_seqs + 1]; max_len bounds every
 * sequence. O / l is O times the hardware reciprocal of l (within one fp32 ulp
 * of the division before the bf16 rounding). */
int lm_prefill_attention(const void *q, int64_t qs0, int64_t qs1,
                         const void *k, int64_t ks0, int64_t ks1,
                         const void *v, int64_t vs0, int64_t vs1,
                         const int32_t *cu_seqlens, int64_t num_seqs,
                         int64_t tokens, int64_t max_len, int64_t q_heads,
                         int64_t kv_heads, int64_t head_dim, float scale,
                         int causal, void *out, void *stream);

/* --------------------------------------------------------------- router -- */

/* Fused router: logits = bf16(x . Wr^T) (fp32 accumulation), then top-k with
 * ties to the lower expert id, then weights:
 *   renormalize != 0: softmax over the k selected logits (fp32);
 *   renormalize == 0: softmax over all E logits, taken at the k selected.
 * ids come out in descending logit order. logits_out (bf16 [tokens, experts])
 * may be NULL. Replaces the router GEMV `linear_rows(z, router.layer)`
 * (litemoe/model.py:110, ops.py:7-12) and vLLM `fused_topk(z, scores, k,
 * renormalize=True)` (model.py:111-113); on the CPU path `topk` + softmax
 * (model.py:115-116). x: [tokens, hidden] bf16, Wr: [experts, hidden] bf16,
 * hidden % 8 == 0, hidden <= 4096, experts <= 256, topk <= min(experts, 16).
 * Ties among the selected are ordered by id; the weights' denominator is
 * summed in selection order. The fp32 accumulation order of the logits
 * depends on the call size: below 1024 tokens a per-token GEMV; from 1024
 * tokens with hidden = 512*{1,2,3,4,6,8} and 16 < experts <= 64, MFMA tiles
 * of 16 tokens (the last tokens % 16 on the GEMV), so a logit can differ by
 * one bf16 ulp between the two, as between any two BLAS orders. The
 * selection is exact given the logits. `renormalize` is a set of flags:
 * bit 0 (1) softmax over the selection, else over every logit; bit 1 (2)
 * each token's selection written in ascending expert id (weights alongside)
 * instead of descending logit, the order lm_moe_routes_combine_packed sums
 * in. The same for every router entry point below. */
int lm_router(const void *x, const void *gate_weight, int64_t tokens,
              int64_t hidden, int64_t experts, int64_t topk, int renormalize,
              void *logits_out, float *topk_weights, int32_t *topk_ids,
              void *stream);

/* Selection alone, from given bf16 logits [tokens, experts]; same rules as
 * lm_router. Replaces vLLM `fused_topk` (litemoe/model.py:112-113) given
 * `scores`. */
int lm_topk_softmax(const void *logits, int64_t tokens, int64_t experts,
                    int64_t topk, int renormalize, float *topk_weights,
                    int32_t *topk_ids, void *stream);

/* Deterministic stable permutation of routes r = t*topk + j by local expert
 * id: key = ids[r] - first_expert when in [0, local_experts), else
 * local_experts (the ignored tail). Writes expert_offsets [local_experts + 1]
 * (exclusive prefix of the counts; entry local_experts = number of local
 * routes), sorted_routes [routes] (route ids in key order, ascending route id
 * within a key: argsort(key, stable=True)) and, if not NULL, inverse [routes]
 * (inverse[sorted_routes[p]] = p). Replaces the dispatch bookkeeping of
 * litemoe/ops.py:163-173 (`Grouped.__call__`: local ids, argsort, counts,
 * offsets) and ops.py:34-40 (`reference_experts`). local_experts <= 511. */
int lm_moe_align(const int32_t *ids, int64_t routes, int64_t first_expert,
                 int64_t local_experts, int32_t *expert_offsets,
                 int32_t *sorted_routes, int32_t *inverse, void *stream);

/* -------------------------------------------------------------- experts -- */

/* Workspace for lm_fused_experts. */
int lm_fused_experts_workspace_size(int64_t tokens, int64_t topk,
                                    int64_t hidden, int64_t inter,
                                    int64_t experts, int64_t *bytes);

/* SwiGLU mixture of experts with the weighted combine:
 *   out[t] = sum_j w[t,j] * W2[e] . (silu(W13[e,:I] . x[t]) * (W13[e,I:] . x[t])),
 *   e = ids[t,j].
 * Rounding follows the reference CPU path: gate/up rounded to bf16, silu
 * rounded, product rounded, each route's W2 output rounded, then the fp32
 * ordered combine of lm_moe_finish (routes of a token summed in ascending
 * (expert id, branch) order, each term bf16(bf16(y) * bf16(w))).
 * Replaces vLLM `fused_experts(x, w1, w2, topk_weights, topk_ids,
 * apply_router_weight_on_input=False, global_num_experts=E)` as called at
 * litemoe/ep.py:40-41 and vllm_moe.py:25-26. x: [tokens, hidden] bf16,
 * w13: [experts, 2*inter, hidden] bf16 (gate rows first, ops.py:45),
 * w2: [experts, hidden, inter] bf16, topk_weights fp32 [tokens, topk],
 * topk_ids int32 [tokens, topk], out: [tokens, hidden] bf16.
 * hidden % 128 == 0, inter % 128 == 0, hidden / 128 and inter / 128 in
 * {1, 2, 3, 4, 6, 8, 12, 16}. block_rows (0 = automatic) is the number of
 * routes one workgroup carries per weight tile (a multiple of 16). logical
 * (int64 [experts] or NULL for identity) only reorders the combine, as in
 * lm_moe_finish.
 * Expert ids are device data, so they are not validated at the call: a token
 * may list an expert more than once (each route is computed and combined,
 * as the reference's reference_experts does, litemoe/ops.py:34-55), and a
 * route whose id lies outside [0, experts) is skipped: it adds nothing to
 * out and its expert rows are never read (the reference CPU path raises on
 * such ids; vLLM leaves them undefined). */
int lm_fused_experts(const void *x, const void *w13, const void *w2,
                     const float *topk_weights, const int32_t *topk_ids,
                     const int64_t *logical, int64_t tokens, int64_t hidden,
                     int64_t inter, int64_t experts, int64_t topk,
                     int64_t block_rows, void *out, void *workspace,
                     int64_t workspace_bytes, void *stream);

/* lm_fused_experts with no workspace argument and no allocation of any kind
 * (no hipMalloc/hipFree, no allocating library call). No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Its
 * scratch is a static device array of 16 MiB per GPU, held from the
 * library's load until the process ends; a call whose workspace
 * (lm_fused_experts_workspace_size) exceeds it returns LM_ETOOLARGE (the
 * decode shapes fit: 64 tokens x top-8 at hidden 1536 needs about 2 MiB,
 * 256 tokens about 8 MiB). stream must belong to the current device.
 * Results are bitwise those of lm_fused_experts. All calls on one GPU share
 * that GPU's array: calls that overlap on one GPU (two streams, or two host
 * threads) race. */
int lm_fused_experts_noalloc(const void *x, const void *w13, const void *w2,
                             const float *topk_weights,
                             const int32_t *topk_ids, const int64_t *logical,
                             int64_t tokens, int64_t hidden, int64_t inter,
                             int64_t experts, int64_t topk, int64_t block_rows,
                             void *out, void *stream);

/* Stage entry points of lm_fused_experts, exposed for parity tests and
 * kernel timing. For a route r = t*topk + j of expert e:
 * gate_up: act[r, :] = bf16(silu(bf16(g)) * bf16(u)),
 *   g/u = W13[e] . x[r / topk]; act is [routes, inter] in route order.
 * down: y[r, :] = bf16(W2[e] . act[r, :]); y is [routes, hidden] in route
 *   order. Routes of the ignored tail are not touched.
 * With topk_ids given (routes <= 2048, routes / topk <= 256 tokens) each
 * expert's workgroups collect its routes themselves (any number of them,
 * so repeated ids within a token are computed) and
 * expert_offsets/sorted_routes may be NULL; otherwise the routes come from
 * lm_moe_align's offsets and permutation. Routes whose id lies outside
 * [0, experts) are not computed and their act/y rows are not written. */
int lm_moe_gate_up(const void *x, const void *w13,
                   const int32_t *expert_offsets, const int32_t *sorted_routes,
                   const int32_t *topk_ids, int64_t routes, int64_t topk,
                   int64_t hidden, int64_t inter, int64_t experts,
                   int64_t block_rows, void *act, void *stream);
int lm_moe_down(const void *act, const void *w2, const int32_t *expert_offsets,
                const int32_t *sorted_routes, const int32_t *topk_ids,
                int64_t routes, int64_t hidden, int64_t inter, int64_t experts,
                int64_t block_rows, void *y, void *stream);

/* Weighted combine of route outputs, fp32 ordered accumulation:
 *   out[t,:] = bf16( sum over j in ascending (logical[ids[t,j]]*K + j) of
 *                    bf16(bf16(y[row]) * bf16(scales[t,j])) ),
 * row = inverse(order)[t*K + j] when order is given (y in sorted order),
 * else t*K + j (y in route order). Routes whose expert id is outside
 * [rank*count, (rank+1)*count) are skipped and their rows never read.
 * Replaces litemoe/moe_finish.py:34-57 (`finish`, Triton `_finish`
 * moe_finish.py:7-31). y: [tokens*K, hidden] bf16; ids int32 [tokens, K];
 * order int64 [tokens*K] or NULL; scales fp32 [tokens, K]; logical int64
 * [experts] or NULL (identity); out [tokens, hidden] bf16; 1 <= K <= 8.
 * workspace: 4*tokens*K bytes when order is given, else may be NULL. */
int lm_moe_finish(const void *y, const int32_t *ids, const int64_t *order,
                  const float *scales, const int64_t *logical, void *out,
                  int64_t tokens, int64_t hidden, int64_t topk, int64_t rank,
                  int64_t count, void *workspace, int64_t workspace_bytes,
                  void *stream);

/* ------------------------------------------------- decode projections -- */

/* Split-K projection for decode-sized row counts:
 *   partials[s][m][n] = sum_{k in slice s} a[m][k] * weight[n][k]   (fp32)
 * over `splits` equal K slices. bf16(sum_s partials[s]) (slices ascending) is
 * F.linear(a, weight)'s bf16 output; lm_linear_splitk_reduce forms it, and
 * lm_flash_decode_qkv / lm_add_rmsnorm_router_splitk consume the partials
 * directly. Replaces the dense projections of litemoe/model.py:47-49 (packed
 * q|k|v) and :73 (o_proj), torch F.linear in the reference. a: bf16 [rows,
 * in_features], row stride lda (a multiple of 8); weight: bf16
 * [out_features, in_features] contiguous. Supported: 1 <= rows <= 128,
 * out_features % 32 == 0, in_features = splits * 128 * kw with kw in
 * {1, 2, 3, 4, 6, 8}; otherwise LM_EUNSUPPORTED. partials: fp32
 * [splits, rows, out_features]. */
int lm_linear_splitk(const void *a, int64_t lda, const void *weight,
                     int64_t rows, int64_t out_features, int64_t in_features,
                     int64_t splits, float *partials, void *stream);

/* lm_linear_splitk with a in the fragment order of lm_flash_decode_qkv_frag
 * (rows padded to 16*mb, padding rows read and their outputs dropped): each
 * A load then reads 1 KB contiguously instead of 16 rows x 64 bytes. Same
 * partials as lm_linear_splitk on the row-major a, same limits,
 * in_features % 32 == 0. No counterpart in the reference (the projections of
 * litemoe/model.py:47-49 and :73 on this build's decode-step layout). */
int lm_linear_splitk_frag(const void *a_frag, const void *weight, int64_t rows,
                          int64_t out_features, int64_t in_features,
                          int64_t splits, float *partials, void *stream);

/* lm_linear_splitk whose input is rmsnorm(x) with the norm formed on the
 * fly: a[m][k] = bf16(bf16(x[m][k] * r_m) * norm_weight[k]),
 * r_m = 1 / sqrt(S_m / in_features + eps), where S_m is summed from
 * sumsq[m][0 .. in_features/64) (lm_moe_routes_combine with a residual) in
 * lm_rmsnorm's reduction order, so a is bitwise lm_rmsnorm(x). Replaces the
 * next layer's input norm (litemoe/model.py:106) and its packed QKV
 * projection (:47-49) in one launch. x: [rows, in_features] bf16
 * contiguous; in_features a multiple of 512 up to 2048; otherwise the limits
 * of lm_linear_splitk. */
int lm_linear_splitk_rmsnorm(const void *x, const float *sumsq,
                             const void *norm_weight, float eps,
                             const void *weight, int64_t rows,
                             int64_t out_features, int64_t in_features,
                             int64_t splits, float *partials, void *stream);

/* out[m][n] = bf16(sum_s partials[s][m][n]), s ascending; out row stride ldo. */
int lm_linear_splitk_reduce(const float *partials, int64_t splits, int64_t rows,
                            int64_t out_features, void *out, int64_t ldo,
                            void *stream);

/* ------------------------------------------------- dense projections -- */

/* Dense projection for any row count:
 *   out[m][n] = bf16( sum_k a[m][k] * weight[n][k] )   (fp32 accumulation)
 * Each output is reduced by one workgroup over all of K in ascending 32-wide
 * k steps, so a row's result is the same bits whatever the row count, the
 * row's position or the launch (no split-K, no atomics). Replaces the
 * F.linear calls of the packed prefill and of decode batches above 128 rows:
 * litemoe/model.py:47-49 (packed q|k|v), :60 and :73 (o_proj), :127 (LM
 * head). a: bf16 [rows, in_features], row stride lda; weight: bf16
 * [out_features, in_features], row stride ldw; out: bf16 [rows,
 * out_features], row stride ldo. lda and ldw multiples of 8, a and weight
 * 16-byte aligned; in_features a multiple of 64 (else LM_EUNSUPPORTED). Any
 * out_features (the last column tile is masked). */
int lm_linear(const void *a, int64_t lda, const void *weight, int64_t ldw,
              int64_t rows, int64_t out_features, int64_t in_features,
              void *out, int64_t ldo, void *stream);

/* The packed QKV projection with RoPE and the KV-cache store in its epilogue:
 *   qkv = lm_linear(a, weight)       (weight [(q_heads + 2*kv_heads)*64, K])
 *   then lm_rope_kv_write on qkv's q|k|v heads with write_k = 1
 * in one launch: each output row's q and k heads are rotated in registers and
 * written to qkv rotated, k and v are stored into k_cache / v_cache at
 * (slots[r], h, positions[r]) under the lm_kv_write mask. qkv and the caches
 * are bitwise those of the two-call sequence. Replaces litemoe/model.py:47-49
 * (F.linear of the packed q|k|v weight), :58 or :63-64 (rotary_embedding)
 * and :59 / :70 (cache.write -> kv_write.py:23-29). Head dim 64. qkv: bf16
 * [rows, (q_heads + 2*kv_heads)*64], row stride ldo (a multiple of 4,
 * 8-byte aligned); active and slots may be NULL (every row stores; slot =
 * row); k_cache and v_cache both NULL store nothing. Otherwise as lm_linear
 * and lm_rope_kv_write. */
int lm_linear_rope_kv(const void *a, int64_t lda, const void *weight,
                      int64_t rows, int64_t q_heads, int64_t kv_heads,
                      int64_t in_features, void *qkv, int64_t ldo,
                      const int64_t *positions, const uint8_t *active,
                      const int64_t *slots, const void *cos_sin,
                      int64_t table_len, void *k_cache, void *v_cache,
                      int64_t capacity, int64_t cache_batch, void *stream);

/* ------------------------------------------------------ fused decode ops -- */

/* Residual add, RMSNorm and the router in one pass per token:
 *   x[t] <- bf16(x[t] + alpha * a[t]);  z[t] = rmsnorm(x[t]) (lm_rmsnorm);
 *   then lm_router on z[t] (logits_out may be NULL).
 * a may be NULL (x only normalised). Fuses litemoe/model.py:108-113: the
 * residual update, the post-attention norm, the router GEMV and vLLM
 * fused_topk. Same limits and logit accumulation orders as lm_router; x and
 * z are bitwise those of lm_add_rmsnorm at every size. */
int lm_add_rmsnorm_router(void *x, const void *a, float alpha,
                          const void *norm_weight, float eps, void *z,
                          const void *gate_weight, int64_t tokens,
                          int64_t hidden, int64_t experts, int64_t topk,
                          int renormalize, void *logits_out,
                          float *topk_weights, int32_t *topk_ids,
                          void *stream);

/* lm_add_rmsnorm_router with the residual branch given as split-K partials
 * (lm_linear_splitk of the attention output projection):
 *   a[t] = bf16(sum_s a_partials[s][t]) (s ascending), then as
 *   lm_add_rmsnorm_router. Bitwise equal to lm_linear_splitk_reduce followed
 * by lm_add_rmsnorm_router. Fuses the o_proj output of litemoe/model.py:73
 * into :108-113. a_partials: fp32 [a_splits][tokens][hidden], 1 <= a_splits
 * <= 4; hidden a multiple of 512 up to 2048 (else LM_EUNSUPPORTED). */
int lm_add_rmsnorm_router_splitk(void *x, const float *a_partials,
                                 int64_t a_splits, float alpha,
                                 const void *norm_weight, float eps, void *z,
                                 const void *gate_weight, int64_t tokens,
                                 int64_t hidden, int64_t experts, int64_t topk,
                                 int renormalize, void *logits_out,
                                 float *topk_weights, int32_t *topk_ids,
                                 void *stream);

/* Workspace for lm_moe_routes. */
int lm_moe_routes_workspace_size(int64_t tokens, int64_t topk, int64_t hidden,
                                 int64_t inter, int64_t experts,
                                 int64_t *bytes);

/* Per-route expert outputs, unweighted, in route order r = t*topk + j:
 *   y[r] = bf16(W2[e] . bf16(silu(bf16(W13[e,:I] x_t)) * bf16(W13[e,I:] x_t)))
 * (the first half of lm_fused_experts; combine with lm_moe_finish or
 * lm_moe_finish_add_rmsnorm). Decode-sized batches (tokens <= 256 and
 * tokens * topk <= 2048) take a
 * path where each expert's workgroups collect that expert's routes
 * themselves (no permutation pass); larger batches use lm_moe_align blocks.
 * Replaces the expert GEMMs inside vLLM fused_experts (litemoe/ep.py:40-41)
 * and the per-expert loop of litemoe/ops.py:43-47. Shapes as
 * lm_fused_experts; y: [tokens*topk, hidden] bf16. Repeated ids within a
 * token are computed on every path; the y rows of routes whose id lies
 * outside [0, experts) are not written. */
int lm_moe_routes(const void *x, const void *w13, const void *w2,
                  const int32_t *topk_ids, int64_t tokens, int64_t hidden,
                  int64_t inter, int64_t experts, int64_t topk,
                  int64_t block_rows, void *y, void *workspace,
                  int64_t workspace_bytes, void *stream);

/* Expert weights in MFMA fragment order, done once when the model is
 * loaded (two launches): for each matrix M [rows][K] (w13 as
 * [experts*2*inter][hidden], w2 as [experts*hidden][inter]), 16-byte chunk
 * (tile, k, lane) of the packed copy = M[16*tile + lane%16][32*k +
 * 8*(lane/16) .. +8], tiles of 16 rows, k-steps of 32. Every MFMA weight
 * fragment a kernel loads (16 rows x 32 k, one per lane) is then 1 KB
 * contiguous, and a decode workgroup's weight tile one contiguous run.
 * Same sizes as the inputs; hidden and inter as lm_fused_experts requires;
 * all four pointers 16-byte aligned; no aliasing. Replaces the reference's
 * load-time weight preparation (litemoe/weights.py:80-108, model.py:37-40),
 * which keeps the checkpoint layout for vLLM. */
int lm_expert_pack(const void *w13, const void *w2, int64_t experts,
                   int64_t hidden, int64_t inter, void *w13_packed,
                   void *w2_packed, void *stream);

/* lm_moe_gate_up, lm_moe_down, lm_moe_routes and lm_fused_experts on
 * weights packed by lm_expert_pack: the same arguments, kernels, arithmetic
 * order and results bit for bit. */
int lm_moe_gate_up_packed(const void *x, const void *w13,
                          const int32_t *expert_offsets,
                          const int32_t *sorted_routes,
                          const int32_t *topk_ids, int64_t routes,
                          int64_t topk, int64_t hidden, int64_t inter,
                          int64_t experts, int64_t block_rows, void *act,
                          void *stream);
int lm_moe_down_packed(const void *act, const void *w2,
                       const int32_t *expert_offsets,
                       const int32_t *sorted_routes, const int32_t *topk_ids,
                       int64_t routes, int64_t hidden, int64_t inter,
                       int64_t experts, int64_t block_rows, void *y,
                       void *stream);
int lm_moe_routes_packed(const void *x, const void *w13, const void *w2,
                         const int32_t *topk_ids, int64_t tokens,
                         int64_t hidden, int64_t inter, int64_t experts,
                         int64_t topk, int64_t block_rows, void *y,
                         void *workspace, int64_t workspace_bytes,
                         void *stream);

/* Workspace for lm_moe_routes_combine[_packed]. */
int lm_moe_routes_combine_workspace_size(int64_t tokens, int64_t topk,
                                         int64_t hidden, int64_t inter,
                                         int64_t experts, int64_t *bytes);

/* The decode MoE in two launches: the gate/up projection, then the down
 * projection with the weighted combine fused in (the last workgroup to finish
 * a 64-column tile sums that tile's route terms, counted with device-scope
 * atomics on counters in the workspace, which the call clears and leaves
 * clear). Each token's ids must be in ascending expert id (the router's id
 * order, `renormalize` bit 1): the sum then runs in the moe_finish order
 * (ascending id*K + branch) and equals lm_moe_routes + lm_moe_finish bit for
 * bit. Two forms:
 *   residual == NULL: out[t] = bf16(sum_j bf16(bf16(y_tj) * bf16(w_tj)));
 *   residual != NULL: residual[t] <- bf16(residual[t] + alpha * that bf16),
 *     and sumsq[t][c] (fp32 [tokens, hidden/64]) = the sum of squares of the
 *     new residual over columns 64c .. 64c+63, formed as lm_rmsnorm forms its
 *     partial sums, so lm_linear_splitk_rmsnorm can finish the next RMSNorm
 *     in the same order.
 * Replaces `ep(...)` -> vLLM fused_experts (litemoe/ep.py:40-41) and, with a
 * residual, also `x.add(y, alpha=residual_multiplier)` (model.py:122). Decode
 * scan path only (tokens <= 256, tokens*topk <= 2048, hidden a multiple of
 * 64, inter <= 1024, topk <= 8); otherwise LM_EUNSUPPORTED. The _packed form
 * reads lm_expert_pack weights. Calls that overlap on one workspace race. */
int lm_moe_routes_combine(const void *x, const void *w13, const void *w2,
                          const int32_t *topk_ids, const float *topk_weights,
                          int64_t tokens, int64_t hidden, int64_t inter,
                          int64_t experts, int64_t topk, void *residual,
                          float alpha, float *sumsq, void *out,
                          void *workspace, int64_t workspace_bytes,
                          void *stream);
int lm_moe_routes_combine_packed(const void *x, const void *w13,
                                 const void *w2, const int32_t *topk_ids,
                                 const float *topk_weights, int64_t tokens,
                                 int64_t hidden, int64_t inter,
                                 int64_t experts, int64_t topk,
                                 void *residual, float alpha, float *sumsq,
                                 void *out, void *workspace,
                                 int64_t workspace_bytes, void *stream);
int lm_fused_experts_packed(const void *x, const void *w13, const void *w2,
                            const float *topk_weights,
                            const int32_t *topk_ids, const int64_t *logical,
                            int64_t tokens, int64_t hidden, int64_t inter,
                            int64_t experts, int64_t topk, int64_t block_rows,
                            void *out, void *workspace,
                            int64_t workspace_bytes, void *stream);

/* The combine of lm_moe_finish (y in route order, all routes owned) fused
 * with the residual add and the next RMSNorm:
 *   m[t] = bf16(finish(y, ids, scales)[t]);  x[t] <- bf16(x[t] + alpha*m[t]);
 *   z[t] = rmsnorm(x[t], norm_weight).
 * Replaces moe_finish (litemoe/moe_finish.py:7-57) followed by
 * litemoe/model.py:122 and the next layer's :106 (or the final norm :126).
 * logical as lm_moe_finish (NULL = identity). Every route is owned: ids must
 * lie in [0, experts) (lm_router's ids always do). */
int lm_moe_finish_add_rmsnorm(const void *y, const int32_t *ids,
                              const float *scales, const int64_t *logical,
                              void *x, float alpha, const void *norm_weight,
                              float eps, void *z, int64_t tokens,
                              int64_t hidden, int64_t topk, void *stream);

/* -------------------------------------------------- greedy decode step ends -- */

/* The start of one decode step, per row b (one launch):
 *   valid[b] = active[b];  positions[b] = valid[b] ? length[b] : 0;
 *   used[b] = positions[b] + 1;
 *   x[b] = bf16(embedding[next[b]] * multiplier);  z[b] = rmsnorm(x[b]).
 * Replaces litemoe/engine.py:89-91 (valid, positions) with model.py:103
 * (used, lean decode), :104 (embedding) and :106 (first layer's norm,
 * lm_rmsnorm's rounding). active/valid are bool bytes; length/next int64;
 * next is clamped to [0, vocab). hidden a multiple of 8, at most 4096
 * (else LM_EUNSUPPORTED). row_order (int32 [rows], may be NULL): the rows
 * by descending used, equal used by ascending row (the stable argsort of
 * -used), for lm_flash_decode_qkv's dispatch order. No counterpart in the
 * reference, whose attention kernel schedules itself. step_counter (int64
 * [1] on the device, may be NULL) is incremented once per call: the step
 * count lm_greedy_epilogue's emit ring is indexed by. */
int lm_decode_prologue(const uint8_t *active, const int64_t *length,
                       const int64_t *next, const void *embedding,
                       float multiplier, const void *norm_weight, float eps,
                       void *x, void *z, uint8_t *valid, int64_t *positions,
                       int32_t *used, int32_t *row_order,
                       int64_t *step_counter, int64_t rows, int64_t hidden,
                       int64_t vocab, void *stream);

/* The end of one greedy decode step, per row b (one launch):
 *   candidate = argmax_v bf16(logits[b][v] * (1 / logits_scaling)), the
 *   first index of the maximum (torch.argmax; NaN counts as the maximum);
 *   emit[b] = (candidate, generated[b], valid[b]);
 *   length[b] += valid[b];  generated[b] += valid[b];
 *   if valid[b]: next[b] = candidate;
 *   done = generated[b] >= budget[b] || (!ignore_eos && candidate in eos);
 *   active[b] = valid[b] && !done.
 * Replaces litemoe/model.py:127 (/ logits_scaling) and engine.py:92-102.
 * logits: bf16 [rows][ld] raw head output; emit int64 [rows][3]; eos int64
 * [neos].
 * emit_ring (may be NULL): the device address (lm_host_device_pointer) of
 * int64 [ring_depth][rows][3] pinned host memory; each emit row is also
 * stored, with system-scope stores, into slot (*step_counter - 1) %
 * ring_depth, step_counter being the device counter lm_decode_prologue
 * increments. This folds the per-step device-to-host copy of the
 * reference's OutputRing (litemoe/execution.py:25-41) into the step.
 * workspace: lm_greedy_epilogue_workspace_size bytes (the argmax of each
 * row is split over slices of the row; two launches). rows <= 65535. */
int lm_greedy_epilogue_workspace_size(int64_t rows, int64_t vocab,
                                      int64_t *bytes);
int lm_greedy_epilogue(const void *logits, int64_t ld, float logits_scaling,
                       int64_t vocab, int64_t rows, const uint8_t *valid,
                       int64_t *next, int64_t *length, int64_t *generated,
                       const int64_t *budget, uint8_t *active, int64_t *emit,
                       const int64_t *eos, int64_t neos, int ignore_eos,
                       int64_t *emit_ring, int64_t ring_depth,
                       const int64_t *step_counter, void *workspace,
                       int64_t workspace_bytes, void *stream);

/* The LM head in MFMA fragment order, for lm_head_greedy (one launch;
 * done once when the model is loaded): 16-byte chunk (k, tile, lane) of
 * packed = head[16*tile + lane%16][32*k + 8*(lane/16) .. +8], k-steps of
 * 32 outermost, then tiles of 16 vocabulary rows; zero rows past the
 * vocabulary.
 * lm_head_pack_size: ceil(vocab/16)*16*hidden*2 bytes. head bf16
 * [vocab][hidden] contiguous; hidden a multiple of 32. No counterpart in the
 * reference, which multiplies by the checkpoint layout (model.py:127). */
int lm_head_pack_size(int64_t vocab, int64_t hidden, int64_t *bytes);
int lm_head_pack(const void *head, int64_t vocab, int64_t hidden, void *packed,
                 void *stream);

/* The LM head product and lm_greedy_epilogue fused (two launches):
 *   logits[b][v] = bf16(sum_k z[b][k] * head[v][k])   (F.linear's output)
 * then the candidate, emit row and state update exactly as
 * lm_greedy_epilogue computes them from those logits. The head weights are
 * streamed once, with the argmax of each vocabulary slice taken in the
 * product's epilogue; the logits are stored only if `logits` is not NULL
 * (bf16 [rows][ldo]). Replaces litemoe/model.py:127 (F.linear(z, head) /
 * logits_scaling) and engine.py:92-102. z: bf16 [rows][ldz], 16-byte
 * aligned, ldz a multiple of 8; head: the lm_head_pack layout of the bf16
 * [vocab][hidden] head, 16-byte aligned. rows <= 128 and hidden in {512, 1024, 1536, 2048}
 * (else LM_EUNSUPPORTED). The fp32 sum runs in the MFMA's order, so a
 * logit may differ from another BLAS's by one bf16 ulp; the candidate is
 * always the argmax of the logits this call computes. Ring arguments as
 * lm_greedy_epilogue; workspace: lm_head_greedy_workspace_size bytes. */
int lm_head_greedy_workspace_size(int64_t rows, int64_t vocab, int64_t hidden,
                                  int64_t *bytes);
int lm_head_greedy(const void *z, int64_t ldz, const void *head, int64_t rows,
                   int64_t vocab, int64_t hidden, float logits_scaling,
                   void *logits, int64_t ldo, const uint8_t *valid,
                   int64_t *next, int64_t *length, int64_t *generated,
                   const int64_t *budget, uint8_t *active, int64_t *emit,
                   const int64_t *eos, int64_t neos, int ignore_eos,
                   int64_t *emit_ring, int64_t ring_depth,
                   const int64_t *step_counter, void *workspace,
                   int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* LITEMOE_AMD_H */
