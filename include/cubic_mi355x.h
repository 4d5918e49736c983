/*
 * cubic_mi355x.h -- C ABI of the MI355X (gfx950) MTP verify-step library.
 *
 * Plain pointers and sizes only.  Every pointer argument named *device* data
 * is a device address on the current HIP device; `stream` is a hipStream_t
 * (NULL = the default stream).  Every entry point returns 0 on success or a
 * negative CUBIC_E* code; cubic_last_error() then describes the failure.
 * Nothing here allocates device memory except cubic_* functions documented as
 * doing so (none do): callers own weights, outputs and workspaces.
 *
 * Reference paths are relative to src/cubic_serve/ of QuantTrio/cubic-serve.
 */
#ifndef CUBIC_MI355X_H
#define CUBIC_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define CUBIC_API __attribute__((visibility("default")))
#else
#define CUBIC_API
#endif

#define CUBIC_OK 0
#define CUBIC_EINVAL (-1)      /* argument outside the admitted ABI (shape, dtype, size) */
#define CUBIC_ENOTSUP (-2)     /* geometry not admitted by this kernel family */
#define CUBIC_EHIP (-3)        /* HIP runtime / launch failure */
#define CUBIC_EWORKSPACE (-4)  /* workspace smaller than the planned size */

/* Metadata formats (quantization/extensions/cubic/checkpoint.py:38-46). */
#define CUBIC_FMT_F32_SCALE_F16_AB 0  /* "float32-scale-float16-ab" */
#define CUBIC_FMT_I8_SCALE_I4_AB 1    /* "int8-scale-int4-ab-global-fp32" */
#define CUBIC_FMT_E5M9_CURVE2 2       /* "e5m9-scale-curve2-tensor-fp16" */

/* ABI revision, raised whenever an entry point's arguments change: 2 added
 * the GEMM dtype, 3 the candidate dtype, 4 the device live/owned counts of
 * cubic_accept(_noalloc) and cubic_candidates, 5 the candidate vocab_start,
 * 6 the grammar-masked logits output of the greedy launches.
 * This header describes revision 6. */
CUBIC_API int cubic_abi_version(void);
CUBIC_API const char* cubic_last_error(void);

/* 16-bit floating-point element types of activations, outputs and prepared
 * level tables (the reference admits FP16 or BF16 activations with the output
 * in the same dtype: ops/cuda/linear/quantized.py:348-405). */
#define CUBIC_DTYPE_BF16 0
#define CUBIC_DTYPE_F16 1
#define CUBIC_DTYPE_F32 2  /* candidate preparation logits only */

/* ---------------------------------------------------------------------------
 * Cubic weight preparation (load time).
 * Replaces the format-prepared derivatives of quantization/extensions/cubic/
 * marlin.py:38-81 (_prepare: repack_signed_codes + prepare_metadata) and
 * marlin_metadata.py:35-100.
 *
 * cubic_prepared_words: sizes (in uint32 words) of the prepared code stream
 * and metadata for an [n, k] matrix.
 * cubic_prepare_weight: device payload -> prepared (codes, meta).
 *   packed        uint8 [n, ceil(k*bits/8)]    weight_packed
 *   fmt 0: m0 = weight_scale f32, m1 = weight_a f16, m2 = weight_b f16   [n/go, ceil(k/gi)]
 *   fmt 1: m0 = weight_scale i8, m1 = weight_ab u8; g0..g2 = *_global f32 [partitions]
 *   fmt 2: m0 = weight_metadata u16; m1 = weight_curve_a f16, m2 = weight_curve_b f16 [partitions, 4]
 *   part_of_row   int32 [n] partition index of each output row (fmt 1, 2; may be NULL for fmt 0)
 *   dtype         CUBIC_DTYPE_BF16 / _F16: the activation dtype the prepared weight
 *                 serves (bits <= 4 store per-group level tables rounded to it;
 *                 the code stream is the same for both)
 *   expanded      device scratch of cubic_prepare_scratch_bytes() bytes
 * Admission (quantization/extensions/cubic/marlin.py:256-336 analogue):
 *   1 <= bits <= 8, group_in % 32 == 0, k % 8 == 0, group_out divides n.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_prepared_words(int64_t n, int64_t k, int bits, int group_in, int64_t* code_words,
                         int64_t* meta_words);
CUBIC_API int64_t cubic_prepare_scratch_bytes(int64_t n, int64_t k, int group_in);
CUBIC_API int cubic_prepare_weight(int fmt, const void* packed, const void* m0, const void* m1,
                         const void* m2, const void* g0, const void* g1, const void* g2,
                         const int32_t* part_of_row, int64_t n, int64_t k, int bits,
                         int group_in, int group_out, int dtype, void* expanded,
                         int64_t expanded_bytes, uint32_t* codes, uint32_t* meta, void* stream);

/* ---------------------------------------------------------------------------
 * Cubic WNA16 GEMM: y = x . decode(W)^T, bf16 or fp16 in/out (dtype; the
 * prepared weight must have been prepared for the same dtype), weights
 * rounded once to that dtype, FP32 accumulation.
 * Replaces the Marlin launch plus _merge_dense_partials of
 * quantization/extensions/cubic/marlin.py:377-521 (bind_planned_linear :339)
 * and the small-row kernel of quantization/common/small_rows.cu:94-241.
 *
 * K plan: the K partition of every output column is a function of its
 * member's (n, k) and bits only -- never of m, nor of how many members share a launch
 * (quantization/extensions/cubic/marlin.py:347-360, common/marlin/cost.py:
 * 59-79) -- so a row's result is bitwise the same for every m of one
 * arithmetic regime and grouped members equal separate launches bit for bit.
 * The regimes, as the reference's: m <= 4 with groups of whole 128-wide
 * k-blocks runs the small-row kernel (bits <= 4 at any k; 5..8 bits while k
 * is at most 64 k-blocks), one partition per wave, a function of k alone;
 * every other m runs the MFMA-tile arithmetic with the K plan above (m <= 64
 * at bits <= 4 on column panels that share each staged activation block over
 * several tiles, the rest one tile per wave; both issue the same MFMA
 * sequence and agree bit for bit).
 *
 * cubic_gemm_workspace_bytes: workspace for (m, n, k); 0 when no K split.
 *   The workspace must be zero-filled before its first use; every completed
 *   launch leaves it zero again (a launch killed mid-kernel can leave an
 *   arrival counter set: zero the workspace again before reusing it).  One
 *   workspace per concurrently running launch.
 * cubic_gemm: single output y[m, ldy] (columns n).
 * cubic_gemm_group: `members` (1..8) matrices of the same [n, k] shape and
 *   encoding sharing x, prepared as one [members * n, k] matrix (member i's
 *   prepared codes/metadata follow member i-1's); member i's columns go to
 *   ys[i] (row stride ldys[i]); n % 16 == 0 when members > 1.  ys and ldys
 *   are host arrays.  Replaces bind_planned_grouped (cubic/marlin.py:
 *   347-360) behind bind_linear_group (ops/cuda/linear/quantized.py:445-507).
 *   Workspace: cubic_gemm_group_workspace_bytes(m, members, n, k, bits).
 * cubic_gemm_grouped: two members (gate/up), prepared as one [n0 + n1, k]
 *   matrix; columns < n0 go to y0, the rest to y1; n0 % 16 == 0.  Equal
 *   widths run as one cubic_gemm_group launch; unequal widths run as two
 *   launches (each member keeps its own K plan).  Workspace:
 *   cubic_gemm_grouped_workspace_bytes(m, n0, n1, k, bits).
 * x: dtype [m, ldx], 16-byte aligned, ldx % 8 == 0; outputs dtype.
 * ------------------------------------------------------------------------- */
CUBIC_API int64_t cubic_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int bits);
CUBIC_API int64_t cubic_gemm_group_workspace_bytes(int64_t m, int members, int64_t n, int64_t k,
                                                   int bits);
CUBIC_API int64_t cubic_gemm_grouped_workspace_bytes(int64_t m, int64_t n0, int64_t n1, int64_t k,
                                                     int bits);
CUBIC_API int cubic_gemm(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
               int64_t m, int64_t n, int64_t k, int bits, int group_in, int dtype, void* y, int64_t ldy,
               void* workspace, int64_t workspace_bytes, void* stream);
CUBIC_API int cubic_gemm_group(const void* x, int64_t ldx, const uint32_t* codes,
                               const uint32_t* meta, int64_t m, int members, int64_t n, int64_t k,
                               int bits, int group_in, int dtype, void* const* ys, const int64_t* ldys,
                               void* workspace, int64_t workspace_bytes, void* stream);
CUBIC_API int cubic_gemm_grouped(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
                       int64_t m, int64_t n0, int64_t n1, int64_t k, int bits, int group_in, int dtype,
                       void* y0, int64_t ldy0, void* y1, int64_t ldy1, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Routed experts (MoE).  Replaces the Cubic Marlin MoE bind
 * (quantization/extensions/cubic/marlin.py:84-253: bind_grouped, bind_routed)
 * with its route padding (quantization/common/marlin/repack.py:253-277,
 * _pad_routes) over RoutedRows (quantization/api.py:123-134).
 *
 * cubic_moe_pad_routes: expert e's compact routes row_map[starts[e] ..
 *   starts[e] + counts[e]) fill padded slots (block_starts[e] + b) * block_m
 *   + i; slots past counts[e] hold `routes` (padding); block_expert[block] =
 *   e; *padded_total = *total_blocks * block_m.  All int32, device.
 *   block_starts are in units of block_m.
 * cubic_moe_max_blocks: capacity of the padded tables, in blocks, for
 *   `routes` routes over `experts` experts (routes + active experts x
 *   (block_m - 1), rounded up).
 * cubic_moe_gemm: y[route, :] = x[route / top_k, :] . decode(W[e])^T for every
 *   route of every padded block of expert e (padding slots write nothing).
 *   Expert e's prepared codes / metadata start at e * expert_code_words /
 *   e * expert_meta_words.  Gate and up of one expert are prepared as one
 *   [n_gate + n_up, k] matrix (columns gate first), as the reference groups
 *   them.  block_m in {16, 32, 64}; top_k = 1 for the down projection.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_moe_pad_routes(const int32_t* counts, const int32_t* starts,
                                   const int32_t* block_starts, const int32_t* total_blocks,
                                   const int32_t* row_map, int experts, int routes, int block_m,
                                   int32_t* padded, int32_t* block_expert, int32_t* padded_total,
                                   void* stream);
CUBIC_API int64_t cubic_moe_max_blocks(int64_t routes, int experts, int block_m);
CUBIC_API int cubic_moe_gemm(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
                             int64_t expert_code_words, int64_t expert_meta_words,
                             const int32_t* padded, const int32_t* block_expert,
                             const int32_t* padded_total, int64_t max_blocks, int block_m,
                             int routes, int top_k, int64_t n, int64_t k, int bits, int group_in,
                             int dtype, void* y, int64_t ldy, void* stream);

/* ---------------------------------------------------------------------------
 * Root top-k/top-p sampling of gathered [tp, rows, k] candidates (non-
 * speculative decode).  Replaces RootTopKTopPSamplingPrimitive.launch and
 * _root_topk_topp_kernel (ops/cuda/sampling/topk_topp.py:22-121, :141-278):
 *   scores       bf16 (scores_fp16 = 0) or fp16 [tp, rows, k]; ids int64
 *   temperatures/top_ps f32 [rows]; top_ks/seeds/ordinals int64 [rows]
 *   constrained_rows bool [rows] or NULL (needs allow_underfilled)
 *   output_tokens int64 [rows] (-1 when invalid), output_valid bool [rows]
 * Global top-k (duplicate (score, id) pairs count once, ties by ascending
 * id), temperature, softmax, top-p over the exclusive CDF, then the first
 * candidate whose retained CDF exceeds u * retained mass, u = Philox4x32-10
 * with key seed ^ (seed >> 32) ^ (ordinal >> 32) (both words) and counter
 * (uint32) ordinal.  Greedy rows (temperature 0) take the top candidate.
 * 1 <= tp <= 8, 1 <= k <= 20.  Reduction orders and exp as cubic_verify_candidates.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_root_sample(const void* scores, int scores_fp16, const int64_t* ids,
                                const float* temperatures, const float* top_ps,
                                const int64_t* top_ks, const int64_t* seeds,
                                const int64_t* ordinals, const uint8_t* constrained_rows,
                                int allow_underfilled, int tp, int rows, int k,
                                int64_t* output_tokens, uint8_t* output_valid, void* stream);

/* ---------------------------------------------------------------------------
 * Greedy sampling for non-speculative decode (CapturedGreedySampler,
 * ops/cuda/sampling/greedy.py:41-420).  metadata is the sampler's device
 * int32 [2] = (active rows, cancel flag), read when the launch runs.
 *
 * cubic_greedy_candidates replaces greedy_partial + greedy_merge
 * (greedy.cu:14-78, bound at greedy.py:255-283): per row r < active, the
 * exact argmax of logits[r, :width] (first maximum, i.e. lowest column, on
 * ties; -0 == +0) among the columns the grammar mask admits, published as
 * (score, vocab_start + column) in slot 0 and (NaN, -1) in the other slots.
 * A row holding any non-finite visible logit (admitted or not) publishes
 * (NaN, -2) in slot 0; a row the mask empties, rows >= active and width 0
 * publish (NaN, -1).  Rows >= active read no logits.
 *   logits       bf16 (logits_fp16 = 0) or fp16 [rows, row_stride]
 *   token_mask   int32 bit words [rows, mask_words] (bit t%32 of word t/32
 *                admits token t) or NULL; needs vocab_start + width <= 32 * mask_words
 *   masked_logits  logits dtype [rows, masked_stride] or NULL (token_mask
 *                required): the grammar-masked logits the reference's candidate
 *                preparation writes for its terminal consumer
 *                (local_candidates.cu:37-53): row r < active, column j < width
 *                gets logits[r, j] if the mask admits token vocab_start + j, else
 *                -inf; rows >= active get -inf.  masked_logits == logits with
 *                masked_stride == row_stride masks in place (consume_logits) and
 *                leaves rows >= active as they are.
 *   scores/ids   logits dtype / int64 [rows, candidates], 1 <= candidates <= 64
 *   1 <= rows <= 65535, 0 <= width <= 2^30
 *   workspace    cubic_greedy_workspace_bytes(rows, width) bytes, zero-filled
 *                once before first use; each launch returns its arrival
 *                counters to zero; one workspace serves launches of the same
 *                rows at any width up to the one it was sized for (launches
 *                sharing a workspace must not overlap)
 *
 * cubic_greedy_root replaces greedy_root (greedy.cu:91-114): over gathered
 * [tp, rows, k] candidates, a row r < active takes the best real candidate
 * (finite score, 0 <= id < vocab_size; highest score, lowest id on ties) when
 * every candidate is real or (NaN, -1) padding, at least one is real,
 * temperature == 0, top_p in (0, 1], 1 <= top_k <= k, seed >= 0 and
 * ordinal >= 0; tokens[r] = that id and valid[r] = 1, else -1 and 0.  Rows
 * >= active publish -1 (-2 at row == active when cancelled), valid 0.
 *   1 <= tp <= 8, 1 <= k <= 64, 1 <= vocab_size <= 2^31 - 1.
 *
 * cubic_sampling_final_guard replaces sampling_final_guard (greedy.cu:117-
 * 139): valid[0] = 0 < active <= capacity and, for every row i < capacity:
 * i < active: 0 <= tokens[i] < vocab_size, root_valid[i] (skipped when
 * root_valid is NULL, the reference's non-root ranks), temperature finite in
 * [0, 2], top_p finite in (0, 1], 1 <= top_k <= k, seed >= 0, ordinal >= 0;
 * i == active: tokens[i] in {-1, -2}; i > active: tokens[i] == -1.
 *
 * cubic_greedy_sample is the single-GPU composition of the three (TP = 1,
 * vocab_start = 0, candidates = k; the reference's all-gather and broadcast
 * are identities there) in one launch: the same candidate publication, root
 * tokens/root_valid and final validity.  width <= vocab_size.
 * ------------------------------------------------------------------------- */
CUBIC_API int64_t cubic_greedy_workspace_bytes(int rows, int width);
CUBIC_API int cubic_greedy_candidates(const void* logits, int logits_fp16, int64_t row_stride,
                                      int rows, int width, int64_t vocab_start,
                                      const int32_t* metadata, const uint32_t* token_mask,
                                      int64_t mask_words, void* masked_logits,
                                      int64_t masked_stride, int candidates, void* scores,
                                      int64_t* ids, void* workspace, int64_t workspace_bytes,
                                      void* stream);
CUBIC_API int cubic_greedy_root(const void* scores, int scores_fp16, const int64_t* ids,
                                const float* temperatures, const float* top_ps,
                                const int64_t* top_ks, const int64_t* seeds,
                                const int64_t* ordinals, const int32_t* metadata, int tp, int rows,
                                int k, int64_t vocab_size, int64_t* tokens, uint8_t* valid,
                                void* stream);
CUBIC_API int cubic_sampling_final_guard(const int64_t* tokens, const uint8_t* root_valid,
                                         const int32_t* metadata, const float* temperatures,
                                         const float* top_ps, const int64_t* top_ks,
                                         const int64_t* seeds, const int64_t* ordinals,
                                         int capacity, int k, int64_t vocab_size, uint8_t* valid,
                                         void* stream);
CUBIC_API int cubic_greedy_sample(const void* logits, int logits_fp16, int64_t row_stride, int rows,
                                  int width, const int32_t* metadata, const uint32_t* token_mask,
                                  int64_t mask_words, void* masked_logits, int64_t masked_stride,
                                  int k, const float* temperatures,
                                  const float* top_ps, const int64_t* top_ks, const int64_t* seeds,
                                  const int64_t* ordinals, int64_t vocab_size, void* scores,
                                  int64_t* ids, int64_t* tokens, uint8_t* root_valid,
                                  uint8_t* final_valid, void* workspace, int64_t workspace_bytes,
                                  void* stream);

/* ---------------------------------------------------------------------------
 * Packed embedding lookup: out[t, :] = decode(W[ids[t], :]) rounded to the
 * output dtype.  Replaces PackedLinearOperators.bind_embedding for Cubic
 * matrices (ops/cuda/linear/quantized.py:786-846) and the Cubic hook
 * bind_embedding (quantization/extensions/cubic/linear.py:266-294, kernel
 * quantization/common/kernels.py:138-164 with load_weight,
 * quantization/extensions/cubic/kernels.py:44-113).  Reads the checkpoint
 * payload as stored (no preparation):
 *   ids          int32 (id_bytes 4) or int64 (id_bytes 8) [tokens]; an id
 *                outside [0, n) yields a zero row
 *   fmt, packed, m0..m2, g0..g2, part_of_row: as cubic_prepare_weight
 *   out          [tokens, k] contiguous, out_dtype CUBIC_DTYPE_BF16 / _F16
 * Bit-exact to the reference decode: every value is evaluated in unfused
 * binary32 in the reference's order and rounded once (RNE).
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_embedding(const void* ids, int id_bytes, int64_t tokens, int fmt,
                              const void* packed, const void* m0, const void* m1, const void* m2,
                              const void* g0, const void* g1, const void* g2,
                              const int32_t* part_of_row, int64_t n, int64_t k, int bits,
                              int group_in, int group_out, void* out, int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * MoE router: per row, the top_k experts by (logit desc, expert id asc), then
 * a softmax over the selected logits, re-ordered by ascending expert id.
 * Replaces the routing launches of PackedRoutedExpertsPrimitive
 * (_bind_route_selection, ops/cuda/moe/quantized.py:58-180, kernels
 * _stable_topk_logits + _sort_and_normalize_topk / _stable_topk_routes,
 * ops/cuda/moe/fused.py:44-156):
 *   logits        bf16 / fp16 [rows, experts] (logits_fp16)
 *   row_activity  int32 [rows]; active_rows int32 device scalar: rows at or
 *                 past it, or with activity 0, publish 0 / -1 / -1 / 0
 *   top_logits f32, top_ids int64 [rows, top_k] in (logit desc) order
 *   route_ids int64, route_weights bf16 / fp16 (weights_fp16) [rows, top_k]
 *   in ascending expert order
 * 1 <= experts <= 1024, 1 <= top_k <= min(experts, 64).  exp and the sum
 * order are build-defined (as cubic_verify_candidates); logits must be finite.
 *
 * cubic_moe_compact: routes of experts [first_expert, first_expert + experts)
 * grouped by expert, ascending route ordinal inside each expert; counts,
 * starts, block starts (blocks of block_m) and the total block count
 * (_compact_local_routes, ops/cuda/moe/fused.py:174-199).  Other routes are
 * skipped; row_map positions past the owned routes are not written.
 * 1 <= experts <= 1024.  The outputs feed cubic_moe_pad_routes.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_moe_route(const void* logits, int logits_fp16, const int32_t* row_activity,
                              const int32_t* active_rows, int rows, int experts, int top_k,
                              float* top_logits, int64_t* top_ids, int64_t* route_ids,
                              void* route_weights, int weights_fp16, void* stream);
CUBIC_API int cubic_moe_compact(const int64_t* route_ids, int routes, int first_expert,
                                int experts, int block_m, int32_t* counts, int32_t* starts,
                                int32_t* block_starts, int32_t* total_blocks, int32_t* row_map,
                                void* stream);

/* ---------------------------------------------------------------------------
 * Candidate preparation: vocab logits -> top-`count` candidates per row.
 * Replaces LocalCandidatePlan.launch (ops/cuda/sampling/local_candidates.py:
 * 206-226: torch.topk + candidate_partial/candidate_publish,
 * local_candidates.cu:19-146) and the greedy argmax (greedy.cu:14-78).
 *   logits        [rows, row_stride], width <= row_stride visible columns;
 *                 dtype CUBIC_DTYPE_BF16, _F16 or _F32 (local_candidates.py:41)
 *   temperatures  f32 [rows]; 0 = greedy row (slot 0 = argmax, lowest id on ties)
 *   vocab_start   first token of this shard: published ids are vocab_start + column
 *   scores/ids    logits dtype / int64 [rows, capacity]; padding (NaN, -1); rows with a
 *                 non-finite logit publish id -2 in every counted slot
 *   owned rows: row < owned_rows, or row < owned_count[0] when owned_count
 *                 (device int32, the reference's metadata) is given, read when
 *                 the launch runs; and row_activity[row] != 0 when that bool
 *                 [rows] array is given.  Other rows publish padding only.
 *   1 <= count <= 20, count <= capacity <= 64; ties ordered by ascending id.
 * ------------------------------------------------------------------------- */
CUBIC_API int64_t cubic_candidates_workspace_bytes(int rows, int width);
CUBIC_API int cubic_candidates(const void* logits, int dtype, int64_t row_stride, int rows, int width,
                     int64_t vocab_start, const float* temperatures, int owned_rows, const int32_t* owned_count,
                     const uint8_t* row_activity, int count, int capacity,
                     int all_random, void* scores, int64_t* ids, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * K1 speculative verification over [tp, rows, k] candidates.
 * Replaces verify_one_draft_candidates (ops/cuda/sampling/speculative.py:
 * 222-328, kernel :46-219); same operand meanings and dtypes:
 *   q_scores/p_scores bf16, q_ids/p_ids int64, target_rows int32 [q_rows],
 *   draft_tokens/top_ks/seeds/ordinals int64 [q_rows], temperatures/top_ps f32,
 *   uniforms f32 [q_rows, 2] or NULL (Philox draws), constrained_rows bool or
 *   NULL, decisions int64 [q_rows, 2] = (accepted, next) or (-1, -1).
 *   1 <= tp <= 8, 1 <= k <= 20, 1 <= active_rows <= q_rows.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_verify_candidates(const void* q_scores, const int64_t* q_ids, const void* p_scores,
                            const int64_t* p_ids, const int32_t* target_rows,
                            const int64_t* draft_tokens, const float* temperatures,
                            const float* top_ps, const int64_t* top_ks, const int64_t* seeds,
                            const int64_t* ordinals, const float* uniforms,
                            const uint8_t* constrained_rows, int allow_underfilled, int tp,
                            int q_rows, int p_rows, int k, int active_rows, int64_t* decisions,
                            void* stream);

/* ---------------------------------------------------------------------------
 * Accepted-prefix merge.  Replaces merge_prefix (executor/draft_graph.py:
 * 146-157): decisions int64 [depth, c, 2] -> out int64 [c, 2] =
 * (accepted length, bonus token) or (-1, -1).  live: device int32 row count
 * (the reference's ctx[0]) or NULL to use live_rows.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_merge_prefix(const int64_t* decisions, int c, int depth, const int32_t* live,
                       int live_rows, int64_t* out, void* stream);

/* ---------------------------------------------------------------------------
 * Fused verify from logits: candidates of the c*(depth+1) target rows, then
 * verification of every depth, then the prefix merge -- the composition of
 * LocalCandidatePlan.launch, verify_one_draft_candidates per depth and
 * merge_prefix in finish_review (executor/draft_graph.py:1034-1067), in one
 * launch and one pass over the logits.  TP = 1.
 *   logits            bf16 [c*(depth+1), row_stride], row c*(depth+1)+d
 *   live sequences    c' < live_rows, or c' < live_count[0] when live_count
 *                     (device int32, the reference's ctx[0]) is given, read
 *                     when the launch runs; other sequences publish padding
 *                     and (-1, -1) decisions
 *   row_temperatures  f32 [c*(depth+1)] candidate publication temperatures
 *   q_scores/q_ids    bf16/int64 [depth, c, capacity] draft candidates
 *   draft_tokens, top_ks, seeds, ordinals  int64 [depth, c];
 *   temperatures, top_ps f32 [depth, c]; uniforms f32 [depth, c, 2] or NULL
 *   cand_scores/ids   bf16/int64 [c*(depth+1), capacity] published candidates
 *   decisions int64 [depth, c, 2]; merged int64 [c, 2]; emitted int64
 *   [c, depth+1] (accepted drafts then the bonus token, -1 padded) or NULL.
 *   1 <= depth <= 8, 1 <= capacity <= 20.
 * ------------------------------------------------------------------------- */
CUBIC_API int64_t cubic_accept_workspace_bytes(int c, int depth, int width);
CUBIC_API int cubic_accept(const void* logits, int64_t row_stride, int width, int c, int depth,
                 int live_rows, const int32_t* live_count, const float* row_temperatures,
                 const void* q_scores,
                 const int64_t* q_ids, int capacity, const int64_t* draft_tokens,
                 const float* temperatures, const float* top_ps, const int64_t* top_ks,
                 const int64_t* seeds, const int64_t* ordinals, const float* uniforms,
                 void* cand_scores, int64_t* cand_ids, int64_t* decisions, int64_t* merged,
                 int64_t* emitted, void* workspace, int64_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * cubic_accept_noalloc: cubic_accept with no workspace argument.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same operands, results and errors as cubic_accept.
 * Its scratch is a 4 MiB static device array per GPU, held until the process
 * ends; calls whose plan needs more (cubic_accept_workspace_bytes(c, depth,
 * width) > 4 MiB) fail with CUBIC_EWORKSPACE.  The array starts zero and
 * every launch leaves its counters zero; the first call on a device only
 * resolves the array's address and enqueues nothing besides the acceptance
 * launches, so that call may itself be under capture.  Nothing here calls hipMalloc,
 * hipFree or an allocating library routine.  Every call on one GPU shares the
 * array and it keeps the last call's contents: calls that overlap on one GPU
 * (launches on concurrent streams) race and must be ordered by the caller.
 * ------------------------------------------------------------------------- */
CUBIC_API int cubic_accept_noalloc(const void* logits, int64_t row_stride, int width, int c,
                                   int depth, int live_rows, const int32_t* live_count,
                                   const float* row_temperatures,
                                   const void* q_scores, const int64_t* q_ids, int capacity,
                                   const int64_t* draft_tokens, const float* temperatures,
                                   const float* top_ps, const int64_t* top_ks,
                                   const int64_t* seeds, const int64_t* ordinals,
                                   const float* uniforms, void* cand_scores, int64_t* cand_ids,
                                   int64_t* decisions, int64_t* merged, int64_t* emitted,
                                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CUBIC_MI355X_H */
