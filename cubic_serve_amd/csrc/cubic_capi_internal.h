// Kernel argument blocks shared between the C-ABI entry points (cubic_capi.cpp)
// and the kernels.  Not part of the public interface (include/cubic_mi355x.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cubic {

// GEMM workgroup: kGemmWaves waves, each owning J 16-column tiles, share one
// LDS activation tile.  Four: two independent workgroups per CU hide latency
// better than one 8-wave workgroup in barrier lockstep, although the latter
// halves the activation bytes per weight byte (measured both); 2-wave
// workgroups measured slower on every cfg2 shape.
constexpr int kGemmWaves = 4;

// Members of one grouped GEMM launch (same K, same per-member width).
constexpr int kMaxGemmMembers = 8;

struct AcceptArgs {
    const uint16_t* logits;       // [rows, row_stride] bf16 (fp16 when scores_fp16, candidates only)
    int64_t row_stride;           // elements
    int scores_fp16;
    int rows, width, tiles, tile_width, vector_loads;
    const float* row_temperatures;  // [rows]: 0 = greedy publication
    int owned_rows, count, capacity, all_random;
    int64_t vocab_start;          // published ids: vocab_start + column (candidates only)
    // device-side counts read when the launch runs (null: the host values):
    // candidates: rows < owned_count[0] are owned, and row_activity[row] must
    // be set; fused: sequences < live_count[0] are live (owned rows follow)
    const int32_t* owned_count;
    const uint8_t* row_activity;
    const int32_t* live_count;
    uint16_t* cand_scores;        // [rows, capacity], the logits' type
    int64_t* cand_ids;            // [rows, capacity]
    int group_rows;               // rows finalised together (1, or depth+1 when fused)
    uint32_t* counters;           // [rows / group_rows], zero between launches
    uint32_t* partial_keys;       // [rows, tiles, 20]
    uint32_t* partial_flags;      // [rows, tiles]
    // fused verify (group = one sequence of depth+1 target rows)
    int c, live_rows, block;
    const uint16_t* q_scores;     // [depth, c, capacity] bf16
    const int64_t* q_ids;
    const int64_t* draft_tokens;  // [depth, c]
    const float* temperatures;    // [depth, c]
    const float* top_ps;
    const int64_t* top_ks;
    const int64_t* seeds;
    const int64_t* ordinals;
    const float* uniforms;        // [depth, c, 2] or null
    int64_t* decisions;           // [depth, c, 2]
    int64_t* merged;              // [c, 2]
    int64_t* emitted;             // [c, depth + 1] or null
};

// fp32 candidate preparation (SCORE_TYPE 2): a tile pass over (tile, row)
// workgroups, then one publishing wave per row.
struct CandF32Args {
    const float* logits;          // [rows, row_stride]
    int64_t row_stride;           // elements
    int rows, width, tiles, vector_loads;
    const float* row_temperatures;  // [rows]: 0 = greedy publication
    int owned_rows, count, capacity, all_random;
    int64_t vocab_start;
    const int32_t* owned_count;   // device: rows < owned_count[0] are owned, or null
    const uint8_t* row_activity;  // [rows] or null
    float* scores;                // [rows, capacity]
    int64_t* ids;                 // [rows, capacity]
    uint64_t* partial;            // [rows, tiles, 20] composite keys of each tile's top
    uint32_t* partial_finite;     // [rows, tiles]
};

struct VerifyArgs {
    const uint16_t* q_scores;  // [tp, q_rows, k] bf16
    const int64_t* q_ids;
    const uint16_t* p_scores;  // [tp, p_rows, k] bf16
    const int64_t* p_ids;
    const int32_t* target_rows;
    const int64_t* draft_tokens;
    const float* temperatures;
    const float* top_ps;
    const int64_t* top_ks;
    const int64_t* seeds;
    const int64_t* ordinals;
    const float* uniforms;        // [q_rows, 2] or null
    const uint8_t* constrained_rows;  // [q_rows] bool or null
    int64_t* decisions;           // [q_rows, 2]
    int tp, q_rows, p_rows, k, block, active_rows, allow_underfilled;
};

struct RootSampleArgs {
    const uint16_t* scores;          // [tp, rows, k] bf16 or fp16
    int scores_fp16;
    const int64_t* ids;              // [tp, rows, k]
    const float* temperatures;       // [rows]
    const float* top_ps;
    const int64_t* top_ks;
    const int64_t* seeds;
    const int64_t* ordinals;
    const uint8_t* constrained_rows;  // [rows] bool or null
    int allow_underfilled;
    int tp, rows, k, block;          // block = next_pow2(tp * k)
    int64_t* output_tokens;          // [rows]
    uint8_t* output_valid;           // [rows] bool
};

// MoE router (cubic_moe.hip)
constexpr int kMaxRouteExperts = 1024;
constexpr int kMaxRouteTopK = 64;
struct MoERouteArgs {
    const uint16_t* logits;       // [rows, experts] bf16 or fp16
    int logits_fp16;
    const int32_t* row_activity;  // [rows]
    const int32_t* active_rows;   // device scalar
    int rows, experts, top_k;
    float* top_logits;            // [rows, top_k] (logit desc order)
    int64_t* top_ids;             // [rows, top_k]
    int64_t* route_ids;           // [rows, top_k] ascending expert id
    uint16_t* route_weights;      // [rows, top_k] bf16 or fp16
    int weights_fp16;
};

// Route compaction (cubic_moe.hip)
constexpr int kMaxCompactExperts = 1024;
constexpr int kCompactExpertBits = 10;  // 2^bits >= kMaxCompactExperts
struct MoECompactArgs {
    const int64_t* route_ids;  // [routes] global expert ids (-1 / others unowned)
    int routes, first_expert, experts, block_m;
    int32_t* counts;           // [experts]
    int32_t* starts;
    int32_t* block_starts;
    int32_t* total_blocks;     // [1]
    int32_t* row_map;          // [routes]; only owned positions written
};

struct GemmArgs {
    const uint16_t* x;            // [m, k] bf16, row stride ldx
    const uint32_t* codes;        // prepared code tiles
    const uint32_t* meta;         // prepared (scale, a|b) per (column, group)
    // member outputs: column n belongs to member n / n_member and lands at
    // column n % n_member of ys[member] (row stride ldys[member])
    uint16_t* ys[kMaxGemmMembers];
    float* partials;              // split-K FP32 partials or null
    uint32_t* counters;           // split-K arrival counters or null
    int64_t ldx;
    int64_t ldys[kMaxGemmMembers];
    int m, n, k, n_member;
    int bits, group_in;
    int k_blocks, groups_k;       // ceil(k / 128), ceil(k / group_in)
    int split, blocks_per_split;  // K partitions and k-blocks per partition
    int n_tiles;                  // ceil(n / 16)
    int tiles_per_wave;           // J: 16-column tiles per wave (1, 2, 4)
    int chunk_rows;               // rows per grid-z chunk: 64, or 32 (M split), or block_m (routed)
    int rows_waves;               // > 0: small-row kernel with this many waves per tile
                                  // (blocks_per_split = k-blocks per wave)
    int f16;                      // activations, prepared levels and outputs are fp16 (else bf16)
    int panel;                    // > 0: column-panel kernel (2: level tables staged in LDS)
    int panel_stages;             // column-panel ring depth S (2 or 4; divides the partition's k-block pairs)
    int panel_waves;              // column-panel waves per workgroup (the kernels take 4)
    // routed experts (MoE, routed != 0): workgroup chunk z covers the
    // 16 * MT padded route slots [z * 16 * MT, ...) of one expert
    // (block_expert[z]); a slot holds a route ordinal, or `routes` for
    // padding; input row = route / top_k, output row = route.  Chunks at or
    // past *padded_total / (16 * MT) exit at once.
    int routed, block_m;          // block_m: 16, 32 or 64 route slots per block
    const int32_t* padded;        // [max blocks * 16 * MT] route ordinals
    const int32_t* block_expert;  // [max blocks] expert of each block
    const int32_t* padded_total;  // device: total blocks * 16 * MT
    int routes, top_k;
    int64_t expert_code_stride, expert_meta_stride;  // uint32 words per expert
};

struct EmbedArgs {
    const void* ids;              // [tokens] int32 or int64 (id_bytes)
    int id_bytes;
    int64_t tokens;
    int fmt;                      // metadata format (group_metadata)
    const uint8_t* packed;        // [n, row_bytes] little-endian bitstream
    const void *m0, *m1, *m2, *g0, *g1, *g2;
    const int32_t* part_of_row;   // [n] output partition of each row (fmt 1, 2)
    int64_t n, k, row_bytes, groups_k;
    int bits, group_in, group_out;
    int aligned;                  // packed base and row_bytes 4-byte aligned
    int chunk_in_group;           // group_in % 16 == 0: a 16-column chunk is in one group
    int lut;                      // chunk_in_group and 4 * 2^bits <= group_in: table path
    uint16_t* out;                // [tokens, k] bf16 or fp16
    int out_fp16;
};

// Per-row sampling parameters read by the greedy root and the final guard.
struct GreedyParams {
    const float* temperatures;    // [rows]
    const float* top_ps;
    const int64_t* top_ks;
    const int64_t* seeds;
    const int64_t* ordinals;
    int k;                        // max_top_k (candidates per rank)
    int64_t vocab_size;           // true vocabulary size
};

struct GreedyArgs {
    const uint16_t* logits;       // [rows, row_stride] bf16 or fp16
    int64_t row_stride;
    int scores_fp16, rows, width;
    int64_t vocab_start;
    const int32_t* metadata;      // [2]: active rows, cancel flag
    const uint32_t* token_mask;   // [rows, mask_words] or null
    int64_t mask_words;
    // grammar-masked logits out (token_mask only): [rows, masked_stride], the
    // logits' type; rows < active get the admitted logits and -inf elsewhere,
    // other rows -inf unless masked == logits (in place: left as they are)
    uint16_t* masked;
    int64_t masked_stride;
    int masked_inplace;
    int candidates;               // published slots per row
    uint16_t* scores;             // [rows, candidates]
    int64_t* ids;
    int tiles, tile_width, vector_loads;
    uint64_t* partial_keys;       // [rows, tiles]
    uint32_t* partial_flags;      // [rows, tiles]
    uint32_t* counters;           // [rows + 1], zero between launches; the last
                                  // counts fused row arrivals (+ 2^16 per failed guard term)
    // fused root and guard (tokens == null: candidates only)
    GreedyParams p;
    int64_t* tokens;              // [rows]
    uint8_t* root_valid;          // [rows]
    uint8_t* final_valid;         // [1]
};

struct GreedyRootArgs {
    const uint16_t* scores;       // [tp, rows, k]
    int scores_fp16;
    const int64_t* ids;
    const int32_t* metadata;
    int tp, rows;
    GreedyParams p;
    int64_t* tokens;
    uint8_t* valid;
};

struct GuardArgs {
    const int64_t* tokens;        // [capacity]
    const uint8_t* root_valid;    // [capacity] or null (not the root rank)
    const int32_t* metadata;
    int capacity;
    GreedyParams p;
    uint8_t* valid;               // [1]
};

hipError_t launch_accept(const AcceptArgs& a, bool fused, hipStream_t s);
hipError_t launch_greedy(const GreedyArgs& a, hipStream_t s);
hipError_t launch_greedy_root(const GreedyRootArgs& a, hipStream_t s);
hipError_t launch_final_guard(const GuardArgs& a, hipStream_t s);
hipError_t launch_verify(const VerifyArgs& a, hipStream_t s);
hipError_t launch_candidates_f32(const CandF32Args& a, hipStream_t s);
constexpr int kCandF32Tile = 4096;  // columns per fp32 candidate tile
hipError_t launch_root_sample(const RootSampleArgs& a, hipStream_t s);
hipError_t launch_merge_prefix(const int64_t* decisions, int c, int depth, const int32_t* live,
                               int live_rows, int64_t* out, hipStream_t s);
// f16: level tables (bits <= 4) in fp16 instead of bf16; codes do not depend on it
hipError_t launch_prepare(const void* packed, const float* scale, const uint16_t* a,
                          const uint16_t* b, int64_t n, int64_t k, int bits, int group_in, int f16,
                          uint32_t* codes, uint32_t* meta, hipStream_t s);
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s);
// Column-panel kernel (cubic_panel.hip), chosen by the host plan (a.panel > 0).
hipError_t launch_panel_gemm(const GemmArgs& a, hipStream_t s);
// Routed-block table from compact routes (quantization/common/marlin/repack.py:253-277)
hipError_t launch_pad_routes(const int32_t* counts, const int32_t* starts, const int32_t* block_starts,
                             const int32_t* total_blocks, const int32_t* row_map, int experts,
                             int routes, int block_m, int32_t* padded, int32_t* block_expert,
                             int32_t* padded_total, hipStream_t s);
// fmt 0: m0 scale f32, m1 a f16, m2 b f16; fmt 1: m0 scale i8, m1 ab u8, g0..g2
// globals f32; fmt 2: m0 metadata u16, m1 curve_a f16, m2 curve_b f16.
hipError_t launch_expand_metadata(int fmt, const void* m0, const void* m1, const void* m2,
                                  const void* g0, const void* g1, const void* g2,
                                  const int32_t* part_of_row,
                                  int64_t n, int64_t groups_k, int group_out, float* scale,
                                  uint16_t* a, uint16_t* b, hipStream_t s);

hipError_t launch_moe_route(const MoERouteArgs& a, hipStream_t s);
hipError_t launch_moe_compact(const MoECompactArgs& a, hipStream_t s);

// Packed embedding lookup (quantization/extensions/cubic/linear.py:266-294)
hipError_t launch_embedding(const EmbedArgs& a, hipStream_t s);
int64_t embedding_column_blocks(int64_t k);  // grid.y of launch_embedding

}  // namespace cubic
