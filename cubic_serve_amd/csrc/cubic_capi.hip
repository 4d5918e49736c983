// C ABI entry points: argument validation, launch planning, kernel dispatch.
// Declarations and the reference interface each entry replaces are in
// include/cubic_mi355x.h.
#include <string>
#include <cstdio>
#include <cstdarg>
#include <cstdlib>
#include <mutex>
#include <algorithm>
#include <climits>

#include "cubic_mi355x.h"
#include "cubic_capi_internal.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return CUBIC_OK;
    return fail(CUBIC_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kKBlock = 128;
constexpr int kTop = 20;
constexpr int kChunk = 2048;
constexpr int kMaxTileChunks = 16;
constexpr int kMaxTiles = 24;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---------------------------------------------------------------------------
// GEMM launch plan.
//
// The K partition (split, blocks_per_split) is a pure function of ONE
// member's (n, k): neither m nor the number of grouped members changes which
// k-blocks a partition holds, so every output element is summed in the same
// order whatever m is and whether or not its matrix shares a launch
// (quantization/extensions/cubic/marlin.py:347-360 plans grouped launches on
// one member for this reason; quantization/common/marlin/cost.py:59-79 keeps
// partitions independent of m).  Tiles per wave (J) and the row chunking only
// choose which wave computes a tile; they never change its arithmetic, so they
// may follow the launch's total width and m.
// ---------------------------------------------------------------------------
struct GemmPlan {
    int n_tiles, k_blocks, tiles_per_wave, col_blocks, split, blocks_per_split;
    int chunk_rows;  // rows per grid-z chunk (64; 32 when M is split across workgroups; 128 past 64 rows)
    int rows_waves;  // > 0: small-row kernel, this many waves per tile, blocks_per_split per wave
    int panel;       // > 0: column-panel kernel (2: level tables staged in LDS)
    int panel_stages;  // column-panel ring depth
    int panel_waves;   // column-panel waves per workgroup
};

#ifdef CUBIC_EXPERIMENTS
// experiment builds only: force the panel plan (J, split, tables in LDS)
static int g_exp_j = 0, g_exp_split = 0, g_exp_tl = -1, g_exp_panel = -1, g_exp_stages = 0, g_exp_waves = 0;
extern "C" __attribute__((visibility("default"))) void cubic_exp_plan(int j, int split, int tl, int panel, int stages, int waves) {
    g_exp_j = j; g_exp_split = split; g_exp_tl = tl; g_exp_panel = panel; g_exp_stages = stages; g_exp_waves = waves;
}
#endif

// Small-row regime (the reference's small_rows path, M <= 4): one tile per
// workgroup, K split over the workgroup's waves; a function of (k, bits) alone.
// Above 4 bits there is no prepared table: 5-6 bits build each k-block's
// levels in LDS, 7-8 bits evaluate every weight from the curve.  Measured
// against the MFMA-tile kernel at M = 1 (Llama-3-70B linears, Qwen3 lm_head):
// 7-8 bits win at every K (down 28672-deep: 95 -> 81 us at 7 bits); 5-6 bits
// win up to 64 k-blocks (gate/up 145 -> 121 us at 5 bits) and lose a few
// percent on the 224-k-block down projection, which stays on the MFMA-tile
// kernel.
bool small_rows(int64_t m, int bits, int group_in, int64_t k) {
    if (m < 1 || m > 4 || bits > 8 || group_in <= 0 || group_in % kKBlock != 0) return false;
    // the small-row kernel sizes a tile's code and metadata buffers in 32 bits
    const int64_t k_blocks = ceil_div(k, kKBlock);
    if (k_blocks * 64 * bits * 4 >= (int64_t(1) << 31) || ceil_div(k, group_in) * 16 * 16 >= (int64_t(1) << 31))
        return false;
    return bits <= 4 || bits >= 7 || ceil_div(k, kKBlock) <= 64;
}

// K partition of one member: split in powers of two (at most 8) until a
// partition holds at most 16 k-blocks -- 32 when the unsplit member already
// gives >= 160 workgroups of one tile per wave, 64 for a K of 128 k-blocks or
// more -- and about 256 workgroups of one tile per wave are in flight; a
// member wide enough to fill the GPU with two tiles per wave keeps K whole.
// The plan is a function of one member's (n, k) alone, so a row's result does
// not depend on M.  Measured per launch, same box, W4, M = 8 / 64 / 512 (us):
//   Llama-3-70B gate/up members, 28672 x 8192: split 2 instead of 4, grouped
//     launch 61 -> 57, equal, 607 -> 521;
//   qkv 10240 x 8192: split 2 instead of 4, 19.6 -> 19.4, 33.3 -> 31.1,
//     123.9 -> 117.0;
//   down 8192 x 28672: split 4 instead of 8, 34.3 -> 31.3, 53.9 -> 56.8,
//     284 -> 255;
//   o 8192 x 8192 stays at 4 (split 2: 13.7 -> 18.3 and 21.6 -> 28.3 at
//     M = 8 and 64, though 99 -> 81 at M = 512).
// Above 4 bits (per-weight curve or LDS-table decode, about twice the work
// per weight) the 160-block and deep-K caps lose: qkv and down at 6 and 8 bits
// take 16-22 us longer at M = 8 and 64 with the halved split, so there the
// cap is 32 only from 384 workgroups.  Bits are a property of the weight, so
// the plan still does not depend on M.
void plan_k(int64_t n_member, int64_t k, int bits, int* split_out, int* bps_out) {
    const int64_t tiles = ceil_div(n_member, 16);
    const int k_blocks = (int)ceil_div(k, kKBlock);
    int split = 1;
    if (ceil_div(tiles, 2 * cubic::kGemmWaves) < 256) {
        const int64_t out_blocks = ceil_div(tiles, cubic::kGemmWaves);
        const int kb_cap = bits > 4 ? (out_blocks >= 384 ? 32 : 16)
                                    : (k_blocks >= 128 ? 64 : out_blocks >= 160 ? 32 : 16);
        while (split < 8 && (ceil_div(k_blocks, split) > kb_cap || out_blocks * split < 256)) split *= 2;
        if (split > k_blocks / 2) split = k_blocks / 2 > 0 ? k_blocks / 2 : 1;
    }
    const int bps = (int)ceil_div(k_blocks, split);
    *bps_out = bps;
    *split_out = (int)ceil_div(k_blocks, bps);
}

GemmPlan plan_gemm(int64_t m, int64_t n_member, int members, int64_t k, int bits, int group_in) {
    GemmPlan p = {};
    const int64_t n = n_member * members;
    p.n_tiles = (int)ceil_div(n, 16);
    p.k_blocks = (int)ceil_div(k, kKBlock);
    p.rows_waves = 0;
    if (small_rows(m, bits, group_in, k)) {
        p.rows_waves = p.k_blocks > 32 ? 8 : 4;
        p.blocks_per_split = (int)ceil_div(p.k_blocks, p.rows_waves);
        p.split = 1;
        p.tiles_per_wave = 1;
        p.col_blocks = p.n_tiles;
        p.chunk_rows = 4;
        return p;
    }
    p.panel = 0;
    p.panel_stages = 2;
    p.panel_waves = cubic::kGemmWaves;
    plan_k(n_member, k, bits, &p.split, &p.blocks_per_split);
#ifdef CUBIC_EXPERIMENTS
    if (g_exp_split > 0) {
        p.split = g_exp_split;
        p.blocks_per_split = (int)ceil_div(p.k_blocks, p.split);
        p.split = (int)ceil_div(p.k_blocks, p.blocks_per_split);
    }
#endif
    // Column panels (M <= 64, bits <= 4, whole-k-block groups): the tiles of
    // a wave share each staged activation block and A fragment.  The
    // kernel addresses activations and metadata with 32-bit buffer offsets.
    const int64_t meta_bytes = (int64_t)p.n_tiles * ceil_div(k, group_in) * 16 * (bits == 4 ? 16 : 8);
    if (m <= 64 && bits <= 4 && group_in % kKBlock == 0 && meta_bytes < (int64_t(1) << 31)) {
        p.panel = bits == 4 ? 2 : 1;
        // Two tiles per wave (each staged activation block feeds twice the
        // MFMAs) while the grid keeps >= 384 workgroups, with a 2-deep ring;
        // one tile per wave otherwise, with a 4-deep ring.  Measured at
        // M = 64, 4 bits, Llama-3-8B shapes: gate/up 26.7 us (one tile per
        // wave in gemm_kernel: 29.9), lm_head 110 (116), down 18.2 (19.2),
        // qkv and o equal; two tiles with a 4-deep ring: lm_head 143.
        int j = ceil_div(p.n_tiles, cubic::kGemmWaves * 2) * p.split >= 384 ? 2 : 1;
        p.panel_stages = j == 2 ? 2 : 4;
#ifdef CUBIC_EXPERIMENTS
        if (g_exp_j > 0) j = g_exp_j;
        if (g_exp_tl >= 0) p.panel = g_exp_tl ? 2 : 1;
        if (g_exp_panel == 0) p.panel = 0;
        if (g_exp_stages > 0) p.panel_stages = g_exp_stages;
        if (g_exp_waves > 0) p.panel_waves = g_exp_waves;
#endif
        if (p.panel) {
            p.tiles_per_wave = j;
            p.col_blocks = (int)ceil_div(p.n_tiles, p.panel_waves * j);
            p.chunk_rows = 64;
            return p;
        }
    }
    // Past 64 rows (whole-k-block groups) a workgroup takes 128 rows: each
    // decoded weight fragment feeds eight m-tiles of MFMA instead of four.
    const bool wide = m > 64 && group_in % kKBlock == 0;
    const int64_t chunks = ceil_div(m, wide ? 128 : 64);
    // Two 16-column tiles per wave (half the activation bytes and A-fragment
    // LDS reads per weight byte) when K is whole and the launch still fills the
    // GPU; one tile per wave otherwise.
    p.tiles_per_wave = (p.split == 1 && ceil_div(p.n_tiles, 2 * cubic::kGemmWaves) * chunks >= 256) ? 2 : 1;
    // Past 64 rows the A-fragment LDS reads bound the loop (one MFMA per
    // fragment at J = 1): two tiles per wave whenever the grid keeps >= 320
    // workgroups (Llama-3-70B layers at M = 65..512: 12-25% faster per layer;
    // a narrower grid, o at M <= 128, measured slower).
    if (wide && ceil_div(p.n_tiles, 2 * cubic::kGemmWaves) * p.split * chunks >= 320) p.tiles_per_wave = 2;
    p.col_blocks = (int)ceil_div(p.n_tiles, cubic::kGemmWaves * p.tiles_per_wave);
    // Rows 33..64 split over two 32-row workgroups when the grid would
    // otherwise hold fewer than two workgroups per CU (qkv, o: measured 7%
    // faster; the weights are read twice, from L2 the second time).
    p.chunk_rows = wide ? 128 : 64;
    if (p.tiles_per_wave == 1 && m > 32 && m <= 64 && (int64_t)p.col_blocks * p.split < 512)
        p.chunk_rows = 32;
    return p;
}

// Split-K workspace: arrival counters per output block, then FP32 partials
// per K partition and output block (64-row chunk x column block): waves x J
// tiles x MT m-tiles x 64 lanes float4 units.
int64_t gemm_workspace(int64_t m, int64_t n_member, int members, int64_t k, int bits, int group_in) {
    const GemmPlan p = plan_gemm(m, n_member, members, k, bits, group_in);
    if (p.split == 1) return 0;
    const int64_t blocks = (int64_t)p.col_blocks * ceil_div(m, p.chunk_rows);
    const int64_t mt = p.chunk_rows == 128 ? 8 : p.chunk_rows == 32 ? 2 : (ceil_div(m, 64) > 1 ? 4 : (m >= 33 ? 4 : (m >= 17 ? 2 : 1)));
    const int64_t units = (p.panel ? p.panel_waves : cubic::kGemmWaves) *
                          p.tiles_per_wave * mt * 64;
    return align256(blocks * 4) + align256((int64_t)p.split * blocks * units * 16);
}

// Workspace when the group width is not known yet: the larger of the two
// chunkings (128-row chunks for whole-k-block groups, 64-row chunks otherwise).
int64_t gemm_workspace_any_group(int64_t m, int64_t n_member, int members, int64_t k, int bits) {
    const int64_t a = gemm_workspace(m, n_member, members, k, bits, kKBlock);
    const int64_t b = gemm_workspace(m, n_member, members, k, bits, 32);
    return a > b ? a : b;
}

int gemm_common(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
                int64_t m, int members, int64_t n_member, int64_t k, int bits, int group_in, int dtype,
                void* const* ys, const int64_t* ldys, void* workspace, int64_t workspace_bytes,
                void* stream) {
    if (!x || !codes || !meta || !ys) return fail(CUBIC_EINVAL, "null operand");
    if (dtype != CUBIC_DTYPE_BF16 && dtype != CUBIC_DTYPE_F16) return fail(CUBIC_ENOTSUP, "dtype=%d", dtype);
    if (members < 1 || members > cubic::kMaxGemmMembers)
        return fail(CUBIC_EINVAL, "members=%d outside 1..%d", members, cubic::kMaxGemmMembers);
    for (int i = 0; i < members; ++i)
        if (!ys[i]) return fail(CUBIC_EINVAL, "null output of member %d", i);
    if (m <= 0 || n_member <= 0 || k <= 0 || m > (1 << 30) || n_member * members > (1 << 30) || k > (1 << 30))
        return fail(CUBIC_EINVAL, "gemm extents must be positive: m=%lld n=%lld k=%lld",
                    (long long)m, (long long)n_member, (long long)k);
    if (members > 1 && n_member % 16)
        return fail(CUBIC_EINVAL, "grouped members need n %% 16 == 0 (n=%lld)", (long long)n_member);
    if (bits < 1 || bits > 8) return fail(CUBIC_ENOTSUP, "bits=%d outside 1..8", bits);
    if (group_in <= 0 || group_in % 32) return fail(CUBIC_ENOTSUP, "group_in=%d must be a multiple of 32", group_in);
    if (k % 8 || ldx % 8 || ldx < k || !aligned16(x))
        return fail(CUBIC_ENOTSUP, "activations need k %% 8 == 0, ldx %% 8 == 0 and 16-byte alignment");
    for (int i = 0; i < members; ++i)
        if (ldys[i] < n_member) return fail(CUBIC_EINVAL, "output leading dimension too small");
    GemmPlan p = plan_gemm(m, n_member, members, k, bits, group_in);
    const int64_t need = gemm_workspace(m, n_member, members, k, bits, group_in);
    if (workspace_bytes < need) return fail(CUBIC_EWORKSPACE, "gemm workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)need);
    if (p.rows_waves && m * ldx * 2 >= (int64_t(1) << 31))
        return fail(CUBIC_ENOTSUP, "small-row GEMM: activation row stride too large (m * ldx * 2 = %lld >= 2^31 bytes)",
                    (long long)(m * ldx * 2));
    if (p.panel && m * ldx * 2 >= (int64_t(1) << 31)) {
        // the column-panel kernel reaches activations through 32-bit buffer
        // offsets: a row stride this large takes the MFMA-tile kernel (same
        // K plan, same arithmetic), whose split-K buffer is no larger
        p.panel = 0;
        p.tiles_per_wave = 1;
        p.col_blocks = (int)ceil_div(p.n_tiles, cubic::kGemmWaves);
        p.chunk_rows = 64;
        const int64_t alt = p.split == 1 ? 0
                          : align256((int64_t)p.col_blocks * 4) +
                                align256((int64_t)p.split * p.col_blocks * cubic::kGemmWaves * 4 * 64 * 16);
        if (workspace_bytes < alt) return fail(CUBIC_EWORKSPACE, "gemm workspace %lld < %lld bytes", (long long)workspace_bytes, (long long)alt);
    }
    if (need && !workspace) return fail(CUBIC_EINVAL, "null workspace");
    cubic::GemmArgs a = {};
    a.x = (const uint16_t*)x;
    a.codes = codes;
    a.meta = meta;
    for (int i = 0; i < members; ++i) {
        a.ys[i] = (uint16_t*)ys[i];
        a.ldys[i] = ldys[i];
    }
    a.ldx = ldx;
    a.m = (int)m;
    a.n = (int)(n_member * members);
    a.k = (int)k;
    a.n_member = (int)n_member;
    a.bits = bits;
    a.group_in = group_in;
    a.k_blocks = p.k_blocks;
    a.groups_k = (int)ceil_div(k, group_in);
    a.split = p.split;
    a.blocks_per_split = p.blocks_per_split;
    a.n_tiles = p.n_tiles;
    a.tiles_per_wave = p.tiles_per_wave;
    a.chunk_rows = p.chunk_rows;
    a.rows_waves = p.rows_waves;
    a.panel = p.panel;
    a.panel_stages = p.panel_stages;
    a.panel_waves = p.panel_waves;
    a.f16 = dtype == CUBIC_DTYPE_F16;
    if (p.split > 1) {
        const int64_t counters = align256((int64_t)p.col_blocks * ceil_div(m, p.chunk_rows) * 4);  // one per output block
        a.counters = (uint32_t*)workspace;
        a.partials = (float*)((char*)workspace + counters);
    }
    return hip_status(cubic::launch_gemm(a, (hipStream_t)stream), "cubic_gemm launch");
}

// words of the prepared code stream / metadata of `tiles` 16-column tiles
int64_t prepared_code_words(int64_t tiles, int64_t k, int bits) { return tiles * ceil_div(k, kKBlock) * 64 * bits; }
int64_t prepared_meta_words(int64_t tiles, int64_t k, int bits, int group_in) {
    return tiles * ceil_div(k, group_in) * 16 * (bits == 4 ? 4 : 2);
}

// ---------------------------------------------------------------------------
// Candidate tiling: enough (row, tile) workgroups to cover the chip.
// ---------------------------------------------------------------------------
struct TilePlan {
    int tiles, tile_width;
};

bool plan_tiles(int rows, int width, TilePlan* out) {
    if (width <= 0 || rows <= 0) return false;
#ifndef CUBIC_TILE_TARGET
#define CUBIC_TILE_TARGET 512
#endif
    int target = (int)ceil_div(CUBIC_TILE_TARGET, rows);
    if (target < 1) target = 1;
    if (target > kMaxTiles) target = kMaxTiles;
    int64_t tw = ceil_div(ceil_div(width, target), kChunk) * kChunk;
    // tiles of at least four chunks (or the whole row): a narrower tile
    // saves less load time than its extra partial lists cost the merge
    // (2 rows x 32768: 16 one-chunk tiles 8.9 us, 4 four-chunk tiles 8.0)
    const int64_t floor_tw = ceil_div(width, kChunk) * kChunk < 4 * kChunk ? ceil_div(width, kChunk) * kChunk : 4 * kChunk;
    if (tw < floor_tw) tw = floor_tw;
    const int64_t min_tw = ceil_div(ceil_div(width, kMaxTiles), kChunk) * kChunk;
    if (tw > (int64_t)kChunk * kMaxTileChunks) tw = (int64_t)kChunk * kMaxTileChunks;
    // tiles of <= 8 chunks keep the per-lane element registers of the tile
    // phase free of spills; wider tiles only when the tile count demands it
    if (tw > (int64_t)kChunk * 8) tw = (int64_t)kChunk * 8;
    if (tw < min_tw) tw = min_tw;
    if (tw > (int64_t)kChunk * kMaxTileChunks) return false;
    out->tile_width = (int)tw;
    out->tiles = (int)ceil_div(width, tw);
    return out->tiles <= kMaxTiles;
}

int64_t accept_workspace(int rows, int groups, int width) {
    TilePlan t;
    if (!plan_tiles(rows, width, &t)) return -1;
    return align256((int64_t)groups * 4) + align256((int64_t)rows * t.tiles * kTop * 4) +
           align256((int64_t)rows * t.tiles * 4);
}

void carve_accept(void* ws, int rows, int groups, int tiles, cubic::AcceptArgs& a) {
    char* p = (char*)ws;
    a.counters = (uint32_t*)p;
    p += align256((int64_t)groups * 4);
    a.partial_keys = (uint32_t*)p;
    p += align256((int64_t)rows * tiles * kTop * 4);
    a.partial_flags = (uint32_t*)p;
}

int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

// ---------------------------------------------------------------------------
// Static acceptance scratch for cubic_accept_noalloc: arrival counters, tile
// survivor keys and flags, in device memory that the library owns for the life
// of the process (one copy per device).  The name below is a host-side handle;
// device code only ever sees the address hipGetSymbolAddress returns for the
// current device.  The array starts zero (a zero-initialised device global)
// and every launch leaves its counters zero again, as cubic_accept does with
// its workspace, so set-up only resolves the address: it enqueues nothing, and
// a first call made under HIP graph capture records only the acceptance
// launches themselves.
// ---------------------------------------------------------------------------
constexpr int64_t kAcceptScratchBytes = int64_t(4) << 20;
__device__ __align__(256) uint32_t scratch[kAcceptScratchBytes / 4];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// Address of the current device's scratch, resolved on the first call per device.
int accept_scratch(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(CUBIC_ENOTSUP, "device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return hip_status(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return CUBIC_OK;
}

int accept_common(const void* logits, int64_t row_stride, int width, int c, int depth,
                  int live_rows, const int32_t* live_count, const float* row_temperatures,
                  const void* q_scores,
                  const int64_t* q_ids, int capacity, const int64_t* draft_tokens,
                  const float* temperatures, const float* top_ps, const int64_t* top_ks,
                  const int64_t* seeds, const int64_t* ordinals, const float* uniforms,
                  void* cand_scores, int64_t* cand_ids, int64_t* decisions, int64_t* merged,
                  int64_t* emitted, void* workspace, int64_t workspace_bytes, void* stream);

}  // namespace

extern "C" {

int cubic_abi_version(void) { return 6; }

const char* cubic_last_error(void) { return g_error.c_str(); }

int cubic_prepared_words(int64_t n, int64_t k, int bits, int group_in, int64_t* code_words,
                         int64_t* meta_words) {
    if (n <= 0 || k <= 0 || bits < 1 || bits > 8 || group_in <= 0 || group_in % 32)
        return fail(CUBIC_EINVAL, "invalid prepared geometry");
    const int64_t n_tiles = ceil_div(n, 16), k_blocks = ceil_div(k, kKBlock);
    if (code_words) *code_words = n_tiles * k_blocks * 64 * bits;
    if (meta_words) *meta_words = n_tiles * ceil_div(k, group_in) * 16 * (bits == 4 ? 4 : 2);
    return CUBIC_OK;
}

int64_t cubic_prepare_scratch_bytes(int64_t n, int64_t k, int group_in) {
    if (n <= 0 || k <= 0 || group_in <= 0) return -1;
    const int64_t groups = n * ceil_div(k, group_in);
    return align256(groups * 4) + 2 * align256(groups * 2);
}

int cubic_prepare_weight(int fmt, const void* packed, const void* m0, const void* m1,
                         const void* m2, const void* g0, const void* g1, const void* g2,
                         const int32_t* part_of_row, int64_t n, int64_t k, int bits,
                         int group_in, int group_out, int dtype, void* expanded, int64_t expanded_bytes,
                         uint32_t* codes, uint32_t* meta, void* stream) {
    if (!packed || !m0 || !m1 || !codes || !meta || !expanded)
        return fail(CUBIC_EINVAL, "null operand");
    if (dtype != CUBIC_DTYPE_BF16 && dtype != CUBIC_DTYPE_F16) return fail(CUBIC_ENOTSUP, "dtype=%d", dtype);
    if (fmt < 0 || fmt > 2) return fail(CUBIC_ENOTSUP, "unknown metadata format %d", fmt);
    if (n <= 0 || k <= 0 || bits < 1 || bits > 8) return fail(CUBIC_EINVAL, "invalid geometry");
    if (group_in <= 0 || group_in % 32) return fail(CUBIC_ENOTSUP, "group_in=%d must be a multiple of 32", group_in);
    if (group_out <= 0 || n % group_out) return fail(CUBIC_EINVAL, "group_out must divide n");
    if (fmt != 0 && !part_of_row) return fail(CUBIC_EINVAL, "format %d needs part_of_row", fmt);
    if (fmt == 1 && (!g0 || !g1 || !g2)) return fail(CUBIC_EINVAL, "format 1 needs the partition globals");
    if (fmt != 1 && !m2) return fail(CUBIC_EINVAL, "format %d needs its third metadata tensor", fmt);
    const int64_t need = cubic_prepare_scratch_bytes(n, k, group_in);
    if (expanded_bytes < need) return fail(CUBIC_EWORKSPACE, "prepare scratch %lld < %lld", (long long)expanded_bytes, (long long)need);
    const int64_t groups_k = ceil_div(k, group_in);
    const int64_t groups = n * groups_k;
    char* p = (char*)expanded;
    float* scale = (float*)p;
    uint16_t* av = (uint16_t*)(p + align256(groups * 4));
    uint16_t* bv = (uint16_t*)(p + align256(groups * 4) + align256(groups * 2));
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = cubic::launch_expand_metadata(fmt, m0, m1, m2, g0, g1, g2, part_of_row, n,
                                                 groups_k, group_out, scale, av, bv, s);
    if (e != hipSuccess) return hip_status(e, "metadata expansion");
    e = cubic::launch_prepare(packed, scale, av, bv, n, k, bits, group_in, dtype == CUBIC_DTYPE_F16, codes, meta, s);
    return hip_status(e, "weight preparation");
}

int64_t cubic_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int bits) {
    if (m <= 0 || n <= 0 || k <= 0 || bits < 1 || bits > 8) return -1;
    return gemm_workspace_any_group(m, n, 1, k, bits);
}

int64_t cubic_gemm_group_workspace_bytes(int64_t m, int members, int64_t n, int64_t k, int bits) {
    if (m <= 0 || n <= 0 || k <= 0 || bits < 1 || bits > 8 || members < 1 ||
        members > cubic::kMaxGemmMembers)
        return -1;
    return gemm_workspace_any_group(m, n, members, k, bits);
}

int64_t cubic_gemm_grouped_workspace_bytes(int64_t m, int64_t n0, int64_t n1, int64_t k, int bits) {
    if (m <= 0 || n0 <= 0 || n1 <= 0 || k <= 0 || bits < 1 || bits > 8) return -1;
    if (n0 == n1) return gemm_workspace_any_group(m, n0, 2, k, bits);
    const int64_t w0 = gemm_workspace_any_group(m, n0, 1, k, bits), w1 = gemm_workspace_any_group(m, n1, 1, k, bits);
    return w0 > w1 ? w0 : w1;
}

int cubic_gemm(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
               int64_t m, int64_t n, int64_t k, int bits, int group_in, int dtype, void* y, int64_t ldy,
               void* workspace, int64_t workspace_bytes, void* stream) {
    void* ys[1] = {y};
    const int64_t ldys[1] = {ldy};
    return gemm_common(x, ldx, codes, meta, m, 1, n, k, bits, group_in, dtype, ys, ldys, workspace,
                       workspace_bytes, stream);
}

int cubic_gemm_group(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
                     int64_t m, int members, int64_t n, int64_t k, int bits, int group_in, int dtype,
                     void* const* ys, const int64_t* ldys, void* workspace,
                     int64_t workspace_bytes, void* stream) {
    if (!ys || !ldys) return fail(CUBIC_EINVAL, "null output table");
    return gemm_common(x, ldx, codes, meta, m, members, n, k, bits, group_in, dtype, ys, ldys, workspace,
                       workspace_bytes, stream);
}

int cubic_gemm_grouped(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
                       int64_t m, int64_t n0, int64_t n1, int64_t k, int bits, int group_in, int dtype,
                       void* y0, int64_t ldy0, void* y1, int64_t ldy1, void* workspace,
                       int64_t workspace_bytes, void* stream) {
    if (!y0 || !y1 || n0 <= 0 || n1 <= 0) return fail(CUBIC_EINVAL, "grouped gemm needs two members");
    if (n0 % 16) return fail(CUBIC_EINVAL, "grouped gemm needs n0 %% 16 == 0 (n0=%lld)", (long long)n0);
    if (n0 == n1) {
        void* ys[2] = {y0, y1};
        const int64_t ldys[2] = {ldy0, ldy1};
        return gemm_common(x, ldx, codes, meta, m, 2, n0, k, bits, group_in, dtype, ys, ldys, workspace,
                           workspace_bytes, stream);
    }
    // members of different widths have different K plans: one launch each, in
    // stream order, sharing the workspace (every launch leaves it zero)
    if (bits < 1 || bits > 8 || group_in <= 0 || group_in % 32 || k <= 0)
        return fail(CUBIC_ENOTSUP, "invalid grouped geometry");
    const int64_t off_c = prepared_code_words(n0 / 16, k, bits), off_m = prepared_meta_words(n0 / 16, k, bits, group_in);
    const int rc = cubic_gemm(x, ldx, codes, meta, m, n0, k, bits, group_in, dtype, y0, ldy0, workspace,
                              workspace_bytes, stream);
    if (rc != CUBIC_OK) return rc;
    return cubic_gemm(x, ldx, codes + off_c, meta + off_m, m, n1, k, bits, group_in, dtype, y1, ldy1,
                      workspace, workspace_bytes, stream);
}

int cubic_moe_route(const void* logits, int logits_fp16, const int32_t* row_activity,
                    const int32_t* active_rows, int rows, int experts, int top_k, float* top_logits,
                    int64_t* top_ids, int64_t* route_ids, void* route_weights, int weights_fp16,
                    void* stream) {
    if (!logits || !row_activity || !active_rows || !top_logits || !top_ids || !route_ids ||
        !route_weights)
        return fail(CUBIC_EINVAL, "null operand");
    if (rows < 1 || experts < 1 || experts > cubic::kMaxRouteExperts)
        return fail(CUBIC_ENOTSUP, "router needs 1 <= experts <= %d", cubic::kMaxRouteExperts);
    if (top_k < 1 || top_k > experts || top_k > cubic::kMaxRouteTopK)
        return fail(CUBIC_EINVAL, "router needs a valid top-k (1..min(experts, %d))", cubic::kMaxRouteTopK);
    cubic::MoERouteArgs a = {};
    a.logits = (const uint16_t*)logits;
    a.logits_fp16 = logits_fp16 != 0;
    a.row_activity = row_activity;
    a.active_rows = active_rows;
    a.rows = rows;
    a.experts = experts;
    a.top_k = top_k;
    a.top_logits = top_logits;
    a.top_ids = top_ids;
    a.route_ids = route_ids;
    a.route_weights = (uint16_t*)route_weights;
    a.weights_fp16 = weights_fp16 != 0;
    return hip_status(cubic::launch_moe_route(a, (hipStream_t)stream), "cubic_moe_route launch");
}

int cubic_moe_compact(const int64_t* route_ids, int routes, int first_expert, int experts,
                      int block_m, int32_t* counts, int32_t* starts, int32_t* block_starts,
                      int32_t* total_blocks, int32_t* row_map, void* stream) {
    if (!route_ids || !counts || !starts || !block_starts || !total_blocks || !row_map)
        return fail(CUBIC_EINVAL, "null operand");
    if (routes < 1 || first_expert < 0 || block_m < 1)
        return fail(CUBIC_EINVAL, "compaction needs routes >= 1, first_expert >= 0, block_m >= 1");
    if (experts < 1 || experts > cubic::kMaxCompactExperts)
        return fail(CUBIC_ENOTSUP, "compaction needs 1 <= experts <= %d", cubic::kMaxCompactExperts);
    cubic::MoECompactArgs a = {};
    a.route_ids = route_ids;
    a.routes = routes;
    a.first_expert = first_expert;
    a.experts = experts;
    a.block_m = block_m;
    a.counts = counts;
    a.starts = starts;
    a.block_starts = block_starts;
    a.total_blocks = total_blocks;
    a.row_map = row_map;
    return hip_status(cubic::launch_moe_compact(a, (hipStream_t)stream), "cubic_moe_compact launch");
}

int cubic_embedding(const void* ids, int id_bytes, int64_t tokens, int fmt, const void* packed,
                    const void* m0, const void* m1, const void* m2, const void* g0, const void* g1,
                    const void* g2, const int32_t* part_of_row, int64_t n, int64_t k, int bits,
                    int group_in, int group_out, void* out, int out_dtype, void* stream) {
    if (!ids || !packed || !m0 || !m1 || !out) return fail(CUBIC_EINVAL, "null operand");
    if (id_bytes != 4 && id_bytes != 8) return fail(CUBIC_EINVAL, "embedding ids must be int32 or int64");
    if (out_dtype != CUBIC_DTYPE_BF16 && out_dtype != CUBIC_DTYPE_F16)
        return fail(CUBIC_EINVAL, "embedding output must be bf16 or fp16");
    if (fmt < 0 || fmt > 2) return fail(CUBIC_ENOTSUP, "unknown metadata format %d", fmt);
    if (tokens <= 0 || tokens > 0x7fffffff) return fail(CUBIC_EINVAL, "embedding needs 1 <= tokens < 2^31");
    if (n <= 0 || k <= 0 || bits < 1 || bits > 8 || group_in <= 0) return fail(CUBIC_EINVAL, "invalid geometry");
    if (group_out <= 0 || n % group_out) return fail(CUBIC_EINVAL, "group_out must divide n");
    if (cubic::embedding_column_blocks(k) > 65535) return fail(CUBIC_ENOTSUP, "embedding width %lld too large", (long long)k);
    if (fmt != 0 && !part_of_row) return fail(CUBIC_EINVAL, "format %d needs part_of_row", fmt);
    if (fmt == 1 && (!g0 || !g1 || !g2)) return fail(CUBIC_EINVAL, "format 1 needs the partition globals");
    if (fmt != 1 && !m2) return fail(CUBIC_EINVAL, "format %d needs its third metadata tensor", fmt);
    cubic::EmbedArgs a = {};
    a.ids = ids;
    a.id_bytes = id_bytes;
    a.tokens = tokens;
    a.fmt = fmt;
    a.packed = (const uint8_t*)packed;
    a.m0 = m0; a.m1 = m1; a.m2 = m2;
    a.g0 = g0; a.g1 = g1; a.g2 = g2;
    a.part_of_row = part_of_row;
    a.n = n;
    a.k = k;
    a.row_bytes = ceil_div(k * bits, 8);
    a.groups_k = ceil_div(k, group_in);
    a.bits = bits;
    a.group_in = group_in;
    a.group_out = group_out;
    a.aligned = ((uintptr_t)packed % 4 == 0) && (a.row_bytes % 4 == 0);
    a.chunk_in_group = group_in % 16 == 0;
    a.lut = a.chunk_in_group && 4 * (1 << bits) <= group_in;
    a.out = (uint16_t*)out;
    a.out_fp16 = out_dtype == CUBIC_DTYPE_F16;
    return hip_status(cubic::launch_embedding(a, (hipStream_t)stream), "cubic_embedding launch");
}

// ---------------------------------------------------------------------------
// Routed experts (MoE)
// ---------------------------------------------------------------------------
int cubic_moe_pad_routes(const int32_t* counts, const int32_t* starts, const int32_t* block_starts,
                         const int32_t* total_blocks, const int32_t* row_map, int experts, int routes,
                         int block_m, int32_t* padded, int32_t* block_expert, int32_t* padded_total,
                         void* stream) {
    if (!counts || !starts || !block_starts || !total_blocks || !row_map || !padded || !block_expert ||
        !padded_total)
        return fail(CUBIC_EINVAL, "null operand");
    if (experts <= 0 || routes < 0 || (block_m != 16 && block_m != 32 && block_m != 64))
        return fail(CUBIC_EINVAL, "moe pad: experts=%d routes=%d block_m=%d", experts, routes, block_m);
    return hip_status(cubic::launch_pad_routes(counts, starts, block_starts, total_blocks, row_map, experts,
                                               routes, block_m, padded, block_expert, padded_total,
                                               (hipStream_t)stream),
                      "cubic_moe_pad_routes launch");
}

int64_t cubic_moe_max_blocks(int64_t routes, int experts, int block_m) {
    if (routes < 0 || experts <= 0 || block_m <= 0) return -1;
    const int64_t active = routes < experts ? routes : experts;  // experts holding a route
    return ceil_div(routes + active * (block_m - 1), block_m);
}

int cubic_moe_gemm(const void* x, int64_t ldx, const uint32_t* codes, const uint32_t* meta,
                   int64_t expert_code_words, int64_t expert_meta_words, const int32_t* padded,
                   const int32_t* block_expert, const int32_t* padded_total, int64_t max_blocks,
                   int block_m, int routes, int top_k, int64_t n, int64_t k, int bits, int group_in,
                   int dtype, void* y, int64_t ldy, void* stream) {
    if (!x || !codes || !meta || !padded || !block_expert || !padded_total || !y)
        return fail(CUBIC_EINVAL, "null operand");
    if (dtype != CUBIC_DTYPE_BF16 && dtype != CUBIC_DTYPE_F16) return fail(CUBIC_ENOTSUP, "dtype=%d", dtype);
    if (block_m != 16 && block_m != 32 && block_m != 64)
        return fail(CUBIC_ENOTSUP, "block_m=%d not in {16, 32, 64}", block_m);
    if (routes <= 0 || top_k <= 0 || routes % top_k || max_blocks <= 0 || max_blocks * block_m > (1 << 30) ||
        n <= 0 || k <= 0 || n > (1 << 30) || k > (1 << 30))
        return fail(CUBIC_EINVAL, "moe gemm extents: routes=%d top_k=%d blocks=%lld n=%lld k=%lld", routes,
                    top_k, (long long)max_blocks, (long long)n, (long long)k);
    if (bits < 1 || bits > 8) return fail(CUBIC_ENOTSUP, "bits=%d outside 1..8", bits);
    if (group_in <= 0 || group_in % 32) return fail(CUBIC_ENOTSUP, "group_in=%d must be a multiple of 32", group_in);
    if (k % 8 || ldx % 8 || ldx < k || !aligned16(x))
        return fail(CUBIC_ENOTSUP, "activations need k %% 8 == 0, ldx %% 8 == 0 and 16-byte alignment");
    if (ldy < n) return fail(CUBIC_EINVAL, "output leading dimension too small");
    int64_t cw = 0, mw = 0;
    cubic_prepared_words(n, k, bits, group_in, &cw, &mw);
    if (expert_code_words < cw || expert_meta_words < mw)
        return fail(CUBIC_EINVAL, "expert strides smaller than one prepared matrix");
    // no K split: routed launches have max_blocks x column blocks workgroups
    const GemmPlan p = plan_gemm(64, n, 1, k, bits, group_in);
    cubic::GemmArgs a = {};
    a.x = (const uint16_t*)x;
    a.codes = codes;
    a.meta = meta;
    a.ys[0] = (uint16_t*)y;
    a.ldx = ldx;
    a.ldys[0] = ldy;
    a.m = (int)(max_blocks * block_m);
    a.n = (int)n;
    a.k = (int)k;
    a.n_member = (int)n;
    a.bits = bits;
    a.group_in = group_in;
    a.k_blocks = p.k_blocks;
    a.groups_k = (int)ceil_div(k, group_in);
    a.split = 1;
    a.blocks_per_split = p.k_blocks;
    a.n_tiles = p.n_tiles;
    // two tiles per wave: half the workgroups of one-tile waves over the many
    // short route blocks (cfg4: gate/up 76 -> 71 us, down 60 -> 57 us)
    a.tiles_per_wave = 2;
    a.chunk_rows = block_m;
    a.f16 = dtype == CUBIC_DTYPE_F16;
    a.routed = 1;
    a.block_m = block_m;
    a.padded = padded;
    a.block_expert = block_expert;
    a.padded_total = padded_total;
    a.routes = routes;
    a.top_k = top_k;
    a.expert_code_stride = expert_code_words;
    a.expert_meta_stride = expert_meta_words;
    return hip_status(cubic::launch_gemm(a, (hipStream_t)stream), "cubic_moe_gemm launch");
}


// fp32 logits: [rows, tiles, 20] composite keys + [rows, tiles] finite flags
int64_t cand_f32_workspace(int rows, int width) {
    if (rows <= 0 || width <= 0) return -1;
    const int64_t tiles = ceil_div(width, cubic::kCandF32Tile);
    return align256((int64_t)rows * tiles * kTop * 8) + align256((int64_t)rows * tiles * 4);
}

int64_t cubic_candidates_workspace_bytes(int rows, int width) {
    // one size for every logits dtype: the larger of the two plans
    const int64_t a16 = accept_workspace(rows, rows, width), a32 = cand_f32_workspace(rows, width);
    return a16 > a32 ? a16 : a32;
}

int cubic_candidates(const void* logits, int dtype, int64_t row_stride, int rows, int width,
                     int64_t vocab_start, const float* temperatures, int owned_rows, const int32_t* owned_count,
                     const uint8_t* row_activity, int count, int capacity,
                     int all_random, void* scores, int64_t* ids, void* workspace,
                     int64_t workspace_bytes, void* stream) {
    if (!logits || !temperatures || !scores || !ids || !workspace) return fail(CUBIC_EINVAL, "null operand");
    if (dtype != CUBIC_DTYPE_BF16 && dtype != CUBIC_DTYPE_F16 && dtype != CUBIC_DTYPE_F32)
        return fail(CUBIC_EINVAL, "candidate logits dtype must be CUBIC_DTYPE_BF16, _F16 or _F32");
    if (vocab_start < 0) return fail(CUBIC_EINVAL, "negative vocabulary start");
    if (rows <= 0 || width <= 0 || row_stride < width) return fail(CUBIC_EINVAL, "invalid logits geometry");
    if (owned_rows < 0 || owned_rows > rows) return fail(CUBIC_EINVAL, "owned_rows outside 0..rows");
    if (count < 1 || count > kTop || capacity < count || capacity > 64)
        return fail(CUBIC_EINVAL, "need 1 <= count <= 20 and count <= capacity <= 64");
    if (dtype == CUBIC_DTYPE_F32) {
        const int64_t need = cand_f32_workspace(rows, width);
        if (workspace_bytes < need)
            return fail(CUBIC_EWORKSPACE, "candidate workspace %lld < %lld", (long long)workspace_bytes, (long long)need);
        const int64_t tiles = ceil_div(width, cubic::kCandF32Tile);
        cubic::CandF32Args f = {};
        f.logits = (const float*)logits;
        f.row_stride = row_stride;
        f.rows = rows;
        f.width = width;
        f.tiles = (int)tiles;
        f.vector_loads = aligned16(logits) && row_stride % 4 == 0;
        f.row_temperatures = temperatures;
        f.owned_rows = owned_rows;
        f.count = count;
        f.capacity = capacity;
        f.all_random = all_random;
        f.vocab_start = vocab_start;
        f.owned_count = owned_count;
        f.row_activity = row_activity;
        f.scores = (float*)scores;
        f.ids = ids;
        f.partial = (uint64_t*)workspace;
        f.partial_finite = (uint32_t*)((char*)workspace + align256((int64_t)rows * tiles * kTop * 8));
        return hip_status(cubic::launch_candidates_f32(f, (hipStream_t)stream), "cubic_candidates launch");
    }
    TilePlan t;
    if (!plan_tiles(rows, width, &t)) return fail(CUBIC_ENOTSUP, "vocabulary width %d too large", width);
    const int64_t need = accept_workspace(rows, rows, width);
    if (workspace_bytes < need) return fail(CUBIC_EWORKSPACE, "candidate workspace %lld < %lld", (long long)workspace_bytes, (long long)need);
    cubic::AcceptArgs a = {};
    a.logits = (const uint16_t*)logits;
    a.scores_fp16 = dtype == CUBIC_DTYPE_F16;
    a.row_stride = row_stride;
    a.rows = rows;
    a.width = width;
    a.tiles = t.tiles;
    a.tile_width = t.tile_width;
    a.vector_loads = aligned16(logits) && row_stride % 8 == 0;
    a.row_temperatures = temperatures;
    a.owned_rows = owned_rows;
    a.owned_count = owned_count;
    a.row_activity = row_activity;
    a.vocab_start = vocab_start;
    a.count = count;
    a.capacity = capacity;
    a.all_random = all_random;
    a.cand_scores = (uint16_t*)scores;
    a.cand_ids = ids;
    a.group_rows = 1;
    carve_accept(workspace, rows, rows, t.tiles, a);
    return hip_status(cubic::launch_accept(a, false, (hipStream_t)stream), "cubic_candidates launch");
}

int cubic_verify_candidates(const void* q_scores, const int64_t* q_ids, const void* p_scores,
                            const int64_t* p_ids, const int32_t* target_rows,
                            const int64_t* draft_tokens, const float* temperatures,
                            const float* top_ps, const int64_t* top_ks, const int64_t* seeds,
                            const int64_t* ordinals, const float* uniforms,
                            const uint8_t* constrained_rows, int allow_underfilled, int tp,
                            int q_rows, int p_rows, int k, int active_rows, int64_t* decisions,
                            void* stream) {
    if (!q_scores || !q_ids || !p_scores || !p_ids || !target_rows || !draft_tokens ||
        !temperatures || !top_ps || !top_ks || !seeds || !ordinals || !decisions)
        return fail(CUBIC_EINVAL, "null operand");
    if (tp < 1 || tp > 8 || k < 1 || k > 20) return fail(CUBIC_EINVAL, "speculative candidates require 1 <= tp <= 8, 1 <= k <= 20");
    if (q_rows < 1 || p_rows < 1 || active_rows < 1 || active_rows > q_rows)
        return fail(CUBIC_EINVAL, "speculative row buffers differ from proposal capacity");
    cubic::VerifyArgs a = {};
    a.q_scores = (const uint16_t*)q_scores;
    a.q_ids = q_ids;
    a.p_scores = (const uint16_t*)p_scores;
    a.p_ids = p_ids;
    a.target_rows = target_rows;
    a.draft_tokens = draft_tokens;
    a.temperatures = temperatures;
    a.top_ps = top_ps;
    a.top_ks = top_ks;
    a.seeds = seeds;
    a.ordinals = ordinals;
    a.uniforms = uniforms;
    a.constrained_rows = constrained_rows;
    a.decisions = decisions;
    a.tp = tp;
    a.q_rows = q_rows;
    a.p_rows = p_rows;
    a.k = k;
    a.block = next_pow2(tp * k);
    a.active_rows = active_rows;
    a.allow_underfilled = allow_underfilled;
    return hip_status(cubic::launch_verify(a, (hipStream_t)stream), "cubic_verify_candidates launch");
}

int cubic_root_sample(const void* scores, int scores_fp16, const int64_t* ids,
                      const float* temperatures, const float* top_ps, const int64_t* top_ks,
                      const int64_t* seeds, const int64_t* ordinals,
                      const uint8_t* constrained_rows, int allow_underfilled, int tp, int rows,
                      int k, int64_t* output_tokens, uint8_t* output_valid, void* stream) {
    if (!scores || !ids || !temperatures || !top_ps || !top_ks || !seeds || !ordinals ||
        !output_tokens || !output_valid)
        return fail(CUBIC_EINVAL, "null operand");
    if (tp < 1 || tp > 8 || k < 1 || k > 20)
        return fail(CUBIC_EINVAL, "scores must be [TP,C,K] with TP<=8 and K<=20");
    if (rows < 1) return fail(CUBIC_EINVAL, "root sampling needs at least one row");
    if (constrained_rows && !allow_underfilled)
        return fail(CUBIC_EINVAL, "invalid constrained-row ownership for root sampling");
    cubic::RootSampleArgs a = {};
    a.scores = (const uint16_t*)scores;
    a.scores_fp16 = scores_fp16 != 0;
    a.ids = ids;
    a.temperatures = temperatures;
    a.top_ps = top_ps;
    a.top_ks = top_ks;
    a.seeds = seeds;
    a.ordinals = ordinals;
    a.constrained_rows = constrained_rows;
    a.allow_underfilled = allow_underfilled != 0;
    a.tp = tp;
    a.rows = rows;
    a.k = k;
    a.block = next_pow2(tp * k);
    a.output_tokens = output_tokens;
    a.output_valid = output_valid;
    return hip_status(cubic::launch_root_sample(a, (hipStream_t)stream), "cubic_root_sample launch");
}

}  // extern "C"

namespace {

// ---------------------------------------------------------------------------
// Greedy sampler.  Workgroups of 256 threads stream tiles of whole
// 2048-column load rounds; a row splits into max(4, 256 / rows) tiles, at
// most 32 (and never more tiles than rounds).  Measured on the Qwen3-8B
// vocabulary (151936 columns) for 1..256 rows: fewer tiles leave a row's
// stream latency-bound inside one workgroup, more tiles add workgroups whose
// fixed cost (parameter loads, reduction, the hand-off to the row's last
// arrival) exceeds their share of the stream.
// ---------------------------------------------------------------------------
struct GreedyPlan {
    int tiles, tile_width;
};

constexpr int64_t kGreedyMaxWidth = int64_t(1) << 30;

GreedyPlan plan_greedy(int rows, int width) {
    const int64_t w = width > 0 ? width : 1;
    int64_t want = std::min<int64_t>(std::max<int64_t>(4, ceil_div(256, rows)), 32);
    want = std::min<int64_t>(want, ceil_div(w, kChunk));
    GreedyPlan g;
    g.tile_width = (int)(ceil_div(ceil_div(w, want), kChunk) * kChunk);
    g.tiles = (int)ceil_div(w, g.tile_width);
    return g;
}

int64_t greedy_workspace(int rows, int width) {
    const GreedyPlan g = plan_greedy(rows, width);
    const int64_t slots = (int64_t)rows * g.tiles;
    return align256((int64_t)(rows + 1) * 4) + align256(slots * 8) + align256(slots * 4);
}

bool greedy_params(const float* temperatures, const float* top_ps, const int64_t* top_ks,
                   const int64_t* seeds, const int64_t* ordinals, int k, int64_t vocab_size,
                   cubic::GreedyParams* p) {
    if (!temperatures || !top_ps || !top_ks || !seeds || !ordinals) return false;
    p->temperatures = temperatures;
    p->top_ps = top_ps;
    p->top_ks = top_ks;
    p->seeds = seeds;
    p->ordinals = ordinals;
    p->k = k;
    p->vocab_size = vocab_size;
    return true;
}

int greedy_pass(const void* logits, int logits_fp16, int64_t row_stride, int rows, int width,
                int64_t vocab_start, const int32_t* metadata, const uint32_t* token_mask,
                int64_t mask_words, void* masked_logits, int64_t masked_stride, int candidates,
                void* scores, int64_t* ids, void* workspace, int64_t workspace_bytes,
                cubic::GreedyArgs& a, const char* who) {
    if (!logits || !metadata || !scores || !ids || !workspace) return fail(CUBIC_EINVAL, "%s: null operand", who);
    if (rows < 1 || rows > 65535 || width < 0 || width > kGreedyMaxWidth || row_stride < width)
        return fail(CUBIC_EINVAL, "%s: invalid logits geometry", who);
    if (vocab_start < 0) return fail(CUBIC_EINVAL, "%s: negative vocabulary start", who);
    if (candidates < 1 || candidates > 64) return fail(CUBIC_EINVAL, "%s: need 1 <= candidates <= 64", who);
    if (token_mask && (mask_words < 1 || vocab_start + width > mask_words * 32))
        return fail(CUBIC_EINVAL, "%s: grammar mask rows do not cover the visible vocabulary", who);
    if (masked_logits && !token_mask)
        return fail(CUBIC_EINVAL, "%s: masked logits need a grammar mask", who);
    const bool inplace = masked_logits == logits;
    if (masked_logits && (masked_stride < width || (inplace && masked_stride != row_stride)))
        return fail(CUBIC_EINVAL, "%s: masked logits geometry (in place: the logits' own row stride)", who);
    const int64_t need = greedy_workspace(rows, width);
    if (workspace_bytes < need)
        return fail(CUBIC_EWORKSPACE, "%s: workspace %lld < %lld", who, (long long)workspace_bytes, (long long)need);
    const GreedyPlan g = plan_greedy(rows, width);
    a.logits = (const uint16_t*)logits;
    a.row_stride = row_stride;
    a.scores_fp16 = logits_fp16 != 0;
    a.rows = rows;
    a.width = width;
    a.vocab_start = vocab_start;
    a.metadata = metadata;
    a.token_mask = token_mask;
    a.mask_words = mask_words;
    a.masked = (uint16_t*)masked_logits;
    a.masked_stride = masked_stride;
    a.masked_inplace = masked_logits && inplace;
    a.candidates = candidates;
    a.scores = (uint16_t*)scores;
    a.ids = ids;
    a.tiles = g.tiles;
    a.tile_width = g.tile_width;
    a.vector_loads = aligned16(logits) && row_stride % 8 == 0;
    // counters first: their place depends on rows only, so one workspace
    // serves launches of the same rows at any width it was sized for
    const int64_t slots = (int64_t)rows * g.tiles;
    char* w = (char*)workspace;
    a.counters = (uint32_t*)w;
    w += align256((int64_t)(rows + 1) * 4);
    a.partial_keys = (uint64_t*)w;
    w += align256(slots * 8);
    a.partial_flags = (uint32_t*)w;
    return CUBIC_OK;
}

}  // namespace

extern "C" {

int64_t cubic_greedy_workspace_bytes(int rows, int width) {
    if (rows < 1 || rows > 65535 || width < 0 || width > kGreedyMaxWidth)
        return fail(CUBIC_EINVAL, "invalid greedy geometry");
    return greedy_workspace(rows, width);
}

int cubic_greedy_candidates(const void* logits, int logits_fp16, int64_t row_stride, int rows,
                            int width, int64_t vocab_start, const int32_t* metadata,
                            const uint32_t* token_mask, int64_t mask_words, void* masked_logits,
                            int64_t masked_stride, int candidates, void* scores, int64_t* ids,
                            void* workspace, int64_t workspace_bytes, void* stream) {
    cubic::GreedyArgs a = {};
    const int rc = greedy_pass(logits, logits_fp16, row_stride, rows, width, vocab_start, metadata,
                               token_mask, mask_words, masked_logits, masked_stride, candidates,
                               scores, ids, workspace, workspace_bytes, a, "cubic_greedy_candidates");
    if (rc != CUBIC_OK) return rc;
    return hip_status(cubic::launch_greedy(a, (hipStream_t)stream), "cubic_greedy_candidates launch");
}

int cubic_greedy_root(const void* scores, int scores_fp16, const int64_t* ids,
                      const float* temperatures, const float* top_ps, const int64_t* top_ks,
                      const int64_t* seeds, const int64_t* ordinals, const int32_t* metadata,
                      int tp, int rows, int k, int64_t vocab_size, int64_t* tokens, uint8_t* valid,
                      void* stream) {
    cubic::GreedyRootArgs a = {};
    if (!scores || !ids || !metadata || !tokens || !valid ||
        !greedy_params(temperatures, top_ps, top_ks, seeds, ordinals, k, vocab_size, &a.p))
        return fail(CUBIC_EINVAL, "null operand");
    if (tp < 1 || tp > 8 || k < 1 || k > 64 || rows < 1)
        return fail(CUBIC_EINVAL, "greedy root needs [TP,C,K] candidates with TP<=8, 1<=K<=64, C>=1");
    if (vocab_size < 1 || vocab_size > INT32_MAX) return fail(CUBIC_EINVAL, "vocabulary size outside 1..2^31-1");
    a.scores = (const uint16_t*)scores;
    a.scores_fp16 = scores_fp16 != 0;
    a.ids = ids;
    a.metadata = metadata;
    a.tp = tp;
    a.rows = rows;
    a.tokens = tokens;
    a.valid = valid;
    return hip_status(cubic::launch_greedy_root(a, (hipStream_t)stream), "cubic_greedy_root launch");
}

int cubic_sampling_final_guard(const int64_t* tokens, const uint8_t* root_valid,
                               const int32_t* metadata, const float* temperatures,
                               const float* top_ps, const int64_t* top_ks, const int64_t* seeds,
                               const int64_t* ordinals, int capacity, int k, int64_t vocab_size,
                               uint8_t* valid, void* stream) {
    cubic::GuardArgs a = {};
    if (!tokens || !metadata || !valid ||
        !greedy_params(temperatures, top_ps, top_ks, seeds, ordinals, k, vocab_size, &a.p))
        return fail(CUBIC_EINVAL, "null operand");
    if (capacity < 1 || k < 1) return fail(CUBIC_EINVAL, "final guard needs capacity >= 1 and K >= 1");
    a.tokens = tokens;
    a.root_valid = root_valid;
    a.metadata = metadata;
    a.capacity = capacity;
    a.valid = valid;
    return hip_status(cubic::launch_final_guard(a, (hipStream_t)stream), "cubic_sampling_final_guard launch");
}

int cubic_greedy_sample(const void* logits, int logits_fp16, int64_t row_stride, int rows,
                        int width, const int32_t* metadata, const uint32_t* token_mask,
                        int64_t mask_words, void* masked_logits, int64_t masked_stride, int k,
                        const float* temperatures, const float* top_ps,
                        const int64_t* top_ks, const int64_t* seeds, const int64_t* ordinals,
                        int64_t vocab_size, void* scores, int64_t* ids, int64_t* tokens,
                        uint8_t* root_valid, uint8_t* final_valid, void* workspace,
                        int64_t workspace_bytes, void* stream) {
    cubic::GreedyArgs a = {};
    if (!tokens || !root_valid || !final_valid ||
        !greedy_params(temperatures, top_ps, top_ks, seeds, ordinals, k, vocab_size, &a.p))
        return fail(CUBIC_EINVAL, "cubic_greedy_sample: null operand");
    if (vocab_size < 1 || vocab_size > INT32_MAX || width > vocab_size)
        return fail(CUBIC_EINVAL, "cubic_greedy_sample: visible width exceeds the vocabulary");
    if (rows > 65535) return fail(CUBIC_EINVAL, "cubic_greedy_sample: at most 65535 rows");
    const int rc = greedy_pass(logits, logits_fp16, row_stride, rows, width, 0, metadata, token_mask,
                               mask_words, masked_logits, masked_stride, k, scores, ids, workspace,
                               workspace_bytes, a, "cubic_greedy_sample");
    if (rc != CUBIC_OK) return rc;
    a.tokens = tokens;
    a.root_valid = root_valid;
    a.final_valid = final_valid;
    return hip_status(cubic::launch_greedy(a, (hipStream_t)stream), "cubic_greedy_sample launch");
}

int cubic_merge_prefix(const int64_t* decisions, int c, int depth, const int32_t* live,
                       int live_rows, int64_t* out, void* stream) {
    if (!decisions || !out) return fail(CUBIC_EINVAL, "null operand");
    if (c < 1 || depth < 1) return fail(CUBIC_EINVAL, "merge needs c >= 1 and depth >= 1");
    return hip_status(cubic::launch_merge_prefix(decisions, c, depth, live, live_rows, out,
                                                 (hipStream_t)stream), "cubic_merge_prefix launch");
}

int64_t cubic_accept_workspace_bytes(int c, int depth, int width) {
    if (c < 1 || depth < 1 || depth > 8) return -1;
    return accept_workspace(c * (depth + 1), c, width);
}

int cubic_accept(const void* logits, int64_t row_stride, int width, int c, int depth,
                 int live_rows, const int32_t* live_count, const float* row_temperatures,
                 const void* q_scores,
                 const int64_t* q_ids, int capacity, const int64_t* draft_tokens,
                 const float* temperatures, const float* top_ps, const int64_t* top_ks,
                 const int64_t* seeds, const int64_t* ordinals, const float* uniforms,
                 void* cand_scores, int64_t* cand_ids, int64_t* decisions, int64_t* merged,
                 int64_t* emitted, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!workspace) return fail(CUBIC_EINVAL, "null operand");
    return accept_common(logits, row_stride, width, c, depth, live_rows, live_count, row_temperatures, q_scores,
                         q_ids, capacity, draft_tokens, temperatures, top_ps, top_ks, seeds, ordinals,
                         uniforms, cand_scores, cand_ids, decisions, merged, emitted, workspace,
                         workspace_bytes, stream);
}

int cubic_accept_noalloc(const void* logits, int64_t row_stride, int width, int c, int depth,
                         int live_rows, const int32_t* live_count, const float* row_temperatures,
                  const void* q_scores,
                         const int64_t* q_ids, int capacity, const int64_t* draft_tokens,
                         const float* temperatures, const float* top_ps, const int64_t* top_ks,
                         const int64_t* seeds, const int64_t* ordinals, const float* uniforms,
                         void* cand_scores, int64_t* cand_ids, int64_t* decisions, int64_t* merged,
                         int64_t* emitted, void* stream) {
    if (c >= 1 && depth >= 1 && depth <= 8) {
        const int64_t need = accept_workspace(c * (depth + 1), c, width);
        if (need > kAcceptScratchBytes)
            return fail(CUBIC_EWORKSPACE, "accept scratch needs %lld bytes; the static scratch holds %lld",
                        (long long)need, (long long)kAcceptScratchBytes);
    }
    void* scratch_ptr = nullptr;
    const int rc = accept_scratch(&scratch_ptr);
    if (rc != CUBIC_OK) return rc;
    return accept_common(logits, row_stride, width, c, depth, live_rows, live_count, row_temperatures, q_scores,
                         q_ids, capacity, draft_tokens, temperatures, top_ps, top_ks, seeds, ordinals,
                         uniforms, cand_scores, cand_ids, decisions, merged, emitted, scratch_ptr,
                         kAcceptScratchBytes, stream);
}

}  // extern "C"

namespace {

int accept_common(const void* logits, int64_t row_stride, int width, int c, int depth,
                  int live_rows, const int32_t* live_count, const float* row_temperatures,
                  const void* q_scores,
                  const int64_t* q_ids, int capacity, const int64_t* draft_tokens,
                  const float* temperatures, const float* top_ps, const int64_t* top_ks,
                  const int64_t* seeds, const int64_t* ordinals, const float* uniforms,
                  void* cand_scores, int64_t* cand_ids, int64_t* decisions, int64_t* merged,
                  int64_t* emitted, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!logits || !row_temperatures || !q_scores || !q_ids || !draft_tokens || !temperatures ||
        !top_ps || !top_ks || !seeds || !ordinals || !cand_scores || !cand_ids || !decisions ||
        !merged || !workspace)
        return fail(CUBIC_EINVAL, "null operand");
    if (c < 1 || depth < 1 || depth > 8) return fail(CUBIC_EINVAL, "need c >= 1 and 1 <= depth <= 8");
    if (live_rows < 0 || live_rows > c) return fail(CUBIC_EINVAL, "live_rows outside 0..c");
    if (capacity < 1 || capacity > kTop) return fail(CUBIC_EINVAL, "capacity must be 1..20");
    if (width <= 0 || row_stride < width) return fail(CUBIC_EINVAL, "invalid logits geometry");
    const int rows = c * (depth + 1);
    TilePlan t;
    if (!plan_tiles(rows, width, &t)) return fail(CUBIC_ENOTSUP, "vocabulary width %d too large", width);
    const int64_t need = accept_workspace(rows, c, width);
    if (workspace_bytes < need) return fail(CUBIC_EWORKSPACE, "accept workspace %lld < %lld", (long long)workspace_bytes, (long long)need);
    cubic::AcceptArgs a = {};
    a.logits = (const uint16_t*)logits;
    a.row_stride = row_stride;
    a.rows = rows;
    a.width = width;
    a.tiles = t.tiles;
    a.tile_width = t.tile_width;
    a.vector_loads = aligned16(logits) && row_stride % 8 == 0;
    a.row_temperatures = row_temperatures;
    a.owned_rows = live_rows * (depth + 1);
    a.count = capacity;
    a.capacity = capacity;
    a.all_random = 0;
    a.cand_scores = (uint16_t*)cand_scores;
    a.cand_ids = cand_ids;
    a.group_rows = depth + 1;
    a.c = c;
    a.live_rows = live_rows;
    a.live_count = live_count;
    a.block = next_pow2(capacity);
    a.q_scores = (const uint16_t*)q_scores;
    a.q_ids = q_ids;
    a.draft_tokens = draft_tokens;
    a.temperatures = temperatures;
    a.top_ps = top_ps;
    a.top_ks = top_ks;
    a.seeds = seeds;
    a.ordinals = ordinals;
    a.uniforms = uniforms;
    a.decisions = decisions;
    a.merged = merged;
    a.emitted = emitted;
    carve_accept(workspace, rows, c, t.tiles, a);
    return hip_status(cubic::launch_accept(a, true, (hipStream_t)stream), "cubic_accept launch");
}

}  // namespace
