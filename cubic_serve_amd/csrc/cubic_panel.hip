// Column-panel Cubic GEMM for gfx950 (M <= 64, bits <= 4, whole-k-block
// groups): the verify-shape path of y[M,N] = x[M,K] . decode(W)[N,K]^T.
//
// Reference semantics (paths under src/cubic_serve/ of QuantTrio/cubic-serve):
//   decode       quantization/extensions/cubic/reference.py:98-121
//   WNA16 linear ops/eager/quantization.py:181-186, ops/eager/linear.py:43-56
//   dispatch     quantization/extensions/cubic/marlin.py:377-521 (Marlin + merge)
#include <type_traits>

#include "cubic_gemm_common.h"

namespace cubic {
#ifdef CUBIC_TIMELINE
__device__ unsigned long long* g_tl;
extern "C" __attribute__((visibility("default"))) int cubic_exp_set_timeline(void* p) {
    return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_tl), &p, sizeof(p));
}
#define TL_STAMP(slot) do { if (tlw && threadIdx.x == 0) tlw[slot] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define TL_STAMP(slot) do { } while (0)
#endif
namespace {
using namespace gemm;

// ---------------------------------------------------------------------------
// Column-panel GEMM (M <= 64, bits <= 4, whole-k-block groups)
//   grid.x: column panels of kGemmWaves waves x J tiles x 16 columns
//   grid.y: K partitions (split)
// Each tile sees exactly gemm_kernel's arithmetic: the same MFMA per
// (m-tile, tile, k-block, fragment) in the same order, the same zero-padded
// k-block pairs, the same split-K exchange and ascending partition sum, so
// the two kernels' outputs are bit-identical under one K plan.
//
// What differs is how the loads are kept in flight.  Under load an HBM read
// takes ~1.4 us to return, and a wave's reads return in issue order, so an
// activation read that hits L2 still waits behind the code reads issued
// before it.  Every stream is therefore issued S k-blocks ahead of its use:
//   * activations go global -> LDS by buffer DMA (no registers held) into a
//     ring of S stages laid out in the MFMA A-fragment swizzle;
//   * with TL (4 bits) the panel's level tables go the same way, one 16-byte
//     record per column instead of four lane copies;
//   * codes (and without TL each lane's table) fill an S-deep register ring.
// One issue group per k-block -- MT activation DMAs, the table DMA, then the
// code loads -- in a fixed order, so one counted `s_waitcnt vmcnt` before the
// iteration's barrier proves the whole group of the k-block about to be used
// has landed, while the S - 2 younger groups stay in flight.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
// f(integral_constant<I>) for I = B .. E - 1, unrolled at compile time
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}
// s_waitcnt immediate that waits for vmcnt <= n and leaves the other counters
// alone (gfx9 layout: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at
// [15:14]).  Issued through the builtin rather than inline assembly, the
// compiler's own wait insertion knows which loads it has retired.
constexpr int vmcnt_only(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }
template <int BITS, int MT, int J, bool TL, int S, int WV, bool F16>
__global__ __launch_bounds__(WV * 64) void panel_kernel(GemmArgs a) {
    static_assert(BITS <= 4, "level-table decode only");
    static_assert(!TL || BITS == 4, "table DMA moves 16-byte records (4-bit tables)");
    static_assert(S == 2 || S == 4, "ring depth");
    constexpr int W = BITS;
    constexpr int MW = meta_words<BITS>();
    constexpr int kAStage = a_stage<MT>();                // bf16 per activation stage
    constexpr int kAStageBytes = kAStage * 2;
    constexpr int kTblStageBytes = WV * J * 256;          // WV J tiles x 16 columns x 16 B
    // activation DMA instructions per wave (a stage is 4 MT KiB); with more
    // waves than instructions the extra waves repeat one (same bytes, same place)
    constexpr int kXInstr = 4 * MT / WV > 0 ? 4 * MT / WV : 1;
    // table DMA instructions per panel (1 KiB each); wave w issues w % kTInstr
    constexpr int kTInstr = WV * J / 4 > 0 ? WV * J / 4 : 1;
    static_assert(WV * J % 4 == 0 || WV * J < 4, "table records fill whole DMA instructions");
    constexpr int kTileBytes = 16 * MT * tile_pitch<J, WV>() * 2;
    // Every ring stage is its own LDS object: the compiler then knows that a
    // DMA into one stage cannot touch the LDS reads of another and issues no
    // drain for it (with one array it waits for the newest DMA before every
    // fragment read).  Stage 0 also holds the epilogue's output tile.
    constexpr int kStage0 = kAStageBytes > kTileBytes ? kAStageBytes : kTileBytes;
    constexpr int kTblBytes = TL ? kTblStageBytes : 16;
    __shared__ __attribute__((aligned(1024))) uint8_t xs0[kStage0];
    __shared__ __attribute__((aligned(1024))) uint8_t xs1[kAStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t xs2[S == 4 ? kAStageBytes : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t xs3[S == 4 ? kAStageBytes : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t ts0[kTblBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t ts1[kTblBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t ts2[S == 4 ? kTblBytes : 16];
    __shared__ __attribute__((aligned(1024))) uint8_t ts3[S == 4 ? kTblBytes : 16];
    auto x_stage = [&](int slot) -> uint8_t* { return slot == 0 ? xs0 : slot == 1 ? xs1 : slot == 2 ? xs2 : xs3; };
    auto t_stage = [&](int slot) -> uint8_t* { return slot == 0 ? ts0 : slot == 1 ? ts1 : slot == 2 ? ts2 : ts3; };
    // target of the DMAs that fetch nothing (never read)
    __shared__ __attribute__((aligned(1024))) uint8_t dummy[1024];
    // VMEM instructions per issue group (the counted wait below relies on it)
    constexpr int kActOps = kXInstr;
    constexpr int kCodeOps = J;
    constexpr int kGroupOps = kActOps + (TL ? 1 : J) + kCodeOps;

    // wave and lane as plain functions of threadIdx.x: their value ranges let
    // the compiler prove that the DMA into one stage never overlaps the LDS
    // reads of another (otherwise it drains the DMA before every read)
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int q = lane >> 4, col = lane & 15;
    const int panel_tile0 = blockIdx.x * WV * J;
    const int tile0 = panel_tile0 + wave * J;
    const int kb_begin = blockIdx.y * a.blocks_per_split;
    const int kb_end = min(kb_begin + a.blocks_per_split, a.k_blocks);
    // whole pairs of k-blocks, the second of an odd partition zero (as
    // gemm_kernel)
    const int n_iter = (kb_end - kb_begin + 1) & ~1;
    const int gpk = a.group_in / kKBlock;  // k-blocks per metadata group
#ifdef CUBIC_TIMELINE
    unsigned long long* tlw = g_tl ? g_tl + 64 * (blockIdx.y * gridDim.x + blockIdx.x) : nullptr;
    TL_STAMP(0);
    if (tlw && threadIdx.x == 0) {
        tlw[1] = ((unsigned long long)__builtin_amdgcn_s_getreg((31 << 11) | 20) << 32) |
                 __builtin_amdgcn_s_getreg((31 << 11) | 4);
        tlw[62] = n_iter;
    }
#endif

    floatx4_t acc[MT][J];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[mt][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // --- activation DMA: instruction p of wave w fills the 64 consecutive
    // 16-byte slots g * 64 + lane of a stage, g = w kXInstr + p; a stage holds
    // 16-row blocks, row r16 of a block in slots r16 * 16 + (c ^ r16) for its
    // 16-byte chunks c, so one instruction reads four whole 256-byte rows of
    // the k-block and the fragment reads (16 lanes: 16 rows, one chunk) hit
    // 16 distinct bank groups.  Rows past M read row M - 1 (outputs
    // discarded); chunks past K or past the partition, and instructions past
    // the stage (more waves than instructions) read an offset past the
    // buffer's extent, which the hardware returns as zero without a fetch;
    // the latter land in a dummy LDS block.
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x), 0, (int)((int64_t)a.m * a.ldx * 2), 0x00020000);
    constexpr uint32_t kOut = 0x80000000u;
    uint32_t x_off[kXInstr];
    int x_k8[kXInstr];
    int x_g[kXInstr];
#pragma unroll
    for (int p = 0; p < kXInstr; ++p) {
        const int g = wave * kXInstr + p;
        const bool real = g < 4 * MT;
        x_g[p] = real ? g : -1;
        const int s = (real ? g : 0) * 64 + lane;
        const int mt = s >> 8, r16 = (s >> 4) & 15, c = (s & 15) ^ r16;
        const int row = min(mt * 16 + r16, a.m - 1);
        x_off[p] = (uint32_t)((int64_t)row * a.ldx * 2) + 16u * c;
        x_k8[p] = real ? 8 * c : 1 << 30;  // a dummy instruction is never live
    }
    // --- table DMA (TL): wave w < kTInstr fills the panel's table slots
    // 64 w + lane (tile slot / 16, column slot % 16); the other waves issue an
    // out-of-extent DMA into the dummy block, so every wave issues the same
    // group shape without fetching duplicates
    __amdgpu_buffer_rsrc_t mr;
    uint32_t t_off = 0;
    if constexpr (TL) {
        mr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(a.meta), 0,
                                               (int)((int64_t)a.n_tiles * a.groups_k * 16 * MW * 4), 0x00020000);
        const int s = (wave % kTInstr) * 64 + lane;
        const int nt = min(panel_tile0 + (s >> 4), a.n_tiles - 1);
        t_off = (uint32_t)(((int64_t)nt * a.groups_k * 16 + (s & 15)) * (MW * 4));
        if (wave >= kTInstr) t_off = kOut;
    }
    // --- codes (and, without TL, each lane's table): S-deep register ring
    const uint32_t* code_base[J];
    const uint32_t* meta_base[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int nt = min(tile0 + j, a.n_tiles - 1);
        code_base[j] = a.codes + ((int64_t)nt * a.k_blocks * kWave + lane) * W;
        meta_base[j] = a.meta + ((int64_t)nt * a.groups_k * 16 + col) * MW;
    }
    uint32_t ring_codes[S][J][W];
    uint32_t ring_meta[S][J][TL ? 1 : MW];

    // one issue group: k-block kb into ring slot / LDS stage `slot`
    // a chunk is live when it lies inside K and inside the partition: one
    // per-lane compare (kb < kb_end <=> kb * 128 + k8 < kb_end * 128 for k8 < 128)
    const int k_live = min(a.k, kb_end * kKBlock);
    // the table DMA's wave condition as a scalar (a plain threadIdx-derived
    // compare would become an exec-masked branch around the DMA)
    const bool tbl_wave = __builtin_amdgcn_readfirstlane(wave) < kTInstr;
    auto issue = [&](int kb, int slot) {
        const int kbc = min(kb, kb_end - 1);
        __attribute__((address_space(3))) uint8_t* xs = (__attribute__((address_space(3))) uint8_t*)(void*)x_stage(slot);
#pragma unroll
        for (int p = 0; p < kActOps; ++p) {
            const uint32_t off = kb * kKBlock + x_k8[p] < k_live ? x_off[p] + (uint32_t)kb * 256u : kOut;
            lds_void_t* dst = x_g[p] >= 0 ? (lds_void_t*)(xs + x_g[p] * 1024) : (lds_void_t*)(void*)dummy;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, dst, 16, off, 0, 0, 0);
        }
        if constexpr (TL) {
            lds_void_t* ts = tbl_wave ? (lds_void_t*)((__attribute__((address_space(3))) uint8_t*)(void*)t_stage(slot) +
                                                      wave * 1024)
                                      : (lds_void_t*)(void*)dummy;
            const uint32_t toff = tbl_wave ? t_off + (uint32_t)((kbc / gpk) * 16 * MW * 4) : kOut;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(mr, ts, 16, toff, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < J; ++j) {
            load_words<W>(code_base[j] + kbc * (kWave * W), ring_codes[slot][j]);
            if constexpr (!TL) {
                const uint32_t* mp = meta_base[j] + (kbc / gpk) * (16 * MW);
                if constexpr (MW == 4) {
                    const uint4 mv = *reinterpret_cast<const uint4*>(mp);
                    ring_meta[slot][j][0] = mv.x; ring_meta[slot][j][1] = mv.y;
                    ring_meta[slot][j][2] = mv.z; ring_meta[slot][j][3] = mv.w;
                } else {
                    const uint2 mv = *reinterpret_cast<const uint2*>(mp);
                    ring_meta[slot][j][0] = mv.x; ring_meta[slot][j][1] = mv.y;
                }
            }
        }
    };

    // prologue: groups for the first S - 1 k-blocks
#pragma unroll
    for (int v = 0; v < S - 1; ++v) issue(kb_begin + v, v);
    __builtin_amdgcn_sched_barrier(0);
    TL_STAMP(2);

    // one k-block: `st` is its ring stage (compile time), `it` its index
    auto iteration = [&](auto st_c, int it) {
            constexpr int st = decltype(st_c)::value;
            const int kb = kb_begin + it;
            // this wave's group for k-block kb has landed (the S - 2 younger
            // groups may still be in flight); after the barrier every wave's
            // has, and every wave is done with k-block kb - 1's stage
            __builtin_amdgcn_s_waitcnt(vmcnt_only((S - 2) * kGroupOps));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            if (it < 19) TL_STAMP(3 + 3 * it);
            // the group for k-block kb + S - 1 goes into the stage and ring
            // slot that the barrier just freed, ahead of this block's math
            issue(kb + S - 1, (st + S - 1) % S);
            __builtin_amdgcn_sched_barrier(0);
            if (it < 19) TL_STAMP(4 + 3 * it);

            const uint16_t* lds = reinterpret_cast<const uint16_t*>(x_stage(st));
            LevelTable tab[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                uint32_t m4[4] = {0u, 0u, 0u, 0u};
                if constexpr (TL) {
                    const uint4 v = *reinterpret_cast<const uint4*>(t_stage(st) + ((wave * J + j) * 16 + col) * 16);
                    m4[0] = v.x; m4[1] = v.y; m4[2] = v.z; m4[3] = v.w;
                } else {
#pragma unroll
                    for (int w = 0; w < MW; ++w) m4[w] = ring_meta[st][j][w];
                }
                tab[j].lo_lo = m4[0];
                tab[j].hi_lo = m4[1];
                tab[j].lo_hi = MW == 4 ? m4[2] : 0u;
                tab[j].hi_hi = MW == 4 ? m4[3] : 0u;
            }
            auto afrag_at = [&](int mt, int f) {
                return *reinterpret_cast<const uint4*>(&lds[(mt * 256 + col * 16 + ((4 * q + f) ^ col)) * 8]);
            };
            __builtin_amdgcn_s_setprio(1);
            uint4 afrag[2][MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) afrag[0][mt] = afrag_at(mt, 0);
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                if (f + 1 < 4) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) afrag[(f + 1) & 1][mt] = afrag_at(mt, f + 1);
                }
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const uint4 bw = decode_fragment<BITS>(ring_codes[st][j], f, tab[j]);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][j] = mfma16<F16>(afrag[f & 1][mt], bw, acc[mt][j]);
                }
            }
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            if (it < 19) TL_STAMP(5 + 3 * it);
    };
    // whole rounds of S k-blocks, then (S = 4, an even count that is not a
    // multiple of 4) the last two.  The tail stays outside the loop: a
    // conditional exit inside the round makes the compiler drain every load
    // at the loop head, the S - 2 groups in flight included.
    const int whole = n_iter - n_iter % S;
    for (int i0 = 0; i0 < whole; i0 += S)
        static_for<0, S>([&](auto st_c) { iteration(st_c, i0 + decltype(st_c)::value); });
    if constexpr (S == 4) {
        if (whole < n_iter) {
            iteration(std::integral_constant<int, 0>{}, whole);
            iteration(std::integral_constant<int, 1>{}, whole + 1);
        }
    }
    TL_STAMP(60);
    // the last groups (k-blocks past the partition) may still be landing in
    // the stages that the output tile reuses
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

    // --- epilogue: the stages hold the block's output tile ------------------
    finish_block<J, MT, F16, WV>(a, acc, reinterpret_cast<uint16_t*>(xs0), 0, wave, lane);
    TL_STAMP(61);
}

template <int BITS, int MT, int J, int S, int WV, bool F16>
hipError_t launch_panel_tl(const GemmArgs& a, dim3 grid, hipStream_t s) {
    if constexpr (BITS == 4) {
        if (a.panel == 2) {
            panel_kernel<BITS, MT, J, true, S, WV, F16><<<grid, WV * 64, 0, s>>>(a);
            return hipGetLastError();
        }
    }
    panel_kernel<BITS, MT, J, false, S, WV, F16><<<grid, WV * 64, 0, s>>>(a);
    return hipGetLastError();
}
template <int BITS, int MT, int J, int S, bool F16>
hipError_t launch_panel_w(const GemmArgs& a, dim3 grid, hipStream_t s) {
#ifdef CUBIC_EXPERIMENTS
    if (a.panel_waves == 8) return launch_panel_tl<BITS, MT, J, S, 8, F16>(a, grid, s);
#endif
    if (a.panel_waves != kGemmWaves) return hipErrorInvalidValue;
    return launch_panel_tl<BITS, MT, J, S, kGemmWaves, F16>(a, grid, s);
}
template <int BITS, int MT, int J, bool F16>
hipError_t launch_panel_s(const GemmArgs& a, dim3 grid, hipStream_t s) {
    if (a.panel_stages == 4) return launch_panel_w<BITS, MT, J, 4, F16>(a, grid, s);
    return launch_panel_w<BITS, MT, J, 2, F16>(a, grid, s);
}
template <int BITS, int MT, bool F16>
hipError_t launch_panel_j(const GemmArgs& a, dim3 grid, hipStream_t s) {
    switch (a.tiles_per_wave) {
        case 1: return launch_panel_s<BITS, MT, 1, F16>(a, grid, s);
        case 2: return launch_panel_s<BITS, MT, 2, F16>(a, grid, s);
#ifdef CUBIC_EXPERIMENTS
        case 3: return launch_panel_s<BITS, MT, 3, F16>(a, grid, s);
        case 4: return launch_panel_s<BITS, MT, 4, F16>(a, grid, s);
#endif
        default: return hipErrorInvalidValue;
    }
}
template <int BITS, bool F16>
hipError_t launch_panel_mt(const GemmArgs& a, dim3 grid, hipStream_t s) {
    if (a.m >= 33) return launch_panel_j<BITS, 4, F16>(a, grid, s);
    if (a.m >= 17) return launch_panel_j<BITS, 2, F16>(a, grid, s);
    return launch_panel_j<BITS, 1, F16>(a, grid, s);
}
template <int BITS>
hipError_t launch_panel_bits(const GemmArgs& a, hipStream_t s) {
    const int cols = a.panel_waves * a.tiles_per_wave * 16;
    dim3 grid((a.n + cols - 1) / cols, a.split, 1);
    return a.f16 ? launch_panel_mt<BITS, true>(a, grid, s) : launch_panel_mt<BITS, false>(a, grid, s);
}
}  // namespace

hipError_t launch_panel_gemm(const GemmArgs& a, hipStream_t s) {
#ifdef CUBIC_EXP_FAST
    if (a.bits != 4 || a.f16 || a.m < 33) return hipErrorInvalidValue;
    const int cols = a.panel_waves * a.tiles_per_wave * 16;
    return launch_panel_j<4, 4, false>(a, dim3((a.n + cols - 1) / cols, a.split, 1), s);
#endif
    switch (a.bits) {
        case 1: return launch_panel_bits<1>(a, s);
        case 2: return launch_panel_bits<2>(a, s);
        case 3: return launch_panel_bits<3>(a, s);
        case 4: return launch_panel_bits<4>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace cubic
