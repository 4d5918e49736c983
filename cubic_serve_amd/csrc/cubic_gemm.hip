// Cubic weight-only GEMM for gfx950: y[M,N] = x[M,K] . decode(W)[N,K]^T
//
// Reference semantics (paths under src/cubic_serve/ of QuantTrio/cubic-serve):
//   decode       quantization/extensions/cubic/reference.py:98-121
//   WNA16 linear ops/eager/quantization.py:181-186, ops/eager/linear.py:43-56
//   dispatch     quantization/extensions/cubic/marlin.py:377-521 (Marlin + merge)
//
// Prepared layout (built once per weight by prepare_kernel):
//   codes  uint32 [n_tiles][k_blocks][64 lanes][W]   (W = bits words)
//   meta   uint32 [n_tiles][groups_k][16 columns][2]  (scale f32, a f16 | b f16 << 16)
// A 16-column x 128-k block is one MFMA B-operand stream: lane l owns column
// l % 16 and the 32 consecutive k of quarter l / 16, split into four 8-k
// fragments (one v_mfma_f32_16x16x32_bf16 each).  Codes are stored in
// sign-magnitude form laid out so that decode is a v_perm_b32 lookup into a
// per-group table of bf16 levels (bits <= 4), or a direct evaluation of the
// curve (bits >= 5).  Activations are staged per k-block through LDS with the
// same k order, so the MFMA contraction pairs every weight with its input.
//
// Every decoded weight equals bf16(decode_cubic(...)) bit for bit: levels are
// evaluated in the reference's unfused binary32 order and rounded once.
// FP32 accumulation runs in MFMA; K partitions (fixed by N, K and the number
// of 64-row chunks) are summed in ascending order by the last workgroup of
// each output block.
#include "cubic_gemm_common.h"


namespace cubic {
namespace {
using namespace gemm;
// OCC3: registers capped for three resident workgroups per CU (the wide
// single-split launches: lm_head-sized N with J = 2, MT = 4; the cap only
// spills in the split-K exchange, which those launches do not run).
template <int BITS, int MT, int J, bool G128, bool OCC3, bool F16>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(OCC3 ? 3 : 1)))
void gemm_kernel(GemmArgs a) {
    constexpr int W = BITS;  // code words per lane per (tile, k-block)
    // Code/metadata prefetch depth (k-blocks) and activation register stages.
    // Deeper rings (S = 4, NA up to 4) measured equal on every cfg2 shape: the
    // loop is not bound by load latency.
    constexpr int S = 2, NA = 1;
    constexpr int kAStage = a_stage<MT>();
    __shared__ __attribute__((aligned(16))) uint16_t a_lds[2][kAStage];
    __shared__ float t_lds[128];
    // bits 5..7, G128: per wave, the bf16 levels of its J x 16 columns for the
    // current k-block's group (wave-private, rebuilt every k-block)
    constexpr bool LT = G128 && BITS >= 5 && BITS <= 7;
    constexpr int NM = 1 << (BITS - 1);
    // rows padded by 4 levels (8 bytes): 16 columns' rows start on 16 distinct
    // bank groups instead of 4, and stay 8-byte aligned for the pair writes
    constexpr int NMP = NM + 4;
    __shared__ __attribute__((aligned(16))) uint16_t lv_lds[LT ? kGemmWaves * J * 16 * NMP : 1];

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int q = lane >> 4, col = lane & 15;
    const int tile0 = (blockIdx.x * kGemmWaves + wave) * J;
    const int split = blockIdx.y;
    const int m0 = blockIdx.z * a.chunk_rows;
    // routed: this chunk's expert, or nothing to do past the routed blocks
    int expert = 0;
    if (a.routed) {
        if (m0 >= *a.padded_total) return;  // uniform: before any barrier
        expert = a.block_expert[blockIdx.z];
    }
    // source row of local row r (rows past M / padding slots read a valid row;
    // their outputs are discarded)
    auto src_row = [&](int r) -> int64_t {
        if (a.routed) {
            const int route = a.padded[m0 + r];
            return route < a.routes ? route / a.top_k : 0;
        }
        return min(m0 + r, a.m - 1);
    };
    const int kb_begin = split * a.blocks_per_split;
    const int kb_end = min(kb_begin + a.blocks_per_split, a.k_blocks);

    if constexpr (BITS >= 5) {
        for (int i = threadIdx.x; i < (1 << (BITS - 1)); i += kGemmThreads)
            t_lds[i] = (float)((double)i / (double)((1 << (BITS - 1)) - 1));
        __syncthreads();
    }

    floatx4_t acc[MT][J];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[mt][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // --- code/metadata ring: stage s holds k-block kb with kb % S == s -------
    // Loads are unconditional: a tile past N or a k-block past this split reads
    // a clamped in-bounds address and its result is never consumed or stored.
    const uint32_t* code_base[J];
    const uint32_t* meta_base[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int nt = min(tile0 + j, a.n_tiles - 1);
        code_base[j] = a.codes + expert * a.expert_code_stride + ((int64_t)nt * a.k_blocks * kWave + lane) * W;
        meta_base[j] = a.meta + expert * a.expert_meta_stride +
                       ((int64_t)nt * a.groups_k * 16 + col) * meta_words<BITS>();
    }
    const int gq = G128 ? 0 : 32 * q;  // G128: group_in is a multiple of 128
    uint32_t ring_codes[S][J][W];
    constexpr int MW = meta_words<BITS>();
    uint32_t ring_meta[S][J][MW];
    auto load_codes = [&](int kb, uint32_t (&codes)[J][W], uint32_t (&meta)[J][MW]) {
        kb = min(kb, kb_end - 1);
        // quarters past K (group_in < 128 with a K tail) would index one group
        // past the last; their codes are zero padding against zero
        // activations, so any in-bounds table serves
        const int g = min((kb * kKBlock + gq) / a.group_in, a.groups_k - 1);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            load_words<W>(code_base[j] + kb * (kWave * W), codes[j]);
            const uint32_t* mp = meta_base[j] + g * (16 * MW);
            if constexpr (MW == 4) {
                const uint4 mv = *reinterpret_cast<const uint4*>(mp);
                meta[j][0] = mv.x; meta[j][1] = mv.y; meta[j][2] = mv.z; meta[j][3] = mv.w;
            } else {
                const uint2 mv = *reinterpret_cast<const uint2*>(mp);
                meta[j][0] = mv.x; meta[j][1] = mv.y;
            }
        }
    };
    // activations: 16 * MT rows x 128 k, chunks of 8 bf16; thread t loads
    // chunk t & 15 (k = 8 * chunk) of rows (t >> 4) + 16 i, i < MT.
    // k % 8 == 0 (admission): a chunk is wholly inside or outside K; rows past
    // M read row M-1 (their outputs are discarded), chunks past K are zero.
    static_assert(kGemmThreads == 256, "one chunk per thread per 16-row block");
    constexpr int kAct = MT;
    uint4 act[NA][kAct];
    const uint16_t* act_row[kAct];
    int act_r[kAct];
    const int act_c8 = (threadIdx.x & 15) * 8;  // same chunk column for every i
#pragma unroll
    for (int i = 0; i < kAct; ++i) {
        act_r[i] = (threadIdx.x >> 4) + 16 * i;
        act_row[i] = a.x + src_row(act_r[i]) * a.ldx + act_c8;
    }
    // The loaded registers are carried unmodified (any use right after the
    // load would make the wave wait for it); chunks past K read chunk 0 and
    // are zeroed when written to LDS.
    auto load_act = [&](int kb, uint4 (&dst)[kAct]) {
        const int kofs = min(kb, kb_end - 1) * kKBlock;
#pragma unroll
        for (int i = 0; i < kAct; ++i)
            dst[i] = *reinterpret_cast<const uint4*>(act_row[i] + (kofs + act_c8 < a.k ? kofs : 0));
    };

#pragma unroll
    for (int st = 0; st < S; ++st) load_codes(kb_begin + st, ring_codes[st], ring_meta[st]);
#pragma unroll
    for (int i = 0; i < NA; ++i) load_act(kb_begin + i, act[i]);
    // Whole groups of S k-blocks, with no exit inside the unrolled group (an
    // exit there makes the wait-count analysis drain the ring at the loop
    // edge).  Blocks past the split's end read clamped addresses and get zero
    // activations, so they add exactly 0 to the accumulators.
    for (int kb0 = kb_begin; kb0 < kb_end; kb0 += S) {
#pragma unroll
        for (int st = 0; st < S; ++st) {
            const int kb = kb0 + st;
            constexpr int kStageMask = 1;
            const int ab = st & kStageMask;  // S is even: the stage alternates every block
            uint16_t* lds = a_lds[ab];
            // a whole k-block inside this split and inside K (wave-uniform)
            // is stored as loaded; otherwise chunks past K or past the
            // split's end are zeroed
            if (kb < kb_end && (kb + 1) * kKBlock <= a.k) {
#pragma unroll
                for (int i = 0; i < kAct; ++i) {
                    const int r = act_r[i];
                    *reinterpret_cast<uint4*>(&lds[((r >> 4) * 256 + a_slot(r & 15, act_c8 >> 3)) * 8]) =
                        act[st % NA][i];
                }
            } else {
                const uint32_t keep =  // same for all i
                    kb < kb_end && kb * kKBlock + act_c8 < a.k ? 0xFFFFFFFFu : 0u;
#pragma unroll
                for (int i = 0; i < kAct; ++i) {
                    const int r = act_r[i];
                    const uint4 v = act[st % NA][i];
                    *reinterpret_cast<uint4*>(&lds[((r >> 4) * 256 + a_slot(r & 15, act_c8 >> 3)) * 8]) =
                        make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
                }
            }
            uint32_t codes[J][W];
            uint32_t meta[J][MW];
#pragma unroll
            for (int j = 0; j < J; ++j) {
#pragma unroll
                for (int w = 0; w < W; ++w) codes[j][w] = ring_codes[st][j][w];
#pragma unroll
                for (int w = 0; w < MW; ++w) meta[j][w] = ring_meta[st][j][w];
            }
            // LDS hand-off only: no vector-memory drain at the barrier
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_s_barrier();
            load_act(kb + NA, act[st % NA]);
            __builtin_amdgcn_sched_barrier(0);  // keep the prefetch where it is issued

            // level tables (bits <= 4, prepared) or curve parameters (bits >= 5)
            LevelTable tab[J];
            float ms[J], ma[J], mb[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                if constexpr (BITS <= 4) {
                    tab[j].lo_lo = meta[j][0];
                    tab[j].hi_lo = meta[j][1];
                    tab[j].lo_hi = MW == 4 ? meta[j][MW == 4 ? 2 : 0] : 0u;
                    tab[j].hi_hi = MW == 4 ? meta[j][MW == 4 ? 3 : 1] : 0u;
                    ms[j] = ma[j] = mb[j] = 0.0f;
                } else {
                    ms[j] = __uint_as_float(meta[j][0]);
                    ma[j] = half_bits_to_float(meta[j][1] & 0xFFFFu);
                    mb[j] = half_bits_to_float(meta[j][1] >> 16);
                }
            }
            if constexpr (LT) {
                // the four lanes of a column (quarters q) evaluate a quarter of
                // its levels each, rounded as direct_fragment rounds them
                constexpr int kPer = NM / 4;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    uint32_t pairs[kPer / 2];
#pragma unroll
                    for (int p = 0; p < kPer / 2; ++p) {
                        const int m = q * kPer + 2 * p;
                        pairs[p] = pack_level2<F16>(curve_level(t_lds[m], ms[j], ma[j], mb[j]),
                                               curve_level(t_lds[m + 1], ms[j], ma[j], mb[j]));
                    }
                    uint32_t* dst = reinterpret_cast<uint32_t*>(&lv_lds[((wave * J + j) * 16 + col) * NMP + q * kPer]);
#pragma unroll
                    for (int p = 0; p < kPer / 2; p += 2)
                        *reinterpret_cast<uint2*>(dst + p) = make_uint2(pairs[p], pairs[p + 1]);
                }
                // every lane reads the levels its column's other lanes wrote
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }

            // fragment f of lane (col, q): chunk 4q + f of row col in each 16-row block
            auto afrag_at = [&](int mt, int f) {
                return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                                        &lds[(mt * 256 + a_slot(col, 4 * q + f)) * 8]));
            };
            // A fragments are double-buffered: the LDS reads of fragment f + 1
            // are in flight while fragment f is decoded and multiplied.
            // Raised wave priority over the fragment reads, decode and MFMA:
            // the arbiter then favours a wave that is in its math phase over
            // one issuing loads or staging activations, which keeps the MFMA
            // pipe fed while other waves wait on memory (cfg2 gate/up 30.1 ->
            // 29.2 us, qkv 14.8 -> 14.5 us, same box).
            __builtin_amdgcn_s_setprio(1);
            bf16x8_t afrag_buf[2][MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) afrag_buf[0][mt] = afrag_at(mt, 0);
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                if (f + 1 < 4) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) afrag_buf[(f + 1) & 1][mt] = afrag_at(mt, f + 1);
                }
                const int fb = f & 1;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    uint4 bw;
                    if constexpr (BITS <= 4)
                        bw = decode_fragment<BITS>(codes[j], f, tab[j]);
                    else if constexpr (LT)
                        bw = table_fragment<BITS>(codes[j], f, &lv_lds[((wave * J + j) * 16 + col) * NMP]);
                    else
                        bw = direct_fragment<BITS, F16>(codes[j], f, ms[j], ma[j], mb[j], t_lds);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][j] = mfma16<F16>(__builtin_bit_cast(uint4, afrag_buf[fb][mt]), bw, acc[mt][j]);
                }
            }
            __builtin_amdgcn_s_setprio(0);
            // Refill this ring slot only now that its codes are consumed: a load
            // issued while the old value is live would land in other registers
            // and be copied back (a wait on the load) at the loop edge.
            __builtin_amdgcn_sched_barrier(0);
            load_codes(kb + S, ring_codes[st], ring_meta[st]);
            __builtin_amdgcn_sched_barrier(0);
            // every wave finished reading this LDS stage before it is rewritten
            // two blocks later (the next barrier orders it)
            __builtin_amdgcn_s_waitcnt(0xC07F);
        }
    }

    // --- epilogue -----------------------------------------------------------
    // The activation stages are free once every wave is past its last MFMA;
    // they hold the block's bf16 output tile.
    static_assert(16 * MT * tile_pitch<J>() <= 2 * kAStage, "output tile fits the activation stages");
    finish_block<J, MT, F16>(a, acc, &a_lds[0][0], m0, wave, lane);
}

// ---------------------------------------------------------------------------
// Small-row GEMM (M <= 4; groups of whole k-blocks; bits <= 4 and 7..8 at any K,
// 5..6 up to 64 k-blocks -- the host plan decides)
//   grid.x: 16-column tiles; a workgroup of G waves owns one tile and all of K.
//   Wave w streams the tile's k-blocks [w * kbw, (w + 1) * kbw) in chunks of
//   D: codes, the group's level table (bits <= 4) or curve parameters, and
//   the k-block's 4 x 128 activations
//   (one 16-byte load per lane; rows past M read zero), all loaded straight
//   into registers -- no LDS staging and no barrier in the loop.  The MFMA
//   A fragments are gathered across lanes with ds_bpermute: the loop is
//   bound by vector-memory instructions issued, and the four per-fragment
//   activation loads it replaces cost as much of that path as 4 KB of codes
//   while carrying at most 1 KB.  The MFMA sums each 32-k fragment; the G per-wave
//   partial sums are added in wave order through LDS at the end, so the K
//   partition depends on K alone (not on M or on grouping).
// (quantization/common/small_rows.cu:94-241 and small_rows_cost.py:438-501
// are the reference's small-row path: a separate arithmetic for M <= 4.)
// ---------------------------------------------------------------------------
template <int BITS, int G, int D, bool F16>
__global__ __launch_bounds__(64 * G) void rows_kernel(GemmArgs a) {
    constexpr int W = BITS;
    constexpr int MW = meta_words<BITS>();
    constexpr int kOut = 0x7FFFFFF0;  // buffer offset past every range: the load returns 0, no fetch
    __shared__ float red[G][16][4];
    // bits >= 5: the curve abscissae t_i = i / (2^(BITS-1) - 1), as the MFMA kernel builds them
    __shared__ float t_lds[BITS >= 5 ? (1 << (BITS - 1)) : 1];
    // bits 5..6: per wave, the current k-block's group levels of the tile's
    // 16 columns (wave-private, rebuilt every k-block; rows padded as in the
    // MFMA kernel).  At 7 and 8 bits a column has 64-128 levels, as many as
    // the lane has weights per k-block, and direct evaluation measured faster.
    constexpr bool LT = BITS >= 5 && BITS <= 6;
    constexpr int NM = 1 << (BITS - 1);
    constexpr int NMP = NM + 4;
    __shared__ __attribute__((aligned(16))) uint16_t lv_lds[LT ? G * 16 * NMP : 1];
    if constexpr (BITS >= 5) {
        for (int i = threadIdx.x; i < (1 << (BITS - 1)); i += 64 * G)
            t_lds[i] = (float)((double)i / (double)((1 << (BITS - 1)) - 1));
        __syncthreads();
    }
    // wave index as a scalar: the per-wave K range and loop bounds stay uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int q = lane >> 4, col = lane & 15;
    const int tile = blockIdx.x;
    const int kb_begin = wave * a.blocks_per_split;
    const int kb_end = min(kb_begin + a.blocks_per_split, a.k_blocks);
    const int nkb = kb_end - kb_begin;  // may be <= 0 for trailing waves
    // Buffer views of this tile's codes and metadata and of the activations.
    // Out-of-range offsets read zero without touching memory: rows at or past
    // M, quarters past K, and k-blocks past the wave's range (the tail of its
    // last chunk) all come back as zero codes / zero activations, so they add
    // exactly 0 to the accumulator with no masking instructions.
    const __amdgpu_buffer_rsrc_t codes = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(a.codes + (int64_t)tile * a.k_blocks * kWave * W), 0,
        a.k_blocks * kWave * W * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t meta = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(a.meta + (int64_t)tile * a.groups_k * 16 * MW), 0, a.groups_k * 16 * MW * 4,
        0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(a.x), 0, (int)((int64_t)a.m * a.ldx * 2), 0x00020000);
    const int gpk = a.group_in / kKBlock;  // k-blocks per metadata group
    // Activations: one 16-byte load per lane and k-block covers the 4 x 128
    // block (lane l: row l / 16, elements 8 (l % 16) .. + 7); the MFMA
    // A fragments are gathered from it across lanes.  Rows past M read zero.
    const int x_row = lane >> 4, x_chunk = lane & 15;
    const int x_lane = x_row < a.m ? (int)((int64_t)x_row * a.ldx * 2) + 16 * x_chunk : 0;
    const int x_dead = x_row < a.m ? 0 : kOut;
    // fragment f of lane (col, q) is chunk 4q + f of row col, k = 32q + 8f
    // (rows 4..15 of the MFMA are never stored; they repeat rows 0..3)
    const int x_src = ((col & 3) * 16 + 4 * q) * 4;

    uint32_t rc[D][W];
    uint32_t rm[D][MW];
    u32x4_dev_t ra[D];
    auto load = [&](int i, uint32_t (&c)[W], uint32_t (&mm)[MW], u32x4_dev_t& av) {
        const int kb = kb_begin + i;
        // Offsets are computed unconditionally and pushed past the buffer by
        // OR-ing kOut, with no select: a uniform condition around a load
        // becomes a branch, and the wait-count pass drains every load in
        // flight where the branches join.
        const int dead = (int)((uint32_t)(nkb - 1 - i) >> 31) * kOut;  // kOut when i >= nkb
        const int co = ((kb * kWave + lane) * W * 4) | dead;
        if constexpr (W == 4) {
            const u32x4_dev_t v = __builtin_amdgcn_raw_buffer_load_b128(codes, co, 0, 2);  // nt
            c[0] = v.x; c[1] = v.y; c[2] = v.z; c[3] = v.w;
        } else if constexpr (W == 2) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(codes, co, 0, 2);
            c[0] = v[0]; c[1] = v[1];
        } else if constexpr (W == 3) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b96(codes, co, 0, 2);
            c[0] = v[0]; c[1] = v[1]; c[2] = v[2];
        } else if constexpr (W == 1) {
            c[0] = __builtin_amdgcn_raw_buffer_load_b32(codes, co, 0, 2);
        } else {  // 5..8 words: 16 bytes, then the rest (dword-aligned buffer loads)
            const u32x4_dev_t v = __builtin_amdgcn_raw_buffer_load_b128(codes, co, 0, 2);
            c[0] = v.x; c[1] = v.y; c[2] = v.z; c[3] = v.w;
            const int co4 = co + 16;  // still past the buffer when dead
            if constexpr (W == 5) {
                c[4] = __builtin_amdgcn_raw_buffer_load_b32(codes, co4, 0, 2);
            } else if constexpr (W == 6) {
                const auto u = __builtin_amdgcn_raw_buffer_load_b64(codes, co4, 0, 2);
                c[4] = u[0]; c[5] = u[1];
            } else if constexpr (W == 7) {
                const auto u = __builtin_amdgcn_raw_buffer_load_b96(codes, co4, 0, 2);
                c[4] = u[0]; c[5] = u[1]; c[6] = u[2];
            } else {
                const u32x4_dev_t u = __builtin_amdgcn_raw_buffer_load_b128(codes, co4, 0, 2);
                c[4] = u.x; c[5] = u.y; c[6] = u.z; c[7] = u.w;
            }
        }
        const int mo = (((kb / gpk) * 16 + col) * MW * 4) | dead;
        if constexpr (MW == 4) {
            const u32x4_dev_t v = __builtin_amdgcn_raw_buffer_load_b128(meta, mo, 0, 0);
            mm[0] = v.x; mm[1] = v.y; mm[2] = v.z; mm[3] = v.w;
        } else {
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(meta, mo, 0, 0);
            mm[0] = v[0]; mm[1] = v[1];
        }
        const int k0 = kb * kKBlock + 8 * x_chunk;
        const int past_k = (int)((uint32_t)(a.k - 1 - k0) >> 31) * kOut;  // kOut when k0 >= K
        const int xo = (x_lane + kb * kKBlock * 2) | dead | past_k | x_dead;
        av = __builtin_bit_cast(u32x4_dev_t, __builtin_amdgcn_raw_buffer_load_b128(xr, xo, 0, 0));
    };
    auto afrag = [&](const u32x4_dev_t& av, int f) {
        const int src = x_src + 4 * f;
        return make_uint4((uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)av.x),
                          (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)av.y),
                          (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)av.z),
                          (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)av.w));
    };
    floatx4_t acc = floatx4_t{0.f, 0.f, 0.f, 0.f};
    // Chunks of D k-blocks: every load of a chunk is issued before its first
    // use and none is carried across the loop edge (a load still in flight at
    // the back-edge makes the compiler drain the counter at the loop head);
    // the other waves of the CU cover each chunk's latency.
    for (int i0 = 0; i0 < nkb; i0 += D) {
#pragma unroll
        for (int st = 0; st < D; ++st) load(i0 + st, rc[st], rm[st], ra[st]);
#pragma unroll
        for (int st = 0; st < D; ++st) {
            LevelTable tab;
            float ms = 0.0f, ma = 0.0f, mb = 0.0f;
            if constexpr (BITS <= 4) {
                tab.lo_lo = rm[st][0];
                tab.hi_lo = rm[st][1];
                tab.lo_hi = MW == 4 ? rm[st][MW == 4 ? 2 : 0] : 0u;
                tab.hi_hi = MW == 4 ? rm[st][MW == 4 ? 3 : 1] : 0u;
            } else {
                ms = __uint_as_float(rm[st][0]);
                ma = half_bits_to_float(rm[st][1] & 0xFFFFu);
                mb = half_bits_to_float(rm[st][1] >> 16);
            }
            uint16_t* lv = &lv_lds[(wave * 16 + col) * NMP];
            if constexpr (LT) {
                // the four lanes of a column evaluate a quarter of its levels
                // each, rounded as direct_fragment rounds them; the previous
                // k-block's lookups are complete before the table is rewritten
                constexpr int kPer = NM / 4;
                uint32_t pairs[kPer / 2];
#pragma unroll
                for (int p = 0; p < kPer / 2; ++p) {
                    const int m = q * kPer + 2 * p;
                    pairs[p] = pack_level2<F16>(curve_level(t_lds[m], ms, ma, mb),
                                                curve_level(t_lds[m + 1], ms, ma, mb));
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                uint32_t* dst = reinterpret_cast<uint32_t*>(lv + q * kPer);
#pragma unroll
                for (int p = 0; p < kPer / 2; p += 2)
                    *reinterpret_cast<uint2*>(dst + p) = make_uint2(pairs[p], pairs[p + 1]);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
#pragma unroll
            for (int f = 0; f < 4; ++f) {
                uint4 bw;
                if constexpr (BITS <= 4) bw = decode_fragment<BITS>(rc[st], f, tab);
                else if constexpr (LT) bw = table_fragment<BITS>(rc[st], f, lv);
                else bw = direct_fragment<BITS, F16>(rc[st], f, ms, ma, mb, t_lds);
                acc = mfma16<F16>(afrag(ra[st], f), bw, acc);
            }
        }
    }
    // rows 0..3 of the tile are lanes 0..15 (quarter 0), one register per row
    if (q == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][col][r] = acc[r];
    }
    __syncthreads();
    if (wave == 0 && q == 0) {
        const int n = tile * 16 + col;
        if (n < a.n) {
            float sum[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[r] = red[0][col][r];
#pragma unroll
            for (int w = 1; w < G; ++w)
#pragma unroll
                for (int r = 0; r < 4; ++r) sum[r] += red[w][col][r];
            const int member = n / a.n_member;
            uint16_t* y = a.ys[member] + (n - member * a.n_member);
            const int64_t ldy = a.ldys[member];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (r < a.m) y[(int64_t)r * ldy] = out_bits<F16>(sum[r]);
        }
    }
}

template <int BITS>
hipError_t launch_rows_bits(const GemmArgs& a, int g, hipStream_t s) {
    dim3 grid(a.n_tiles);
    if (a.f16) {
        if (g == 8) rows_kernel<BITS, 8, 4, true><<<grid, 8 * 64, 0, s>>>(a);
        else rows_kernel<BITS, 4, 4, true><<<grid, 4 * 64, 0, s>>>(a);
    } else {
        if (g == 8) rows_kernel<BITS, 8, 4, false><<<grid, 8 * 64, 0, s>>>(a);
        else rows_kernel<BITS, 4, 4, false><<<grid, 4 * 64, 0, s>>>(a);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Load-time preparation
// ---------------------------------------------------------------------------
// Metadata: per (column, group) words; padding columns are zero.  bits <= 4:
// the group's level table as byte planes (lo bytes of L0..3, hi bytes of L0..3,
// lo bytes of L4..7, hi bytes of L4..7), each level bf16(curve) evaluated in
// the reference's operation order; bits >= 5: (scale, a | b << 16).
template <int BITS, bool F16>
__global__ void prepare_meta_kernel(const float* scale, const uint16_t* av, const uint16_t* bv,
                                    int64_t n, int groups_k, int n_tiles, uint32_t* meta) {
    constexpr int MW = meta_words<BITS>();
    const int64_t total = (int64_t)n_tiles * groups_k * 16;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % 16);
        const int64_t g = (i / 16) % groups_k, nt = i / (16 * (int64_t)groups_k);
        const int64_t row = nt * 16 + c;
        uint32_t w[4] = {0, 0, 0, 0};
        if (row < n) {
            const int64_t src = row * groups_k + g;
            if constexpr (BITS <= 4) {
                const float sc = scale[src], a = half_bits_to_float(av[src]), b = half_bits_to_float(bv[src]);
                const uint32_t p0 = level_pair<BITS, F16>(0, sc, a, b);
                const uint32_t p1 = BITS >= 3 ? level_pair<BITS, F16>(2, sc, a, b) : 0u;
                const uint32_t p2 = BITS >= 4 ? level_pair<BITS, F16>(4, sc, a, b) : 0u;
                const uint32_t p3 = BITS >= 4 ? level_pair<BITS, F16>(6, sc, a, b) : 0u;
                const LevelTable t = table_from_pairs(p0, p1, p2, p3);
                w[0] = t.lo_lo; w[1] = t.hi_lo; w[2] = t.lo_hi; w[3] = t.hi_hi;
            } else {
                w[0] = __float_as_uint(scale[src]);
                w[1] = (uint32_t)av[src] | ((uint32_t)bv[src] << 16);
            }
        }
#pragma unroll
        for (int x = 0; x < MW; ++x) meta[MW * i + x] = w[x];
    }
}

template <int BITS>
__device__ __forceinline__ uint32_t level_sign_mask(float s, float a, float b) {
    // bit m = sign of bf16(L[m]), m = 0..7, for the stored-sign convention (bits <= 4)
    uint32_t mask = 0;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        float l = 0.0f;
        if constexpr (BITS == 1) l = m == 1 ? s : 0.0f;
        else if (m < (1 << (BITS - 1))) l = curve_level(t_of<BITS>(m), s, a, b);
        mask |= ((pack_bf16x2(l, 0.0f) >> 15) & 1u) << m;
    }
    return mask;
}

template <int BITS>
__global__ __launch_bounds__(kThreads) void prepare_codes_kernel(
        const uint8_t* packed, const float* scale, const uint16_t* av, const uint16_t* bv, int64_t n,
        int64_t k, int group_in, int groups_k, int n_tiles, int k_blocks, int aligned, uint32_t* codes) {
    const int64_t total = (int64_t)n_tiles * k_blocks * kWave;
    const int64_t row_bytes = (k * BITS + 7) / 8;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % kWave);
        const int64_t kb = (i / kWave) % k_blocks, nt = i / ((int64_t)kWave * k_blocks);
        const int q = lane >> 4, col = lane & 15;
        const int64_t row = nt * 16 + col;
        const int64_t k0 = kb * kKBlock + 32 * q;
        float s = 0.0f, a = 0.0f, b = 0.0f;
        if (row < n && k0 < k) {
            const int64_t g = k0 / group_in;
            s = scale[row * groups_k + g];
            a = half_bits_to_float(av[row * groups_k + g]);
            b = half_bits_to_float(bv[row * groups_k + g]);
        }
        const uint32_t sigma = BITS <= 4 ? level_sign_mask<BITS>(s, a, b) : 0u;
        // codes k0 .. k0+31 of the row: 4 * BITS bytes of the little-endian
        // bitstream starting at byte k0 * BITS / 8 (a multiple of 4)
        uint32_t rw[BITS + 1];
#pragma unroll
        for (int x = 0; x <= BITS; ++x) rw[x] = 0;
        if (row < n && k0 < k) {
            const uint8_t* src = packed + row * row_bytes + k0 * BITS / 8;
            if (aligned && k0 + 32 <= k) {
#pragma unroll
                for (int x = 0; x < BITS; ++x) rw[x] = reinterpret_cast<const uint32_t*>(src)[x];
            } else {
                const int64_t left = row_bytes - k0 * BITS / 8;
#pragma unroll
                for (int y = 0; y < 4 * BITS; ++y)
                    if (y < left) rw[y >> 2] |= (uint32_t)src[y] << (8 * (y & 3));
            }
        }
        int mag[32], neg[32];
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const int p = BITS * e, word = p >> 5, shift = p & 31;
            const uint64_t pair = ((uint64_t)rw[word + 1] << 32) | rw[word];
            const int raw = (int)((pair >> shift) & ((1u << BITS) - 1u));
            int qv;
            if constexpr (BITS == 1) {
                qv = raw * 2 - 1;
            } else {
                constexpr int kSign = 1 << (BITS - 1);
                qv = raw >= kSign ? raw - (1 << BITS) : raw;
                if (qv == -kSign) qv = 0;  // reserved code
            }
            if (row >= n || k0 + e >= k) qv = 0;
            const int m = qv < 0 ? -qv : qv;
            mag[e] = m;
            if (BITS <= 4)  // stored sign = sign(q) xor sign(bf16(L[|q|]))
                neg[e] = (int)((qv < 0 ? 1u : 0u) ^ ((sigma >> (m & 7)) & 1u));
            else
                neg[e] = qv < 0;
        }
        uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (BITS == 4) {
#pragma unroll
            for (int f = 0; f < 4; ++f)
#pragma unroll
                for (int byte = 0; byte < 4; ++byte) {
                    const int ea = 8 * f + byte, eb = 8 * f + 4 + byte;
                    const uint32_t v = (uint32_t)(mag[ea] & 7) | ((uint32_t)neg[eb] << 3) |
                                       ((uint32_t)(mag[eb] & 7) << 4) | ((uint32_t)neg[ea] << 7);
                    w[f] |= v << (8 * byte);
                }
        } else if (BITS == 3 || BITS == 2 || BITS == 1) {
#pragma unroll
            for (int f = 0; f < 4; ++f)
#pragma unroll
                for (int byte = 0; byte < 4; ++byte) {
                    const int ea = 8 * f + byte, eb = 8 * f + 4 + byte;
                    if (BITS == 3) {
                        const uint32_t v = (uint32_t)(mag[ea] & 3) | ((uint32_t)(mag[eb] & 3) << 2);
                        w[f >> 1] |= v << (8 * byte + 4 * (f & 1));
                    } else if (BITS == 2) {
                        const uint32_t v = (uint32_t)(mag[ea] & 1) | ((uint32_t)(mag[eb] & 1) << 1);
                        w[0] |= v << (8 * byte + 2 * f);
                    }
                    const int sw = BITS == 3 ? 2 : (BITS == 2 ? 1 : 0);
                    w[sw] |= ((uint32_t)neg[ea] << (8 * byte + 7 - 2 * f)) |
                             ((uint32_t)neg[eb] << (8 * byte + 6 - 2 * f));
                }
        } else {
#pragma unroll
            for (int e = 0; e < 32; ++e) {
                const uint32_t code = ((uint32_t)neg[e] << (BITS - 1)) | (uint32_t)mag[e];
                const int p = BITS * e, word = p >> 5, shift = p & 31;
                w[word] |= code << shift;
                if (shift + BITS > 32) w[word + 1] |= code >> (32 - shift);
            }
        }
#pragma unroll
        for (int x = 0; x < BITS; ++x) codes[i * BITS + x] = w[x];
    }
}

// fmt1 / fmt2 metadata -> per-group (scale f32, a f16, b f16) per output row
// (reference.py:67-95), replicating output groups (group_out) to rows.
__global__ void expand_metadata_kernel(int fmt, const void* m0, const void* m1, const void* m2,
                                       const void* g0, const void* g1, const void* g2,
                                       const int32_t* part_of_row,
                                       int64_t n, int64_t groups_k, int group_out, float* scale,
                                       uint16_t* av, uint16_t* bv) {
    const int64_t total = n * groups_k;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / groups_k, g = i % groups_k;
        const int64_t src = (row / group_out) * groups_k + g;
        const int p = part_of_row ? part_of_row[row] : 0;
        group_metadata(fmt, m0, m1, m2, g0, g1, g2, src, p, scale[i], av[i], bv[i]);
    }
}

template <int BITS, int MT, bool G128, bool F16>
hipError_t launch_g(const GemmArgs& a, int j, dim3 grid, hipStream_t s) {
    if constexpr (MT == 4 && BITS <= 5 && !F16) {
        if (j == 2 && a.split == 1) {
            gemm_kernel<BITS, MT, 2, G128, true, F16><<<grid, kGemmThreads, 0, s>>>(a);
            return hipGetLastError();
        }
    }
    if (j == 2) gemm_kernel<BITS, MT, 2, G128, false, F16><<<grid, kGemmThreads, 0, s>>>(a);
    else gemm_kernel<BITS, MT, 1, G128, false, F16><<<grid, kGemmThreads, 0, s>>>(a);
    return hipGetLastError();
}

template <int BITS, int MT, bool F16>
hipError_t launch_j(const GemmArgs& a, int j, dim3 grid, hipStream_t s) {
    if (a.group_in % kKBlock == 0) return launch_g<BITS, MT, true, F16>(a, j, grid, s);
    return launch_g<BITS, MT, false, F16>(a, j, grid, s);
}

template <int BITS, bool F16>
hipError_t launch_mt(const GemmArgs& a, int mt, int j, dim3 grid, hipStream_t s) {
    if (mt == 1) return launch_j<BITS, 1, F16>(a, j, grid, s);
    if (mt == 2) return launch_j<BITS, 2, F16>(a, j, grid, s);
    if (mt == 8) {  // 128-row chunks: host plan, whole-k-block groups only
        if (a.group_in % kKBlock) return hipErrorInvalidValue;
        return launch_g<BITS, 8, true, F16>(a, j, grid, s);
    }
    return launch_j<BITS, 4, F16>(a, j, grid, s);
}

template <int BITS>
hipError_t launch_bits(const GemmArgs& a, int mt, int j, dim3 grid, hipStream_t s) {
    return a.f16 ? launch_mt<BITS, true>(a, mt, j, grid, s) : launch_mt<BITS, false>(a, mt, j, grid, s);
}

}  // namespace

// MT (16-row tiles per 64-row chunk) follows m; J and the K split come from the
// host plan: J from n, the K split from the number of output blocks (so a
// row's result is the same for every m up to one 64-row chunk).
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    if (a.rows_waves > 0) {  // small-row plan (host: M <= 4, whole-k-block groups)
        switch (a.bits) {
            case 1: return launch_rows_bits<1>(a, a.rows_waves, s);
            case 2: return launch_rows_bits<2>(a, a.rows_waves, s);
            case 3: return launch_rows_bits<3>(a, a.rows_waves, s);
            case 4: return launch_rows_bits<4>(a, a.rows_waves, s);
            case 5: return launch_rows_bits<5>(a, a.rows_waves, s);
            case 6: return launch_rows_bits<6>(a, a.rows_waves, s);
            case 7: return launch_rows_bits<7>(a, a.rows_waves, s);
            case 8: return launch_rows_bits<8>(a, a.rows_waves, s);
            default: return hipErrorInvalidValue;
        }
    }
    if (a.panel) return launch_panel_gemm(a, s);  // host plan: M <= 64, bits <= 4, whole-k-block groups
    // routed: one grid chunk per padded route block (a.m = block capacity)
    const int mt = a.routed ? a.block_m / 16 : (a.m >= 33 ? 4 : (a.m >= 17 ? 2 : 1));
    const int rows_chunks = (a.m + a.chunk_rows - 1) / a.chunk_rows;
    const int mt_eff = a.routed ? mt
                                : (a.chunk_rows == 128 ? 8 : (a.chunk_rows == 32 ? 2 : (rows_chunks == 1 ? mt : 4)));
    const int j = a.tiles_per_wave;  // chosen by the host plan
    const int cols_per_block = kGemmWaves * j * 16;
    dim3 grid((a.n + cols_per_block - 1) / cols_per_block, a.split, rows_chunks);
    switch (a.bits) {
        case 1: return launch_bits<1>(a, mt_eff, j, grid, s);
        case 2: return launch_bits<2>(a, mt_eff, j, grid, s);
        case 3: return launch_bits<3>(a, mt_eff, j, grid, s);
        case 4: return launch_bits<4>(a, mt_eff, j, grid, s);
        case 5: return launch_bits<5>(a, mt_eff, j, grid, s);
        case 6: return launch_bits<6>(a, mt_eff, j, grid, s);
        case 7: return launch_bits<7>(a, mt_eff, j, grid, s);
        case 8: return launch_bits<8>(a, mt_eff, j, grid, s);
        default: return hipErrorInvalidValue;
    }
}

// Routed-block table (repack.py:253-277 semantics): expert e's compact routes
// row_map[starts[e] ..) fill padded slots (block_starts[e] + b) * block_m + i;
// slots past counts[e] hold `routes` (padding); block_expert[block] = e.
__global__ void pad_routes_kernel(const int32_t* counts, const int32_t* starts,
                                  const int32_t* block_starts, const int32_t* total_blocks,
                                  const int32_t* row_map, int routes, int block_m, int32_t* padded,
                                  int32_t* block_expert, int32_t* padded_total) {
    const int e = blockIdx.x;
    const int count = counts[e], start = starts[e], block = block_starts[e];
    const int blocks = (count + block_m - 1) / block_m;
    for (int i = threadIdx.x; i < blocks * block_m; i += blockDim.x) {
        padded[block * block_m + i] = i < count ? row_map[start + i] : routes;
        if (i % block_m == 0) block_expert[block + i / block_m] = e;
    }
    if (e == 0 && threadIdx.x == 0) *padded_total = *total_blocks * block_m;
}

hipError_t launch_pad_routes(const int32_t* counts, const int32_t* starts, const int32_t* block_starts,
                             const int32_t* total_blocks, const int32_t* row_map, int experts,
                             int routes, int block_m, int32_t* padded, int32_t* block_expert,
                             int32_t* padded_total, hipStream_t s) {
    pad_routes_kernel<<<experts, kThreads, 0, s>>>(counts, starts, block_starts, total_blocks, row_map,
                                                   routes, block_m, padded, block_expert, padded_total);
    return hipGetLastError();
}

hipError_t launch_prepare(const void* packed, const float* scale, const uint16_t* av,
                          const uint16_t* bv, int64_t n, int64_t k, int bits, int group_in, int f16,
                          uint32_t* codes, uint32_t* meta, hipStream_t s) {
    const int n_tiles = (int)((n + 15) / 16);
    const int k_blocks = (int)((k + kKBlock - 1) / kKBlock);
    const int groups_k = (int)((k + group_in - 1) / group_in);
    const int64_t code_threads = (int64_t)n_tiles * k_blocks * kWave;
    const int blocks = (int)((code_threads + 255) / 256 < 65535 ? (code_threads + 255) / 256 : 65535);
    const uint8_t* p = (const uint8_t*)packed;
    const int aligned = ((uintptr_t)packed % 4 == 0) && (((k * bits + 7) / 8) % 4 == 0);
    switch (bits) {
#define CUBIC_PREP(B) case B: prepare_codes_kernel<B><<<blocks, 256, 0, s>>>(p, scale, av, bv, n, k, group_in, groups_k, n_tiles, k_blocks, aligned, codes); break;
        CUBIC_PREP(1) CUBIC_PREP(2) CUBIC_PREP(3) CUBIC_PREP(4)
        CUBIC_PREP(5) CUBIC_PREP(6) CUBIC_PREP(7) CUBIC_PREP(8)
#undef CUBIC_PREP
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t meta_threads = (int64_t)n_tiles * groups_k * 16;
    const int mblocks = (int)((meta_threads + 255) / 256 < 65535 ? (meta_threads + 255) / 256 : 65535);
    switch (bits) {
#define CUBIC_META(B) case B: \
        if (f16) prepare_meta_kernel<B, true><<<mblocks, 256, 0, s>>>(scale, av, bv, n, groups_k, n_tiles, meta); \
        else prepare_meta_kernel<B, false><<<mblocks, 256, 0, s>>>(scale, av, bv, n, groups_k, n_tiles, meta); \
        break;
        CUBIC_META(1) CUBIC_META(2) CUBIC_META(3) CUBIC_META(4)
        CUBIC_META(5) CUBIC_META(6) CUBIC_META(7) CUBIC_META(8)
#undef CUBIC_META
    }
    return hipGetLastError();
}

hipError_t launch_expand_metadata(int fmt, const void* m0, const void* m1, const void* m2,
                                  const void* g0, const void* g1, const void* g2,
                                  const int32_t* part_of_row,
                                  int64_t n, int64_t groups_k, int group_out, float* scale,
                                  uint16_t* a, uint16_t* b, hipStream_t s) {
    const int64_t total = n * groups_k;
    const int blocks = (int)((total + 255) / 256 < 65535 ? (total + 255) / 256 : 65535);
    expand_metadata_kernel<<<blocks > 0 ? blocks : 1, 256, 0, s>>>(fmt, m0, m1, m2, g0, g1, g2,
                                                                 part_of_row, n, groups_k, group_out, scale, a, b);
    return hipGetLastError();
}

}  // namespace cubic
