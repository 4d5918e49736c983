// Device helpers shared by the Cubic GEMM kernels (cubic_gemm.hip,
// cubic_panel.hip): the activation LDS swizzle, the level-table decode, the
// prepared-code loads and the output / split-K epilogue.  Every kernel that
// uses them performs the same per-tile arithmetic, so their outputs agree bit
// for bit under one K plan.
#pragma once
#include "cubic_device.h"
#include "cubic_capi_internal.h"

namespace cubic {
namespace gemm {


constexpr int kWave = 64;
constexpr int kThreads = 256;                  // prepare / expand kernels
constexpr int kGemmThreads = kGemmWaves * 64;  // gemm_kernel
constexpr int kKBlock = 128;
// Activation stage in LDS: per 16-row block, 16-byte chunk c (k = 8c..8c+7 of
// the k-block) of row r sits in 16-byte slot c * 16 + (r ^ (c & 3) << 2 ^ c >> 2).
// An MFMA A-fragment read (lane (col, q) reads row col, chunk 4q + f) then
// lands in position col ^ 4f ^ q of its 256-byte line, and the staging write
// (lanes 0..15 store rows 0..15 of one chunk) in position r ^ g(c): both run at
// the b128 peak rate of gfx950's LDS (measured 243 B/clk/CU for the reads,
// 83 B/clk/CU for the writes; the plain r ^ c swizzle reads at 128).
// bf16 per activation stage of a workgroup with MT m-tiles (at least 64 rows:
// the output tile of the epilogue reuses the stages)
template <int MT>
__host__ __device__ constexpr int a_stage() { return (MT > 4 ? MT : 4) * 16 * kKBlock; }
__device__ __forceinline__ int a_slot(int r16, int c) { return c * 16 + (r16 ^ ((c & 3) << 2) ^ (c >> 2)); }

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float floatx4_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;

// Activation / weight / output element type: bf16, or fp16 (F16).  The
// reference rounds each decoded weight once to the activation dtype and
// accumulates in FP32 (ops/eager/quantization.py:181-186).
template <bool F16>
__device__ __forceinline__ uint32_t pack_level2(float lo, float hi) {
    if constexpr (F16) return float_to_f16_bits(lo) | (float_to_f16_bits(hi) << 16);
    else return pack_bf16x2(lo, hi);
}

template <bool F16>
__device__ __forceinline__ uint16_t out_bits(float f) {
    if constexpr (F16) return (uint16_t)float_to_f16_bits(f);
    else return (uint16_t)float_to_bf16_bits(f);
}

template <bool F16>
__device__ __forceinline__ floatx4_t mfma16(uint4 a, uint4 b, floatx4_t c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Prepared metadata words per (column, group): bits <= 4 store the group's bf16
// level table as v_perm byte planes (4 words at 4 bits, 2 words below);
// bits >= 5 store (scale f32, a f16 | b f16 << 16).
template <int BITS>
__host__ __device__ constexpr int meta_words() { return BITS == 4 ? 4 : 2; }

// ---------------------------------------------------------------------------
// Level tables for bits <= 4: magnitudes 0..7 -> bf16, split into low-byte and
// high-byte planes so one v_perm_b32 looks up four magnitudes.
// ---------------------------------------------------------------------------
struct LevelTable {
    uint32_t lo_lo, lo_hi, hi_lo, hi_hi;  // low bytes of L0..3, L4..7; high bytes of L0..3, L4..7
};

template <int BITS, bool F16>
__device__ __forceinline__ uint32_t level_pair(int m0, float s, float a, float b) {
    // bf16 pair (L[m0], L[m0 + 1]) for the compile-time-unrolled callers below
    float l0, l1;
    if (BITS == 1) {
        l0 = 0.0f;  // unused: bipolar codes always select magnitude 1
        l1 = s;
    } else {
        constexpr int kMags = 1 << (BITS - 1);
        l0 = m0 < kMags ? curve_level(t_of<BITS>(m0), s, a, b) : 0.0f;
        l1 = m0 + 1 < kMags ? curve_level(t_of<BITS>(m0 + 1), s, a, b) : 0.0f;
    }
    return pack_level2<F16>(l0, l1);
}

__device__ __forceinline__ LevelTable table_from_pairs(uint32_t p0, uint32_t p1, uint32_t p2,
                                                       uint32_t p3) {
    LevelTable t;
    t.lo_lo = perm(p1, p0, 0x06040200u);
    t.hi_lo = perm(p1, p0, 0x07050301u);
    t.lo_hi = perm(p3, p2, 0x06040200u);
    t.hi_hi = perm(p3, p2, 0x07050301u);
    return t;
}

// Four bf16 pairs (k = 8f .. 8f+7) from magnitude selectors and sign bytes.
// selA/selB: magnitude per byte of weights 0..3 / 4..7; sgnA/sgnB: the stored
// sign in bit 7 of each byte.  The stored sign replaces the level's sign bit.
__device__ __forceinline__ uint4 lut_decode(const LevelTable& t, uint32_t selA, uint32_t selB,
                                            uint32_t sgnA, uint32_t sgnB) {
    const uint32_t loA = perm(t.lo_hi, t.lo_lo, selA);
    uint32_t hiA = perm(t.hi_hi, t.hi_lo, selA);
    const uint32_t loB = perm(t.lo_hi, t.lo_lo, selB);
    uint32_t hiB = perm(t.hi_hi, t.hi_lo, selB);
    hiA = (sgnA & 0x80808080u) | (hiA & 0x7F7F7F7Fu);
    hiB = (sgnB & 0x80808080u) | (hiB & 0x7F7F7F7Fu);
    uint4 r;
    r.x = perm(hiA, loA, 0x05010400u);
    r.y = perm(hiA, loA, 0x07030602u);
    r.z = perm(hiB, loB, 0x05010400u);
    r.w = perm(hiB, loB, 0x07030602u);
    return r;
}

// Fragment f of one lane's words, bits <= 4 layouts (see prepare_kernel).
template <int BITS>
__device__ __forceinline__ uint4 decode_fragment(const uint32_t* w, int f, const LevelTable& t) {
    if (BITS == 4) {
        const uint32_t x = w[f];
        return lut_decode(t, x & 0x07070707u, (x >> 4) & 0x07070707u, x, x << 4);
    } else if (BITS == 3) {
        const uint32_t mw = w[f >> 1] >> (4 * (f & 1));
        const uint32_t sg = w[2];
        return lut_decode(t, mw & 0x03030303u, (mw >> 2) & 0x03030303u, sg << (2 * f),
                          sg << (2 * f + 1));
    } else if (BITS == 2) {
        const uint32_t mw = w[0];
        const uint32_t sg = w[1];
        return lut_decode(t, (mw >> (2 * f)) & 0x01010101u, (mw >> (2 * f + 1)) & 0x01010101u,
                          sg << (2 * f), sg << (2 * f + 1));
    } else {  // BITS == 1: every code has magnitude 1
        const uint32_t sg = w[0];
        return lut_decode(t, 0x01010101u, 0x01010101u, sg << (2 * f), sg << (2 * f + 1));
    }
}

// bits >= 5: code i of the lane (k order) is bit-packed at bits [B*i, B*i+B)
// as (sign << (B-1)) | magnitude; the level is evaluated directly.
template <int BITS>
__device__ __forceinline__ uint32_t code_at(const uint32_t* w, int i) {
    const int p = BITS * i, word = p >> 5, shift = p & 31;
    uint32_t v = w[word] >> shift;
    if (shift + BITS > 32) v |= w[word + 1] << (32 - shift);
    return v & ((1u << BITS) - 1u);
}

template <int BITS, bool F16>
__device__ __forceinline__ uint4 direct_fragment(const uint32_t* w, int f, float s, float a,
                                                 float b, const float* t_table) {
    uint32_t out[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        float v[2];
        uint32_t sg[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t code = code_at<BITS>(w, 8 * f + 2 * h + e);
            const uint32_t mag = code & ((1u << (BITS - 1)) - 1u);
            sg[e] = (code >> (BITS - 1)) << 15;
            v[e] = curve_level(t_table[mag], s, a, b);
        }
        out[h] = pack_level2<F16>(v[0], v[1]) ^ (sg[0] | (sg[1] << 16));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// bits 5..7 with one metadata group per k-block: the group's bf16 levels of
// the lane's column sit in LDS (lv, indexed by magnitude); a weight is a
// lookup plus the stored sign, bit for bit what direct_fragment computes.
template <int BITS>
__device__ __forceinline__ uint4 table_fragment(const uint32_t* w, int f, const uint16_t* lv) {
    constexpr uint32_t kMagMask = (1u << (BITS - 1)) - 1u;
    uint32_t out[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const uint32_t c0 = code_at<BITS>(w, 8 * f + 2 * h), c1 = code_at<BITS>(w, 8 * f + 2 * h + 1);
        const uint32_t l0 = lv[c0 & kMagMask], l1 = lv[c1 & kMagMask];
        const uint32_t sg = ((c0 >> (BITS - 1)) << 15) | ((c1 >> (BITS - 1)) << 31);
        out[h] = (l0 | (l1 << 16)) ^ sg;
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// ---------------------------------------------------------------------------
// GEMM kernel
//   grid.x: column blocks of kGemmWaves waves x J tiles x 16 columns
//   grid.y: K partitions (split)
//   grid.z: 64-row chunks of M
// ---------------------------------------------------------------------------
// Code words of one lane for one (tile, k-block): vector loads, streamed once.
template <int W>
__device__ __forceinline__ void load_words(const uint32_t* src, uint32_t (&dst)[W]) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    if constexpr (W == 4) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    } else if constexpr (W == 2) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src));
        dst[0] = v.x; dst[1] = v.y;
    } else if constexpr (W == 3) {
        typedef unsigned u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 v = __builtin_nontemporal_load(reinterpret_cast<const u32x3*>(src));
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z;
    } else if constexpr (W == 8) {
        const u32x4 v0 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src));
        const u32x4 v1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + 1);
        dst[0] = v0.x; dst[1] = v0.y; dst[2] = v0.z; dst[3] = v0.w;
        dst[4] = v1.x; dst[5] = v1.y; dst[6] = v1.z; dst[7] = v1.w;
    } else {
#pragma unroll
        for (int w = 0; w < W; ++w) dst[w] = __builtin_nontemporal_load(src + w);
    }
}


// Output block staging: the block's bf16 results (16 * MT rows x C columns)
// sit row-major in LDS with a row pitch of C + 8 elements (16-byte aligned
// rows; the 2-byte writes of the four lane quarters land 16 banks apart).
// store_tile then writes 16-byte row segments: eight consecutive columns of
// one member, when the address is 16-byte aligned; otherwise (a ragged N, a
// member boundary, an unaligned output) column by column.
__host__ __device__ constexpr int largest_divisor_at_most(int n, int cap) {
    int d = cap < n ? cap : n;
    while (d > 1 && n % d) --d;
    return d;
}

template <int J, int WV = kGemmWaves>
__host__ __device__ constexpr int tile_cols() { return WV * J * 16; }
template <int J, int WV = kGemmWaves>
__host__ __device__ constexpr int tile_pitch() { return tile_cols<J, WV>() + 8; }

// Output row m of a member, and a member's row stride, by constant indices
// into the argument arrays: indexing them with a register makes the compiler
// copy the whole argument block to private memory (scratch) in the
// register-heavy kernels.
__device__ __forceinline__ int64_t member_ldy(const GemmArgs& a, int member) {
    int64_t ld = a.ldys[0];
#pragma unroll
    for (int i = 1; i < kMaxGemmMembers; ++i)
        if (member == i) ld = a.ldys[i];
    return ld;
}

__device__ __forceinline__ uint16_t* member_row(const GemmArgs& a, int member, int64_t m) {
    uint16_t* y = a.ys[0];
#pragma unroll
    for (int i = 1; i < kMaxGemmMembers; ++i)
        if (member == i) y = a.ys[i];
    return y + m * member_ldy(a, member);
}

template <int J, int MT, int WV = kGemmWaves>
__device__ __forceinline__ void store_tile(const GemmArgs& a, const uint16_t* tile, int m0) {
    constexpr int C = tile_cols<J, WV>(), P = tile_pitch<J, WV>();
    constexpr int kThr = WV * kWave;
    constexpr int kSegs = C / 8, kChunks = 16 * MT * kSegs;
    const int n_base = blockIdx.x * C;
    const int rows = a.routed ? a.routes : a.m;
    // Whole block inside one member, in range and 16-byte aligned in every
    // row: the member, its pointer and its row stride are block-uniform
    // (scalar registers), and every segment is one 16-byte store.
    const int member0 = n_base / a.n_member;
    const int nl0 = n_base - member0 * a.n_member;
    if (n_base + C <= a.n && nl0 + C <= a.n_member) {
        uint16_t* y0 = member_row(a, member0, 0) + nl0;
        const int64_t ldy = member_ldy(a, member0);
        if (((reinterpret_cast<uintptr_t>(y0) | (uintptr_t)ldy * 2) & 15) == 0) {
#pragma unroll
            for (int i = 0; i < (kChunks + kThr - 1) / kThr; ++i) {
                const int c = threadIdx.x + kThr * i;
                if (c >= kChunks) break;
                const int row = c / kSegs, seg = c % kSegs;
                const int m = a.routed ? a.padded[m0 + row] : m0 + row;
                if (m >= rows) continue;
                *reinterpret_cast<uint4*>(y0 + (int64_t)m * ldy + seg * 8) =
                    *reinterpret_cast<const uint4*>(&tile[row * P + seg * 8]);
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < (kChunks + kThr - 1) / kThr; ++i) {
        const int c = threadIdx.x + kThr * i;
        if (c >= kChunks) break;
        const int row = c / kSegs, seg = c % kSegs;
        const int n = n_base + seg * 8;
        const int m = a.routed ? a.padded[m0 + row] : m0 + row;
        if (m >= rows || n >= a.n) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(&tile[row * P + seg * 8]);
        const int member = n / a.n_member;
        const int nl = n - member * a.n_member;
        uint16_t* y = member_row(a, member, m) + nl;
        if (nl + 8 <= a.n_member && n + 8 <= a.n && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
            *reinterpret_cast<uint4*>(y) = v;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int ne = n + e;
                if (ne < a.n) {
                    const int me = ne / a.n_member;
                    const uint32_t word = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
                    member_row(a, me, m)[ne - me * a.n_member] = (uint16_t)(word >> (16 * (e & 1)));
                }
            }
        }
    }
}

// Last arrival of a split-K output block: sums the S partitions of each unit
// in ascending K order into the LDS output tile.  Every partition load of a
// batch of units is in flight at once (the exchange is latency bound, not
// bandwidth bound); thread t owns units t, t + WV * 64, ...
template <int S, int J, int MT, bool F16, int WV = kGemmWaves>
__device__ __forceinline__ void reduce_partials(__amdgpu_buffer_rsrc_t part, int split_bytes, uint16_t* tile) {
    constexpr int kThr = WV * kWave;
    constexpr int kPer = J * MT;  // units per thread
    // at most 16 partition loads (64 registers) in flight: a larger batch
    // would set the whole kernel's register allocation, main loop included
    // (the batch divides the units per thread: a partial batch would read
    // past this block's partitions)
    constexpr int kCap = 16 / S > 0 ? 16 / S : 1;
    constexpr int kBatch = largest_divisor_at_most(kPer, kCap);
    static_assert(kBatch >= 1 && kPer % kBatch == 0, "whole batches of units");
    constexpr int P = tile_pitch<J, WV>();
#pragma unroll 1
    for (int b0 = 0; b0 < kPer; b0 += kBatch) {
        floatx4_dev_t v[kBatch][S];
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
#pragma unroll
            for (int sp = 0; sp < S; ++sp)
                v[b][sp] = load_device4(part, sp * split_bytes + ((b0 + b) * kThr + threadIdx.x) * 16);
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            floatx4_dev_t sum = v[b][0];
#pragma unroll
            for (int sp = 1; sp < S; ++sp) sum += v[b][sp];
            const int u = (b0 + b) * kThr + threadIdx.x;
            const int uw = u / (J * MT * kWave), uj = (u / (MT * kWave)) % J;
            const int umt = (u / kWave) % MT, ul = u % kWave;
            const int cl = (uw * J + uj) * 16 + (ul & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r)
                tile[(umt * 16 + 4 * (ul >> 4) + r) * P + cl] = out_bits<F16>(sum[r]);
        }
    }
}

// Second arrival of a two-partition output block: each thread adds the two
// partitions of the units it computed itself (its J x MT accumulators), in K
// order, reading the first arrival's partials from the workspace and taking
// its own partition `mine` from its registers.
template <int J, int MT, bool F16, int WV = kGemmWaves>
__device__ __forceinline__ void reduce_pair(__amdgpu_buffer_rsrc_t part, int split_bytes, int mine,
                                            const floatx4_t (&acc)[MT][J], uint16_t* tile, int wave, int lane) {
    constexpr int kPer = J * MT;
    constexpr int kBatch = largest_divisor_at_most(kPer, 8);
    constexpr int P = tile_pitch<J, WV>();
    const int q = lane >> 4, col = lane & 15;
    const int other = (1 - mine) * split_bytes;
#pragma unroll
    for (int b0 = 0; b0 < kPer; b0 += kBatch) {
        floatx4_dev_t v[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int u = b0 + b, j = u / MT, mt = u % MT;
            v[b] = load_device4(part, other + (((wave * J + j) * MT + mt) * kWave + lane) * 16);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int u = b0 + b, j = u / MT, mt = u % MT;
            const floatx4_dev_t own = acc[mt][j];
            const floatx4_dev_t sum = mine == 0 ? own + v[b] : v[b] + own;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                tile[(mt * 16 + 4 * q + r) * P + (wave * J + j) * 16 + col] = out_bits<F16>(sum[r]);
        }
    }
}

// Output of one block: split = 1 stores bf16 through the LDS tile; a K split
// stores the FP32 accumulators in the MFMA-native layout (one 16-byte unit per
// tile, m-tile and lane) and the last arrival sums the K partitions in
// ascending order.  `tile` is LDS no longer in use by any wave's main loop.
template <int J, int MT, bool F16, int WV = kGemmWaves>
__device__ __forceinline__ void finish_block(const GemmArgs& a, const floatx4_t (&acc)[MT][J], uint16_t* tile,
                                             int m0, int wave, int lane) {
    const int q = lane >> 4, col = lane & 15;
    if (a.split == 1) {
        constexpr int P = tile_pitch<J, WV>();
        __syncthreads();
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    tile[(mt * 16 + 4 * q + r) * P + (wave * J + j) * 16 + col] =
                        out_bits<F16>(acc[mt][j][r]);
        __syncthreads();
        store_tile<J, MT, WV>(a, tile, m0);
        return;
    }
    constexpr int kUnits = WV * J * MT * kWave;  // float4 units per output block
    const int block = blockIdx.z * gridDim.x + blockIdx.x;
    const int split_bytes = (int)(gridDim.x * gridDim.z) * kUnits * 16;  // < 2^31: split > 1 only below 256 blocks of <= 64 KiB
    const __amdgpu_buffer_rsrc_t part =
        device_rsrc(reinterpret_cast<char*>(a.partials) + (int64_t)block * kUnits * 16);
    const auto store_partials = [&]() {
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                store_device4(part, blockIdx.y * split_bytes + (((wave * J + j) * MT + mt) * kWave + lane) * 16,
                              acc[mt][j]);
    };
    if (a.split == 2) {
        // Two partitions: the block's counter word counts arrivals in its low
        // half and stored partitions in its high half.  A workgroup takes its
        // arrival ticket first; the first stores its FP32 partials (device-
        // scope stores, performed before the count goes up) and counts
        // itself stored; the second never stores: it waits until the first
        // is stored and sums both in K order, its own from registers.  (With
        // more partitions the last arrival waits on the slowest of several
        // partners' ticket-then-store sequences, which measured slower than
        // storing first.)
        __shared__ uint32_t ticket;
        __syncthreads();
        if (threadIdx.x == 0)
            ticket = __hip_atomic_fetch_add(&a.counters[block], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                     0xFFFFu;
        __syncthreads();
        if (ticket == 0) {
            store_partials();
            __builtin_amdgcn_s_waitcnt(0);  // this thread's partials are performed
            __syncthreads();
            if (threadIdx.x == 0)
                __hip_atomic_fetch_add(&a.counters[block], 1u << 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        if (threadIdx.x == 0) {
            // the first has taken its ticket, so it is running and only has
            // its stores left; the bound only keeps a broken workspace (a
            // counter not zero at launch) from spinning forever
            for (int spin = 0; spin < (1 << 24) && (load_device(&a.counters[block]) >> 16) == 0u; ++spin)
                __builtin_amdgcn_s_sleep(1);
        }
        __syncthreads();
        reduce_pair<J, MT, F16, WV>(part, split_bytes, (int)blockIdx.y, acc, tile, wave, lane);
    } else {
        store_partials();
        __shared__ uint32_t last;
        if (!arrive_last(&a.counters[block], (uint32_t)a.split, &last)) return;
        switch (a.split) {  // arrive_last's barriers leave the tile free
            case 3: reduce_partials<3, J, MT, F16, WV>(part, split_bytes, tile); break;
            case 4: reduce_partials<4, J, MT, F16, WV>(part, split_bytes, tile); break;
            case 5: reduce_partials<5, J, MT, F16, WV>(part, split_bytes, tile); break;
            case 6: reduce_partials<6, J, MT, F16, WV>(part, split_bytes, tile); break;
            case 7: reduce_partials<7, J, MT, F16, WV>(part, split_bytes, tile); break;
            default: reduce_partials<8, J, MT, F16, WV>(part, split_bytes, tile); break;
        }
    }
    if (threadIdx.x == 0) store_device(&a.counters[block], 0u);
    __syncthreads();
    store_tile<J, MT, WV>(a, tile, m0);
}

}  // namespace gemm
}  // namespace cubic
