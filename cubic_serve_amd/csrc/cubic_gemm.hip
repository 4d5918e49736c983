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
// FP32 accumulation runs in MFMA; K partitions (fixed by N and K only) are
// summed in ascending order by the last workgroup of each output block.
#include "cubic_device.h"
#include "cubic_capi_internal.h"

namespace cubic {
namespace {

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kKBlock = 128;
constexpr int kALd = kKBlock + 8;  // LDS row pitch in bf16 (16-byte pad: conflict-free b128 reads)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float floatx4_t;

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// fl32(m / D) with the division done in binary64 and rounded once to binary32,
// as reference.py:120 does.  Evaluated at compile time for unrolled m.
template <int BITS>
__host__ __device__ constexpr float t_of(int m) {
    return (float)((double)m / (double)((1 << (BITS - 1)) - 1));
}

// One Cubic level: s * (t * (a + t * (b + t * ((1 - a) - b)))), unfused fp32.
__device__ __forceinline__ float curve_level(float t, float s, float a, float b) {
    const float c = (1.0f - a) - b;
    const float inner = b + t * c;
    const float mid = a + t * inner;
    return s * (t * mid);
}

// ---------------------------------------------------------------------------
// Level tables for bits <= 4: magnitudes 0..7 -> bf16, split into low-byte and
// high-byte planes so one v_perm_b32 looks up four magnitudes.
// ---------------------------------------------------------------------------
struct LevelTable {
    uint32_t lo_lo, lo_hi, hi_lo, hi_hi;  // low bytes of L0..3, L4..7; high bytes of L0..3, L4..7
};

template <int BITS>
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
    return pack_bf16x2(l0, l1);
}

template <int BITS>
__device__ __forceinline__ uint32_t level_pair_dyn(int q, float s, float a, float b) {
    // q in 0..3 selects the pair (2q, 2q + 1); unrolled so t stays a constant
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i == q) r = level_pair<BITS>(2 * i, s, a, b);
    return r;
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

// Table for this lane's (column, group).  When a group spans the whole
// 128-k block the four lanes sharing it (l, l^16, l^32, l^48) each evaluate
// one level pair and exchange them; otherwise the lane evaluates all pairs.
template <int BITS>
__device__ __forceinline__ LevelTable make_table(float s, float a, float b, int lane, bool shared) {
    if (shared) {
        const int q = lane >> 4;
        const uint32_t mine = level_pair_dyn<BITS>(q, s, a, b);
        const int base = lane & 15;
        const uint32_t p0 = __shfl(mine, base);
        const uint32_t p1 = __shfl(mine, base + 16);
        const uint32_t p2 = __shfl(mine, base + 32);
        const uint32_t p3 = __shfl(mine, base + 48);
        return table_from_pairs(p0, p1, p2, p3);
    }
    const uint32_t p0 = level_pair<BITS>(0, s, a, b);
    const uint32_t p1 = BITS >= 3 ? level_pair<BITS>(2, s, a, b) : 0u;
    const uint32_t p2 = BITS >= 4 ? level_pair<BITS>(4, s, a, b) : 0u;
    const uint32_t p3 = BITS >= 4 ? level_pair<BITS>(6, s, a, b) : 0u;
    return table_from_pairs(p0, p1, p2, p3);
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

template <int BITS>
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
        out[h] = pack_bf16x2(v[0], v[1]) ^ (sg[0] | (sg[1] << 16));
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

// ---------------------------------------------------------------------------
// GEMM kernel
//   grid.x: column blocks of 4 waves x J tiles x 16 columns
//   grid.y: K partitions (split)
//   grid.z: 64-row chunks of M
// ---------------------------------------------------------------------------
template <int BITS, int MT, int J>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmArgs a) {
    constexpr int W = BITS;  // code words per lane per (tile, k-block)
    __shared__ __attribute__((aligned(16))) uint16_t a_lds[2][64 * kALd];
    __shared__ float t_lds[128];

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int q = lane >> 4, col = lane & 15;
    const int tile0 = (blockIdx.x * 4 + wave) * J;
    const int split = blockIdx.y;
    const int m0 = blockIdx.z * 64;
    const int kb_begin = split * a.blocks_per_split;
    const int kb_end = min(kb_begin + a.blocks_per_split, a.k_blocks);

    if constexpr (BITS >= 5) {
        for (int i = threadIdx.x; i < (1 << (BITS - 1)); i += kThreads)
            t_lds[i] = (float)((double)i / (double)((1 << (BITS - 1)) - 1));
    }

    floatx4_t acc[MT][J];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[mt][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // --- per-k-block loads -------------------------------------------------
    uint32_t nxt_codes[J][W];
    uint32_t nxt_meta[J][2];
    uint4 nxt_a[4];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int nt = tile0 + j;
            if (nt < a.n_tiles) {
                const uint32_t* src = a.codes + (((int64_t)nt * a.k_blocks + kb) * kWave + lane) * W;
#pragma unroll
                for (int w = 0; w < W; ++w) nxt_codes[j][w] = src[w];
                const int g = (kb * kKBlock + 32 * q) / a.group_in;
                const uint32_t* ms = a.meta + (((int64_t)nt * a.groups_k + g) * 16 + col) * 2;
                nxt_meta[j][0] = ms[0];
                nxt_meta[j][1] = ms[1];
            } else {
#pragma unroll
                for (int w = 0; w < W; ++w) nxt_codes[j][w] = 0u;
                nxt_meta[j][0] = nxt_meta[j][1] = 0u;
            }
        }
        // activations: 64 rows x 128 k = 1024 chunks of 8 bf16, 4 per thread
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int chunk = threadIdx.x + kThreads * i;
            const int r = chunk >> 4, c8 = (chunk & 15) * 8;
            const int m = m0 + r, k = kb * kKBlock + c8;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (r < MT * 16 && m < a.m) {
                const uint16_t* src = a.x + (int64_t)m * a.ldx + k;
                if (k + 8 <= a.k) {
                    v = *reinterpret_cast<const uint4*>(src);
                } else if (k < a.k) {
                    uint32_t wv[4] = {0, 0, 0, 0};
                    for (int e = 0; e < 8; ++e)
                        if (k + e < a.k) wv[e >> 1] |= (uint32_t)src[e] << ((e & 1) * 16);
                    v = make_uint4(wv[0], wv[1], wv[2], wv[3]);
                }
            }
            nxt_a[i] = v;
        }
    };

    if (kb_begin < kb_end) load_block(kb_begin);
    const bool shared_groups = (a.group_in % kKBlock) == 0;
    int buf = 0;
    for (int kb = kb_begin; kb < kb_end; ++kb) {
        // publish this block's activations, take its codes/metadata
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int chunk = threadIdx.x + kThreads * i;
            const int r = chunk >> 4, c8 = (chunk & 15) * 8;
            if (r < MT * 16)
                *reinterpret_cast<uint4*>(&a_lds[buf][r * kALd + c8]) = nxt_a[i];
        }
        uint32_t codes[J][W];
        uint32_t meta[J][2];
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
            for (int w = 0; w < W; ++w) codes[j][w] = nxt_codes[j][w];
            meta[j][0] = nxt_meta[j][0];
            meta[j][1] = nxt_meta[j][1];
        }
        __syncthreads();
        if (kb + 1 < kb_end) load_block(kb + 1);

        // level tables for this block
        LevelTable tab[J];
        float ms[J], ma[J], mb[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            ms[j] = __uint_as_float(meta[j][0]);
            ma[j] = half_bits_to_float(meta[j][1] & 0xFFFFu);
            mb[j] = half_bits_to_float(meta[j][1] >> 16);
            if constexpr (BITS <= 4) tab[j] = make_table<BITS>(ms[j], ma[j], mb[j], lane, shared_groups);
        }

        const uint16_t* abase = &a_lds[buf][col * kALd + 32 * q];
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            bf16x8_t afrag[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const uint4 v = *reinterpret_cast<const uint4*>(abase + mt * 16 * kALd + 8 * f);
                afrag[mt] = __builtin_bit_cast(bf16x8_t, v);
            }
#pragma unroll
            for (int j = 0; j < J; ++j) {
                uint4 bw;
                if constexpr (BITS <= 4)
                    bw = decode_fragment<BITS>(codes[j], f, tab[j]);
                else
                    bw = direct_fragment<BITS>(codes[j], f, ms[j], ma[j], mb[j], t_lds);
                const bf16x8_t bfrag = __builtin_bit_cast(bf16x8_t, bw);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag[mt], bfrag,
                                                                         acc[mt][j], 0, 0, 0);
            }
        }
        buf ^= 1;
    }

    // --- epilogue -----------------------------------------------------------
    if (a.split == 1) {
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int n = (tile0 + j) * 16 + col;
            if (n >= a.n) continue;
            uint16_t* y = n < a.n_split ? a.y0 + n : a.y1 + (n - a.n_split);
            const int64_t ldy = n < a.n_split ? a.ldy0 : a.ldy1;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = m0 + mt * 16 + 4 * q + r;
                    if (m < a.m) y[(int64_t)m * ldy] = (uint16_t)float_to_bf16_bits(acc[mt][j][r]);
                }
        }
        return;
    }
    // split-K: FP32 partials [split][m][n], then the last arrival sums them in order
    float* part = a.partials + (int64_t)split * a.m * a.n;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int n = (tile0 + j) * 16 + col;
        if (n >= a.n) continue;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + mt * 16 + 4 * q + r;
                if (m < a.m) part[(int64_t)m * a.n + n] = acc[mt][j][r];
            }
    }
    __shared__ uint32_t last;
    __threadfence();
    __syncthreads();
    const int counter = blockIdx.z * gridDim.x + blockIdx.x;
    if (threadIdx.x == 0) last = atomicAdd(&a.counters[counter], 1u) == (uint32_t)(a.split - 1);
    __syncthreads();
    if (!last) return;
    __threadfence();
    const int cols = 4 * J * 16, rows = MT * 16;
    const int n0 = blockIdx.x * cols;
    for (int e = threadIdx.x; e < rows * cols; e += kThreads) {
        const int m = m0 + e / cols, n = n0 + e % cols;
        if (m >= a.m || n >= a.n) continue;
        const int64_t off = (int64_t)m * a.n + n;
        float sum = a.partials[off];
        for (int sp = 1; sp < a.split; ++sp) sum = sum + a.partials[(int64_t)sp * a.m * a.n + off];
        const uint16_t bits = (uint16_t)float_to_bf16_bits(sum);
        if (n < a.n_split) a.y0[(int64_t)m * a.ldy0 + n] = bits;
        else a.y1[(int64_t)m * a.ldy1 + (n - a.n_split)] = bits;
    }
    if (threadIdx.x == 0) a.counters[counter] = 0u;
}

// ---------------------------------------------------------------------------
// Load-time preparation
// ---------------------------------------------------------------------------
// Metadata: per (column, group) words (scale, a | b << 16); padding columns 0.
__global__ void prepare_meta_kernel(const float* scale, const uint16_t* av, const uint16_t* bv,
                                    int64_t n, int groups_k, int n_tiles, uint32_t* meta) {
    const int64_t total = (int64_t)n_tiles * groups_k * 16;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % 16);
        const int64_t g = (i / 16) % groups_k, nt = i / (16 * (int64_t)groups_k);
        const int64_t row = nt * 16 + c;
        uint32_t w0 = 0, w1 = 0;
        if (row < n) {
            const int64_t src = row * groups_k + g;
            w0 = __float_as_uint(scale[src]);
            w1 = (uint32_t)av[src] | ((uint32_t)bv[src] << 16);
        }
        meta[2 * i] = w0;
        meta[2 * i + 1] = w1;
    }
}

// Signed code at logical k of row `row` (reference.py:31-47 semantics).
__device__ __forceinline__ int unpack_code(const uint8_t* rowp, int64_t row_bytes, int64_t k, int bits) {
    const int64_t pos = k * bits, byte = pos >> 3;
    const int shift = (int)(pos & 7);
    uint32_t v = rowp[byte] >> shift;
    if (shift + bits > 8) v |= (uint32_t)rowp[byte + 1 < row_bytes ? byte + 1 : row_bytes - 1] << (8 - shift);
    const uint32_t raw = v & ((1u << bits) - 1u);
    if (bits == 1) return (int)raw * 2 - 1;
    const int sign = 1 << (bits - 1);
    int q = (int)raw >= sign ? (int)raw - (1 << bits) : (int)raw;
    return q == -sign ? 0 : q;
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
__global__ void prepare_codes_kernel(const uint8_t* packed, const float* scale, const uint16_t* av,
                                     const uint16_t* bv, int64_t n, int64_t k, int group_in,
                                     int groups_k, int n_tiles, int k_blocks, uint32_t* codes) {
    const int64_t total = (int64_t)n_tiles * k_blocks * kWave;
    const int64_t row_bytes = (k * BITS + 7) / 8;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int lane = (int)(i % kWave);
        const int64_t kb = (i / kWave) % k_blocks, nt = i / ((int64_t)kWave * k_blocks);
        const int q = lane >> 4, col = lane & 15;
        const int64_t row = nt * 16 + col;
        const int64_t k0 = kb * kKBlock + 32 * q;
        int mag[32], neg[32];
        float s = 0.0f, a = 0.0f, b = 0.0f;
        if (row < n && k0 < k) {
            const int64_t g = k0 / group_in;
            s = scale[row * groups_k + g];
            a = half_bits_to_float(av[row * groups_k + g]);
            b = half_bits_to_float(bv[row * groups_k + g]);
        }
        const uint32_t sigma = BITS <= 4 ? level_sign_mask<BITS>(s, a, b) : 0u;
        for (int e = 0; e < 32; ++e) {
            int qv = 0;
            if (row < n && k0 + e < k) qv = unpack_code(packed + row * row_bytes, row_bytes, k0 + e, BITS);
            const int m = qv < 0 ? -qv : qv;
            mag[e] = m;
            if (BITS <= 4)  // stored sign = sign(q) xor sign(bf16(L[|q|]))
                neg[e] = (int)((qv < 0 ? 1u : 0u) ^ ((sigma >> (m & 7)) & 1u));
            else
                neg[e] = qv < 0;
        }
        uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        if (BITS == 4) {
            for (int f = 0; f < 4; ++f)
                for (int byte = 0; byte < 4; ++byte) {
                    const int ea = 8 * f + byte, eb = 8 * f + 4 + byte;
                    const uint32_t v = (uint32_t)(mag[ea] & 7) | ((uint32_t)neg[eb] << 3) |
                                       ((uint32_t)(mag[eb] & 7) << 4) | ((uint32_t)neg[ea] << 7);
                    w[f] |= v << (8 * byte);
                }
        } else if (BITS == 3 || BITS == 2 || BITS == 1) {
            for (int f = 0; f < 4; ++f)
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
            for (int e = 0; e < 32; ++e) {
                const uint32_t code = ((uint32_t)neg[e] << (BITS - 1)) | (uint32_t)mag[e];
                const int p = BITS * e, word = p >> 5, shift = p & 31;
                w[word] |= code << shift;
                if (shift + BITS > 32) w[word + 1] |= code >> (32 - shift);
            }
        }
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
        if (fmt == 0) {
            scale[i] = ((const float*)m0)[src];
            av[i] = ((const uint16_t*)m1)[src];
            bv[i] = ((const uint16_t*)m2)[src];
        } else if (fmt == 1) {
            const int8_t si = ((const int8_t*)m0)[src];
            const uint32_t ab = ((const uint8_t*)m1)[src];
            const int lo = (int)(ab & 15u), hi = (int)(ab >> 4);
            const float af = (float)(lo >= 8 ? lo - 16 : lo), bf = (float)(hi >= 8 ? hi - 16 : hi);
            scale[i] = (float)si * ((const float*)g0)[p];
            const float prod = af * ((const float*)g1)[p];
            av[i] = __half_as_ushort(__float2half_rn(1.0f + prod));
            bv[i] = __half_as_ushort(__float2half_rn(bf * ((const float*)g2)[p]));
        } else {
            const uint32_t md = ((const uint16_t*)m0)[src];
            scale[i] = half_bits_to_float((md & 0x3FFFu) << 1);
            av[i] = ((const uint16_t*)m1)[p * 4 + (md >> 14)];
            bv[i] = ((const uint16_t*)m2)[p * 4 + (md >> 14)];
        }
    }
}

template <int BITS, int MT>
hipError_t launch_j(const GemmArgs& a, int j, dim3 grid, hipStream_t s) {
    if (j == 4) gemm_kernel<BITS, MT, 4><<<grid, kThreads, 0, s>>>(a);
    else if (j == 2) gemm_kernel<BITS, MT, 2><<<grid, kThreads, 0, s>>>(a);
    else gemm_kernel<BITS, MT, 1><<<grid, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

template <int BITS>
hipError_t launch_bits(const GemmArgs& a, int mt, int j, dim3 grid, hipStream_t s) {
    if (mt == 1) return launch_j<BITS, 1>(a, j, grid, s);
    if (mt == 2) return launch_j<BITS, 2>(a, j, grid, s);
    return launch_j<BITS, 4>(a, j, grid, s);
}

}  // namespace

// MT (16-row tiles per 64-row chunk) follows m; J and the K split come from the
// host plan, which depends on (n, k) only so results are invariant to m.
hipError_t launch_gemm(const GemmArgs& a, hipStream_t s) {
    const int mt = a.m >= 33 ? 4 : (a.m >= 17 ? 2 : 1);
    const int rows_chunks = (a.m + 63) / 64;
    const int mt_eff = rows_chunks > 1 ? 4 : mt;
    const int j = a.tiles_per_wave;  // chosen by the host plan
    const int cols_per_block = 4 * j * 16;
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

hipError_t launch_prepare(const void* packed, const float* scale, const uint16_t* av,
                          const uint16_t* bv, int64_t n, int64_t k, int bits, int group_in,
                          uint32_t* codes, uint32_t* meta, hipStream_t s) {
    const int n_tiles = (int)((n + 15) / 16);
    const int k_blocks = (int)((k + kKBlock - 1) / kKBlock);
    const int groups_k = (int)((k + group_in - 1) / group_in);
    const int64_t code_threads = (int64_t)n_tiles * k_blocks * kWave;
    const int blocks = (int)((code_threads + 255) / 256 < 65535 ? (code_threads + 255) / 256 : 65535);
    const uint8_t* p = (const uint8_t*)packed;
    switch (bits) {
#define CUBIC_PREP(B) case B: prepare_codes_kernel<B><<<blocks, 256, 0, s>>>(p, scale, av, bv, n, k, group_in, groups_k, n_tiles, k_blocks, codes); break;
        CUBIC_PREP(1) CUBIC_PREP(2) CUBIC_PREP(3) CUBIC_PREP(4)
        CUBIC_PREP(5) CUBIC_PREP(6) CUBIC_PREP(7) CUBIC_PREP(8)
#undef CUBIC_PREP
        default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t meta_threads = (int64_t)n_tiles * groups_k * 16;
    const int mblocks = (int)((meta_threads + 255) / 256 < 65535 ? (meta_threads + 255) / 256 : 65535);
    prepare_meta_kernel<<<mblocks, 256, 0, s>>>(scale, av, bv, n, groups_k, n_tiles, meta);
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
