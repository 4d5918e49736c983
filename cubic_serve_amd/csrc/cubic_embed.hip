// Packed Cubic embedding lookup for gfx950: out[t, :] = decode(W[ids[t], :]).
//
// Reference semantics (paths under src/cubic_serve/ of QuantTrio/cubic-serve):
//   bind_embedding   ops/cuda/linear/quantized.py:786-846 (validation)
//   Cubic hook       quantization/extensions/cubic/linear.py:266-294
//   per-weight value quantization/extensions/cubic/kernels.py:44-113 (load_weight)
//   eager oracle     ops/eager/quantization.py:189-202 (embedding_matrix)
//
// The lookup reads the checkpoint payload as stored (no prepared copy of the
// table): one workgroup per (token, 4096-column slice), one thread per 16
// consecutive columns.  Sixteen columns of a row are 2 * bits consecutive bytes
// of the little-endian bitstream, so a wave reads one contiguous 128 * bits
// byte run and writes one contiguous 2 KiB run of the output row: HBM bound,
// with traffic = row bytes + metadata + 2 bytes per output column.
//
// Every value is the reference's unfused binary32 expression
//   (q < 0 ? -n : n) * scale,   n = t * (a + t * (b + t * ((1 - a) - b)))
// with t = fl32(|q| / D) (a per-workgroup LDS table), rounded once to the
// output dtype (RNE; v_cvt_pk_bf16_f32 for bf16).  bits = 1 is the bipolar
// code: (2 * raw - 1) * scale.
// Token ids outside [0, n) produce a zero row.
#include "cubic_device.h"
#include "cubic_capi_internal.h"

namespace cubic {
namespace {

constexpr int kEmbedThreads = 256;
constexpr int kEmbedCols = 16;  // columns per thread: 2 * bits bytes of the bitstream

// The 16 columns of chunk c are bits 16c*BITS .. 16(c+1)*BITS-1 of the row:
// 2*BITS bytes starting at byte 2c*BITS, returned as little-endian words.
template <int BITS>
__device__ __forceinline__ void load_chunk(const uint8_t* row, int64_t c, int64_t row_bytes,
                                           bool aligned, uint32_t (&w)[5]) {
    constexpr int kBytes = 2 * BITS;
    const int64_t off = c * kBytes;
#pragma unroll
    for (int i = 0; i < 5; ++i) w[i] = 0;
    if (aligned && off + kBytes <= row_bytes) {
        if constexpr (BITS % 2 == 0) {  // 4-byte aligned: BITS/2 dwords
#pragma unroll
            for (int i = 0; i < BITS / 2; ++i) w[i] = ((const uint32_t*)(row + off))[i];
        } else {                        // 2-byte aligned: BITS halfwords
#pragma unroll
            for (int i = 0; i < BITS; ++i)
                w[i >> 1] |= (uint32_t)((const uint16_t*)(row + off))[i] << (16 * (i & 1));
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kBytes; ++i)
        if (off + i < row_bytes) w[i >> 2] |= (uint32_t)row[off + i] << (8 * (i & 3));
}

template <int BITS>
__device__ __forceinline__ int raw_code(const uint32_t (&w)[5], int e) {
    const int p = e * BITS, word = p >> 5, sh = p & 31;
    const uint64_t pair = ((uint64_t)w[word + 1 < 5 ? word + 1 : 4] << 32) | w[word];
    return (int)((pair >> sh) & ((1u << BITS) - 1u));
}

// One value in the reference's order: (q < 0 ? -n : n) * s with
// n = t * (a + t * (b + t * c)), c = (1 - a) - b; bits = 1: (2 * raw - 1) * s.
template <int BITS>
__device__ __forceinline__ float cubic_value(int raw, const float* t_table, float s, float a,
                                             float b, float c) {
    if constexpr (BITS == 1) {
        return (float)(raw * 2 - 1) * s;
    } else {
        constexpr int kMags = 1 << (BITS - 1);
        int q = raw >= kMags ? raw - 2 * kMags : raw;
        if (q == -kMags) q = 0;  // reserved code
        const float t = t_table[q < 0 ? -q : q];
        const float nrm = t * (a + t * (b + t * c));
        return (q < 0 ? -nrm : nrm) * s;
    }
}

// Output bits of one value (bf16 or fp16, RNE).
__device__ __forceinline__ uint32_t out_bits(float v, bool fp16) {
    return fp16 ? float_to_f16_bits(v) : float_to_bf16_bits(v);
}

// LUT = true (bits <= 4-ish, group_in % 16 == 0, 2^bits * 4 <= group_in): the
// workgroup first evaluates every code of every group in its slice into an LDS
// table of output bits (the reference expression, once per (group, code)),
// then each column is one table read.  LUT = false evaluates every column.
template <int BITS, bool LUT>
__global__ __launch_bounds__(kEmbedThreads) void embedding_kernel(EmbedArgs a) {
    constexpr int kMags = 1 << (BITS - 1);
    constexpr int kSlice = kEmbedThreads * kEmbedCols;
    __shared__ float t_table[kMags];
    __shared__ uint16_t lut[LUT ? kSlice / 4 : 1];
    const int64_t token = blockIdx.x;
    const int64_t row = a.id_bytes == 8 ? ((const int64_t*)a.ids)[token]
                                        : (int64_t)((const int32_t*)a.ids)[token];
    const bool live = row >= 0 && row < a.n;  // uniform over the workgroup
    const int64_t c = (int64_t)blockIdx.y * kEmbedThreads + threadIdx.x;
    const int64_t col0 = c * kEmbedCols;
    // the row's codes are requested first: their latency overlaps the tables
    uint32_t w[5] = {0, 0, 0, 0, 0};
    if (live && col0 < a.k) load_chunk<BITS>(a.packed + row * a.row_bytes, c, a.row_bytes, a.aligned, w);
    if (BITS > 1) {
        for (int m = threadIdx.x; m < kMags; m += kEmbedThreads)
            t_table[m] = (float)((double)m / (double)(kMags - 1));
        __syncthreads();
    }
    const int p = live && a.fmt != 0 ? a.part_of_row[row] : 0;
    const int64_t meta_row = (row / a.group_out) * a.groups_k;
    const int64_t slice0 = (int64_t)blockIdx.y * kSlice;
    if constexpr (LUT) {
        if (live) {
            const int64_t g0 = slice0 / a.group_in;
            const int64_t left = a.groups_k - g0;
            const int groups = (int)(kSlice / a.group_in < left ? kSlice / a.group_in : left);
            for (int i = threadIdx.x; i < (groups << BITS); i += kEmbedThreads) {
                float s;
                uint16_t au, bu;
                group_metadata(a.fmt, a.m0, a.m1, a.m2, a.g0, a.g1, a.g2, meta_row + g0 + (i >> BITS), p,
                               s, au, bu);
                const float ga = half_bits_to_float(au), gb = half_bits_to_float(bu);
                lut[i] = (uint16_t)out_bits(
                    cubic_value<BITS>(i & ((1 << BITS) - 1), t_table, s, ga, gb, (1.0f - ga) - gb), a.out_fp16);
            }
        }
        __syncthreads();
    }
    if (col0 >= a.k) return;
    const int cnt = a.k - col0 < kEmbedCols ? (int)(a.k - col0) : kEmbedCols;
    uint32_t h[kEmbedCols / 2];
#pragma unroll
    for (int i = 0; i < kEmbedCols / 2; ++i) h[i] = 0;
    if (live) {
        if constexpr (LUT) {
            const uint16_t* tab = lut + (((col0 - slice0) / a.group_in) << BITS);
#pragma unroll
            for (int i = 0; i < kEmbedCols / 2; ++i)
                h[i] = (uint32_t)tab[raw_code<BITS>(w, 2 * i)] | ((uint32_t)tab[raw_code<BITS>(w, 2 * i + 1)] << 16);
        } else {
            float v[kEmbedCols];
            float s, ga, gb;
            uint16_t au, bu;
            if (a.chunk_in_group) {  // group_in % 16 == 0: one group per chunk
                group_metadata(a.fmt, a.m0, a.m1, a.m2, a.g0, a.g1, a.g2, meta_row + col0 / a.group_in, p,
                               s, au, bu);
                ga = half_bits_to_float(au);
                gb = half_bits_to_float(bu);
                const float gc = (1.0f - ga) - gb;
#pragma unroll
                for (int e = 0; e < kEmbedCols; ++e)
                    v[e] = cubic_value<BITS>(raw_code<BITS>(w, e), t_table, s, ga, gb, gc);
            } else {
                int64_t last_g = -1;
                s = ga = gb = 0.0f;
#pragma unroll
                for (int e = 0; e < kEmbedCols; ++e) v[e] = 0.0f;
                for (int e = 0; e < cnt; ++e) {
                    const int64_t g = (col0 + e) / a.group_in;
                    if (g != last_g) {
                        group_metadata(a.fmt, a.m0, a.m1, a.m2, a.g0, a.g1, a.g2, meta_row + g, p, s, au, bu);
                        ga = half_bits_to_float(au);
                        gb = half_bits_to_float(bu);
                        last_g = g;
                    }
                    v[e] = cubic_value<BITS>(raw_code<BITS>(w, e), t_table, s, ga, gb, (1.0f - ga) - gb);
                }
            }
#pragma unroll
            for (int i = 0; i < kEmbedCols / 2; ++i) {
                if (a.out_fp16)
                    h[i] = out_bits(v[2 * i], true) | (out_bits(v[2 * i + 1], true) << 16);
                else
                    h[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
            }
        }
    }
    uint16_t* dst = a.out + token * a.k + col0;
    if (cnt == kEmbedCols && ((uintptr_t)dst & 15) == 0) {
        uint4* d4 = (uint4*)dst;
        d4[0] = make_uint4(h[0], h[1], h[2], h[3]);
        d4[1] = make_uint4(h[4], h[5], h[6], h[7]);
    } else {
        for (int e = 0; e < cnt; ++e) dst[e] = (uint16_t)(h[e >> 1] >> (16 * (e & 1)));
    }
}

}  // namespace

int64_t embedding_column_blocks(int64_t k) {
    return (k + kEmbedCols * kEmbedThreads - 1) / (kEmbedCols * kEmbedThreads);
}

hipError_t launch_embedding(const EmbedArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)a.tokens, (unsigned)embedding_column_blocks(a.k));
    switch (a.bits) {
#define CUBIC_EMB(B) case B: \
    if (a.lut) embedding_kernel<B, true><<<grid, kEmbedThreads, 0, s>>>(a); \
    else embedding_kernel<B, false><<<grid, kEmbedThreads, 0, s>>>(a); \
    break;
        CUBIC_EMB(1) CUBIC_EMB(2) CUBIC_EMB(3) CUBIC_EMB(4)
        CUBIC_EMB(5) CUBIC_EMB(6) CUBIC_EMB(7) CUBIC_EMB(8)
#undef CUBIC_EMB
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cubic
