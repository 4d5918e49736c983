// Device helpers shared by the Cubic GEMM and acceptance kernels (gfx950).
//
// Compile every file that includes this header with -ffp-contract=off: the
// Cubic decoder and the acceptance transform are specified as unfused IEEE
// binary32 operations.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace cubic {

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even binary32 -> bfloat16 bits (NaN stays a quiet NaN).
__device__ __forceinline__ uint32_t float_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Two binary32 -> packed bfloat16 pair (lo, hi), RNE, one instruction on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    typedef __attribute__((ext_vector_type(2))) float float2_t;
    const float2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));  // v_cvt_pk_bf16_f32
}

// Binary32 -> fp16 bits, RNE, of the binary32 value as computed: the empty asm
// pins the value, so the compiler cannot fold a producing multiply into the
// conversion (v_fma_mix*_f16 rounds once, where the reference rounds to
// binary32 and then to fp16; the two differ on ties of the fp16 grid).
__device__ __forceinline__ uint32_t float_to_f16_bits(float f) {
    asm volatile("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
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

// Per-group metadata of a Cubic payload as (scale f32, a f16 bits, b f16 bits)
// (quantization/extensions/cubic/reference.py:67-95; the same roundings as
// kernels.py:82-97).  src = (row / group_out) * groups_k + group; p = the
// row's output partition.
//   fmt 0: m0 scale f32, m1 a f16, m2 b f16
//   fmt 1: m0 scale i8, m1 ab u8 (two signed nibbles), g0..g2 partition globals f32
//   fmt 2: m0 e5m9 scale | curve << 14 u16, m1/m2 curve a/b f16 [partitions][4]
__device__ __forceinline__ void group_metadata(int fmt, const void* m0, const void* m1, const void* m2,
                                               const void* g0, const void* g1, const void* g2,
                                               int64_t src, int p, float& scale, uint16_t& a,
                                               uint16_t& b) {
    if (fmt == 0) {
        scale = ((const float*)m0)[src];
        a = ((const uint16_t*)m1)[src];
        b = ((const uint16_t*)m2)[src];
    } else if (fmt == 1) {
        const int8_t si = ((const int8_t*)m0)[src];
        const uint32_t ab = ((const uint8_t*)m1)[src];
        const int lo = (int)(ab & 15u), hi = (int)(ab >> 4);
        const float af = (float)(lo >= 8 ? lo - 16 : lo), bf = (float)(hi >= 8 ? hi - 16 : hi);
        scale = (float)si * ((const float*)g0)[p];
        const float prod = af * ((const float*)g1)[p];
        a = (uint16_t)float_to_f16_bits(1.0f + prod);
        b = (uint16_t)float_to_f16_bits(bf * ((const float*)g2)[p]);
    } else {
        const uint32_t md = ((const uint16_t*)m0)[src];
        scale = half_bits_to_float((md & 0x3FFFu) << 1);
        a = ((const uint16_t*)m1)[p * 4 + (md >> 14)];
        b = ((const uint16_t*)m2)[p * 4 + (md >> 14)];
    }
}

// exp for the acceptance transform: Cody & Waite (1980) two-constant additive
// reduction x = n*ln2 + r, |r| <= ln2/2, exp(r) by the degree-7 Taylor
// polynomial in Horner form, times 2^n.  Unfused binary32 operations in a
// fixed order, so every evaluation of the same x gives the same bits on the
// device and in the CPU restatement.
__device__ __forceinline__ float accept_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_huge_valf();
    if (x < -103.972084045410156f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    const float r = (x - n * 0.693359375f) - n * -2.12194440e-4f;
    float p = 1.98412698e-4f;
    p = 1.38888889e-3f + r * p;
    p = 8.33333377e-3f + r * p;
    p = 4.16666679e-2f + r * p;
    p = 1.66666672e-1f + r * p;
    p = 0.5f + r * p;
    p = 1.0f + r * p;
    p = 1.0f + r * p;
    const int e = (int)n;
    if (e > 127) {
        p = p * __uint_as_float((uint32_t)(e - 64 + 127) << 23);
        return p * __uint_as_float((uint32_t)(64 + 127) << 23);
    }
    if (e < -126) {
        p = p * __uint_as_float((uint32_t)(e + 64 + 127) << 23);
        return p * __uint_as_float((uint32_t)(-64 + 127) << 23);
    }
    return p * __uint_as_float((uint32_t)(e + 127) << 23);
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) first output word for
// counter (ordinal, 0, 0, 0) and key (key, 0), mapped to [0, 1) the way
// tl.rand does: int32 bit pattern, negative x -> -x-1, times 2^-31 (rounded
// constant 4.6566127342e-10).
// Two-word key (k0, k1) = (low, high) 32 bits of tl.rand's 64-bit seed.
__device__ __forceinline__ float philox_uniform2(uint32_t key_lo, uint32_t key_hi, uint32_t ordinal) {
    uint32_t c0 = ordinal, c1 = 0, c2 = 0, c3 = 0, k0 = key_lo, k1 = key_hi;
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        const uint64_t a = (uint64_t)0xD2511F53u * c0, b = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(b >> 32) ^ c1 ^ k0, n2 = (uint32_t)(a >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)b;
        c3 = (uint32_t)a;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    int64_t sv = (int32_t)c0;
    if (sv < 0) sv = -sv - 1;
    return (float)sv * 4.6566127342e-10f;
}

__device__ __forceinline__ float philox_uniform(uint32_t key, uint32_t ordinal) {
    return philox_uniform2(key, 0u, ordinal);
}

// ---------------------------------------------------------------------------
// Wave reductions in fixed orders (the CPU restatement follows the same
// orders).  DPP exchanges (gfx9 encodings): quad_perm [1,0,3,2] 0xB1,
// [2,3,0,1] 0x4E, row_half_mirror 0x141, row_mirror 0x140, row_shr:d 0x110+d,
// row_bcast:15 0x142, row_bcast:31 0x143.  A lane whose source is invalid,
// or whose row is masked off, reads 0.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_or_zero(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}

// Butterfly sum x[i] += x[i ^ m] for m = 1, 2, 4, ... < width (width a power of
// two <= 64): every lane of an aligned width-group ends with the group total.
// m = 4 and m = 8 read the half-row / row mirror: after the steps below m
// every lane of a quad (of an 8-group) holds the same value, so the mirror
// lane's value is the xor partner's.
// m = 16 and m = 32 use the gfx950 lane swaps: v_permlane16_swap exchanges the
// odd 16-lane rows of its first operand with the even rows of its second, and
// v_permlane32_swap the upper half of the first with the lower half of the
// second.  With x in both operands, lane i then holds {x[i], x[i ^ m]} in the
// two results, in an order that depends on i; IEEE addition is commutative, so
// their sum is x[i] + x[i ^ m] bit for bit.
__device__ __forceinline__ float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// x[i ^ 16] / x[i ^ 32] (lanes whose bit m is clear take the second result).
__device__ __forceinline__ uint32_t xor16_u32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (__lane_id() & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t xor32_u32(uint32_t x) {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (__lane_id() & 32) ? r[0] : r[1];
}

__device__ __forceinline__ float wave_butterfly_sum(float x, int width) {
    if (width > 1) x = x + dpp_or_zero<0xB1>(x);
    if (width > 2) x = x + dpp_or_zero<0x4E>(x);
    if (width > 4) x = x + dpp_or_zero<0x141>(x);
    if (width > 8) x = x + dpp_or_zero<0x140>(x);
    if (width > 16) x = xor16_sum(x);
    if (width > 32) x = xor32_sum(x);
    return x;
}

// Maximum over the 64 lanes (exact in any order; NaN-ignoring).
__device__ __forceinline__ float wave_max_f32(float x) {
    float o;
    o = dpp_or_zero<0xB1>(x); x = o > x ? o : x;
    o = dpp_or_zero<0x4E>(x); x = o > x ? o : x;
    o = dpp_or_zero<0x141>(x); x = o > x ? o : x;
    o = dpp_or_zero<0x140>(x); x = o > x ? o : x;
    o = __uint_as_float(xor16_u32(__float_as_uint(x))); x = o > x ? o : x;
    o = __uint_as_float(xor32_u32(__float_as_uint(x))); x = o > x ? o : x;
    return x;
}

// Maxima over the 64 lanes of unsigned keys (every lane ends with the maximum).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    uint32_t o;
    o = dpp_u32<0xB1>(v); v = o > v ? o : v;
    o = dpp_u32<0x4E>(v); v = o > v ? o : v;
    o = dpp_u32<0x141>(v); v = o > v ? o : v;
    o = dpp_u32<0x140>(v); v = o > v ? o : v;
    o = xor16_u32(v); v = o > v ? o : v;
    o = xor32_u32(v); v = o > v ? o : v;
    return v;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    auto step = [&](uint32_t olo, uint32_t ohi) {
        const uint64_t o = ((uint64_t)ohi << 32) | olo;
        v = o > v ? o : v;
    };
    step(dpp_u32<0xB1>((uint32_t)v), dpp_u32<0xB1>((uint32_t)(v >> 32)));
    step(dpp_u32<0x4E>((uint32_t)v), dpp_u32<0x4E>((uint32_t)(v >> 32)));
    step(dpp_u32<0x141>((uint32_t)v), dpp_u32<0x141>((uint32_t)(v >> 32)));
    step(dpp_u32<0x140>((uint32_t)v), dpp_u32<0x140>((uint32_t)(v >> 32)));
    step(xor16_u32((uint32_t)v), xor16_u32((uint32_t)(v >> 32)));
    step(xor32_u32((uint32_t)v), xor32_u32((uint32_t)(v >> 32)));
    return v;
}

// x[i ^ M] for M = 1, 2, 4, ..., 32 without an LDS permute: quad_perm for 1
// and 2; for 4 and 8 the lanes whose bit M is set take row_shr:M (lane i - M)
// and the others row_shl:M (lane i + M); the lane swaps for 16 and 32.
// Callers keep every lane of the wave active.
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (M == 1) return dpp_u32<0xB1>(v);
    else if constexpr (M == 2) return dpp_u32<0x4E>(v);
    else if constexpr (M == 4 || M == 8) {
        // both reads with every lane active (a read from a lane disabled by a
        // branch returns 0), then a bitwise blend rather than a select
        const uint32_t down = dpp_u32<0x110 + M>(v), up = dpp_u32<0x100 + M>(v);
        const uint32_t m = 0u - ((__lane_id() >> (M == 4 ? 2 : 3)) & 1u);
        return (down & m) | (up & ~m);
    }
    else if constexpr (M == 16) return xor16_u32(v);
    else return xor32_u32(v);
}
template <int M>
__device__ __forceinline__ uint64_t xor_lane(uint64_t v) {
    return ((uint64_t)xor_lane<M>((uint32_t)(v >> 32)) << 32) | xor_lane<M>((uint32_t)v);
}
__device__ __forceinline__ uint32_t xor_lane_rt(uint32_t v, int m) {
    switch (m) {
        case 1: return xor_lane<1>(v);
        case 2: return xor_lane<2>(v);
        case 4: return xor_lane<4>(v);
        case 8: return xor_lane<8>(v);
        case 16: return xor_lane<16>(v);
        default: return xor_lane<32>(v);
    }
}
__device__ __forceinline__ uint64_t xor_lane_rt(uint64_t v, int m) {
    switch (m) {
        case 1: return xor_lane<1>(v);
        case 2: return xor_lane<2>(v);
        case 4: return xor_lane<4>(v);
        case 8: return xor_lane<8>(v);
        case 16: return xor_lane<16>(v);
        default: return xor_lane<32>(v);
    }
}

// Value of lane l (wave-uniform l) without a cross-lane permute.
__device__ __forceinline__ float lane_f32(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Inclusive scan over the 64 lanes: inside each 16-lane row x[i] += x[i - d]
// for d = 1, 2, 4, 8 (i % 16 >= d); then rows 1 and 3 add lane 15 and lane 47;
// then rows 2 and 3 add lane 31.
__device__ __forceinline__ float wave_row_scan(float x) {
    x = x + dpp_or_zero<0x111>(x);
    x = x + dpp_or_zero<0x112>(x);
    x = x + dpp_or_zero<0x114>(x);
    x = x + dpp_or_zero<0x118>(x);
    x = x + dpp_or_zero<0x142, 0xA>(x);
    x = x + dpp_or_zero<0x143, 0xC>(x);
    return x;
}

// Cross-workgroup hand-off without a full cache write-back: the producer
// writes the exchanged words with device-scope atomic stores, drains its
// memory counters, then bumps an arrival counter; the last arrival reads the
// words with device-scope atomic loads.  (A device-scope fence would write
// back every dirty L2 line of the XCD instead.)
template <typename T>
__device__ __forceinline__ void store_device(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename T>
__device__ __forceinline__ T load_device(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 128-bit device-scope hand-off through buffer instructions: cache policy sc1
// makes the access coherent across the XCDs' L2s (what a device-scope atomic
// dword access compiles to), four words per instruction.
constexpr int kCpolDevice = 16;
typedef unsigned u32x4_dev_t __attribute__((ext_vector_type(4)));
typedef float floatx4_dev_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t device_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ void store_device4(__amdgpu_buffer_rsrc_t r, int byte_offset, floatx4_dev_t v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_dev_t, v), r, byte_offset, 0, kCpolDevice);
}

__device__ __forceinline__ floatx4_dev_t load_device4(__amdgpu_buffer_rsrc_t r, int byte_offset) {
    return __builtin_bit_cast(floatx4_dev_t, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, kCpolDevice));
}

// Called by every thread after its store_device() writes; returns true in
// every thread of the workgroup that arrives last (count = expected arrivals).
// The caller resets the counter to zero when it is done.
__device__ __forceinline__ bool arrive_last(uint32_t* counter, uint32_t expected, uint32_t* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's device-scope stores are performed
    __syncthreads();
    if (threadIdx.x == 0)
        *lds_flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    expected - 1;
    __syncthreads();
    return *lds_flag != 0;
}

}  // namespace cubic
