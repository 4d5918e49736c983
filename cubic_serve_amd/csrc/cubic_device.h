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

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
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
__device__ __forceinline__ float philox_uniform(uint32_t key, uint32_t ordinal) {
    uint32_t c0 = ordinal, c1 = 0, c2 = 0, c3 = 0, k0 = key, k1 = 0;
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
