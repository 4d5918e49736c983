// MoE router and route compaction for gfx950 (the front of the routed-expert
// GEMM).
//
// Reference semantics (paths under src/cubic_serve/ of QuantTrio/cubic-serve):
//   router      ops/cuda/moe/fused.py:44-156 (_stable_topk_logits +
//               _sort_and_normalize_topk, fused as _stable_topk_routes),
//               bound by ops/cuda/moe/quantized.py:58-180
//   compaction  ops/cuda/moe/fused.py:174-199 (_compact_local_routes)
//
// Router, per row: the top_k experts by (logit desc, expert id asc); their
// logits and ids in that order; softmax over the selected logits (max
// subtracted, build-defined exp, ascending butterfly sum) and the (id, weight) pairs
// re-ordered by ascending expert id.  Rows at or past *active_rows, or with
// row_activity 0, publish logits 0, ids -1, route ids -1 and weights 0.
//
// Compaction: the routes owned by experts [first, first + experts) grouped by
// expert, in ascending route ordinal inside each expert (a stable counting
// sort), with per-expert counts, starts, block starts (blocks of block_m) and
// the total block count.  Unowned routes are skipped and never written.
#include "cubic_device.h"
#include "cubic_capi_internal.h"

namespace cubic {
namespace {

constexpr int kWave = 64;
constexpr int kRouteThreads = 256;
constexpr int kCompactWaves = 8;
constexpr int kCompactThreads = kCompactWaves * kWave;

// Ranking key of one logit: NaN ranks as -inf (finite logits are the
// contract; this keeps ranks a strict total order whatever the input).
__device__ __forceinline__ float rank_value(float x) { return x != x ? -__builtin_huge_valf() : x; }

template <typename T>
__device__ __forceinline__ T wave_inclusive_sum(T x, int lane) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const T y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(MoERouteArgs a) {
    __shared__ float value[kMaxRouteExperts];
    __shared__ float sel_logit[kWave];
    __shared__ int sel_id[kWave];
    const int row = blockIdx.x, t = threadIdx.x;
    const bool active = row < *a.active_rows && a.row_activity[row] > 0;  // uniform
    const uint16_t* src = a.logits + (int64_t)row * a.experts;
    for (int e = t; e < a.experts; e += kRouteThreads)
        value[e] = rank_value(a.logits_fp16 ? half_bits_to_float(src[e]) : bf16_bits_to_float(src[e]));
    __syncthreads();
    // rank of expert e: experts strictly ahead in (value desc, id asc)
    for (int e = t; e < a.experts; e += kRouteThreads) {
        const float v = value[e];
        int rank = 0;
#pragma unroll 8
        for (int j = 0; j < a.experts; ++j) {
            const float o = value[j];
            rank += (int)((uint32_t)(o > v) | ((uint32_t)(o == v) & (uint32_t)(j < e)));
        }
        if (rank < a.top_k) {
            sel_id[rank] = e;
            sel_logit[rank] = a.logits_fp16 ? half_bits_to_float(src[e]) : bf16_bits_to_float(src[e]);
        }
    }
    __syncthreads();
    if (t >= kWave) return;
    const int lane = t, k = a.top_k;
    const bool slot = lane < k;
    const float score = slot ? sel_logit[lane] : -__builtin_huge_valf();
    const int id = slot ? sel_id[lane] : 0x7FFFFFFF;
    if (slot) {
        a.top_logits[(int64_t)row * k + lane] = active ? score : 0.0f;
        a.top_ids[(int64_t)row * k + lane] = active ? id : -1;
    }
    // softmax over the selected logits: max, exp(s - max), butterfly sum
    const float mx = wave_max_f32(score);
    const float p = slot ? accept_expf(score - mx) : 0.0f;
    const float sum = wave_butterfly_sum(p, kWave);
    // output slot = number of selected ids below this one
    int out = 0;
    for (int j = 0; j < k; ++j) out += __shfl(id, j) < id ? 1 : 0;
    if (slot) {
        const float w = p / sum;
        const uint32_t wb = a.weights_fp16 ? float_to_f16_bits(w) : float_to_bf16_bits(w);
        a.route_ids[(int64_t)row * k + out] = active ? id : -1;
        a.route_weights[(int64_t)row * k + out] = active ? (uint16_t)wb : (uint16_t)0;
    }
}

// One workgroup of kCompactWaves waves.  Wave w owns the contiguous segment
// [w * seg, (w + 1) * seg) of route ordinals: a per-wave histogram, a scan
// over experts and waves, then an in-order walk that places each owned route
// at base[w][e] + (earlier routes of e in the segment).
__global__ __launch_bounds__(kCompactThreads) void moe_compact_kernel(MoECompactArgs a) {
    __shared__ int hist[kCompactWaves][kMaxCompactExperts];
    __shared__ int wave_totals[2][kCompactWaves];
    const int t = threadIdx.x, w = t / kWave, lane = t % kWave;
    const int experts = a.experts;
    for (int i = t; i < kCompactWaves * kMaxCompactExperts; i += kCompactThreads) (&hist[0][0])[i] = 0;
    __syncthreads();
    const int seg = ((a.routes + kCompactWaves - 1) / kCompactWaves + kWave - 1) / kWave * kWave;
    const int r0 = w * seg, r1 = min(a.routes, r0 + seg);
    for (int r = r0 + lane; r < r1; r += kWave) {
        const int64_t e = a.route_ids[r] - a.first_expert;
        if (e >= 0 && e < experts) atomicAdd(&hist[w][e], 1);
    }
    __syncthreads();
    // per expert: exclusive prefix over waves, count; then scans over experts
    // (each thread owns kPer consecutive experts)
    constexpr int kPer = kMaxCompactExperts / kCompactThreads;
    int cnt[kPer], blk[kPer], csum = 0, bsum = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = t * kPer + i;
        int run = 0;
        if (e < experts) {
#pragma unroll
            for (int v = 0; v < kCompactWaves; ++v) {
                const int h = hist[v][e];
                hist[v][e] = run;
                run += h;
            }
        }
        cnt[i] = run;
        blk[i] = (run + a.block_m - 1) / a.block_m;
        csum += cnt[i];
        bsum += blk[i];
    }
    const int cinc = wave_inclusive_sum(csum, lane), binc = wave_inclusive_sum(bsum, lane);
    if (lane == kWave - 1) { wave_totals[0][w] = cinc; wave_totals[1][w] = binc; }
    __syncthreads();
    int cbase = cinc - csum, bbase = binc - bsum;
    for (int v = 0; v < w; ++v) { cbase += wave_totals[0][v]; bbase += wave_totals[1][v]; }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = t * kPer + i;
        if (e < experts) {
            a.counts[e] = cnt[i];
            a.starts[e] = cbase;
            a.block_starts[e] = bbase;
#pragma unroll
            for (int v = 0; v < kCompactWaves; ++v) hist[v][e] += cbase;
        }
        cbase += cnt[i];
        bbase += blk[i];
    }
    if (t == kCompactThreads - 1) *a.total_blocks = bbase;
    __syncthreads();
    // in-order placement: peers = lanes of this 64-route chunk with the same expert
    for (int base = r0; base < r1; base += kWave) {
        const int r = base + lane;
        int64_t e = r < r1 ? a.route_ids[r] - a.first_expert : -1;
        const bool owned = e >= 0 && e < experts;
        uint64_t peers = __ballot(owned);
#pragma unroll
        for (int b = 0; b < kCompactExpertBits; ++b) {
            const uint64_t ones = __ballot(owned && ((e >> b) & 1));
            peers &= ((e >> b) & 1) ? ones : ~ones;
        }
        const uint64_t below = lane ? (~0ull >> (kWave - lane)) : 0ull;
        int pos = 0;
        if (owned) pos = hist[w][e] + __builtin_popcountll(peers & below);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // every lane has read its cursor
        if (owned) {
            a.row_map[pos] = r;
            if ((peers >> lane) == 1ull) hist[w][e] += __builtin_popcountll(peers);  // last peer
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
    }
}

}  // namespace

hipError_t launch_moe_route(const MoERouteArgs& a, hipStream_t s) {
    moe_route_kernel<<<a.rows, kRouteThreads, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_moe_compact(const MoECompactArgs& a, hipStream_t s) {
    moe_compact_kernel<<<1, kCompactThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace cubic
