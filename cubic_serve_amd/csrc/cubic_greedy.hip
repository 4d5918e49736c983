// Greedy sampling for non-speculative decode on gfx950: exact argmax over the
// vocabulary (lowest token id on ties) with a finiteness guard, the root
// decision over gathered candidates, and the batch-wide final guard.
//
// Reference semantics (paths under src/cubic_serve/ of QuantTrio/cubic-serve):
//   candidates   ops/cuda/sampling/greedy.cu:14-53 (greedy_partial) and
//                :55-78 (greedy_merge), bound by greedy.py:230-283
//   root         greedy.cu:91-114 (greedy_root), bound by greedy.py:284-303
//   final guard  greedy.cu:117-139 (sampling_final_guard), greedy.py:304-320
//
// The candidate pass is one launch over (tile, row) workgroups: each reduces
// its vocabulary tile to one ordering key and a finiteness flag, and the last
// workgroup of a row merges the tiles and publishes the row.  In the fused
// single-GPU composition (cubic_greedy_sample) that workgroup also takes the
// root decision for its row and contributes the row's guard term; the last
// row to finish writes the batch validity.  Arrival counters live in the
// caller's workspace and return to zero when a launch completes.
#include "cubic_device.h"
#include "cubic_capi_internal.h"

namespace cubic {
namespace {

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kLoadElems = 8;                       // one 16-byte load
constexpr int kRound = kThreads * kLoadElems;       // elements per load round
constexpr uint32_t kNanBf16 = 0x7FC0u, kNanF16 = 0x7E00u;

// Order of a sign-magnitude 16-bit float (bf16 and fp16 alike): compares like
// the values, -0 and +0 equal, NaN patterns above +inf / below -inf (they are
// only ever chosen in rows the finiteness guard rejects).
__device__ __forceinline__ uint32_t order16(uint32_t u) {
    const uint32_t m = u & 0x7FFFu;
    return (u & 0x8000u) ? 0x8000u - m : 0x8000u + m;
}
__device__ __forceinline__ uint32_t bits_of_order16(uint32_t k) {
    return k >= 0x8000u ? k - 0x8000u : (0x8000u | (0x8000u - k));
}

// Tile-local composite of an element: order16 in the high half, 0xFFFF minus
// the element's index inside its tile in the low half (larger = lower index on
// equal values; tiles hold at most 65536 columns).  Zero is reserved for
// "nothing admitted": every finite value has order16 >= 0x81.

// Two sign-magnitude 16-bit values -> two order keys, packed 16-bit ops:
// 0x8000 + |u| for positive, 0x8000 - |u| for negative (-0 == +0).
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t order16x2(uint32_t w, uint32_t mag) {
    const u16x2_t m = __builtin_bit_cast(u16x2_t, mag);
    const u16x2_t bias = {0x8000, 0x8000};
    const uint32_t pos = __builtin_bit_cast(uint32_t, (u16x2_t)(bias + m));
    const uint32_t neg = __builtin_bit_cast(uint32_t, (u16x2_t)(bias - m));
    const uint32_t sgn = __builtin_bit_cast(uint32_t, (i16x2_t)(__builtin_bit_cast(i16x2_t, w) >> 15));
    return (sgn & neg) | (~sgn & pos);
}
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
    const u16x2_t x = __builtin_bit_cast(u16x2_t, a), y = __builtin_bit_cast(u16x2_t, b);
    return __builtin_bit_cast(uint32_t, (u16x2_t)__builtin_elementwise_max(x, y));
}

// Row key of a column across tiles: order16, then lower column first.
__device__ __forceinline__ uint64_t column_key(uint32_t order, uint32_t col) {
    return ((uint64_t)order << 32) | (0xFFFFFFFFu - col);
}
__device__ __forceinline__ uint32_t column_of_key(uint64_t key) {
    return 0xFFFFFFFFu - (uint32_t)key;
}

template <bool HALF>
__device__ __forceinline__ bool nonfinite16(uint32_t u) {
    return HALF ? (u & 0x7C00u) == 0x7C00u : (u & 0x7F80u) == 0x7F80u;
}

__device__ __forceinline__ bool wave_all(bool p) {
    return __builtin_amdgcn_ballot_w64(!p) == 0;
}

// Workgroup maximum of a key and AND of a flag; every thread gets both.
struct KeyFlag {
    uint64_t key;
    uint32_t good;
};
template <int WAVES = kWaves>
__device__ __forceinline__ KeyFlag block_reduce(uint64_t key, bool good, uint64_t* lds_key,
                                                uint32_t* lds_good) {
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    key = wave_max_u64(key);
    good = wave_all(good);
    if (lane == 0) { lds_key[w] = key; lds_good[w] = good; }
    __syncthreads();
    KeyFlag r = {lds_key[0], lds_good[0]};
#pragma unroll
    for (int i = 1; i < WAVES; ++i) {
        r.key = lds_key[i] > r.key ? lds_key[i] : r.key;
        r.good &= lds_good[i];
    }
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// Root decision for one row (greedy.cu:106-110): a row is sampled when every
// gathered candidate is real (finite, 0 <= id < vocab) or padding (NaN, -1),
// at least one is real, and the row's parameters are admissible for greedy
// sampling (temperature exactly 0, top_p in (0, 1], 1 <= top_k <= K,
// non-negative seed and ordinal).  Rows past the active count publish -1,
// except the row at the active count of a cancelled batch, which publishes -2.
// ---------------------------------------------------------------------------
struct RowParams {
    float t, top_p;
    int64_t top_k, seed, ordinal;
};
__device__ __forceinline__ RowParams row_params(const GreedyParams& p, int row) {
    return {p.temperatures[row], p.top_ps[row], p.top_ks[row], p.seeds[row], p.ordinals[row]};
}
__device__ __forceinline__ bool sampling_params_ok(const RowParams& r, int k) {
    return __builtin_isfinite(r.top_p) && r.top_p > 0.0f && r.top_p <= 1.0f && r.top_k >= 1 &&
           r.top_k <= k && r.seed >= 0 && r.ordinal >= 0;
}

struct RowDecision {
    int64_t token;
    bool valid;
};
__device__ __forceinline__ RowDecision root_decision(const RowParams& r, int k, int row, int active,
                                                     int cancel, bool good, bool any_real,
                                                     int64_t best_id) {
    if (row >= active) return {(cancel && row == active) ? -2 : -1, false};
    const bool ok = good && any_real && r.t == 0.0f && sampling_params_ok(r, k);
    return {ok ? best_id : -1, ok};
}

// One row's term of the final guard (greedy.cu:121-130); r is read only for
// rows below the active count.
__device__ __forceinline__ bool guard_term(const RowParams& r, int k, int64_t vocab_size, int i,
                                           int active, int64_t token, bool root_valid) {
    if (i < active)
        return token >= 0 && token < vocab_size && root_valid && __builtin_isfinite(r.t) &&
               r.t >= 0.0f && r.t <= 2.0f && sampling_params_ok(r, k);
    return i == active ? (token == -1 || token == -2) : token == -1;
}

// ---------------------------------------------------------------------------
// Candidate pass.  Grid (tiles, rows).  Rows at or past the active count read
// no logits.  Column j of a row is admitted when the grammar mask (if any)
// allows token vocab_start + j; every visible column counts for finiteness.
// ---------------------------------------------------------------------------
template <int NT, int UNROLL, bool HALF, bool MASK, bool FUSED>
__global__ __launch_bounds__(NT) void greedy_kernel(GreedyArgs a) {
    constexpr int kUnroll = UNROLL;                     // load rounds in flight
    constexpr int kRoundNT = NT * kLoadElems;           // elements per load round
    constexpr int kWavesNT = NT / kWave;
    __shared__ uint64_t lds_key[kWavesNT];
    __shared__ uint32_t lds_good[kWavesNT];
    __shared__ uint32_t last;
    const int tile = blockIdx.x, row = blockIdx.y;
    // the root decision's inputs, fetched while the logits stream
    RowParams rp = {};
    int cancel = 0;
    if (FUSED && threadIdx.x == 0) {
        rp = row_params(a.p, row);
        cancel = a.metadata[1];
    }
    const int active = a.metadata[0];
    const uint32_t begin = (uint32_t)tile * a.tile_width;
    const uint32_t first = begin + threadIdx.x * kLoadElems;   // this thread's first column
    // acc[e]: best composite among this thread's elements at offset e of its
    // 8-column groups: order16 << 16 | (0xFFFF - load round), so equal values
    // keep the earlier round (the lower column)
    uint32_t acc[kLoadElems] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t mag_max = 0;                 // packed running max of |u| (finiteness)
    bool good = true;
    if (row < active) {
        const uint32_t end = min(begin + (uint32_t)a.tile_width, (uint32_t)a.width);
        const uint16_t* src = a.logits + (int64_t)row * a.row_stride;
        const uint32_t* mask_row = MASK ? a.token_mask + (int64_t)row * a.mask_words : nullptr;
        uint32_t round = 0;
        for (uint32_t base = first; base < end; base += kUnroll * kRoundNT, round += kUnroll) {
            uint4 v[kUnroll];
#pragma unroll
            for (int r = 0; r < kUnroll; ++r) {
                const uint32_t j = base + r * kRoundNT;
                if (a.vector_loads && j + kLoadElems <= end) {
                    v[r] = *reinterpret_cast<const uint4*>(src + j);
                } else {
                    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int e = 0; e < kLoadElems; ++e)
                        if (j + e < end) w[e / 2] |= (uint32_t)src[j + e] << (16 * (e % 2));
                    v[r] = make_uint4(w[0], w[1], w[2], w[3]);
                }
            }
#pragma unroll
            for (int r = 0; r < kUnroll; ++r) {
                const uint32_t j = base + r * kRoundNT;
                const uint32_t c = 0xFFFFu - (round + r);
                const uint32_t words[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
                if (!MASK && j + kLoadElems <= end) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t mag = words[q] & 0x7FFF7FFFu;
                        mag_max = max_u16x2(mag_max, mag);
                        const uint32_t ko = order16x2(words[q], mag);
                        acc[2 * q] = max(acc[2 * q], (ko << 16) | c);
                        acc[2 * q + 1] = max(acc[2 * q + 1], (ko & 0xFFFF0000u) | c);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < kLoadElems; ++e) {
                        const uint32_t u = (words[e / 2] >> (16 * (e % 2))) & 0xFFFFu;
                        if (j + e < end) {
                            good &= !nonfinite16<HALF>(u);
                            bool admitted = true;
                            if constexpr (MASK) {
                                const int64_t token = a.vocab_start + j + e;
                                admitted = (mask_row[token >> 5] >> (token & 31)) & 1u;
                                if (a.masked)
                                    a.masked[(int64_t)row * a.masked_stride + j + e] =
                                        admitted ? (uint16_t)u : (uint16_t)(HALF ? 0xFC00u : 0xFF80u);
                            }
                            if (admitted) acc[e] = max(acc[e], (order16(u) << 16) | c);
                        }
                    }
                }
            }
        }
    }
    if (MASK && a.masked && !a.masked_inplace && row >= active) {
        // rows past the active count: every visible column of the tile is -inf
        const uint32_t end = min(begin + (uint32_t)a.tile_width, (uint32_t)a.width);
        for (uint32_t j = begin + threadIdx.x; j < end; j += NT)
            a.masked[(int64_t)row * a.masked_stride + j] = (uint16_t)(HALF ? 0xFC00u : 0xFF80u);
    }
    good &= max(mag_max & 0xFFFFu, mag_max >> 16) < (HALF ? 0x7C00u : 0x7F80u);
    uint64_t key = 0;
#pragma unroll
    for (int e = 0; e < kLoadElems; ++e) {
        const uint32_t col = first + (0xFFFFu - (acc[e] & 0xFFFFu)) * kRoundNT + e;
        const uint64_t k = acc[e] ? column_key(acc[e] >> 16, col) : 0;
        key = k > key ? k : key;
    }
    KeyFlag t = block_reduce<kWavesNT>(key, good, lds_key, lds_good);
    if (a.tiles > 1) {
        const int slot = row * a.tiles + tile;
        if (threadIdx.x == 0) {
            store_device(&a.partial_keys[slot], t.key);
            store_device(&a.partial_flags[slot], t.good);
        }
        if (!arrive_last(&a.counters[row], (uint32_t)a.tiles, &last)) return;
        // last workgroup of the row: merge the tiles (at most NT of them)
        key = 0;
        good = true;
        if ((int)threadIdx.x < a.tiles) {
            key = load_device(&a.partial_keys[row * a.tiles + threadIdx.x]);
            good = load_device(&a.partial_flags[row * a.tiles + threadIdx.x]) != 0;
        }
        t = block_reduce<kWavesNT>(key, good, lds_key, lds_good);
    }
    const bool live = row < active && a.width > 0;
    const bool valid = live && t.good && t.key != 0;   // key 0: the mask admitted nothing
    const bool rejected = live && !t.good;
    const int64_t best_id = (int64_t)column_of_key(t.key) + a.vocab_start;
    const uint32_t nan_bits = HALF ? kNanF16 : kNanBf16;
    const uint32_t order = (uint32_t)(t.key >> 32);
    // the order key holds the value except the sign of a zero: read a zero back
    const uint32_t score = !valid ? nan_bits
                           : order == 0x8000u ? (uint32_t)a.logits[(int64_t)row * a.row_stride + column_of_key(t.key)]
                                              : bits_of_order16(order);
    for (int j = threadIdx.x; j < a.candidates; j += kThreads) {
        const bool first = j == 0;
        a.scores[(int64_t)row * a.candidates + j] = (uint16_t)(first ? score : nan_bits);
        a.ids[(int64_t)row * a.candidates + j] = first && valid ? best_id : (first && rejected ? -2 : -1);
    }
    if constexpr (FUSED) {
        // Root over this row's published candidates: slot 0 is real when
        // valid, every other slot is (NaN, -1) padding; (NaN, -2) is neither.
        // The row's guard term rides on its arrival: +1, plus 2^16 when the
        // term fails, so the last arrival reads the verdict from the count.
        if (threadIdx.x == 0) {
            const bool real = valid && best_id < a.p.vocab_size;
            const RowDecision d = root_decision(rp, a.p.k, row, active, cancel,
                                                !rejected && (real || !valid), real, best_id);
            const bool term = guard_term(rp, a.p.k, a.p.vocab_size, row, active, d.token, d.valid);
            a.tokens[row] = d.token;
            a.root_valid[row] = d.valid;
            if (a.tiles > 1) store_device(&a.counters[row], 0u);
            const uint32_t prior = __hip_atomic_fetch_add(&a.counters[a.rows], term ? 1u : 0x10001u,
                                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t total = prior + (term ? 1u : 0x10001u);
            if ((total & 0xFFFFu) == (uint32_t)a.rows) {
                a.final_valid[0] = (total >> 16) == 0 && active > 0 && active <= a.rows;
                store_device(&a.counters[a.rows], 0u);
            }
        }
    } else {
        if (threadIdx.x == 0 && a.tiles > 1) store_device(&a.counters[row], 0u);
    }
}

// ---------------------------------------------------------------------------
// Root over gathered [tp, rows, k] candidates: one wave per row, four rows per
// workgroup.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void greedy_root_kernel(GreedyRootArgs a) {
    const int row = blockIdx.x * kWaves + threadIdx.x / kWave, lane = threadIdx.x % kWave;
    if (row >= a.rows) return;
    const int active = a.metadata[0];
    uint64_t best = 0;
    bool good = true, real_any = false;
    if (row < active) {
        for (int j = lane; j < a.tp * a.p.k; j += kWave) {
            const int64_t pos = ((int64_t)(j / a.p.k) * a.rows + row) * a.p.k + j % a.p.k;
            const uint32_t u = a.scores[pos];
            const int64_t id = a.ids[pos];
            const bool nan = (u & 0x7FFFu) > (a.scores_fp16 ? 0x7C00u : 0x7F80u);
            const bool finite = !(a.scores_fp16 ? nonfinite16<true>(u) : nonfinite16<false>(u));
            const bool real = finite && id >= 0 && id < a.p.vocab_size;
            good &= real || (nan && id == -1);
            real_any |= real;
            // real ids are below the vocabulary size (< 2^31): the low word
            // orders them, lower id first
            const uint64_t key = ((uint64_t)order16(u) << 32) | (0xFFFFFFFFu - (uint32_t)id);
            if (real && key > best) best = key;
        }
    }
    best = wave_max_u64(best);
    good = wave_all(good);
    real_any = !wave_all(!real_any);
    const int64_t best_id = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
    const RowDecision d = root_decision(row_params(a.p, row), a.p.k, row, active, a.metadata[1], good,
                                        real_any, best_id);
    if (lane == 0) {
        a.tokens[row] = d.token;
        a.valid[row] = d.valid;
    }
}

// Final guard: one workgroup over the capacity.
__global__ __launch_bounds__(kThreads) void final_guard_kernel(GuardArgs a) {
    __shared__ uint64_t lds_key[kWaves];
    __shared__ uint32_t lds_good[kWaves];
    const int active = a.metadata[0];
    bool good = true;
    for (int i = threadIdx.x; i < a.capacity; i += kThreads)
        good &= guard_term(i < active ? row_params(a.p, i) : RowParams{}, a.p.k, a.p.vocab_size, i,
                           active, a.tokens[i], a.root_valid ? a.root_valid[i] != 0 : true);
    const KeyFlag t = block_reduce(0, good, lds_key, lds_good);
    if (threadIdx.x == 0) a.valid[0] = t.good && active > 0 && active <= a.capacity;
}

template <int NT, int U, bool HALF, bool MASK>
hipError_t launch_greedy_t(const GreedyArgs& a, hipStream_t s) {
    const dim3 grid(a.tiles, a.rows);
    if (a.tokens) greedy_kernel<NT, U, HALF, MASK, true><<<grid, NT, 0, s>>>(a);
    else greedy_kernel<NT, U, HALF, MASK, false><<<grid, NT, 0, s>>>(a);
    return hipGetLastError();
}

template <int NT, int U>
hipError_t launch_greedy_nt(const GreedyArgs& a, hipStream_t s) {
    if (a.scores_fp16)
        return a.token_mask ? launch_greedy_t<NT, U, true, true>(a, s) : launch_greedy_t<NT, U, true, false>(a, s);
    return a.token_mask ? launch_greedy_t<NT, U, false, true>(a, s) : launch_greedy_t<NT, U, false, false>(a, s);
}

}  // namespace

hipError_t launch_greedy(const GreedyArgs& a, hipStream_t s) {
    if (a.tiles < 1 || a.tiles > kThreads || a.rows < 1 || a.tile_width % kRound ||
        (int64_t)a.tile_width > (int64_t)65536 * kRound)
        return hipErrorInvalidValue;
    // 256 threads with four 16-byte loads in flight each: measured best on
    // the Qwen3-8B vocabulary for 1..256 rows against 1024 threads and 8 or
    // 16 loads (those hold more bytes in flight per workgroup but fewer
    // workgroups per CU)
    return launch_greedy_nt<kThreads, 4>(a, s);
}

hipError_t launch_greedy_root(const GreedyRootArgs& a, hipStream_t s) {
    greedy_root_kernel<<<(a.rows + kWaves - 1) / kWaves, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_final_guard(const GuardArgs& a, hipStream_t s) {
    final_guard_kernel<<<1, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace cubic
