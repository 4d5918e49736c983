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
constexpr int kUnroll = 4;                          // load rounds in flight
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

// Candidate key of column j (j < 2^31): value order, then lower column, then
// bit 0 = the value is -0 (columns are distinct, so bit 0 never decides).
// Zero is reserved for "no admitted column".
__device__ __forceinline__ uint64_t column_key(uint32_t u, uint32_t j) {
    return ((uint64_t)order16(u) << 32) | ((uint64_t)(0x7FFFFFFFu - j) << 1) | (u == 0x8000u);
}
__device__ __forceinline__ uint32_t column_of_key(uint64_t key) {
    return 0x7FFFFFFFu - (uint32_t)((key & 0xFFFFFFFFu) >> 1);
}
__device__ __forceinline__ uint32_t score_of_key(uint64_t key) {
    return (key & 1u) ? 0x8000u : bits_of_order16((uint32_t)(key >> 32));
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
__device__ __forceinline__ KeyFlag block_reduce(uint64_t key, bool good, uint64_t* lds_key,
                                                uint32_t* lds_good) {
    const int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    key = wave_max_u64(key);
    good = wave_all(good);
    if (lane == 0) { lds_key[w] = key; lds_good[w] = good; }
    __syncthreads();
    KeyFlag r = {lds_key[0], lds_good[0]};
#pragma unroll
    for (int i = 1; i < kWaves; ++i) {
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
struct RowDecision {
    int64_t token;
    bool valid;
};
__device__ __forceinline__ RowDecision root_decision(const GreedyParams& p, int row, int active,
                                                     int cancel, bool good, bool any_real,
                                                     int64_t best_id) {
    if (row >= active) return {(cancel && row == active) ? -2 : -1, false};
    const float t = p.temperatures[row], tp = p.top_ps[row];
    const int64_t k = p.top_ks[row];
    const bool ok = good && any_real && t == 0.0f && __builtin_isfinite(tp) && tp > 0.0f &&
                    tp <= 1.0f && k >= 1 && k <= p.k && p.seeds[row] >= 0 && p.ordinals[row] >= 0;
    return {ok ? best_id : -1, ok};
}

// One row's term of the final guard (greedy.cu:121-130).
__device__ __forceinline__ bool guard_term(const GreedyParams& p, int i, int active, int64_t token,
                                           bool root_valid) {
    if (i < active) {
        const float t = p.temperatures[i], tp = p.top_ps[i];
        const int64_t k = p.top_ks[i];
        return token >= 0 && token < p.vocab_size && root_valid && __builtin_isfinite(t) &&
               t >= 0.0f && t <= 2.0f && __builtin_isfinite(tp) && tp > 0.0f && tp <= 1.0f &&
               k >= 1 && k <= p.k && p.seeds[i] >= 0 && p.ordinals[i] >= 0;
    }
    return i == active ? (token == -1 || token == -2) : token == -1;
}

// ---------------------------------------------------------------------------
// Candidate pass.  Grid (tiles, rows).  Rows at or past the active count read
// no logits.  Column j of a row is admitted when the grammar mask (if any)
// allows token vocab_start + j; every visible column counts for finiteness.
// ---------------------------------------------------------------------------
template <bool HALF, bool MASK>
__device__ __forceinline__ void scan_word(uint32_t word, uint32_t j, uint32_t end,
                                          const uint32_t* mask_row, int64_t vocab_start,
                                          uint64_t& best, bool& good) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t u = (word >> (16 * h)) & 0xFFFFu, jj = j + h;
        if (jj < end) {
            good &= !nonfinite16<HALF>(u);
            bool admitted = true;
            if constexpr (MASK) {
                const int64_t token = vocab_start + jj;
                admitted = (mask_row[token >> 5] >> (token & 31)) & 1u;
            }
            const uint64_t key = column_key(u, jj);
            if (admitted && key > best) best = key;
        }
    }
}

template <bool HALF, bool MASK, bool FUSED>
__global__ __launch_bounds__(kThreads) void greedy_kernel(GreedyArgs a) {
    __shared__ uint64_t lds_key[kWaves];
    __shared__ uint32_t lds_good[kWaves];
    __shared__ uint32_t last;
    const int tile = blockIdx.x, row = blockIdx.y;
    const int active = a.metadata[0];
    uint64_t best = 0;
    bool good = true;
    if (row < active) {
        const uint32_t begin = (uint32_t)tile * a.tile_width;
        const uint32_t end = min(begin + (uint32_t)a.tile_width, (uint32_t)a.width);
        const uint16_t* src = a.logits + (int64_t)row * a.row_stride;
        const uint32_t* mask_row = MASK ? a.token_mask + (int64_t)row * a.mask_words : nullptr;
        for (uint32_t base = begin; base < end; base += kUnroll * kRound) {
            uint4 v[kUnroll];
#pragma unroll
            for (int r = 0; r < kUnroll; ++r) {
                const uint32_t j = base + r * kRound + threadIdx.x * kLoadElems;
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
                const uint32_t j = base + r * kRound + threadIdx.x * kLoadElems;
                const uint32_t words[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    scan_word<HALF, MASK>(words[q], j + 2 * q, end, mask_row, a.vocab_start, best, good);
            }
        }
    }
    KeyFlag t = block_reduce(best, good, lds_key, lds_good);
    const int slot = row * a.tiles + tile;
    if (threadIdx.x == 0) {
        store_device(&a.partial_keys[slot], t.key);
        store_device(&a.partial_flags[slot], t.good);
    }
    if (!arrive_last(&a.counters[row], (uint32_t)a.tiles, &last)) return;

    // Last workgroup of the row: merge the tiles (at most kThreads of them).
    best = 0;
    good = true;
    if ((int)threadIdx.x < a.tiles) {
        best = load_device(&a.partial_keys[row * a.tiles + threadIdx.x]);
        good = load_device(&a.partial_flags[row * a.tiles + threadIdx.x]) != 0;
    }
    t = block_reduce(best, good, lds_key, lds_good);
    const bool live = row < active && a.width > 0;
    const bool valid = live && t.good && t.key != 0;   // key 0: the mask admitted nothing
    const bool rejected = live && !t.good;
    const int64_t best_id = (int64_t)column_of_key(t.key) + a.vocab_start;
    const uint32_t nan_bits = HALF ? kNanF16 : kNanBf16;
    for (int j = threadIdx.x; j < a.candidates; j += kThreads) {
        const bool first = j == 0;
        a.scores[(int64_t)row * a.candidates + j] =
            (uint16_t)(first && valid ? score_of_key(t.key) : nan_bits);
        a.ids[(int64_t)row * a.candidates + j] = first && valid ? best_id : (first && rejected ? -2 : -1);
    }
    if constexpr (FUSED) {
        // Root over this row's published candidates: slot 0 is real when
        // valid, every other slot is (NaN, -1) padding; (NaN, -2) is neither.
        const bool real = valid && best_id < a.p.vocab_size;
        const RowDecision d = root_decision(a.p, row, active, a.metadata[1], !rejected && (real || !valid),
                                            real, best_id);
        const bool term = guard_term(a.p, row, active, d.token, d.valid);
        if (threadIdx.x == 0) {
            a.tokens[row] = d.token;
            a.root_valid[row] = d.valid;
            store_device(&a.row_terms[row], (uint32_t)term);
            store_device(&a.counters[row], 0u);
        }
        if (!arrive_last(&a.counters[a.rows], (uint32_t)a.rows, &last)) return;
        bool all = true;
        for (int i = threadIdx.x; i < a.rows; i += kThreads) all &= load_device(&a.row_terms[i]) != 0;
        t = block_reduce(0, all, lds_key, lds_good);
        if (threadIdx.x == 0) {
            a.final_valid[0] = t.good && active > 0 && active <= a.rows;
            store_device(&a.counters[a.rows], 0u);
        }
    } else {
        if (threadIdx.x == 0) store_device(&a.counters[row], 0u);
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
    const RowDecision d = root_decision(a.p, row, active, a.metadata[1], good, real_any, best_id);
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
        good &= guard_term(a.p, i, active, a.tokens[i], a.root_valid ? a.root_valid[i] != 0 : true);
    const KeyFlag t = block_reduce(0, good, lds_key, lds_good);
    if (threadIdx.x == 0) a.valid[0] = t.good && active > 0 && active <= a.capacity;
}

template <bool HALF, bool MASK>
hipError_t launch_greedy_t(const GreedyArgs& a, hipStream_t s) {
    const dim3 grid(a.tiles, a.rows);
    if (a.tokens) greedy_kernel<HALF, MASK, true><<<grid, kThreads, 0, s>>>(a);
    else greedy_kernel<HALF, MASK, false><<<grid, kThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_greedy(const GreedyArgs& a, hipStream_t s) {
    if (a.tiles < 1 || a.tiles > kThreads || a.rows < 1) return hipErrorInvalidValue;
    if (a.scores_fp16)
        return a.token_mask ? launch_greedy_t<true, true>(a, s) : launch_greedy_t<true, false>(a, s);
    return a.token_mask ? launch_greedy_t<false, true>(a, s) : launch_greedy_t<false, false>(a, s);
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
