// MTP acceptance on gfx950: candidate selection over the vocabulary, p/q
// verification of each draft depth, and the accepted-prefix merge.
//
// Reference semantics (paths under src/cubic_serve/ of QuantTrio/cubic-serve):
//   candidates   ops/cuda/sampling/local_candidates.py:206-226,
//                local_candidates.cu:19-146, greedy.cu:14-78
//   verify       ops/cuda/sampling/speculative.py:46-219
//   merge        executor/draft_graph.py:146-157
//
// One HBM pass over the logits: each workgroup owns a (row, vocab tile) and
// reduces it to its 20 best (value desc, id asc) entries plus a finiteness
// flag; the last workgroup to finish a group of rows (one row for plain
// candidate preparation, the k+1 rows of one sequence for the fused verify)
// merges the tiles, publishes the candidates and, in fused mode, verifies
// every depth and merges the prefix.  Arrival counters live in the caller's
// workspace; the finishing workgroup returns its counter to zero.  Candidate
// preparation also takes fp16 logits; the live and owned row counts may be
// device values read when the launch runs (one captured graph, any count).
//
// Wave-level reductions follow fixed orders (butterfly sums in ascending
// lane distance, row-wise scans; cubic_device.h) that the CPU restatement
// reproduces operation for operation.
#include <type_traits>

#include "cubic_device.h"
#include "cubic_capi_internal.h"


namespace cubic {
namespace {

constexpr int kWave = 64;
constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kTop = 20;              // tile candidates kept per (row, tile)
constexpr int kMaxTileChunks = 16;    // 16 x 2048 = 32768 elements per tile
constexpr int kMaxTiles = 24;         // tiles per row (final merge holds 8 entries per lane)
constexpr int kChunk = kThreads * 8;  // elements per 16-byte load round
constexpr int64_t kInt64Max = 0x7FFFFFFFFFFFFFFFLL;

// --------------------------------------------------------------------------
// Ordering keys.  key16 maps sign-magnitude 16-bit floats (bf16 and fp16
// alike) to an unsigned order that compares like the values and treats -0
// and +0 as equal; the low 16 bits hold 0xFFFF - local index so that the
// larger composite is the lower id on ties.
// --------------------------------------------------------------------------
__device__ __forceinline__ uint32_t order_key16(uint32_t u) {
    const uint32_t m = u & 0x7FFFu;
    return (u & 0x8000u) ? 0x8000u - m : 0x8000u + m;
}

// Two bf16 -> two order keys (low / high half), with packed 16-bit integer
// ops: 0x8000 + |u| for positive, 0x8000 - |u| for negative (-0 == +0).
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
typedef short i16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t order_key16x2(uint32_t w) {
    const u16x2_t mag = __builtin_bit_cast(u16x2_t, w & 0x7FFF7FFFu);
    const u16x2_t bias = {0x8000, 0x8000};
    const uint32_t pos = __builtin_bit_cast(uint32_t, (u16x2_t)(bias + mag));
    const uint32_t neg = __builtin_bit_cast(uint32_t, (u16x2_t)(bias - mag));
    const uint32_t sgn = __builtin_bit_cast(uint32_t, (i16x2_t)(__builtin_bit_cast(i16x2_t, w) >> 15));
    return (sgn & neg) | (~sgn & pos);
}

__device__ __forceinline__ uint32_t bits_of_key16(uint32_t k) {
    return k >= 0x8000u ? k - 0x8000u : (0x8000u | (0x8000u - k));
}


__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), l);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Descending bitonic sort of one u32 per lane across the wave.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v, int lane) {
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride >= 1; stride >>= 1) {
            const uint32_t o = xor_lane_rt(v, stride);  // stride is a constant once unrolled
            const bool upper = (lane & stride) != 0;
            const bool desc = (lane & size) == 0;
            const uint32_t hi = o > v ? o : v, lo = o > v ? v : o;
            v = (upper == desc) ? lo : hi;
        }
    }
    return v;
}

// Descending bitonic sort of one u64 per lane across the wave.
__device__ __forceinline__ uint64_t wave_sort_desc_u64(uint64_t v, int lane) {
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride >= 1; stride >>= 1) {
            const uint64_t o = xor_lane_rt(v, stride);  // stride is a constant once unrolled
            const bool upper = (lane & stride) != 0;
            const bool desc = (lane & size) == 0;
            const uint64_t hi = o > v ? o : v, lo = o > v ? v : o;
            v = (upper == desc) ? lo : hi;
        }
    }
    return v;
}

// Top `want` (<= kTop) nonzero u64 keys of entries e[q] held round-robin
// (entry index = lane + 64 q); lane r returns the rank-r key (0 if none).
// Any `want` lanes whose maxima are >= tau carry `want` distinct entries >= tau,
// so tau = want-th largest lane maximum bounds the answer from below.
template <int P>
__device__ uint64_t wave_topk_u64(const uint64_t (&e)[P], int n_entries, int want, int lane,
                                  uint64_t* buf) {
    if (n_entries <= kWave) return wave_sort_desc_u64(e[0], lane);
    uint64_t lm = 0ull;
#pragma unroll
    for (int q = 0; q < P; ++q) lm = e[q] > lm ? e[q] : lm;
    const uint64_t tau = (uint64_t)readlane64((int64_t)wave_sort_desc_u64(lm, lane), want - 1);
    int mine = 0;
#pragma unroll
    for (int q = 0; q < P; ++q) mine += (e[q] != 0ull && e[q] >= tau);
    // inclusive prefix count: the row-wise DPP scan of wave_row_scan on integers
    int incl = mine;
    incl += (int)__builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, false);
    incl += (int)__builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, false);
    incl += (int)__builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, false);
    incl += (int)__builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, false);
    incl += (int)__builtin_amdgcn_update_dpp(0, incl, 0x142, 0xA, 0xF, false);
    incl += (int)__builtin_amdgcn_update_dpp(0, incl, 0x143, 0xC, 0xF, false);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (total <= kWave) {
        int pos = incl - mine;
#pragma unroll
        for (int q = 0; q < P; ++q)
            if (e[q] != 0ull && e[q] >= tau) buf[pos++] = e[q];
        wave_lds_sync();
        const uint64_t v = lane < total ? buf[lane] : 0ull;
        wave_lds_sync();
        return wave_sort_desc_u64(v, lane);
    }
    uint64_t prev = ~0ull, my = 0ull;  // many equal keys: one rank per round
    for (int round = 0; round < want; ++round) {
        uint64_t best = 0ull;
#pragma unroll
        for (int q = 0; q < P; ++q)
            if (e[q] < prev && e[q] > best) best = e[q];
        best = wave_max_u64(best);
        if (lane == round) my = best;
        prev = best;
    }
    return my;
}

// --------------------------------------------------------------------------
// Verification of one proposal row by one wave (speculative.py:46-219).
// Virtual lanes v = lane + 64 * s, s < SLOTS, cover BLOCK = next_pow2(TP*K).
// --------------------------------------------------------------------------
struct VerifyRow {
    const uint16_t* q_scores;  // rank 0 entry of this row; rank r at + r * q_rank_stride
    const int64_t* q_ids;
    const uint16_t* p0_scores;
    const int64_t* p0_ids;
    const uint16_t* p1_scores;
    const int64_t* p1_ids;
    int64_t q_rank_stride, p_rank_stride;
    int tp, k, block;
    bool active, rows_ok;
    int64_t draft;
    float temperature, top_p;
    int64_t top_k, seed, ordinal;
    bool has_uniforms;      // explicit draws u0 (accept), u1 (resample); else Philox
    float u0, u1;
    bool underfilled;
    // staged: lane j < tp*k already holds candidate j of q, p0 and p1 (tp = 1;
    // the pointers above are not read)
    bool staged;
    uint32_t st_q_s, st_p0_s, st_p1_s;
    int64_t st_q_i, st_p0_i, st_p1_i;
};

template <int SLOTS>
struct VerifyScratch {
    float score[SLOTS * kWave];   // rank-ordered scores of the set being selected
    int64_t id[SLOTS * kWave];
    int64_t q_id[SLOTS * kWave];  // selected draft candidates (for q_at_p)
    float q_prob[SLOTS * kWave];
};

// Per-lane candidate set: virtual lane v = lane + 64 * s.
template <int SLOTS>
struct LaneSet {
    float s[SLOTS];
    int64_t i[SLOTS];
    bool r[SLOTS];
};

template <int SLOTS>
__device__ __forceinline__ float vl_tree_sum(float (&x)[SLOTS], int block) {
    // butterfly x[i] += x[i ^ m], m = 1, 2, ..., block/2: lanes, then slots
    const int width = block < kWave ? block : kWave;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) x[s] = wave_butterfly_sum(x[s], width);
    // slot strides sm = 1, 2, .. while 64 sm < block, as compile-time
    // indices (a runtime x[s ^ sm] keeps the array in scratch memory)
#pragma unroll
    for (int sm = 1; sm < SLOTS; sm <<= 1) {
        if (kWave * sm < block) {
            float y[SLOTS];
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) y[s] = x[s] + x[s ^ sm];
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) x[s] = y[s];
        }
    }
    return lane_f32(x[0], 0);
}

template <int SLOTS>
__device__ __forceinline__ void vl_scan(float (&x)[SLOTS], int block, int lane) {
    // inclusive scan: row-wise order of wave_row_scan inside each slot, then
    // each slot adds the previous slot's last lane, slot after slot
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) x[s] = wave_row_scan(x[s]);
#pragma unroll
    for (int s = 1; s < SLOTS; ++s)
        if (kWave * s < block) x[s] = x[s] + lane_f32(x[s - 1], kWave - 1);
    (void)lane;
}

template <int SLOTS>
__device__ __forceinline__ float vl_max(const float (&x)[SLOTS], int block) {
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) m = x[s] > m ? x[s] : m;  // NaN-ignoring
    (void)block;  // lanes past the block hold -inf
    return lane_f32(wave_max_f32(m), 0);
}


__device__ __forceinline__ float readlanef(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// speculative.py:11-29.  Output: the selected (score, id) of rank v in
// virtual lane v (v < k), (-inf, INT64_MAX) elsewhere; returns the number of
// real lanes.  A real lane is the first of its (score, id) pair if no earlier
// real lane repeats it; its rank is the number of first lanes strictly ahead
// in (score desc, id asc) order, so a duplicated pair occupies one slot,
// exactly as the reference removes every copy of the pair it selects.
// Fast path: real lanes already form a strictly ordered prefix (the layout
// candidate publication produces), where selection is the identity.
template <int SLOTS>
__device__ __forceinline__ int select_set(const LaneSet<SLOTS>& in, int block, int k, int lane,
                          VerifyScratch<SLOTS>& sc, LaneSet<SLOTS>& out) {
    int count = 0;
    bool ok = true;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        count += __builtin_popcountll(__ballot(v < block && in.r[s]));
        // neighbour v + 1
        const int src = lane + 1 < kWave ? lane + 1 : 0;
        const int ss = lane + 1 < kWave ? s : (s + 1 < SLOTS ? s + 1 : s);
        float ns = 0.0f;
        int64_t ni = 0;
        bool nr = false;
#pragma unroll
        for (int t = 0; t < SLOTS; ++t) {
            const float ts = __shfl(in.s[t], src);
            const int64_t ti = __shfl(in.i[t], src);
            const bool tr = __shfl((int)in.r[t], src) != 0;
            if (t == ss) { ns = ts; ni = ti; nr = tr; }
        }
        if (v + 1 < block && !(lane + 1 >= kWave && s + 1 >= SLOTS)) {
            const bool r0 = in.r[s];
            if (nr && !r0) ok = false;
            if (r0 && nr && !(in.s[s] > ns || (in.s[s] == ns && in.i[s] < ni))) ok = false;
        }
    }
    if (__all(ok)) {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const int v = lane + kWave * s;
            const bool take = v < block && v < k && in.r[s];
            out.s[s] = take ? in.s[s] : -__builtin_huge_valf();
            out.i[s] = take ? in.i[s] : kInt64Max;
            out.r[s] = take;
        }
        return count;
    }
    // general path: first-occurrence flags, then ranks, by uniform lane walks
    bool first[SLOTS];
    int rank[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) { first[s] = in.r[s]; rank[s] = 0; }
#pragma unroll
    for (int sj = 0; sj < SLOTS; ++sj)
        for (int l = 0; l < kWave; ++l) {
            const int j = l + kWave * sj;
            if (j >= block) break;
            if (!__builtin_amdgcn_readlane((int)in.r[sj], l)) continue;
            const float vs = readlanef(in.s[sj], l);
            const int64_t vi = readlane64(in.i[sj], l);
#pragma unroll
            for (int s = 0; s < SLOTS; ++s)
                if (in.r[s] && j < lane + kWave * s && vs == in.s[s] && vi == in.i[s]) first[s] = false;
        }
#pragma unroll
    for (int sj = 0; sj < SLOTS; ++sj)
        for (int l = 0; l < kWave; ++l) {
            const int j = l + kWave * sj;
            if (j >= block) break;
            if (!__builtin_amdgcn_readlane((int)first[sj], l)) continue;
            const float vs = readlanef(in.s[sj], l);
            const int64_t vi = readlane64(in.i[sj], l);
#pragma unroll
            for (int s = 0; s < SLOTS; ++s)
                rank[s] += (vs > in.s[s] || (vs == in.s[s] && vi < in.i[s])) ? 1 : 0;
        }
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        if (v < block) { sc.score[v] = -__builtin_huge_valf(); sc.id[v] = kInt64Max; }
    }
    wave_lds_sync();
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
        if (lane + kWave * s < block && first[s] && rank[s] < k) {
            sc.score[rank[s]] = in.s[s];
            sc.id[rank[s]] = in.i[s];
        }
    wave_lds_sync();
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        out.s[s] = v < block ? sc.score[v] : -__builtin_huge_valf();
        out.i[s] = v < block ? sc.id[v] : kInt64Max;
        out.r[s] = out.i[s] != kInt64Max;
    }
    wave_lds_sync();
    return count;
}

// speculative.py:32-43 for one selected set (scores in rank order).
// NORMALIZE = false returns the retained probabilities before the division by
// their mass (topk_topp.py:94-100 samples from those).
template <int SLOTS, bool NORMALIZE = true>
__device__ __forceinline__ void probabilities(const float (&sorted)[SLOTS], float temperature,
                                              int64_t top_k, float top_p, int block, int lane,
                                              float (&out)[SLOTS], float& mass) {
    const float safe_t = temperature == 0.0f ? 1.0f : temperature;
    float logit[SLOTS], w[SLOTS], p[SLOTS], incl[SLOTS], tmp[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        const bool sel = v < block && v < top_k;
        logit[s] = sel ? sorted[s] / safe_t : -__builtin_huge_valf();
    }
    const float mx = vl_max<SLOTS>(logit, block);
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        const bool sel = v < block && v < top_k;
        w[s] = sel ? accept_expf(logit[s] - mx) : 0.0f;
        tmp[s] = w[s];
    }
    const float sum = vl_tree_sum<SLOTS>(tmp, block);
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) { p[s] = w[s] / sum; incl[s] = p[s]; }
    vl_scan<SLOTS>(incl, block, lane);
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        const float excl = incl[s] - p[s];
        p[s] = (v < block && v < top_k && excl <= top_p) ? p[s] : 0.0f;
        tmp[s] = p[s];
    }
    mass = vl_tree_sum<SLOTS>(tmp, block);
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) out[s] = NORMALIZE ? p[s] / mass : p[s];
}

// One candidate set of a verified row (which: 0 = q, 1 = p0, 2 = p1), selected
// and turned into probabilities; ok = every lane's pair is real or padding.
template <int SLOTS>
struct VerifySet {
    LaneSet<SLOTS> sel;
    float prob[SLOTS];
    float mass;
    int count;
    bool ok;
};

template <int SLOTS>
__device__ __forceinline__ void verify_set(const VerifyRow& r, int which, VerifyScratch<SLOTS>& sc, int lane,
                                           VerifySet<SLOTS>& out) {
    const int block = r.block;
    bool lane_ok = true;
    LaneSet<SLOTS> in;
    const uint16_t* scores = which == 0 ? r.q_scores : (which == 1 ? r.p0_scores : r.p1_scores);
    const int64_t* ids = which == 0 ? r.q_ids : (which == 1 ? r.p0_ids : r.p1_ids);
    const int64_t stride = which == 0 ? r.q_rank_stride : r.p_rank_stride;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        const bool cm = v < r.tp * r.k;
        const int rank = cm ? v / r.k : 0, local = cm ? v % r.k : 0;
        const bool load = r.active && cm && (which == 0 || r.rows_ok);
        float xs = -__builtin_huge_valf();
        int64_t xi = -1;
        if (load) {
            if (SLOTS == 1 && r.staged) {
                // a branch on the (uniform) set, not a select of the three
                // fields: the compiler turns that select into a load at a
                // runtime offset into the row, which keeps the whole row in
                // scratch memory (greedy acceptance of 64 rows x 151936: 15.3 -> 13.0 us)
                uint32_t st_s;
                switch (__builtin_amdgcn_readfirstlane(which)) {
                    case 0: st_s = r.st_q_s; xi = r.st_q_i; break;
                    case 1: st_s = r.st_p0_s; xi = r.st_p0_i; break;
                    default: st_s = r.st_p1_s; xi = r.st_p1_i; break;
                }
                xs = bf16_bits_to_float(st_s);
            } else {
                xs = bf16_bits_to_float(scores[rank * stride + local]);
                xi = ids[rank * stride + local];
            }
        }
        const bool real = cm && xi >= 0 && __builtin_fabsf(xs) < __builtin_huge_valf();
        const bool pad = cm && xi == -1 && xs != xs;
        if (v < block) lane_ok = lane_ok && (!cm || real || pad);
        in.s[s] = xs; in.i[s] = xi; in.r[s] = v < block && real;
    }
    out.ok = __all(lane_ok);
    out.count = select_set<SLOTS>(in, block, r.k, lane, sc, out.sel);
    probabilities<SLOTS>(out.sel.s, r.temperature, r.top_k, r.top_p, block, lane, out.prob, out.mass);
}

// Acceptance, the residual draw and the row's decision from its three sets.
template <int SLOTS>
__device__ __forceinline__ void verify_finish(const VerifyRow& r, const VerifySet<SLOTS>& qs, const VerifySet<SLOTS>& p0s,
                              const VerifySet<SLOTS>& p1s, VerifyScratch<SLOTS>& sc, int lane, int64_t* out2) {
    const int block = r.block;
    const LaneSet<SLOTS>& q = qs.sel;
    const LaneSet<SLOTS>& p0 = p0s.sel;
    const LaneSet<SLOTS>& p1 = p1s.sel;
    const float(&qp)[SLOTS] = qs.prob;
    const float(&p0p)[SLOTS] = p0s.prob;
    const float(&p1p)[SLOTS] = p1s.prob;
    const bool pairs_valid = qs.ok && p0s.ok && p1s.ok;
    float t1[SLOTS], t2[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int v = lane + kWave * s;
        t1[s] = q.i[s] == r.draft ? qp[s] : 0.0f;
        t2[s] = p0.i[s] == r.draft ? p0p[s] : 0.0f;
        if (v < block) { sc.q_id[v] = q.i[s]; sc.q_prob[v] = qp[s]; }
    }
    const float q_draft = vl_tree_sum<SLOTS>(t1, block);
    const bool greedy = r.temperature == 0.0f;
    const int64_t p0_top = readlane64(p0.i[0], 0), p1_top = readlane64(p1.i[0], 0);
    const bool greedy_accepted = r.draft == p0_top;
    if (greedy) {
        const bool accepted = greedy_accepted;
        // a greedy row's decision does not depend on the residual: valid below
        // reduces to this, and next is the target argmax after the prefix
        const int64_t need = 1;
        const bool valid = r.active && pairs_valid && r.rows_ok && r.top_k >= 1 && r.top_k <= r.k &&
                           r.top_p > 0.0f && r.top_p <= 1.0f && r.seed >= 0 && r.ordinal >= 0 &&
                           qs.count >= need && p0s.count >= need && p1s.count >= need && qs.mass > 0.0f &&
                           p0s.mass > 0.0f && p1s.mass > 0.0f && q_draft > 0.0f;
        if (lane == 0) {
            out2[0] = valid ? (int64_t)accepted : -1;
            out2[1] = valid ? (greedy_accepted ? p1_top : p0_top) : -1;
        }
        wave_lds_sync();
        return;
    }
    const float p_draft = vl_tree_sum<SLOTS>(t2, block);
    const float quotient = p_draft / q_draft;
    const float ratio = quotient < 1.0f ? quotient : 1.0f;
    const uint32_t key = (uint32_t)(r.seed ^ (r.seed >> 32) ^ 0x9E3779B9LL);
    const float u_accept = r.has_uniforms ? r.u0 : philox_uniform(key, (uint32_t)(r.ordinal * 2));
    const bool accepted = u_accept < ratio;
    wave_lds_sync();

    float q_at_p[SLOTS], residual[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) q_at_p[s] = 0.0f;
    for (int pos = 0; pos < r.k; ++pos) {
        const int64_t qid = sc.q_id[pos];
        const float qpr = sc.q_prob[pos];
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) q_at_p[s] = p0.i[s] == qid ? qpr : q_at_p[s];
    }
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const float d = p0p[s] - q_at_p[s];
        residual[s] = d > 0.0f ? d : 0.0f;
        t1[s] = residual[s];
    }
    const float rmass = vl_tree_sum<SLOTS>(t1, block);
    const float u_sample = r.has_uniforms ? r.u1
                                      : philox_uniform(key ^ 0x85EBCA6Bu, (uint32_t)(r.ordinal * 2 + 1));
    float c1[SLOTS], cr[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) { c1[s] = p1p[s]; cr[s] = residual[s]; }
    vl_scan<SLOTS>(c1, block, lane);
    vl_scan<SLOTS>(cr, block, lane);
    const float scaled_u = u_sample * rmass;
    int p1_slot = block, res_slot = block;
#pragma unroll
    for (int s = SLOTS - 1; s >= 0; --s) {
        const int v = lane + kWave * s;
        const uint64_t b1 = __ballot(v < block && c1[s] > u_sample);
        const uint64_t br = __ballot(v < block && cr[s] > scaled_u);
        if (b1) p1_slot = kWave * s + __builtin_ctzll(b1);
        if (br) res_slot = kWave * s + __builtin_ctzll(br);
    }
    int64_t p1_token = kInt64Max, res_token = kInt64Max;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int64_t a1 = readlane64(p1.i[s], p1_slot & (kWave - 1));
        const int64_t ar = readlane64(p0.i[s], res_slot & (kWave - 1));
        if (p1_slot < block && p1_slot / kWave == s) p1_token = a1;
        if (res_slot < block && res_slot / kWave == s) res_token = ar;
    }
    const int64_t need = (greedy || r.underfilled) ? 1 : r.top_k;
    const bool valid = r.active && pairs_valid && r.rows_ok && r.temperature >= 0.0f &&
                       r.temperature < __builtin_huge_valf() && r.top_k >= 1 && r.top_k <= r.k &&
                       r.top_p > 0.0f && r.top_p <= 1.0f && r.seed >= 0 && r.ordinal >= 0 &&
                       qs.count >= need && p0s.count >= need && p1s.count >= need && qs.mass > 0.0f &&
                       p0s.mass > 0.0f && p1s.mass > 0.0f && q_draft > 0.0f &&
                       (greedy || accepted || rmass > 0.0f);
    const int64_t greedy_next = greedy_accepted ? p1_top : p0_top;
    const int64_t next = greedy ? greedy_next : (accepted ? p1_token : res_token);
    if (lane == 0) {
        out2[0] = valid ? (int64_t)accepted : -1;
        out2[1] = valid ? next : -1;
    }
    wave_lds_sync();
}

template <int SLOTS>
__device__ __forceinline__ void verify_wave(const VerifyRow& r, VerifyScratch<SLOTS>& sc, int lane, int64_t* out2) {
    VerifySet<SLOTS> q, p0, p1;
    verify_set<SLOTS>(r, 0, sc, lane, q);
    verify_set<SLOTS>(r, 1, sc, lane, p0);
    verify_set<SLOTS>(r, 2, sc, lane, p1);
    verify_finish<SLOTS>(r, q, p0, p1, sc, lane, out2);
}

// --------------------------------------------------------------------------
// Root top-k/top-p sampling (ops/cuda/sampling/topk_topp.py:22-121).  One
// workgroup per row, one thread per gathered candidate (TP * K <= 160):
//   1. load; a pair is real (finite score, id >= 0) or the NaN/-1 sentinel;
//   2. a real pair is first unless an earlier lane holds the same (score, id);
//   3. the rank of a first pair = first pairs strictly ahead in (score desc,
//      id asc); ranks < K land in LDS.  This is the reference's K rounds of
//      max / min-id / remove-all-copies, as one counting pass;
//   4. wave 0 runs temperature, softmax, top-p over the exclusive CDF and the
//      inverse-CDF draw over the K ranked slots (slots past the selection are
//      (-inf, INT64_MAX) and carry zero weight, so reducing over 64 lanes
//      gives the same bits as over next_pow2(TP * K)).
// Reduction orders and exp as verify_wave.
// --------------------------------------------------------------------------
constexpr int kRootThreads = 256;

struct RootScratch {
    uint64_t key[kRootThreads];      // (sortable score << 32) | ~id32 of real lanes, else 0
    float score[kRootThreads];
    int64_t id[kRootThreads];
    uint32_t real[kRootThreads];
    float sorted_score[kRootThreads];  // real pairs at their (score desc, id asc, lane asc) rank
    int64_t sorted_id[kRootThreads];
    int counts[kRootThreads / kWave][4];
    float sel_score[kWave];
    int64_t sel_id[kWave];
};

// Monotone map of a finite float to uint32 (-0 and +0 map alike).
__device__ __forceinline__ uint32_t sortable_score(float f) {
    const uint32_t u = f == 0.0f ? 0u : __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(kRootThreads) void root_sample_kernel(RootSampleArgs a) {
    __shared__ RootScratch sc;
    const int row = blockIdx.x, v = threadIdx.x, w = v / kWave, lane = v % kWave;
    const int count = a.tp * a.k;
    const bool cm = v < count;
    float score = -__builtin_huge_valf();
    int64_t id = -1;
    if (cm) {
        const int64_t off = ((int64_t)(v / a.k) * a.rows + row) * a.k + v % a.k;
        const uint32_t bits = a.scores[off];
        score = a.scores_fp16 ? half_bits_to_float(bits) : bf16_bits_to_float(bits);
        id = a.ids[off];
    }
    const bool real = cm && id >= 0 && __builtin_fabsf(score) < __builtin_huge_valf();
    const bool sentinel = cm && score != score && id == -1;
    const bool wide = real && (uint64_t)id > 0xFFFFFFFFull;
    const uint64_t key = real ? ((uint64_t)sortable_score(score) << 32) | (0xFFFFFFFFu - (uint32_t)id) : 0ull;
    sc.key[v] = key;
    sc.score[v] = score;
    sc.id[v] = id;
    sc.real[v] = real;
    if (v < kWave) { sc.sel_score[v] = -__builtin_huge_valf(); sc.sel_id[v] = kInt64Max; }
    {
        const uint64_t bm = __ballot(cm && !real && !sentinel), br = __ballot(real), bw = __ballot(wide);
        if (lane == 0) {
            sc.counts[w][0] = __builtin_popcountll(bm);
            sc.counts[w][1] = __builtin_popcountll(br);
            sc.counts[w][2] = __builtin_popcountll(bw);
        }
    }
    __syncthreads();
    int malformed = 0, real_count = 0, wide_count = 0;
#pragma unroll
    for (int x = 0; x < kRootThreads / kWave; ++x) {
        malformed += sc.counts[x][0];
        real_count += sc.counts[x][1];
        wide_count += sc.counts[x][2];
    }
    // rank of a real pair in (score desc, id asc, lane asc): unique 0 .. real_count-1.
    // One pass over broadcast LDS entries; 64-bit keys unless an id needs more
    // than 32 bits.
    int rank = 0;
    if (wide_count == 0) {
#pragma unroll 8
        for (int j = 0; j < count; ++j) {
            const uint64_t o = sc.key[j];
            rank += (int)((uint32_t)(o > key) | ((uint32_t)(o == key) & (uint32_t)(j < v)));
        }
    } else {
#pragma unroll 4
        for (int j = 0; j < count; ++j) {
            const float os = sc.score[j];
            const int64_t oi = sc.id[j];
            const uint32_t ahead = (uint32_t)(os > score) |
                                   ((uint32_t)(os == score) & ((uint32_t)(oi < id) | ((uint32_t)(oi == id) & (uint32_t)(j < v))));
            rank += (int)(sc.real[j] & ahead);
        }
    }
    if (real) { sc.sorted_score[rank] = score; sc.sorted_id[rank] = id; }
    __syncthreads();
    // a sorted pair equal to its predecessor is a duplicate: it takes no slot
    // (the reference removes every copy of the pair it selects)
    const bool in = v < real_count;
    const float ps = in ? sc.sorted_score[v] : 0.0f;
    const int64_t pi = in ? sc.sorted_id[v] : 0;
    const bool dup = in && v > 0 && sc.sorted_score[v - 1] == ps && sc.sorted_id[v - 1] == pi;
    const uint64_t bd = __ballot(dup);
    if (lane == 0) sc.counts[w][3] = __builtin_popcountll(bd);
    __syncthreads();
    int dups_before = __builtin_popcountll(bd & (lane ? (~0ull >> (kWave - lane)) : 0ull));
    for (int x = 0; x < w; ++x) dups_before += sc.counts[x][3];
    const int distinct = v - dups_before;
    if (in && !dup && distinct < a.k) { sc.sel_score[distinct] = ps; sc.sel_id[distinct] = pi; }
    __syncthreads();
    if (v >= kWave) return;

    const float temperature = a.temperatures[row], top_p = a.top_ps[row];
    const int64_t top_k = a.top_ks[row], seed = a.seeds[row], ordinal = a.ordinals[row];
    const bool greedy = temperature == 0.0f;
    const bool params_ok = temperature == temperature && temperature >= 0.0f &&
                           temperature < __builtin_huge_valf() && top_p == top_p && top_p > 0.0f &&
                           top_p <= 1.0f && top_k >= 1 && top_k <= a.k && seed >= 0 && ordinal >= 0;
    bool under = a.allow_underfilled != 0;
    if (a.constrained_rows) under = under && a.constrained_rows[row];
    const bool enough = (greedy || under) ? real_count >= 1 : real_count >= top_k;

    float sorted[1] = {sc.sel_score[lane]};
    const int64_t sel_id = sc.sel_id[lane];
    float retained[1], mass;
    probabilities<1, false>(sorted, temperature, top_k, top_p, kWave, lane, retained, mass);
    const int64_t random_seed = seed ^ (seed >> 32) ^ (ordinal >> 32);
    const float uniform = philox_uniform2((uint32_t)random_seed, (uint32_t)((uint64_t)random_seed >> 32),
                                          (uint32_t)ordinal);
    const float target = uniform * mass;
    vl_scan<1>(retained, kWave, lane);
    const uint64_t hit = __ballot(retained[0] > target);
    const int sampled = hit ? __builtin_ctzll(hit) : kWave;
    const int chosen = greedy ? 0 : sampled;
    const int64_t token = readlane64(sel_id, chosen & (kWave - 1));
    const bool valid = malformed == 0 && params_ok && enough &&
                       (greedy || (mass > 0.0f && sampled < kWave));
    if (lane == 0) {
        a.output_tokens[row] = valid ? token : -1;
        a.output_valid[row] = valid ? 1 : 0;
    }
}

// --------------------------------------------------------------------------
// Standalone verify: one wave per proposal row.
// --------------------------------------------------------------------------
template <int SLOTS>
__global__ __launch_bounds__(kWave) void verify_candidates_kernel(VerifyArgs a) {
    __shared__ VerifyScratch<SLOTS> sc;
    const int row = blockIdx.x, lane = threadIdx.x;
    VerifyRow r;
    r.active = row < a.active_rows;
    const int32_t target = r.active ? a.target_rows[row] : 0;
    r.rows_ok = target >= 0 && target + 1 < a.p_rows;
    const int64_t t = r.rows_ok ? target : 0;
    r.q_scores = a.q_scores + (int64_t)row * a.k;
    r.q_ids = a.q_ids + (int64_t)row * a.k;
    r.p0_scores = a.p_scores + t * a.k;
    r.p0_ids = a.p_ids + t * a.k;
    r.p1_scores = r.p0_scores + a.k;
    r.p1_ids = r.p0_ids + a.k;
    r.q_rank_stride = (int64_t)a.q_rows * a.k;
    r.p_rank_stride = (int64_t)a.p_rows * a.k;
    r.tp = a.tp;
    r.k = a.k;
    r.block = a.block;
    r.draft = r.active ? a.draft_tokens[row] : -1;
    r.temperature = r.active ? a.temperatures[row] : 1.0f;
    r.top_p = r.active ? a.top_ps[row] : 1.0f;
    r.top_k = r.active ? a.top_ks[row] : 1;
    r.seed = r.active ? a.seeds[row] : 0;
    r.ordinal = r.active ? a.ordinals[row] : 0;
    r.has_uniforms = a.uniforms != nullptr;
    r.u0 = r.has_uniforms ? a.uniforms[2 * (int64_t)row] : 0.0f;
    r.u1 = r.has_uniforms ? a.uniforms[2 * (int64_t)row + 1] : 0.0f;
    r.staged = false;
    bool under = a.allow_underfilled != 0;
    if (a.constrained_rows) under = under && r.active && a.constrained_rows[row];
    r.underfilled = under;
    verify_wave<SLOTS>(r, sc, lane, a.decisions + 2 * (int64_t)row);
}

// merge_prefix: decisions [depth, c, 2] -> out [c, 2]
__global__ __launch_bounds__(kThreads) void merge_prefix_kernel(const int64_t* decisions, int c,
                                                                 int depth, const int32_t* live,
                                                                 int live_rows, int64_t* out) {
    const int live_count = live ? live[0] : live_rows;
    for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < c; r += gridDim.x * blockDim.x) {
        int64_t accepted = depth, bonus = decisions[((int64_t)(depth - 1) * c + r) * 2 + 1];
        bool good = true;
        for (int d = depth - 1; d >= 0; --d) {
            const int64_t av = decisions[((int64_t)d * c + r) * 2];
            const int64_t tok = decisions[((int64_t)d * c + r) * 2 + 1];
            if (av == 0) { accepted = d; bonus = tok; }
            good = good && (av == 0 || av == 1) && tok >= 0;
        }
        const bool ok = r < live_count && good;
        out[2 * (int64_t)r] = ok ? accepted : -1;
        out[2 * (int64_t)r + 1] = ok ? bonus : -1;
    }
}

// --------------------------------------------------------------------------
// Candidate tiles + group finalisation (plain candidates or fused verify).
// --------------------------------------------------------------------------
// One wave's selected candidate set, handed to the wave that finishes the row.
struct VerifySetLds {
    float s[kWave];
    int64_t i[kWave];
    float prob[kWave];
    uint8_t r[kWave];
    float mass;
    int count, ok;
};

struct TileScratch {
    uint32_t survivors[kWaves][kWave] __attribute__((aligned(16)));
    uint32_t wave_top[kWaves * kTop] __attribute__((aligned(16)));
    uint32_t flags[kWaves];
    uint32_t last;
    // finalisation: candidates of the group rows (count <= 64, rows <= 9)
    uint16_t cand_score[9][64];
    int64_t cand_id[9][64];
    int64_t decisions[8][2];
    uint64_t merge[kWaves][kWave];
    VerifySetLds sets[3];  // one-depth groups: the sets of the three verifying waves
};

// Inputs of one verified depth (proposal row pi of the fused verify), loaded
// at kernel start by the wave that verifies it should its workgroup finish
// the group: lane j < capacity holds the q candidate j.
struct VerifyPrefetch {
    uint32_t q_score;
    int64_t q_id;
    int64_t draft, top_k, seed, ordinal;
    float temperature, top_p, u0, u1;
};

__device__ __forceinline__ VerifyPrefetch prefetch_verify(const AcceptArgs& a, int64_t pi, int lane) {
    VerifyPrefetch p;
    const bool in = lane < a.capacity;
    p.q_score = in ? a.q_scores[pi * a.capacity + lane] : 0x7FC0u;
    p.q_id = in ? a.q_ids[pi * a.capacity + lane] : -1;
    p.draft = a.draft_tokens[pi];
    p.temperature = a.temperatures[pi];
    p.top_p = a.top_ps[pi];
    p.top_k = a.top_ks[pi];
    p.seed = a.seeds[pi];
    p.ordinal = a.ordinals[pi];
    p.u0 = a.uniforms ? a.uniforms[2 * pi] : 0.0f;
    p.u1 = a.uniforms ? a.uniforms[2 * pi + 1] : 0.0f;
    return p;
}

// Exact top-`kTop` composites of the lane-held elements of one wave.
// keys are recomputed from the raw bf16 words (E chunks of 8 per lane).
template <int EMAX>
__device__ __forceinline__ uint32_t elem_composite(const uint4 (&raw)[EMAX], int e, int j,
                                                   uint32_t base_idx, int width_left) {
    const uint32_t word = (&raw[e].x)[j >> 1];
    const uint32_t u = (j & 1) ? (word >> 16) : (word & 0xFFFFu);
    const int idx = (int)base_idx + e * kChunk + j;
    if (idx >= width_left) return 0u;
    return (order_key16(u) << 16) | (0xFFFFu - (uint32_t)idx);
}

// Prefilter key of a bf16 pair, one per half: the bits with the sign bit
// flipped for positive values and all bits flipped for negative ones (three
// VALU per word).  It orders like the values except that -0 (0x7FFF) sits
// just below +0 (0x8000), where the exact order ties them; inf and positive
// NaN map to >= 0xFF80, -inf and negative NaN to <= 0x007F.
__device__ __forceinline__ uint32_t prefilter_key2(uint32_t w) {
    const uint32_t s = __builtin_bit_cast(uint32_t, (i16x2_t)(__builtin_bit_cast(i16x2_t, w) >> 15));
    return w ^ (s | 0x80008000u);
}
// Exact order key (order_key16) of a nonzero 16-bit prefilter key.
__device__ __forceinline__ uint32_t exact_of_prefilter(uint32_t k) {
    const uint32_t raw = k >= 0x8000u ? k ^ 0x8000u : (~k & 0xFFFFu);
    return order_key16(raw);
}

// Returns whether any element of the lane's share is non-finite.  HALF:
// fp16 elements (same sign-magnitude order; non-finite from 0x7C00 up).
template <int EMAX, bool HALF>
__device__ bool tile_top(const uint4 (&raw)[EMAX], int chunks, uint32_t base_idx, int width_left,
                         TileScratch& ts, uint32_t* kw, int lane, int wave, uint32_t* out_top) {
    // 1. prefilter keys, two per word (elements 2w, 2w + 1 of a chunk), 0 =
    //    empty; the lane maximum and, for whole tiles, the lane minimum: a
    //    whole tile is non-finite iff its extreme keys reach the inf/NaN ranges
    uint32_t key2[EMAX][4];
    uint32_t nonfinite = 0;
    const bool whole = chunks == EMAX && chunks * kChunk <= width_left;  // wave-uniform
    u16x2_t m2 = {0, 0};
    if (whole) {
        u16x2_t n2 = {0xFFFF, 0xFFFF};
#pragma unroll
        for (int e = 0; e < EMAX; ++e)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                key2[e][w] = prefilter_key2((&raw[e].x)[w]);
                const u16x2_t k = __builtin_bit_cast(u16x2_t, key2[e][w]);
                m2 = __builtin_elementwise_max(m2, k);
                n2 = __builtin_elementwise_min(n2, k);
            }
        // prefilter keys of inf/NaN: >= 0xFF80 / <= 0x007F (bf16), >= 0xFC00 / <= 0x03FF (fp16)
        constexpr uint32_t kHi = HALF ? 0xFC00u : 0xFF80u, kLo = HALF ? 0x03FFu : 0x007Fu;
        nonfinite = (m2.x >= kHi) | (m2.y >= kHi) | (n2.x <= kLo) | (n2.y <= kLo);
    } else {
        const bool partial = chunks * kChunk > width_left;  // wave-uniform
#pragma unroll
        for (int e = 0; e < EMAX; ++e)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t word = (&raw[e].x)[w];
                uint32_t valid = e < chunks ? 0xFFFFFFFFu : 0u;
                if (partial) {
                    const int idx = (int)base_idx + e * kChunk + 2 * w;
                    valid &= (idx < width_left ? 0x0000FFFFu : 0u) | (idx + 1 < width_left ? 0xFFFF0000u : 0u);
                }
                const u16x2_t mag = __builtin_bit_cast(u16x2_t, word & 0x7FFF7FFFu);
                const u16x2_t inf = {HALF ? 0x7C00 : 0x7F80, HALF ? 0x7C00 : 0x7F80};
                nonfinite |= __builtin_bit_cast(uint32_t, (i16x2_t)(mag >= inf)) & valid;
                key2[e][w] = prefilter_key2(word) & valid;
                m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2_t, key2[e][w]));
            }
    }
    // 2. tau = the kTop-th largest lane maximum (ballot radix select): kTop
    //    lanes hold distinct elements with keys >= tau, so every element of
    //    the exact top kTop has a prefilter key >= tau -- or is -0 (0x7FFF)
    //    tied with a +0 tau (0x8000), which the threshold then admits too.
    const uint32_t lane_max = m2.x > m2.y ? m2.x : m2.y;
    uint32_t tau = 0;
#pragma unroll
    for (int b = 15; b >= 0; --b) {
        const uint32_t cand = tau | (1u << b);
        if (__popcll(__ballot(lane_max >= cand)) >= kTop) tau = cand;
    }
    const uint32_t thr = tau == 0x8000u ? 0x7FFFu : (tau > 0u ? tau : 1u);  // empty never survives
    // 3. compact survivors (prefilter key >= thr) as exact composites.  Each
    //    lane marks the words holding a survivor (saturating packed subtract:
    //    nonzero iff a half is >= thr) and spills its keys to LDS word-major
    //    (lane-distinct banks); the wave then takes one marked word per lane
    //    per round, so the rounds number the largest per-lane count of marked
    //    words, not the words.  Survivor order is irrelevant: ranks count
    //    composites.
    static_assert(EMAX * 4 <= 64, "word mask");
    using Marks = typename std::conditional<EMAX * 4 <= 32, uint32_t, uint64_t>::type;
    Marks marks = 0;
    const u16x2_t thr_m1 = {(unsigned short)(thr - 1u), (unsigned short)(thr - 1u)};
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t k2 = key2[e][w];
            const uint32_t d = __builtin_bit_cast(
                uint32_t, (u16x2_t)__builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2_t, k2), thr_m1));
            marks |= (Marks)(d < 1u ? d : 1u) << (e * 4 + w);
            kw[(e * 4 + w) * kWave + lane] = k2;
        }
    wave_lds_sync();
    uint32_t total = 0;  // wave-uniform
    while (__ballot(marks != 0)) {
        const bool has = marks != 0;
        const int i = has ? (int)__builtin_ctzll((uint64_t)marks) : 0;
        marks &= marks - 1;
        const uint32_t k2 = kw[i * kWave + lane];
        const uint32_t idx0 = base_idx + (uint32_t)((i >> 2) * kChunk + 2 * (i & 3));
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t k = h ? k2 >> 16 : k2 & 0xFFFFu;
            const bool sv = has && k >= thr;
            const uint64_t m = __ballot(sv);
            const uint32_t pos = total + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            if (sv && pos < kWave)
                ts.survivors[wave][pos] = (exact_of_prefilter(k) << 16) | (0xFFFFu - (idx0 + (uint32_t)h));
            total += (uint32_t)__popcll(m);
        }
    }
    wave_lds_sync();  // the spill is rewritten by this wave's next tile only
    if (total <= kWave) {
        // 4. sort the survivors (distinct composites) in registers: lane r
        //    holds rank r
        const uint32_t v = wave_sort_desc(lane < (int)total ? ts.survivors[wave][lane] : 0u, lane);
        if (lane < kTop) out_top[lane] = v;
    } else {
        // many equal values: kTop rounds of "largest composite below the previous"
        uint32_t prev = 0xFFFFFFFFu, mine_top = 0u;
        for (int round = 0; round < kTop; ++round) {
            uint32_t best = 0u;
#pragma unroll
            for (int e = 0; e < EMAX; ++e)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    // recomputed every round: hoisting 64 composites out of the
                    // round loop would cost 64 registers for a rare path
                    uint32_t kw = key2[e][j >> 1];
                    __asm__ volatile("" : "+v"(kw));
                    const uint32_t k = j & 1 ? kw >> 16 : kw & 0xFFFFu;
                    const uint32_t c = k ? (exact_of_prefilter(k) << 16) |
                                               (0xFFFFu - (base_idx + (uint32_t)(e * kChunk + j)))
                                         : 0u;
                    if (c < prev && c > best) best = c;
                }
            best = wave_max_u32(best);
            if (lane == round) mine_top = best;
            prev = best;
        }
        wave_lds_sync();
        if (lane < kTop) out_top[lane] = mine_top;
    }
    return nonfinite != 0u;
}

// Greedy rows publish only their argmax: the tile keeps its single largest
// composite (value desc, then lowest id; the composite order of tile_top) in
// out_top[0] and zeros in the other slots.  Returns the non-finite flag as
// tile_top does.
// Whole tiles (every element of the lane's EMAX chunks exists): one pass of
// six VALU per word.  Prefilter keys (prefilter_key2) order like the values
// except that -0 sits just below +0, which the exact order ties; the lane's
// composite is (prefilter key << 16 | last - local position), its maximum the
// largest key at the lowest position, found with a three-input maximum per
// word.  A wave whose maximum key is -0 or +0 (the one place the two orders
// differ) returns false and takes the general path; otherwise out_top[0] is
// the exact composite tile_max_general computes.  *nonfinite: as tile_top.
template <int EMAX, bool HALF>
__device__ bool tile_max_whole(const uint4 (&raw)[EMAX], uint32_t base_idx, int lane, uint32_t* out_top,
                               bool* nonfinite) {
    constexpr uint32_t kLast = EMAX * 8 - 1;  // the lane's last position
    uint32_t best = 0;
    u16x2_t kmin = {0xFFFF, 0xFFFF};
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t k2 = prefilter_key2((&raw[e].x)[w]);
            kmin = __builtin_elementwise_min(kmin, __builtin_bit_cast(u16x2_t, k2));
            const uint32_t pos = (uint32_t)(e * 8 + 2 * w);  // lane-local position of the low half
            const uint32_t c_lo = (k2 << 16) | (kLast - pos);
            const uint32_t c_hi = (k2 & 0xFFFF0000u) | (kLast - 1u - pos);
            const uint32_t m = c_lo > c_hi ? c_lo : c_hi;
            best = m > best ? m : best;
        }
    const uint32_t key = best >> 16, pos = kLast - (best & 0xFFFFu);
    constexpr uint32_t kHi = HALF ? 0xFC00u : 0xFF80u, kLo = HALF ? 0x03FFu : 0x007Fu;
    *nonfinite = key >= kHi || kmin.x <= kLo || kmin.y <= kLo;
    const uint32_t wave_key = wave_max_u32(key);
    if (wave_key == 0x7FFFu || wave_key == 0x8000u) return false;  // wave-uniform
    // position (chunk e, element j of the lane's 8) -> tile index
    const uint32_t idx = base_idx + (pos >> 3) * kChunk + (pos & 7u);
    uint32_t lane_best = (exact_of_prefilter(key) << 16) | (0xFFFFu - idx);
    lane_best = wave_max_u32(lane_best);
    if (lane < kTop) out_top[lane] = lane == 0 ? lane_best : 0u;
    return true;
}

template <int EMAX, bool HALF>
__device__ bool tile_max(const uint4 (&raw)[EMAX], int chunks, uint32_t base_idx, int width_left,
                         int lane, uint32_t* out_top) {
    if (chunks == EMAX && chunks * kChunk <= width_left) {  // wave-uniform
        bool nonfinite = false;
        if (tile_max_whole<EMAX, HALF>(raw, base_idx, lane, out_top, &nonfinite)) return nonfinite;
    }
    // Per word (two elements): packed order keys, masked to 0 (empty) past the
    // tile; the word's larger key and the word's position form a composite
    // whose maximum is the lane's largest key in its lowest word; inside that
    // word the even element (lower index) wins a tie.
    // Valid halves of the last chunk (only it can be partial): element
    // base_idx + (chunks - 1) * kChunk + j exists iff j < lim.
    const int lim = width_left - (int)base_idx - (chunks - 1) * kChunk;
    uint32_t last_mask[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
        last_mask[w] = (2 * w < lim ? 0x0000FFFFu : 0u) | (2 * w + 1 < lim ? 0xFFFF0000u : 0u);
    uint32_t magmax = 0, best = 0;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t word = (&raw[e].x)[w];
            const uint32_t valid = e < chunks - 1 ? 0xFFFFFFFFu : (e == chunks - 1 ? last_mask[w] : 0u);
            const uint32_t mag = word & 0x7FFF7FFFu & valid;
            magmax = __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, magmax),
                                                                            __builtin_bit_cast(u16x2_t, mag)));
            const uint32_t k2 = order_key16x2(word) & valid;  // 0 = empty element
            const uint32_t lo = k2 & 0xFFFFu, hi = k2 >> 16;
            const uint32_t m = lo > hi ? lo : hi;
            const uint32_t c = (m << 16) | (0xFFFFu - (uint32_t)(e * 4 + w));
            best = c > best ? c : best;
        }
    // the winning word: its key and which half holds it (lo first)
    const uint32_t wi = 0xFFFFu - (best & 0xFFFFu), key = best >> 16;
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < EMAX; ++e)
#pragma unroll
        for (int w = 0; w < 4; ++w) word = wi == (uint32_t)(e * 4 + w) ? (&raw[e].x)[w] : word;
    const uint32_t lo_key = order_key16(word & 0xFFFFu);
    const uint32_t half = lo_key == key ? 0u : 1u;
    const uint32_t idx = base_idx + (wi >> 2) * kChunk + 2 * (wi & 3) + half;
    uint32_t lane_best = key ? (key << 16) | (0xFFFFu - idx) : 0u;
    lane_best = wave_max_u32(lane_best);
    if (lane < kTop) out_top[lane] = lane == 0 ? lane_best : 0u;
    const u16x2_t mm = __builtin_bit_cast(u16x2_t, magmax);
    constexpr unsigned short kInf = HALF ? 0x7C00 : 0x7F80;
    return mm.x >= kInf || mm.y >= kInf;
}

template <int EMAX, bool FUSED, int SLOTS, bool HALF>
__global__ __launch_bounds__(kThreads) void accept_kernel(AcceptArgs a) {
    __shared__ TileScratch ts;
    __shared__ VerifyScratch<SLOTS> vs[kWaves];
    __shared__ uint32_t key_spill[kWaves * EMAX * 4 * kWave];  // tile_top's key words, word-major
    const int tile = blockIdx.x, row = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    // live sequences and owned rows: host values, or device counts read now
    int live_rows = a.live_rows, owned_rows = a.owned_rows;
    if (FUSED && a.live_count) {
        const int v = a.live_count[0];
        live_rows = v < 0 ? 0 : (v > a.c ? a.c : v);
        owned_rows = live_rows * a.group_rows;
    } else if (!FUSED && a.owned_count) {
        const int v = a.owned_count[0];
        owned_rows = v < 0 ? 0 : (v > a.rows ? a.rows : v);
    }
    auto row_owned = [&](int r) {
        return r < owned_rows && (FUSED || !a.row_activity || a.row_activity[r] != 0);
    };
    const bool owned = row_owned(row);
    const int64_t begin = (int64_t)tile * a.tile_width;
    const int width_left = (int)((a.width - begin) < a.tile_width ? (a.width - begin) : a.tile_width);
    const int chunks = (width_left + kChunk - 1) / kChunk;
    const uint16_t* src = a.logits + (int64_t)row * a.row_stride + begin;

    uint4 raw[EMAX];
    const bool vec = a.vector_loads != 0;
    if (owned && vec && chunks * kChunk <= width_left) {
        // every chunk complete: all loads in one straight run so that they are
        // in flight together (per-chunk branches made the compiler wait for
        // each load before issuing the next); chunks past the tile repeat the
        // last one and are masked out by the tile reductions (e >= chunks)
#pragma unroll
        for (int e = 0; e < EMAX; ++e)
            raw[e] = *reinterpret_cast<const uint4*>(src + (e < chunks ? e : chunks - 1) * kChunk + threadIdx.x * 8);
    } else if (owned) {
#pragma unroll
        for (int e = 0; e < EMAX; ++e) {
            raw[e] = make_uint4(0, 0, 0, 0);
            if (e >= chunks) continue;
            const int off = e * kChunk + threadIdx.x * 8;
            if (vec && off + 8 <= width_left) {
                raw[e] = *reinterpret_cast<const uint4*>(src + off);
            } else {
                uint32_t w[4] = {0, 0, 0, 0};
                for (int j = 0; j < 8; ++j)
                    if (off + j < width_left) w[j >> 1] |= (uint32_t)src[off + j] << ((j & 1) * 16);
                raw[e] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < EMAX; ++e) raw[e] = make_uint4(0, 0, 0, 0);
    }
    // the fused verify's inputs for depth d = wave of this row's group, read
    // now so that their latency hides under the tile phase (only the group's
    // last workgroup uses them; deeper depths read them when verified)
    const int group = row / a.group_rows;
    VerifyPrefetch pre = {};
    // (a one-depth group verifies on three waves, each needing depth 0's inputs)
    const bool split_verify = FUSED && SLOTS == 1 && a.group_rows == 2;
    const int pre_depth = split_verify ? 0 : wave;
    if (FUSED && (wave < a.group_rows - 1 || (split_verify && wave < 3)))
        pre = prefetch_verify(a, (int64_t)pre_depth * a.c + group, lane);
    const bool greedy_row = a.row_temperatures[row] == 0.0f;  // row-uniform
    // wave top-kTop of this wave's share (the maximum alone for a greedy
    // row), then the workgroup's top-kTop
    const uint32_t base_idx = (uint32_t)(threadIdx.x * 8);
    const bool nonfinite =
        greedy_row ? tile_max<EMAX, HALF>(raw, owned ? chunks : 0, base_idx, width_left, lane, &ts.wave_top[wave * kTop])
                   : tile_top<EMAX, HALF>(raw, owned ? chunks : 0, base_idx, width_left, ts,
                                    &key_spill[wave * EMAX * 4 * kWave], lane, wave, &ts.wave_top[wave * kTop]);
    const uint32_t bad = __any(nonfinite);
    if (lane == 0) ts.flags[wave] = bad;
    __syncthreads();
    uint32_t* part = a.partial_keys + ((int64_t)row * a.tiles + tile) * kTop;
    // workgroup top-kTop: wave 0 sorts the waves' lists in registers, waves
    // 0-2 first (60 entries), then its top kTop with wave 3's list (a greedy
    // row takes the largest of the waves' maxima)
    if (wave == 0) {
        uint32_t v;
        if (greedy_row) {
            // a greedy tile keeps only slot 0 of each wave's list
            v = wave_max_u32(lane < kWaves ? ts.wave_top[lane * kTop] : 0u);
            v = lane == 0 ? v : 0u;
        } else {
            v = wave_sort_desc(lane < 3 * kTop ? ts.wave_top[lane] : 0u, lane);
            v = lane < kTop ? v : (lane < 2 * kTop ? ts.wave_top[3 * kTop + lane - kTop] : 0u);
            v = wave_sort_desc(v, lane);
        }
        if (lane < kTop) store_device(&part[lane], v);
        if (lane == 0)
            store_device(&a.partial_flags[(int64_t)row * a.tiles + tile],
                         ts.flags[0] | ts.flags[1] | ts.flags[2] | ts.flags[3]);
    }
    // arrival: the last workgroup of this row group finalises it
    if (!arrive_last(&a.counters[group], (uint32_t)(a.group_rows * a.tiles), &ts.last)) return;

    // ---- finalise the group's rows: merge tiles, publish candidates -------
    const int row0 = group * a.group_rows;
    for (int gr = wave; gr < a.group_rows; gr += kWaves) {
        const int r = row0 + gr;
        const bool own = row_owned(r);
        // tiles <= kMaxTiles < 64: one flag per lane; a greedy row's tile
        // maxima (slot 0) are loaded with it, before either is used
        const float temp = a.row_temperatures[r];
        const bool greedy_pub = temp == 0.0f;
        const bool tile_lane = lane < a.tiles;
        uint32_t bad_row = tile_lane ? load_device(&a.partial_flags[(int64_t)r * a.tiles + lane]) : 0u;
        const uint32_t k32_slot0 =
            greedy_pub && tile_lane ? load_device(&a.partial_keys[((int64_t)r * a.tiles + lane) * kTop]) : 0u;
        bad_row = __any(bad_row != 0);
        const int want = a.count < kTop ? a.count : kTop;
        uint64_t my = 0ull;
        if (greedy_pub) {
            // the tiles of a greedy row hold their maximum in slot 0: the
            // row's argmax is the largest of those (lane 0 = rank 0)
            uint64_t e = 0ull;
            if (tile_lane) {
                const uint32_t k32 = k32_slot0;
                if (k32 != 0u) {
                    const uint32_t id = (uint32_t)lane * (uint32_t)a.tile_width + (0xFFFFu - (k32 & 0xFFFFu));
                    e = ((uint64_t)(k32 >> 16) << 32) | (0xFFFFFFFFu - id);
                }
            }
            e = wave_max_u64(e);
            my = lane == 0 ? e : 0ull;
        } else {
            // kTop global winners by (value desc, id asc) over tiles * kTop entries
            constexpr int kPer = (kMaxTiles * kTop + kWave - 1) / kWave;
            uint64_t entry[kPer];
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                const int i = lane + q * kWave;
                entry[q] = 0ull;
                if (i < a.tiles * kTop) {
                    const uint32_t k32 = load_device(&a.partial_keys[(int64_t)r * a.tiles * kTop + i]);
                    if (k32 != 0u) {
                        const uint32_t t = (uint32_t)(i / kTop);
                        const uint32_t id = t * (uint32_t)a.tile_width + (0xFFFFu - (k32 & 0xFFFFu));
                        entry[q] = ((uint64_t)(k32 >> 16) << 32) | (0xFFFFFFFFu - id);
                    }
                }
            }
            my = wave_topk_u64<kPer>(entry, a.tiles * kTop, want, lane, ts.merge[wave]);
        }
        const int j = lane;  // capacity <= 64
        if (j < a.capacity) {
            uint16_t sc = HALF ? 0x7E00u : 0x7FC0u;  // quiet NaN padding
            int64_t id = -1;
            if (j < a.count && own) {
                const bool filled = j < want && my != 0ull;
                const int64_t gid = (int64_t)(0xFFFFFFFFu - (uint32_t)(my & 0xFFFFFFFFu));
                // the score's bits from its order key, which is one-to-one
                // except that -0 and +0 share key 0x8000: only then re-read
                const uint32_t k16 = (uint32_t)(my >> 32);
                auto exact = [&]() -> uint16_t {
                    return k16 != 0x8000u ? (uint16_t)bits_of_key16(k16) : a.logits[(int64_t)r * a.row_stride + gid];
                };
                if (bad_row) {
                    id = -2;
                } else if (!greedy_pub) {
                    if (filled) { sc = exact(); id = gid + a.vocab_start; }
                } else if (!a.all_random && j == 0 && filled) {
                    sc = exact();
                    id = gid + a.vocab_start;
                }
            }
            a.cand_scores[(int64_t)r * a.capacity + j] = sc;
            a.cand_ids[(int64_t)r * a.capacity + j] = id;
            if (FUSED) {
                ts.cand_score[gr][j] = sc;
                ts.cand_id[gr][j] = id;
            }
        }
    }
    if (!FUSED) {
        if (threadIdx.x == 0) store_device(&a.counters[group], 0u);
        return;
    }
    __syncthreads();
    // ---- fused: verify each depth of sequence `group`, merge the prefix ----
    const int c = group, depth = a.group_rows - 1;
    // the verified row of depth d: q candidates from the prefetch (or global),
    // the target rows d and d + 1 from LDS
    auto make_row = [&](int d, bool prefetched) {
        const int64_t pi = (int64_t)d * a.c + c;
        VerifyRow vr;
        vr.active = c < live_rows;
        vr.rows_ok = true;
        const bool in = lane < a.capacity;
        vr.staged = true;
        vr.st_q_s = prefetched ? pre.q_score : (in ? (uint32_t)a.q_scores[pi * a.capacity + lane] : 0x7FC0u);
        vr.st_q_i = prefetched ? pre.q_id : (in ? a.q_ids[pi * a.capacity + lane] : -1);
        vr.st_p0_s = ts.cand_score[d][lane];
        vr.st_p0_i = ts.cand_id[d][lane];
        vr.st_p1_s = ts.cand_score[d + 1][lane];
        vr.st_p1_i = ts.cand_id[d + 1][lane];
        vr.q_scores = a.q_scores + pi * a.capacity;
        vr.q_ids = a.q_ids + pi * a.capacity;
        vr.p0_scores = ts.cand_score[d];
        vr.p0_ids = ts.cand_id[d];
        vr.p1_scores = ts.cand_score[d + 1];
        vr.p1_ids = ts.cand_id[d + 1];
        vr.q_rank_stride = 0;
        vr.p_rank_stride = 0;
        vr.tp = 1;
        vr.k = a.capacity;
        vr.block = a.block;
        if (prefetched) {
            vr.draft = vr.active ? pre.draft : -1;
            vr.temperature = vr.active ? pre.temperature : 1.0f;
            vr.top_p = vr.active ? pre.top_p : 1.0f;
            vr.top_k = vr.active ? pre.top_k : 1;
            vr.seed = vr.active ? pre.seed : 0;
            vr.ordinal = vr.active ? pre.ordinal : 0;
            vr.u0 = pre.u0;
            vr.u1 = pre.u1;
        } else {
            vr.draft = vr.active ? a.draft_tokens[pi] : -1;
            vr.temperature = vr.active ? a.temperatures[pi] : 1.0f;
            vr.top_p = vr.active ? a.top_ps[pi] : 1.0f;
            vr.top_k = vr.active ? a.top_ks[pi] : 1;
            vr.seed = vr.active ? a.seeds[pi] : 0;
            vr.ordinal = vr.active ? a.ordinals[pi] : 0;
            vr.u0 = a.uniforms ? a.uniforms[2 * pi] : 0.0f;
            vr.u1 = a.uniforms ? a.uniforms[2 * pi + 1] : 0.0f;
        }
        vr.has_uniforms = a.uniforms != nullptr;
        vr.underfilled = false;
        return vr;
    };
    if (split_verify) {
        // one depth: waves 0, 1, 2 select and weigh q, p0 and p1 at once; wave
        // 0 then finishes the row from the three sets (the same operations as
        // verify_wave, in the same order)
        const VerifyRow vr = make_row(0, true);
        if (wave < 3) {
            VerifySet<SLOTS> mine;
            verify_set<SLOTS>(vr, wave, vs[wave], lane, mine);
            VerifySetLds& o = ts.sets[wave];
            o.s[lane] = mine.sel.s[0];
            o.i[lane] = mine.sel.i[0];
            o.r[lane] = mine.sel.r[0];
            o.prob[lane] = mine.prob[0];
            if (lane == 0) { o.mass = mine.mass; o.count = mine.count; o.ok = mine.ok; }
        }
        __syncthreads();
        if (wave == 0) {
            VerifySet<SLOTS> set[3];
#pragma unroll
            for (int w = 0; w < 3; ++w) {
                const VerifySetLds& o = ts.sets[w];
                set[w].sel.s[0] = o.s[lane];
                set[w].sel.i[0] = o.i[lane];
                set[w].sel.r[0] = o.r[lane] != 0;
                set[w].prob[0] = o.prob[lane];
                set[w].mass = o.mass;
                set[w].count = o.count;
                set[w].ok = o.ok != 0;
            }
            verify_finish<SLOTS>(vr, set[0], set[1], set[2], vs[0], lane, ts.decisions[0]);
            if (lane == 0) {
                a.decisions[2 * (int64_t)c] = ts.decisions[0][0];
                a.decisions[2 * (int64_t)c + 1] = ts.decisions[0][1];
            }
        }
    } else {
        for (int d = wave; d < depth; d += kWaves) {
            const int64_t pi = (int64_t)d * a.c + c;
            const VerifyRow vr = make_row(d, d == wave);  // first depth of this wave: prefetched
            verify_wave<SLOTS>(vr, vs[wave], lane, ts.decisions[d]);
            if (lane == 0) {
                a.decisions[2 * pi] = ts.decisions[d][0];
                a.decisions[2 * pi + 1] = ts.decisions[d][1];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t accepted = depth, bonus = ts.decisions[depth - 1][1];
        bool good = true;
        for (int d = depth - 1; d >= 0; --d) {
            const int64_t av = ts.decisions[d][0], tok = ts.decisions[d][1];
            if (av == 0) { accepted = d; bonus = tok; }
            good = good && (av == 0 || av == 1) && tok >= 0;
        }
        const bool ok = c < live_rows && good;
        a.merged[2 * (int64_t)c] = ok ? accepted : -1;
        a.merged[2 * (int64_t)c + 1] = ok ? bonus : -1;
        if (a.emitted) {
            for (int d = 0; d <= depth; ++d) {
                int64_t tok = -1;
                if (ok && d < accepted) tok = a.draft_tokens[(int64_t)d * a.c + c];
                if (ok && d == accepted) tok = bonus;
                a.emitted[(int64_t)c * (depth + 1) + d] = tok;
            }
        }
        store_device(&a.counters[group], 0u);
    }
}

// --------------------------------------------------------------------------
// fp32 candidate preparation (local_candidates.py:41 SCORE_TYPE 2, kernels
// local_candidates.cu:19-146).  Same rules as the 16-bit path: order by value
// (-0 == +0), ties by ascending column, raw scores published, -2 in every
// counted slot of a row with a non-finite logit, greedy rows publish the
// argmax in slot 0 (padding when all_random).  A 64-bit composite carries the
// order key of the value above 0xFFFFFFFF - column, so the larger composite
// is the better candidate and every composite of a real column is nonzero.
// --------------------------------------------------------------------------
__device__ __forceinline__ uint64_t f32_composite(uint32_t u, uint32_t col) {
    const uint32_t m = u & 0x7FFFFFFFu;
    const uint32_t key = (u & 0x80000000u) ? 0x80000000u - m : 0x80000000u + m;
    return ((uint64_t)key << 32) | (0xFFFFFFFFu - col);
}

__device__ __forceinline__ bool f32_row_owned(const CandF32Args& a, int row) {
    int owned = a.owned_rows;
    if (a.owned_count) {
        const int v = a.owned_count[0];
        owned = v < 0 ? 0 : (v > a.rows ? a.rows : v);
    }
    return row < owned && (!a.row_activity || a.row_activity[row] != 0);
}

__device__ __forceinline__ int f32_want(const CandF32Args& a, int row) {
    return a.row_temperatures[row] == 0.0f ? 1 : a.count;
}

constexpr int kF32Waves = kThreads / kWave;
constexpr int kF32WaveCols = kCandF32Tile / kF32Waves;  // 1024
constexpr int kF32PerLane = kF32WaveCols / kWave;       // 16

// Workgroup (tile, row): the top `want` composites of kCandF32Tile columns
// and whether all of them are finite.  Wave w reads columns
// [w * 1024, (w + 1) * 1024) of the tile: 16-byte loads of four columns per
// lane per round when the rows are 16-byte aligned, else one column per lane.
__global__ __launch_bounds__(kThreads) void cand_f32_tile_kernel(CandF32Args a) {
    __shared__ uint64_t buf[kF32Waves][kWave];
    __shared__ uint64_t wave_top[kF32Waves * kTop];
    __shared__ uint32_t wave_good[kF32Waves];
    const int tile = blockIdx.x, row = blockIdx.y;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (!f32_row_owned(a, row)) return;  // published as padding; partials unread
    const int want = f32_want(a, row);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.logits) + (int64_t)row * a.row_stride;
    const int c0 = tile * kCandF32Tile + wave * kF32WaveCols;
    uint64_t e[kF32PerLane];
    uint32_t bad = 0;
    if (a.vector_loads) {
#pragma unroll
        for (int q = 0; q < kF32PerLane / 4; ++q) {
            const int c = c0 + q * 4 * kWave + lane * 4;
            uint32_t u[4];
            if (c + 4 <= a.width) {
                const uint4 v = *reinterpret_cast<const uint4*>(src + c);
                u[0] = v.x; u[1] = v.y; u[2] = v.z; u[3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) u[i] = c + i < a.width ? src[c + i] : 0u;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool in = c + i < a.width;
                bad |= in && (u[i] & 0x7F800000u) == 0x7F800000u;
                e[q * 4 + i] = in ? f32_composite(u[i], (uint32_t)(c + i)) : 0ull;
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < kF32PerLane; ++q) {
            const int c = c0 + q * kWave + lane;
            const bool in = c < a.width;
            const uint32_t u = in ? src[c] : 0u;
            bad |= in && (u & 0x7F800000u) == 0x7F800000u;
            e[q] = in ? f32_composite(u, (uint32_t)c) : 0ull;
        }
    }
    const uint64_t top = wave_topk_u64<kF32PerLane>(e, kF32WaveCols, want, lane, buf[wave]);
    if (lane < want) wave_top[wave * kTop + lane] = top;
    const bool wave_bad = __any(bad);
    if (lane == 0) wave_good[wave] = !wave_bad;
    __syncthreads();
    if (wave != 0) return;
    uint64_t m[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int i = lane + h * kWave, w = i / kTop, r = i % kTop;
        m[h] = (w < kF32Waves && r < want) ? wave_top[i] : 0ull;
    }
    const uint64_t best = wave_topk_u64<2>(m, 2 * kWave, want, lane, buf[0]);
    const int64_t slot = (int64_t)row * a.tiles + tile;
    if (lane < want) a.partial[slot * kTop + lane] = best;
    if (lane == 0) {
        uint32_t g = 1;
#pragma unroll
        for (int w = 0; w < kF32Waves; ++w) g &= wave_good[w];
        a.partial_finite[slot] = g;
    }
}

// One wave per row: merges the tiles' lists (7 * 64 entries per round, the
// running top carried in the first entry of each lane) and publishes.
__global__ __launch_bounds__(kWave) void cand_f32_publish_kernel(CandF32Args a) {
    __shared__ uint64_t buf[kWave];
    constexpr int kP = 8;
    const int row = blockIdx.x, lane = threadIdx.x;
    const bool owned = f32_row_owned(a, row);
    const bool greedy = a.row_temperatures[row] == 0.0f;
    const int want = f32_want(a, row);
    uint32_t good = 1;
    uint64_t run = 0;
    if (owned) {
        for (int t = lane; t < a.tiles; t += kWave) good &= a.partial_finite[(int64_t)row * a.tiles + t];
        good = !__any(!good);
        if (good) {
            const int n = a.tiles * want;
            for (int base = 0; base < n; base += (kP - 1) * kWave) {
                uint64_t e[kP];
                e[0] = lane < want ? run : 0ull;
#pragma unroll
                for (int q = 1; q < kP; ++q) {
                    const int i = base + (q - 1) * kWave + lane;
                    e[q] = i < n ? a.partial[((int64_t)row * a.tiles + i / want) * kTop + i % want] : 0ull;
                }
                run = wave_topk_u64<kP>(e, kP * kWave, want, lane, buf);
            }
        }
    }
    const uint32_t* src = reinterpret_cast<const uint32_t*>(a.logits) + (int64_t)row * a.row_stride;
    // capacity <= 64: lane j publishes slot j, and holds rank j of `run`
    if (lane < a.capacity) {
        uint32_t score = 0x7FC00000u;
        int64_t id = -1;
        if (owned && lane < a.count) {
            if (!good) {
                id = -2;
            } else if ((!greedy || (!a.all_random && lane == 0)) && run != 0ull) {
                const uint32_t col = 0xFFFFFFFFu - (uint32_t)run;
                score = src[col];
                id = a.vocab_start + col;
            }
        }
        reinterpret_cast<uint32_t*>(a.scores)[(int64_t)row * a.capacity + lane] = score;
        a.ids[(int64_t)row * a.capacity + lane] = id;
    }
}

template <int EMAX, bool FUSED>
hipError_t launch_accept_slots(const AcceptArgs& a, hipStream_t s) {
    dim3 grid(a.tiles, a.rows), block(kThreads);
    if (a.block > 64) return hipErrorInvalidValue;
    if constexpr (!FUSED) {
        // fp16 logits: candidate preparation only (the verification takes bf16)
        if (a.scores_fp16) {
            accept_kernel<EMAX, false, 1, true><<<grid, block, 0, s>>>(a);
            return hipGetLastError();
        }
    } else {
        if (a.scores_fp16) return hipErrorInvalidValue;
    }
    accept_kernel<EMAX, FUSED, 1, false><<<grid, block, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_accept(const AcceptArgs& a, bool fused, hipStream_t s) {
    const int chunks = (a.tile_width + kChunk - 1) / kChunk;
    if (chunks <= 4) return fused ? launch_accept_slots<4, true>(a, s) : launch_accept_slots<4, false>(a, s);
    if (chunks <= 8) return fused ? launch_accept_slots<8, true>(a, s) : launch_accept_slots<8, false>(a, s);
    if (chunks <= kMaxTileChunks)
        return fused ? launch_accept_slots<16, true>(a, s) : launch_accept_slots<16, false>(a, s);
    return hipErrorInvalidValue;
}

hipError_t launch_candidates_f32(const CandF32Args& a, hipStream_t s) {
    if (a.count < 1 || a.count > kTop || a.capacity < a.count || a.capacity > kWave) return hipErrorInvalidValue;
    cand_f32_tile_kernel<<<dim3(a.tiles, a.rows), kThreads, 0, s>>>(a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    cand_f32_publish_kernel<<<a.rows, kWave, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_verify(const VerifyArgs& a, hipStream_t s) {
    dim3 grid(a.q_rows), block(kWave);
    if (a.block <= 64) verify_candidates_kernel<1><<<grid, block, 0, s>>>(a);
    else if (a.block <= 128) verify_candidates_kernel<2><<<grid, block, 0, s>>>(a);
    else if (a.block <= 256) verify_candidates_kernel<4><<<grid, block, 0, s>>>(a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_root_sample(const RootSampleArgs& a, hipStream_t s) {
    if (a.tp * a.k > kRootThreads || a.k > kWave) return hipErrorInvalidValue;
    root_sample_kernel<<<a.rows, kRootThreads, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_merge_prefix(const int64_t* decisions, int c, int depth, const int32_t* live,
                               int live_rows, int64_t* out, hipStream_t s) {
    const int blocks = (c + kThreads - 1) / kThreads;
    merge_prefix_kernel<<<blocks > 0 ? blocks : 1, kThreads, 0, s>>>(decisions, c, depth, live,
                                                                   live_rows, out);
    return hipGetLastError();
}

}  // namespace cubic
