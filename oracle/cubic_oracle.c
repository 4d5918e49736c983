/*
 * cubic_oracle.c -- CPU restatement of cubic-serve's MTP verify-step algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or the timed
 * CPU baseline.  No product code path may call it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * src/cubic_serve/ of QuantTrio/cubic-serve v0.1.1).  Build with
 * -ffp-contract=off: the reference's FP32 arithmetic is unfused.
 *
 * Pinning (what checks each function independently of this text) is listed in
 * oracle/README.md and exercised by tests/test_oracle_*.py.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>
#include <stdlib.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* IEEE binary16 / bfloat16 conversions (round to nearest even).            */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

EXPORT float oracle_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24 is exact in binary32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112) << 23) | (man << 13));
}

EXPORT uint16_t oracle_float_to_half(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t ax = u & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {
        /* half subnormal range: value = m * 2^-24; round |f| * 2^24 to integer (RNE) */
        float a = u2f(ax) * 16777216.0f; /* exact scaling by 2^24 */
        float r = rintf(a);              /* default rounding mode = nearest even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t mant = ax & 0x7fffffu, e = (ax >> 23) - 112;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* carries into exponent correctly */
    return (uint16_t)(sign | h);
}

EXPORT uint16_t oracle_float_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

EXPORT float oracle_bf16_to_float(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ------------------------------------------------------------------------ */
/* A1  unpack_cubic  -- quantization/extensions/cubic/reference.py:31-47    */
/* Little-endian bitstream, code i at bit offset i*bits, straddling bytes.  */
/* bits==1: 2*raw-1.  Else two's complement, the most negative code is the  */
/* reserved zero.                                                           */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_unpack_cubic(const uint8_t* packed, int64_t rows, int64_t k, int bits,
                               int8_t* codes) {
    if (bits < 1 || bits > 8 || k <= 0 || rows < 0) return -1;
    const int64_t row_bytes = (k * bits + 7) / 8;
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* src = packed + r * row_bytes;
        for (int64_t i = 0; i < k; ++i) {
            const int64_t pos = i * bits, byte = pos / 8;
            const int shift = (int)(pos % 8);
            uint32_t low = (uint32_t)src[byte] >> shift;
            int64_t hi_byte = byte + 1 < row_bytes ? byte + 1 : row_bytes - 1; /* clamp as :41 */
            uint32_t high = (uint32_t)src[hi_byte] << (8 - shift);
            uint32_t raw = (shift + bits > 8 ? (low | high) : low) & ((1u << bits) - 1u);
            int v;
            if (bits == 1) {
                v = (int)raw * 2 - 1;
            } else {
                const int sign = 1 << (bits - 1);
                v = (int)raw >= sign ? (int)raw - (1 << bits) : (int)raw;
                if (v == -sign) v = 0;
            }
            codes[r * k + i] = (int8_t)v;
        }
    }
    return 0;
}

/* Inverse of unpack (test fixture helper): pack signed codes into the       */
/* little-endian bitstream the reference decodes.  Reserved code never used. */
EXPORT int oracle_pack_cubic(const int8_t* codes, int64_t rows, int64_t k, int bits,
                             uint8_t* packed) {
    if (bits < 1 || bits > 8) return -1;
    const int64_t row_bytes = (k * bits + 7) / 8;
    memset(packed, 0, (size_t)(rows * row_bytes));
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < k; ++i) {
            int q = codes[r * k + i];
            uint32_t raw = bits == 1 ? (uint32_t)((q + 1) / 2) : (uint32_t)q & ((1u << bits) - 1u);
            int64_t pos = i * bits;
            for (int b = 0; b < bits; ++b, ++pos)
                if (raw >> b & 1u) packed[r * row_bytes + pos / 8] |= (uint8_t)(1u << (pos % 8));
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* A2  cubic_metadata -- reference.py:50-95.  All three formats expand to   */
/* per-group (scale f32, a f16, b f16); groups = [N/go, ceil(K/gi)].        */
/* `part_of_group_row[g]` = partition index of output-group row g.          */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_metadata_fmt1(const int8_t* scale_i8, const uint8_t* ab,
                                const float* scale_global, const float* a_global,
                                const float* b_global, const int32_t* part_of_group_row,
                                int64_t group_rows, int64_t group_cols,
                                float* s, uint16_t* a, uint16_t* b) {
    /* :67-85  s = i8 * gS[p];  a = fp16(1 + a4*gA[p]);  b = fp16(b4*gB[p]) */
    for (int64_t g = 0; g < group_rows; ++g) {
        const int p = part_of_group_row[g];
        for (int64_t c = 0; c < group_cols; ++c) {
            const int64_t i = g * group_cols + c;
            int lo = ab[i] & 15, hi = ab[i] >> 4;
            float av = (float)(lo >= 8 ? lo - 16 : lo);
            float bv = (float)(hi >= 8 ? hi - 16 : hi);
            s[i] = (float)scale_i8[i] * scale_global[p];
            float prod = av * a_global[p];
            a[i] = oracle_float_to_half(1.0f + prod);
            b[i] = oracle_float_to_half(bv * b_global[p]);
        }
    }
    return 0;
}

EXPORT int oracle_metadata_fmt2(const uint16_t* metadata, const uint16_t* curve_a,
                                const uint16_t* curve_b, const int32_t* part_of_group_row,
                                int64_t group_rows, int64_t group_cols,
                                float* s, uint16_t* a, uint16_t* b) {
    /* :86-95  scale = fp16 bits ((m & 0x3FFF) << 1); curve = m >> 14 picks (a,b)[p, curve] */
    for (int64_t g = 0; g < group_rows; ++g) {
        const int p = part_of_group_row[g];
        for (int64_t c = 0; c < group_cols; ++c) {
            const int64_t i = g * group_cols + c;
            uint32_t m = metadata[i];
            s[i] = oracle_half_to_float((uint16_t)((m & 0x3FFFu) << 1));
            a[i] = curve_a[p * 4 + (m >> 14)];
            b[i] = curve_b[p * 4 + (m >> 14)];
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* A3  decode_cubic -- reference.py:98-121.                                 */
/*   t = fl32(|q| / D) computed in fp64 then rounded (:120), D = 2^(b-1)-1   */
/*   w = sign(q) * (s * (t * (a + t * (b + t * ((1 - a) - b)))))  in fp32   */
/*   bits == 1: w = q * s                                                   */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_decode_cubic(const int8_t* codes, const float* s, const uint16_t* a,
                               const uint16_t* b, int64_t n, int64_t k, int bits,
                               int64_t group_in, int64_t group_out, float* w) {
    const int64_t gcols = (k + group_in - 1) / group_in;
    const double den = (double)((1 << (bits - 1)) - 1);
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) {
            const int64_t g = (r / group_out) * gcols + i / group_in;
            const float q = (float)codes[r * k + i];
            const float sc = s[g];
            if (bits == 1) { w[r * k + i] = q * sc; continue; }
            const float aa = oracle_half_to_float(a[g]), bb = oracle_half_to_float(b[g]);
            const float t = (float)(fabs((double)q) / den);
            const float c = (1.0f - aa) - bb;
            const float inner = bb + t * c;
            const float mid = aa + t * inner;
            const float v = sc * (t * mid);
            const float sg = q > 0 ? 1.0f : (q < 0 ? -1.0f : 0.0f);
            w[r * k + i] = sg * v;
        }
    return 0;
}

EXPORT void oracle_round_bf16(const float* in, uint16_t* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) out[i] = oracle_float_to_bf16(in[i]);
}

/* ------------------------------------------------------------------------ */
/* A5  linear -- ops/eager/linear.py:43-56 with the WNA16 weight rounding of */
/* ops/eager/quantization.py:181-182: y[m, n] = bf16( sum_k fp32(x) *        */
/* fp32(bf16(W)) ).  The reference's FP32 matmul order is backend-defined;   */
/* this restatement sums k in ascending order.  Parity against it is the    */
/* enclosure bound of guardrail/quantization.py:256-310, not bit equality.  */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_linear_bf16(const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                              int64_t n, uint16_t* y, float* y32) {
    float* xf = (float*)malloc(sizeof(float) * (size_t)k);
    if (!xf) return -1;
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t i = 0; i < k; ++i) xf[i] = oracle_bf16_to_float(x[r * k + i]);
        for (int64_t c = 0; c < n; ++c) {
            const uint16_t* wr = w + c * k;
            float acc = 0.0f;
            for (int64_t i = 0; i < k; ++i) acc += xf[i] * oracle_bf16_to_float(wr[i]);
            if (y32) y32[r * n + c] = acc;
            if (y) y[r * n + c] = oracle_float_to_bf16(acc);
        }
    }
    free(xf);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* exp for the acceptance transform.  The reference leaves exp to Triton    */
/* (tl.exp, speculative.py:38) whose rounding is backend-defined; this      */
/* build fixes one: Cody & Waite (1980) two-constant additive reduction     */
/* x = n*ln2 + r, |r| <= ln2/2, exp(r) by the degree-7 Taylor polynomial in */
/* Horner form, times 2^n.  Unfused IEEE binary32 throughout.  The device  */
/* kernel evaluates the identical sequence, so both agree bit for bit; its  */
/* accuracy against libm expf is pinned by tests.                           */
/* ------------------------------------------------------------------------ */
EXPORT float oracle_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    const float r = (x - n * 0.693359375f) - n * -2.12194440e-4f;
    float p = 1.98412698e-4f;                 /* 1/5040 */
    p = 1.38888889e-3f + r * p;               /* 1/720 */
    p = 8.33333377e-3f + r * p;               /* 1/120 */
    p = 4.16666679e-2f + r * p;               /* 1/24 */
    p = 1.66666672e-1f + r * p;               /* 1/6 */
    p = 0.5f + r * p;
    p = 1.0f + r * p;
    p = 1.0f + r * p;
    int e = (int)n;
    if (e > 127) {
        p = p * u2f((uint32_t)(e - 64 + 127) << 23);
        return p * u2f((uint32_t)(64 + 127) << 23);
    }
    if (e < -126) {
        /* two exact power-of-two scalings; the second rounds once into the subnormals */
        p = p * u2f((uint32_t)(e + 64 + 127) << 23);
        return p * u2f((uint32_t)(-64 + 127) << 23);
    }
    return p * u2f((uint32_t)(e + 127) << 23);
}

/* ------------------------------------------------------------------------ */
/* philox_uniform -- guardrail/quantized_graph/speculative.py:15-30, the     */
/* coordinates of tl.rand(key, offset) used at ops/cuda/sampling/            */
/* speculative.py:143-148, :171-175.  Philox4x32-10 (Salmon et al., SC'11). */
/* ------------------------------------------------------------------------ */
EXPORT void oracle_philox4x32_10(const uint32_t* ctr_in, const uint32_t* key_in, uint32_t* out) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int i = 0; i < 10; ++i) {
        uint64_t a = (uint64_t)0xD2511F53u * c0, b = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(b >> 32) ^ c1 ^ k0, n1 = (uint32_t)b;
        uint32_t n2 = (uint32_t)(a >> 32) ^ c3 ^ k1, n3 = (uint32_t)a;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

EXPORT float oracle_philox_uniform(uint64_t seed, uint64_t ordinal) {
    uint32_t ctr[4] = {(uint32_t)ordinal, 0, 0, 0}, key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    oracle_philox4x32_10(ctr, key, out);
    int64_t sv = (int32_t)out[0];
    if (sv < 0) sv = -sv - 1;
    return (float)sv * 4.6566127342e-10f;
}

/* ------------------------------------------------------------------------ */
/* A13  candidate preparation -- ops/cuda/sampling/local_candidates.py:206- */
/* 226 with local_candidates.cu:19-146 (TP=1, vocab_start=0, no grammar).   */
/* Per owned row: `good` = every logit finite.  Non-greedy rows publish the */
/* top-`count` (score, id) pairs; this build orders them by (score desc, id */
/* asc) -- torch.topk's tie order at the count cutoff is unspecified.       */
/* Greedy rows (temperature == 0) publish the exact argmax, lowest id on    */
/* ties (greedy.cu:28-33), in slot 0 only.  Rows with a non-finite logit    */
/* publish id -2 (NaN score) in every counted slot.  Padding is (NaN, -1).  */
/* ------------------------------------------------------------------------ */
static inline int better(float v, int64_t id, float bv, int64_t bid) {
    return v > bv || (v == bv && id < bid);
}

/* logits and published scores in the reference's SCORE_TYPE (local_candidates.py:41,
   :188): kind 0 = bf16 bits, 1 = fp16 bits, 2 = fp32; scores are published unchanged */
static float candidate_value(const void* logits, int kind, int64_t i, uint32_t* raw) {
    if (kind == 2) {
        float v;
        memcpy(raw, (const uint32_t*)logits + i, 4);
        memcpy(&v, raw, 4);
        return v;
    }
    const uint16_t b = ((const uint16_t*)logits)[i];
    *raw = b;
    return kind ? oracle_half_to_float(b) : oracle_bf16_to_float(b);
}

static void candidate_store(void* out, int kind, int64_t i, uint32_t raw) {
    if (kind == 2) ((uint32_t*)out)[i] = raw;
    else ((uint16_t*)out)[i] = (uint16_t)raw;
}

static int candidates_kind(const void* logits, int kind, int64_t rows, int64_t width, int64_t stride,
                           const float* temperatures, int64_t owned_rows, int count, int capacity,
                           int all_random, void* out_scores, int64_t* out_ids) {
    if (count < 1 || count > capacity || count > 64 || kind < 0 || kind > 2) return -1;
    const uint32_t qnan = kind == 2 ? 0x7fc00000u : kind ? 0x7e00u : 0x7fc0u;
    for (int64_t r = 0; r < rows; ++r) {
        int64_t* id = out_ids + r * capacity;
        for (int j = 0; j < capacity; ++j) { candidate_store(out_scores, kind, r * capacity + j, qnan); id[j] = -1; }
        if (r >= owned_rows) continue;
        uint32_t raw;
        int good = 1;
        for (int64_t j = 0; j < width; ++j) {
            if (!isfinite(candidate_value(logits, kind, r * stride + j, &raw))) { good = 0; break; }
        }
        const int greedy = temperatures[r] == 0.0f;
        if (!good) { for (int j = 0; j < count; ++j) id[j] = -2; continue; }
        /* top-count by (value desc, id asc): insertion into a sorted list; its
           slot 0 is the exact argmax with the lowest id on ties */
        float bv[64]; int64_t bi[64]; uint32_t braw[64]; int filled = 0;
        const int want = count;
        for (int64_t j = 0; j < width; ++j) {
            const float v = candidate_value(logits, kind, r * stride + j, &raw);
            if (filled == want && !better(v, j, bv[want - 1], bi[want - 1])) continue;
            int pos = filled < want ? filled++ : want - 1;
            while (pos > 0 && better(v, j, bv[pos - 1], bi[pos - 1])) {
                bv[pos] = bv[pos - 1]; bi[pos] = bi[pos - 1]; braw[pos] = braw[pos - 1]; --pos;
            }
            bv[pos] = v; bi[pos] = j; braw[pos] = raw;
        }
        if (!greedy) {
            for (int j = 0; j < filled; ++j) { candidate_store(out_scores, kind, r * capacity + j, braw[j]); id[j] = bi[j]; }
        } else if (!all_random && filled) {
            candidate_store(out_scores, kind, r * capacity, braw[0]); id[0] = bi[0];
        }
    }
    return 0;
}

EXPORT int oracle_candidates_dtype(const uint16_t* logits, int64_t rows, int64_t width, int64_t stride,
                                   const float* temperatures, int64_t owned_rows, int count,
                                   int capacity, int all_random, int fp16, uint16_t* out_scores,
                                   int64_t* out_ids) {
    return candidates_kind(logits, fp16 ? 1 : 0, rows, width, stride, temperatures, owned_rows, count,
                           capacity, all_random, out_scores, out_ids);
}

/* fp32 logits -> fp32 scores (SCORE_TYPE 2) */
EXPORT int oracle_candidates_f32(const float* logits, int64_t rows, int64_t width, int64_t stride,
                                 const float* temperatures, int64_t owned_rows, int count,
                                 int capacity, int all_random, float* out_scores, int64_t* out_ids) {
    return candidates_kind(logits, 2, rows, width, stride, temperatures, owned_rows, count, capacity,
                           all_random, out_scores, out_ids);
}

EXPORT int oracle_candidates(const uint16_t* logits, int64_t rows, int64_t width, int64_t stride,
                             const float* temperatures, int64_t owned_rows, int count,
                             int capacity, int all_random, uint16_t* out_scores, int64_t* out_ids) {
    return oracle_candidates_dtype(logits, rows, width, stride, temperatures, owned_rows, count,
                                   capacity, all_random, 0, out_scores, out_ids);
}

/* ------------------------------------------------------------------------ */
/* A14  _verify_k1_kernel -- ops/cuda/sampling/speculative.py:46-219,        */
/* restated lane by lane (BLOCK = next_pow2(TP*K) lanes).  Triton leaves     */
/* the order of tl.sum / tl.cumsum reductions open; this build fixes it as  */
/* ascending lane order, and `/` as IEEE division.                          */
/* ------------------------------------------------------------------------ */
#define INT64_MAXV 0x7FFFFFFFFFFFFFFFLL
#define MAX_LANES 256

static void select_topk(float* scores, int64_t* ids, const int* real, int lanes, int k,
                        float* out_s, int64_t* out_i, int* count) {
    /* speculative.py:11-29 */
    int avail[MAX_LANES];
    int cnt = 0;
    for (int l = 0; l < lanes; ++l) {
        out_s[l] = -INFINITY; out_i[l] = INT64_MAXV; avail[l] = real[l]; cnt += real[l];
    }
    for (int p = 0; p < k; ++p) {
        float best = -INFINITY;
        for (int l = 0; l < lanes; ++l) if (avail[l] && scores[l] > best) best = scores[l];
        int64_t bid = INT64_MAXV;
        for (int l = 0; l < lanes; ++l)
            if (avail[l] && scores[l] == best && ids[l] < bid) bid = ids[l];
        out_s[p] = best; out_i[p] = bid;
        for (int l = 0; l < lanes; ++l)
            if (scores[l] == best && ids[l] == bid) avail[l] = 0;
    }
    *count = cnt;
}

/* Reduction orders.  Triton leaves tl.sum / tl.cumsum order open; this
 * build fixes them to what a 64-lane wavefront does with DPP lane exchanges:
 *   tree_sum: butterfly, x[i] += x[i ^ m] for m = 1, 2, 4, .. BLOCK/2 (every
 *             lane ends with the same total because binary32 + commutes);
 *   row_scan: inclusive scan in 64-lane groups: inside each 16-lane row
 *             x[i] += x[i - d] for d = 1, 2, 4, 8 (i % 16 >= d); rows 1 and 3
 *             add lane 15 / lane 47; rows 2 and 3 add lane 31; then each
 *             64-lane group adds the last lane of the group before it. */
static float tree_sum(const float* in, int lanes) {
    float x[MAX_LANES], y[MAX_LANES];
    for (int l = 0; l < lanes; ++l) x[l] = in[l];
    for (int m = 1; m < lanes; m <<= 1) {
        for (int l = 0; l < lanes; ++l) y[l] = x[l] + x[l ^ m];
        for (int l = 0; l < lanes; ++l) x[l] = y[l];
    }
    return x[0];
}

static void ks_scan(const float* in, int lanes, float* out) {
    float x[MAX_LANES], y[MAX_LANES];
    for (int l = 0; l < lanes; ++l) x[l] = in[l];
    for (int g = 0; g < lanes; g += 64) {
        const int n = lanes - g < 64 ? lanes - g : 64;
        float* z = x + g;
        for (int d = 1; d <= 8; d <<= 1) {
            for (int l = 0; l < n; ++l) y[l] = (l % 16 >= d) ? z[l] + z[l - d] : z[l];
            for (int l = 0; l < n; ++l) z[l] = y[l];
        }
        for (int l = 0; l < n; ++l) {
            const int r = l / 16;
            y[l] = (r == 1) ? z[l] + z[15] : (r == 3) ? z[l] + z[47] : z[l];
        }
        for (int l = 0; l < n; ++l) z[l] = y[l];
        for (int l = 0; l < n; ++l) y[l] = (l / 16 >= 2) ? z[l] + z[31] : z[l];
        for (int l = 0; l < n; ++l) z[l] = y[l];
    }
    for (int g = 64; g < lanes; g += 64)
        for (int l = 0; l < 64 && g + l < lanes; ++l) x[g + l] = x[g + l] + x[g - 1];
    for (int l = 0; l < lanes; ++l) out[l] = x[l];
}

/* speculative.py:32-43 up to the retained mass; topk_topp.py:89-100 samples
 * from these retained (not renormalised) probabilities. */
static void retained_probabilities(const float* scores, float temperature, int64_t top_k,
                                   float top_p, int lanes, float* p, float* mass_out) {
    float logits[MAX_LANES] = {0}, w[MAX_LANES] = {0}, incl[MAX_LANES] = {0};
    const float safe_t = temperature == 0.0f ? 1.0f : temperature;
    float mx = -INFINITY; /* NaN-ignoring maximum, as Triton's tl.max */
    for (int l = 0; l < lanes; ++l) {
        logits[l] = l < top_k ? scores[l] / safe_t : -INFINITY;
        if (logits[l] > mx) mx = logits[l];
    }
    for (int l = 0; l < lanes; ++l) w[l] = l < top_k ? oracle_expf(logits[l] - mx) : 0.0f;
    const float sum = tree_sum(w, lanes);
    for (int l = 0; l < lanes; ++l) p[l] = w[l] / sum;
    ks_scan(p, lanes, incl);
    for (int l = 0; l < lanes; ++l) {
        const float excl = incl[l] - p[l];
        p[l] = (l < top_k && excl <= top_p) ? p[l] : 0.0f;
    }
    *mass_out = tree_sum(p, lanes);
}

static void probabilities(const float* scores, float temperature, int64_t top_k, float top_p,
                          int lanes, float* out, float* mass_out) {
    /* speculative.py:32-43 */
    float p[MAX_LANES] = {0};
    retained_probabilities(scores, temperature, top_k, top_p, lanes, p, mass_out);
    for (int l = 0; l < lanes; ++l) out[l] = p[l] / *mass_out;
}

static int next_pow2(int v) { int p = 1; while (p < v) p <<= 1; return p; }

EXPORT int oracle_verify_k1(const uint16_t* q_scores, const int64_t* q_ids,
                            const uint16_t* p_scores, const int64_t* p_ids,
                            const int32_t* target_rows, const int64_t* draft_tokens,
                            const float* temperatures, const float* top_ps,
                            const int64_t* top_ks, const int64_t* seeds,
                            const int64_t* ordinals, const float* uniforms,
                            const uint8_t* constrained_rows, int allow_underfilled,
                            int tp, int q_rows, int p_rows, int k, int active_rows,
                            int64_t* decisions) {
    const int lanes = next_pow2(tp * k);
    if (lanes > MAX_LANES) return -1;
    for (int row = 0; row < q_rows; ++row) {
        const int active = row < active_rows;
        const int32_t target_row = active ? target_rows[row] : 0;
        const int rows_ok = target_row >= 0 && target_row + 1 < p_rows;
        float qs[MAX_LANES], p0s[MAX_LANES], p1s[MAX_LANES];
        int64_t qi[MAX_LANES], p0i[MAX_LANES], p1i[MAX_LANES];
        int qr[MAX_LANES], p0r[MAX_LANES], p1r[MAX_LANES];
        int pairs_valid = 1;
        for (int l = 0; l < lanes; ++l) {
            const int cm = l < tp * k, rank = l / k, local = l % k;
            const int load = active && cm;
            const int load_p = load && rows_ok; /* out-of-range rows are never valid */
            qs[l] = load ? oracle_bf16_to_float(q_scores[((int64_t)rank * q_rows + row) * k + local]) : -INFINITY;
            qi[l] = load ? q_ids[((int64_t)rank * q_rows + row) * k + local] : -1;
            p0s[l] = load_p ? oracle_bf16_to_float(p_scores[((int64_t)rank * p_rows + target_row) * k + local]) : -INFINITY;
            p0i[l] = load_p ? p_ids[((int64_t)rank * p_rows + target_row) * k + local] : -1;
            p1s[l] = load_p ? oracle_bf16_to_float(p_scores[((int64_t)rank * p_rows + target_row + 1) * k + local]) : -INFINITY;
            p1i[l] = load_p ? p_ids[((int64_t)rank * p_rows + target_row + 1) * k + local] : -1;
            qr[l] = cm && qi[l] >= 0 && fabsf(qs[l]) < INFINITY;
            p0r[l] = cm && p0i[l] >= 0 && fabsf(p0s[l]) < INFINITY;
            p1r[l] = cm && p1i[l] >= 0 && fabsf(p1s[l]) < INFINITY;
            const int qpad = cm && qi[l] == -1 && qs[l] != qs[l];
            const int p0pad = cm && p0i[l] == -1 && p0s[l] != p0s[l];
            const int p1pad = cm && p1i[l] == -1 && p1s[l] != p1s[l];
            if (!(!cm || qr[l] || qpad)) pairs_valid = 0;
            if (!(!cm || p0r[l] || p0pad)) pairs_valid = 0;
            if (!(!cm || p1r[l] || p1pad)) pairs_valid = 0;
        }
        float sq[MAX_LANES], sp0[MAX_LANES], sp1[MAX_LANES];
        int64_t iq[MAX_LANES], ip0[MAX_LANES], ip1[MAX_LANES];
        int qc, p0c, p1c;
        select_topk(qs, qi, qr, lanes, k, sq, iq, &qc);
        select_topk(p0s, p0i, p0r, lanes, k, sp0, ip0, &p0c);
        select_topk(p1s, p1i, p1r, lanes, k, sp1, ip1, &p1c);
        const float temperature = active ? temperatures[row] : 1.0f;
        const float top_p = active ? top_ps[row] : 1.0f;
        const int64_t top_k = active ? top_ks[row] : 1;
        float qp[MAX_LANES], p0p[MAX_LANES], p1p[MAX_LANES], qm, p0m, p1m;
        probabilities(sq, temperature, top_k, top_p, lanes, qp, &qm);
        probabilities(sp0, temperature, top_k, top_p, lanes, p0p, &p0m);
        probabilities(sp1, temperature, top_k, top_p, lanes, p1p, &p1m);
        const int64_t draft = active ? draft_tokens[row] : -1;
        float tmp[MAX_LANES];
        for (int l = 0; l < lanes; ++l) tmp[l] = iq[l] == draft ? qp[l] : 0.0f;
        const float q_draft = tree_sum(tmp, lanes);
        for (int l = 0; l < lanes; ++l) tmp[l] = ip0[l] == draft ? p0p[l] : 0.0f;
        const float p_draft = tree_sum(tmp, lanes);
        const float quotient = p_draft / q_draft;
        const float ratio = quotient < 1.0f ? quotient : 1.0f; /* NaN -> 1 (minnum) */
        const int64_t seed = active ? seeds[row] : 0;
        const int64_t ordinal = active ? ordinals[row] : 0;
        const uint32_t key = (uint32_t)(seed ^ (seed >> 32) ^ 0x9E3779B9LL);
        const float u_accept = uniforms ? uniforms[row * 2]
                                        : oracle_philox_uniform(key, (uint32_t)(ordinal * 2));
        const int random_accepted = u_accept < ratio;
        const int greedy = temperature == 0.0f;
        const int64_t p0_top = ip0[0], p1_top = ip1[0];
        const int greedy_accepted = draft == p0_top;
        const int accepted = greedy ? greedy_accepted : random_accepted;
        float q_at_p[MAX_LANES];
        for (int l = 0; l < lanes; ++l) q_at_p[l] = 0.0f;
        for (int pos = 0; pos < k; ++pos)
            for (int l = 0; l < lanes; ++l)
                if (ip0[l] == iq[pos]) q_at_p[l] = qp[pos];
        float residual[MAX_LANES];
        for (int l = 0; l < lanes; ++l) {
            const float d = p0p[l] - q_at_p[l];
            residual[l] = d > 0.0f ? d : 0.0f; /* tl.maximum(x, 0) */
        }
        const float rmass = tree_sum(residual, lanes);
        const float u_sample = uniforms ? uniforms[row * 2 + 1]
                                        : oracle_philox_uniform(key ^ 0x85EBCA6Bu, (uint32_t)(ordinal * 2 + 1));
        int p1_slot = lanes, res_slot = lanes;
        float c1[MAX_LANES], cr[MAX_LANES];
        ks_scan(p1p, lanes, c1);
        ks_scan(residual, lanes, cr);
        const float scaled_u = u_sample * rmass;
        for (int l = 0; l < lanes; ++l) {
            if (p1_slot == lanes && c1[l] > u_sample) p1_slot = l;
            if (res_slot == lanes && cr[l] > scaled_u) res_slot = l;
        }
        const int64_t p1_token = p1_slot < lanes ? ip1[p1_slot] : INT64_MAXV;
        const int64_t res_token = res_slot < lanes ? ip0[res_slot] : INT64_MAXV;
        int underfilled = allow_underfilled;
        if (constrained_rows) underfilled = underfilled && active && constrained_rows[row];
        const int64_t need = (greedy || underfilled) ? 1 : top_k;
        const int valid = active && pairs_valid && rows_ok && temperature >= 0.0f &&
                          temperature < INFINITY && top_k >= 1 && top_k <= k && top_p > 0.0f &&
                          top_p <= 1.0f && seed >= 0 && ordinal >= 0 && qc >= need &&
                          p0c >= need && p1c >= need && qm > 0.0f && p0m > 0.0f && p1m > 0.0f &&
                          q_draft > 0.0f && (greedy || accepted || rmass > 0.0f);
        const int64_t greedy_next = greedy_accepted ? p1_top : p0_top;
        const int64_t next = greedy ? greedy_next : (accepted ? p1_token : res_token);
        decisions[row * 2] = valid ? (int64_t)accepted : -1;
        decisions[row * 2 + 1] = valid ? next : -1;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* F2  _root_topk_topp_kernel -- ops/cuda/sampling/topk_topp.py:22-121,      */
/* lane by lane over BLOCK = next_pow2(TP*K) lanes, with the reduction      */
/* orders and exp of A14.  `uniforms` (test hook, may be NULL) replaces the */
/* Philox draw per row, as the reference test oracle makes it explicit       */
/* (tests/ops/test_cuda_topk_topp_sampling.py:16-62).                       */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_root_sample(const uint16_t* scores, int scores_fp16, const int64_t* ids,
                              const float* temperatures, const float* top_ps,
                              const int64_t* top_ks, const int64_t* seeds,
                              const int64_t* ordinals, const float* uniforms,
                              const uint8_t* constrained_rows, int allow_underfilled, int tp,
                              int rows, int k, int64_t* out_tokens, uint8_t* out_valid) {
    const int lanes = next_pow2(tp * k);
    if (lanes > MAX_LANES) return -1;
    for (int row = 0; row < rows; ++row) {
        float sc[MAX_LANES];
        int64_t id[MAX_LANES];
        int real[MAX_LANES];
        int pairs_valid = 1;
        for (int l = 0; l < lanes; ++l) {
            const int cm = l < tp * k;
            const int64_t off = ((int64_t)(l / k) * rows + row) * k + l % k;
            const uint16_t b = cm ? scores[off] : 0;
            sc[l] = !cm ? -INFINITY : scores_fp16 ? oracle_half_to_float(b) : oracle_bf16_to_float(b);
            id[l] = cm ? ids[off] : -1;
            real[l] = cm && isfinite(sc[l]) && id[l] >= 0;
            const int sentinel = cm && sc[l] != sc[l] && id[l] == -1;
            if (cm && !real[l] && !sentinel) pairs_valid = 0;
        }
        float ss[MAX_LANES];
        int64_t si[MAX_LANES];
        int real_count;
        select_topk(sc, id, real, lanes, k, ss, si, &real_count);
        const float temperature = temperatures[row], top_p = top_ps[row];
        const int64_t top_k = top_ks[row], seed = seeds[row], ordinal = ordinals[row];
        const int greedy = temperature == 0.0f;
        const int params_ok = temperature == temperature && temperature >= 0.0f &&
                              temperature < INFINITY && top_p == top_p && top_p > 0.0f &&
                              top_p <= 1.0f && top_k >= 1 && top_k <= k && seed >= 0 && ordinal >= 0;
        int underfilled = allow_underfilled;
        if (constrained_rows) underfilled = underfilled && constrained_rows[row];
        const int enough = (greedy || underfilled) ? real_count >= 1 : real_count >= top_k;
        float retained[MAX_LANES] = {0}, cdf[MAX_LANES], mass;
        retained_probabilities(ss, temperature, top_k, top_p, lanes, retained, &mass);
        const int64_t random_seed = seed ^ (seed >> 32) ^ (ordinal >> 32);
        const float u = uniforms ? uniforms[row]
                                 : oracle_philox_uniform((uint64_t)random_seed, (uint32_t)ordinal);
        const float target = u * mass;
        ks_scan(retained, lanes, cdf);
        int sampled = lanes;
        for (int l = 0; l < lanes; ++l)
            if (cdf[l] > target) { sampled = l; break; }
        const int chosen = greedy ? 0 : sampled;
        const int64_t token = chosen < lanes ? si[chosen] : INT64_MAXV;
        const int valid = pairs_valid && params_ok && enough &&
                          (greedy || (mass > 0.0f && sampled < lanes));
        out_tokens[row] = valid ? token : -1;
        out_valid[row] = (uint8_t)valid;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* F4  MoE router -- ops/cuda/moe/fused.py:44-100 (_stable_topk_logits then */
/* _sort_and_normalize_topk; the fused _stable_topk_routes :103-156 gives   */
/* the same bits).  K rounds of (max logit, lowest expert among equals);    */
/* softmax over the selected logits with the build's exp and a butterfly    */
/* sum over next_pow2(K) lanes; ids re-ordered ascending.                   */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_moe_route(const uint16_t* logits, int logits_fp16, const int32_t* activity,
                            int active_rows, int rows, int experts, int top_k, float* top_logits,
                            int64_t* top_ids, int64_t* route_ids, uint16_t* route_weights,
                            int weights_fp16) {
    if (top_k < 1 || top_k > experts || top_k > MAX_LANES) return -1;
    float* v = (float*)malloc(sizeof(float) * (size_t)experts);
    int* taken = (int*)malloc(sizeof(int) * (size_t)experts);
    if (!v || !taken) { free(v); free(taken); return -2; }
    const int lanes = next_pow2(top_k);
    for (int r = 0; r < rows; ++r) {
        const int active = r < active_rows && activity[r] > 0;
        for (int e = 0; e < experts; ++e) {
            const uint16_t b = logits[(int64_t)r * experts + e];
            v[e] = logits_fp16 ? oracle_half_to_float(b) : oracle_bf16_to_float(b);
            taken[e] = 0;
        }
        float sc[MAX_LANES];
        int64_t id[MAX_LANES];
        for (int i = 0; i < top_k; ++i) {
            int best = -1;
            for (int e = 0; e < experts; ++e)
                if (!taken[e] && (best < 0 || v[e] > v[best])) best = e;  /* first = lowest id on ties */
            taken[best] = 1;
            sc[i] = v[best];
            id[i] = best;
            top_logits[(int64_t)r * top_k + i] = active ? v[best] : 0.0f;
            top_ids[(int64_t)r * top_k + i] = active ? best : -1;
        }
        float mx = -INFINITY, p[MAX_LANES];
        for (int i = 0; i < top_k; ++i) if (sc[i] > mx) mx = sc[i];
        for (int l = 0; l < lanes; ++l) p[l] = l < top_k ? oracle_expf(sc[l] - mx) : 0.0f;
        const float den = tree_sum(p, lanes);
        for (int i = 0; i < top_k; ++i) {
            int out = 0;
            for (int j = 0; j < top_k; ++j) out += id[j] < id[i];
            const float w = p[i] / den;
            route_ids[(int64_t)r * top_k + out] = active ? id[i] : -1;
            route_weights[(int64_t)r * top_k + out] =
                !active ? 0 : weights_fp16 ? oracle_float_to_half(w) : oracle_float_to_bf16(w);
        }
    }
    free(v);
    free(taken);
    return 0;
}

/* F4  route compaction -- ops/cuda/moe/fused.py:174-199 (_compact_local_routes). */
EXPORT int oracle_moe_compact(const int64_t* route_ids, int routes, int first_expert, int experts,
                              int block_m, int32_t* counts, int32_t* starts, int32_t* block_starts,
                              int32_t* total_blocks, int32_t* row_map) {
    int32_t c = 0, b = 0;
    for (int e = 0; e < experts; ++e) {
        int32_t n = 0;
        for (int r = 0; r < routes; ++r) n += route_ids[r] - first_expert == e;
        counts[e] = n;
        starts[e] = c;
        block_starts[e] = b;
        for (int r = 0; r < routes; ++r)
            if (route_ids[r] - first_expert == e) row_map[c++] = r;
        b += (n + block_m - 1) / block_m;
    }
    *total_blocks = b;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* A15  merge_prefix -- executor/draft_graph.py:146-157.                     */
/* decisions [depth, c, 2] -> out [c, 2]: accepted = first depth whose      */
/* accept flag is 0 (else depth); bonus = that depth's next token (else the */
/* last depth's); (-1,-1) unless the row is live and every depth is a       */
/* well-formed (0|1, token >= 0) decision.                                  */
/* ------------------------------------------------------------------------ */
EXPORT int oracle_merge_prefix(const int64_t* decisions, int c, int depth, int live_rows,
                               int64_t* out) {
    for (int r = 0; r < c; ++r) {
        int64_t accepted = depth, bonus = decisions[((int64_t)(depth - 1) * c + r) * 2 + 1];
        int good = 1;
        for (int d = depth - 1; d >= 0; --d) {
            const int64_t a = decisions[((int64_t)d * c + r) * 2];
            const int64_t tok = decisions[((int64_t)d * c + r) * 2 + 1];
            if (a == 0) { accepted = d; bonus = tok; }
            good = good && (a == 0 || a == 1) && tok >= 0;
        }
        const int live = r < live_rows;
        out[r * 2] = live && good ? accepted : -1;
        out[r * 2 + 1] = live && good ? bonus : -1;
    }
    return 0;
}
