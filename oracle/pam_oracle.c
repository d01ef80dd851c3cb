/*
 * pam_oracle.c - CPU restatement of PagedAttentionMetal's paged-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never linked into libpam.
 *
 * Algorithm sources (reference checkout paths):
 *   Reference/paged_attention_sim.py:12-138    online-softmax paged attention (fp64 here)
 *   Sources/PagedAttentionMetal/kernels.metal:553-601    FP8 e4m3 codec
 *   Sources/PagedAttentionMetal/kernels.metal:1417-1620  decode semantics (scale, GQA, window)
 *   Sources/PagedAttentionMetal/kernels.metal:693-917    prefill semantics (causal, window start)
 *   Sources/PagedAttentionMetal/kernels.metal:1804-1961  KV append, FP8 scale + quantize
 *
 * Pinning (tests/test_oracle.py): binary16 conversion is checked exhaustively against
 * numpy's float16; the FP8 decode table against torch.float8_e4m3fn; attention against
 * dense fp64 softmax(QK^T)V and the closed forms (L = 1, identical keys, block
 * permutation and block-size invariance).
 */
#include "pam_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ binary16 */

uint16_t pamo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                  /* below 2^-14: subnormal */
        int e = (int)(ax >> 23);
        if (e == 0) return (uint16_t)sign; /* float subnormal: far below 2^-25 */
        uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        int shift = 126 - e; /* value / 2^-24 = mant * 2^(e-126) */
        if (shift > 24) return (uint16_t)sign;
        uint32_t r = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t h = (e << 10) | ((ax >> 13) & 0x3ffu);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float pamo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* half multiply: the float product of two halves is exact, so one RNE rounding
 * to binary16 is the correctly rounded half product. */
static uint16_t hmul(uint16_t a, uint16_t b) {
    return pamo_f32_to_f16(pamo_f16_to_f32(a) * pamo_f16_to_f32(b));
}

/* ------------------------------------------------------------------ FP8 codec */

/* kernels.metal:564-601 (quantize_fp8): value / scale in float, clamp to +-448,
 * subnormal range below 2^-6 rounds v*512 (clamped to 7), otherwise frexp with a
 * 3-bit mantissa rounded half-away-from-zero (MSL round == C roundf), saturating
 * to 0x7E / 0xFE. */
uint8_t pamo_quantize_fp8(uint16_t value_h, uint16_t scale_h) {
    float v = pamo_f16_to_f32(value_h) / pamo_f16_to_f32(scale_h);
    v = fminf(fmaxf(v, -448.0f), 448.0f);
    uint32_t sign = v < 0.0f ? 1u : 0u;
    v = fabsf(v);
    if (v == 0.0f) return 0;
    if (v < 0x1p-6f) {
        int mant_int = (int)roundf(v * 512.0f);
        if (mant_int > 7) mant_int = 7;
        if (mant_int < 0) mant_int = 0;
        return (uint8_t)((sign << 7) | (uint32_t)mant_int);
    }
    int exp;
    float mant = frexpf(v, &exp);
    mant = 2.0f * mant;
    exp -= 1;
    if (exp > 8) return (uint8_t)((sign << 7) | (0xFu << 3) | 0x6u);
    int exp_bits = exp + 7;
    float mant_frac = mant - 1.0f;
    int mant_int = (int)roundf(mant_frac * 8.0f);
    if (mant_int > 7) {
        mant_int = 0;
        exp_bits++;
    }
    if (exp_bits > 0xF) return (uint8_t)((sign << 7) | (0xFu << 3) | 0x6u);
    if (exp_bits == 0xF && mant_int > 6) mant_int = 6;
    return (uint8_t)((sign << 7) | ((uint32_t)exp_bits << 3) | (uint32_t)mant_int);
}

/* kernels.metal:553-562 (dequant_fp8), evaluated in half left to right:
 *   exp == 0: (+-1 * scale) * (m/8) * 2^-6
 *   else    : (+-1 * scale) * (1 + m/8) * 2^(exp-7)
 * code 0x00 and 0x80 both give +0. */
uint16_t pamo_dequant_fp8(uint8_t v, uint16_t scale_h) {
    int sign = (v >> 7) & 1;
    int exp = (v >> 3) & 0xF;
    int mant = v & 0x7;
    if (exp == 0 && mant == 0) return 0;
    uint16_t s = (uint16_t)(sign ? (scale_h ^ 0x8000u) : scale_h);
    if (exp == 0) {
        uint16_t m8 = pamo_f32_to_f16((float)mant / 8.0f);
        return hmul(hmul(s, m8), 0x2400u /* 0.015625 */);
    }
    uint16_t mx = pamo_f32_to_f16(1.0f + (float)mant / 8.0f);
    uint16_t p2 = pamo_f32_to_f16(ldexpf(1.0f, exp - 7));
    return hmul(hmul(s, mx), p2);
}

void pamo_quantize_fp8_n(const uint16_t *values, const uint16_t *scales, uint8_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = pamo_quantize_fp8(values[i], scales[i]);
}

void pamo_dequant_fp8_n(const uint8_t *codes, const uint16_t *scales, uint16_t *out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = pamo_dequant_fp8(codes[i], scales[i]);
}

/* kernels.metal:1944-1957: max(new_max, float(old_scale) * 448) / 448 rounded to
 * half, or 1.0h when that max is zero. */
uint16_t pamo_fp8_scale(float new_max_abs, uint16_t old_scale_h) {
    float mk = fmaxf(new_max_abs, pamo_f16_to_f32(old_scale_h) * 448.0f);
    return mk > 0.0f ? pamo_f32_to_f16(mk / 448.0f) : (uint16_t)0x3C00u;
}

/* ------------------------------------------------------------------ append */

int64_t pamo_slot(const int32_t *bt, int64_t pos, int32_t bs) {
    return (int64_t)bt[pos / bs] * bs + pos % bs;
}

static size_t dtype_bytes(int dtype) { return dtype == 0 ? 4 : (dtype == 1 ? 2 : 1); }

int pamo_append(int dtype, const void *keys, const void *values, void *k_pool, void *v_pool,
                uint16_t *k_scale, uint16_t *v_scale, const int32_t *bt, int32_t n_bt,
                int32_t token_offset, int32_t n_new, int32_t hkv, int32_t d, int32_t bs) {
    const int64_t row = (int64_t)hkv * d; /* elements per token */
    for (int32_t t = 0; t < n_new; t++) {
        int64_t pos = (int64_t)token_offset + t;
        if (pos / bs >= n_bt) return -1;
    }
    if (dtype != 2) {
        size_t eb = dtype_bytes(dtype);
        for (int32_t t = 0; t < n_new; t++) {
            int64_t slot = pamo_slot(bt, (int64_t)token_offset + t, bs);
            memcpy((char *)k_pool + (size_t)(slot * row) * eb, (const char *)keys + (size_t)(t * row) * eb,
                   (size_t)row * eb);
            memcpy((char *)v_pool + (size_t)(slot * row) * eb, (const char *)values + (size_t)(t * row) * eb,
                   (size_t)row * eb);
        }
        return 0;
    }
    /* FP8: kernels.metal:1876-1905 gathers max|x| per physical block over this
     * append's elements (all heads); :1907-1961 derives each block's new scale and
     * quantizes with it.  Blocks not touched by this append keep their scale. */
    const uint16_t *kh = (const uint16_t *)keys;
    const uint16_t *vh = (const uint16_t *)values;
    uint8_t *kp = (uint8_t *)k_pool;
    uint8_t *vp = (uint8_t *)v_pool;
    int64_t first_lb = (int64_t)token_offset / bs;
    int64_t last_lb = ((int64_t)token_offset + n_new - 1) / bs;
    if (n_new <= 0) return 0;
    for (int64_t lb = first_lb; lb <= last_lb; lb++) {
        int64_t t0 = lb * bs - token_offset, t1 = t0 + bs;
        if (t0 < 0) t0 = 0;
        if (t1 > n_new) t1 = n_new;
        float mk = 0.0f, mv = 0.0f;
        for (int64_t t = t0; t < t1; t++)
            for (int64_t e = 0; e < row; e++) {
                mk = fmaxf(mk, fabsf(pamo_f16_to_f32(kh[t * row + e])));
                mv = fmaxf(mv, fabsf(pamo_f16_to_f32(vh[t * row + e])));
            }
        int32_t p = bt[lb];
        uint16_t ks = pamo_fp8_scale(mk, k_scale[p]);
        uint16_t vs = pamo_fp8_scale(mv, v_scale[p]);
        for (int64_t t = t0; t < t1; t++) {
            int64_t slot = pamo_slot(bt, (int64_t)token_offset + t, bs);
            for (int64_t e = 0; e < row; e++) {
                kp[slot * row + e] = pamo_quantize_fp8(kh[t * row + e], ks);
                vp[slot * row + e] = pamo_quantize_fp8(vh[t * row + e], vs);
            }
        }
        k_scale[p] = ks;
        v_scale[p] = vs;
    }
    return 0;
}

/* ------------------------------------------------------------------ attention */

/* Reference/paged_attention_sim.py:12-138, line for line in fp64 (prints dropped). */
void pamo_sim_forward(const float *q, const float *k_pool, const float *v_pool,
                      const int32_t *block_table, int32_t nlb, int32_t S, int32_t bs, int32_t d,
                      double *out, double *m_hist, double *l_hist) {
    double *m = (double *)malloc(sizeof(double) * (size_t)S);
    double *l = (double *)calloc((size_t)S, sizeof(double));
    double *O = (double *)calloc((size_t)S * d, sizeof(double));
    double *sc = (double *)malloc(sizeof(double) * (size_t)bs);
    for (int32_t i = 0; i < S; i++) m[i] = -INFINITY;
    for (int32_t lb = 0; lb < nlb; lb++) {
        int32_t p = block_table[lb];
        int32_t start = lb * bs, end = start + bs < S ? start + bs : S;
        int32_t n = end - start; /* sim :75-76 */
        for (int32_t i = 0; i < S; i++) {
            double mb = -INFINITY;
            for (int32_t j = 0; j < n; j++) {
                double s = 0.0;
                for (int32_t e = 0; e < d; e++)
                    s += (double)q[(size_t)i * d + e] * (double)k_pool[((size_t)p * bs + j) * d + e];
                sc[j] = s;
                if (s > mb) mb = s;
            }
            double mn = m[i] > mb ? m[i] : mb;
            double rescale = (m[i] == -INFINITY) ? 0.0 : exp(m[i] - mn);
            double lsum = 0.0;
            for (int32_t j = 0; j < n; j++) {
                sc[j] = exp(sc[j] - mn);
                lsum += sc[j];
            }
            for (int32_t e = 0; e < d; e++) {
                double acc = O[(size_t)i * d + e] * rescale;
                for (int32_t j = 0; j < n; j++) acc += sc[j] * (double)v_pool[((size_t)p * bs + j) * d + e];
                O[(size_t)i * d + e] = acc;
            }
            l[i] = l[i] * rescale + lsum;
            m[i] = mn;
            if (m_hist) m_hist[(size_t)lb * S + i] = m[i];
            if (l_hist) l_hist[(size_t)lb * S + i] = l[i];
        }
    }
    for (int32_t i = 0; i < S; i++)
        for (int32_t e = 0; e < d; e++) out[(size_t)i * d + e] = O[(size_t)i * d + e] / l[i];
    free(m);
    free(l);
    free(O);
    free(sc);
}

/* element loaders: pools in the cache's element type, q in the I/O type */
static inline double load_elem(int dtype, const void *pool, size_t idx, const uint16_t *scale,
                               int32_t p) {
    if (dtype == 0) return (double)((const float *)pool)[idx];
    if (dtype == 1) return (double)pamo_f16_to_f32(((const uint16_t *)pool)[idx]);
    return (double)pamo_f16_to_f32(pamo_dequant_fp8(((const uint8_t *)pool)[idx], scale[p]));
}

static inline double load_q(int dtype, const void *q, size_t idx) {
    if (dtype == 0) return (double)((const float *)q)[idx];
    return (double)pamo_f16_to_f32(((const uint16_t *)q)[idx]);
}

/* One query row against keys [k_lo, k_hi) of a paged sequence, processed per
 * logical block with the sim's online-softmax update (sim :70-136).  qs = q/sqrt(d). */
static void row_attention(int dtype, const double *qs, const void *k_pool, const void *v_pool,
                          const uint16_t *k_scale, const uint16_t *v_scale, const int32_t *bt,
                          int64_t k_lo, int64_t k_hi, int32_t hkv, int32_t kvh, int32_t d,
                          int32_t bs, double *out) {
    double m = -INFINITY, l = 0.0;
    double *O = (double *)calloc((size_t)d, sizeof(double));
    double *sc = (double *)malloc(sizeof(double) * (size_t)bs);
    const size_t row = (size_t)hkv * d;
    if (k_hi > k_lo) {
        for (int64_t lb = k_lo / bs; lb * bs < k_hi; lb++) {
            int32_t p = bt[lb];
            int64_t j0 = lb * bs > k_lo ? lb * bs : k_lo;
            int64_t j1 = lb * bs + bs < k_hi ? lb * bs + bs : k_hi;
            int32_t n = (int32_t)(j1 - j0);
            double mb = -INFINITY;
            for (int32_t t = 0; t < n; t++) {
                size_t base = ((size_t)p * bs + (size_t)(j0 + t - lb * bs)) * row + (size_t)kvh * d;
                double s = 0.0;
                for (int32_t e = 0; e < d; e++) s += qs[e] * load_elem(dtype, k_pool, base + e, k_scale, p);
                sc[t] = s;
                if (s > mb) mb = s;
            }
            double mn = m > mb ? m : mb;
            double rescale = (m == -INFINITY) ? 0.0 : exp(m - mn);
            double lsum = 0.0;
            for (int32_t t = 0; t < n; t++) {
                sc[t] = exp(sc[t] - mn);
                lsum += sc[t];
            }
            for (int32_t e = 0; e < d; e++) O[e] *= rescale;
            for (int32_t t = 0; t < n; t++) {
                size_t base = ((size_t)p * bs + (size_t)(j0 + t - lb * bs)) * row + (size_t)kvh * d;
                for (int32_t e = 0; e < d; e++) O[e] += sc[t] * load_elem(dtype, v_pool, base + e, v_scale, p);
            }
            l = l * rescale + lsum;
            m = mn;
        }
    }
    /* an empty key range leaves l = 0 and gives 0/0 = NaN, as the reference does */
    for (int32_t e = 0; e < d; e++) out[e] = O[e] / l;
    free(O);
    free(sc);
}

int pamo_decode(int dtype, const void *q, const void *k_pool, const void *v_pool,
                const uint16_t *k_scale, const uint16_t *v_scale, const int32_t *block_tables,
                const uint32_t *seq_lengths, int32_t B, int32_t max_nb, int32_t H, int32_t hkv,
                int32_t d, int32_t bs, int32_t window, double *out, int n_threads) {
    const int32_t g = H / hkv;
    const double scale = 1.0 / sqrt((double)d);
    const int64_t total = (int64_t)B * H;
#ifdef _OPENMP
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel for schedule(dynamic, 4) num_threads(n_threads)
#endif
    for (int64_t bh = 0; bh < total; bh++) {
        int32_t b = (int32_t)(bh / H), h = (int32_t)(bh % H);
        int64_t L = seq_lengths[b];
        /* kernels.metal:1442 token-granular window; :1448-1449 block-table clamp */
        int64_t ws = (window > 0 && L > window) ? L - window : 0;
        int64_t nlb = (L + bs - 1) / bs;
        if (nlb > max_nb) nlb = max_nb;
        int64_t k_hi = L < nlb * bs ? L : nlb * bs;
        double qs[1024];
        for (int32_t e = 0; e < d; e++) qs[e] = load_q(dtype, q, ((size_t)b * H + h) * d + e) * scale;
        row_attention(dtype, qs, k_pool, v_pool, k_scale, v_scale, block_tables + (size_t)b * max_nb, ws,
                      k_hi, hkv, h / g, d, bs, out + ((size_t)b * H + h) * d);
    }
    (void)n_threads;
    return 0;
}

int pamo_prefill(int dtype, const void *q, const void *k_pool, const void *v_pool,
                 const uint16_t *k_scale, const uint16_t *v_scale, const int32_t *bt, int32_t n_bt,
                 int32_t q_offset, int32_t T, int32_t H, int32_t hkv, int32_t d, int32_t bs,
                 int32_t window, int32_t causal, double *out, int n_threads) {
    const int32_t g = H / hkv;
    const double scale = 1.0 / sqrt((double)d);
    const int64_t kv_len = (int64_t)q_offset + T;
    if ((kv_len + bs - 1) / bs > n_bt) return -1;
    const int64_t ws = window > 0 ? (kv_len - window > 0 ? kv_len - window : 0) : 0;
    const int64_t total = (int64_t)T * H;
#ifdef _OPENMP
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel for schedule(dynamic, 4) num_threads(n_threads)
#endif
    for (int64_t th = 0; th < total; th++) {
        int32_t t = (int32_t)(th / H), h = (int32_t)(th % H);
        int64_t hi = causal ? (int64_t)q_offset + t + 1 : kv_len;
        double qs[1024];
        for (int32_t e = 0; e < d; e++) qs[e] = load_q(dtype, q, ((size_t)t * H + h) * d + e) * scale;
        row_attention(dtype, qs, k_pool, v_pool, k_scale, v_scale, bt, ws, hi, hkv, h / g, d, bs,
                      out + ((size_t)t * H + h) * d);
    }
    (void)n_threads;
    return 0;
}

void pamo_merge(int32_t P, const double *m, const double *l, const double *o, int32_t d, double *out) {
    double M = -INFINITY;
    for (int32_t p = 0; p < P; p++)
        if (m[p] > M) M = m[p];
    double den = 0.0;
    for (int32_t e = 0; e < d; e++) out[e] = 0.0;
    for (int32_t p = 0; p < P; p++) {
        double w = (m[p] == -INFINITY) ? 0.0 : exp(m[p] - M);
        den += w * l[p];
        for (int32_t e = 0; e < d; e++) out[e] += w * o[(size_t)p * d + e];
    }
    for (int32_t e = 0; e < d; e++) out[e] /= den;
}
