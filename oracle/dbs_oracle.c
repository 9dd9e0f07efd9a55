/* SPDX-License-Identifier: MIT
 *
 * CPU oracle: a scalar C restatement of beamgrad's decode and surrogate
 * backward (test infrastructure only; see dbs_oracle.h). Built with
 * -ffp-contract=off and without fast-math so every float operation is a single
 * IEEE-rounded operation in program order, as the reference requires
 * (CMakeLists.txt:44-50).
 *
 * The structure is this file's own: per step it collects the candidates of
 * every beam into a small sorted buffer under the reference's total order and
 * keeps the best K; the backward walks the trace from the last step and
 * merges the produced entries by index.
 */
#include "dbs_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_INF (__builtin_inff())

/* ------------------------------------------------------------------------ */
/* Numerics                                                                  */
/* ------------------------------------------------------------------------ */

static float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* IEEE binary16 -> binary32, exact. Restates src/half.hpp:16-27. */
float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero / subnormal: m * 2^-24 is exact in binary32 */
        const float mag = (float)m * 5.9604644775390625e-8f;
        return sign ? -mag : mag;
    }
    if (e == 31) return bits_to_float(sign | 0x7f800000u | (m << 13));
    return bits_to_float(sign | ((e + 112u) << 23) | (m << 13));
}

/* bfloat16 -> binary32: the pattern in the high half. Restates src/half.hpp:29. */
float orc_bf16_to_f32(uint16_t h) { return bits_to_float((uint32_t)h << 16); }

static float load_elem(const void* base, int dtype, int64_t i) {
    if (dtype == ORC_F32) return ((const float*)base)[i];
    const uint16_t h = ((const uint16_t*)base)[i];
    return dtype == ORC_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}

/* ln(x) for x >= 1 in double from basic operations: x = m 2^e with
 * m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(s), s = (m-1)/(m+1), the series
 * 1 + s^2/3 + ... + s^22/23 by Horner, and ln 2 split in two parts.
 * Restates src/penalty.hpp:40-68 (same constants and operation order, which
 * the bit-exact penalty and logsumexp depend on). */
double orc_log_ge1(double x) {
    int e = 0;
    double m = frexp(x, &e);
    if (m < 0.70710678118654752440) {
        m = m * 2.0;
        e -= 1;
    }
    const double s = (m - 1.0) / (m + 1.0);
    const double z = s * s;
    static const double inv_odd[12] = {1.0 / 23.0, 1.0 / 21.0, 1.0 / 19.0, 1.0 / 17.0, 1.0 / 15.0, 1.0 / 13.0,
                                       1.0 / 11.0, 1.0 / 9.0,  1.0 / 7.0,  1.0 / 5.0,  1.0 / 3.0,  1.0};
    double poly = inv_odd[0];
    for (int i = 1; i < 12; ++i) poly = poly * z + inv_odd[i];
    const double log_m = (2.0 * s) * poly;
    const double hi = 6.93147180369123816490e-01;
    const double lo = 1.90821492927058770002e-10;
    const double de = (double)e;
    return de * hi + (de * lo + log_m);
}

/* exp(y) for y >= 0 in double: y = k ln2 + r, exp(r) by its Taylor series to
 * 1/15! (Horner), scaled by 2^k. Restates src/penalty.hpp:72-97. */
double orc_exp_ge0(double y) {
    if (y > 709.0) return HUGE_VAL;
    const double inv_ln2 = 1.44269504088896338700e+00;
    const double hi = 6.93147180369123816490e-01;
    const double lo = 1.90821492927058770002e-10;
    const int k = (int)(y * inv_ln2 + 0.5);
    const double dk = (double)k;
    const double r = (y - dk * hi) - dk * lo;
    /* 1/n! for n = 15 .. 2, then the two unit terms */
    static const double inv_fact[14] = {1.0 / 1307674368000.0, 1.0 / 87178291200.0, 1.0 / 6227020800.0,
                                        1.0 / 479001600.0,     1.0 / 39916800.0,    1.0 / 3628800.0,
                                        1.0 / 362880.0,        1.0 / 40320.0,       1.0 / 5040.0,
                                        1.0 / 720.0,           1.0 / 120.0,         1.0 / 24.0,
                                        1.0 / 6.0,             0.5};
    double p = inv_fact[0];
    for (int i = 1; i < 14; ++i) p = p * r + inv_fact[i];
    p = p * r + 1.0;
    p = p * r + 1.0;
    return ldexp(p, k);
}

/* GNMT penalty ((5 + max(len,1)) / 6)^alpha: 1 for alpha 0; exact repeated
 * squaring for integer alpha <= 64; else exp(alpha ln base) in double.
 * Restates src/penalty.hpp:101-122. */
float orc_length_penalty(int length, float alpha) {
    if (alpha == 0.0f) return 1.0f;
    const int l = length > 1 ? length : 1;
    const double base = (5.0 + (double)l) / 6.0;
    if (alpha <= 64.0f && alpha == (float)(int)alpha) {
        int n = (int)alpha;
        double acc = 1.0, sq = base;
        while (n > 0) {
            if (n & 1) acc = acc * sq;
            sq = sq * sq;
            n >>= 1;
        }
        return (float)acc;
    }
    return (float)orc_exp_ge0((double)alpha * orc_log_ge1(base));
}

void orc_length_penalty_array(const int32_t* lengths, int64_t count, float alpha, float* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = orc_length_penalty(lengths[i], alpha);
}

/* exp(x) for x <= 0 with the Cephes expf reduction and degree-5 polynomial
 * (S. L. Moshier, Cephes Math Library), evaluated without FMA; 0 below -87.
 * Restates src/logits.hpp:22-40 (constants) and :59-73 (operation order). */
float orc_exp_nonpositive(float x) {
    if (!(x >= -87.0f)) return 0.0f;
    const float k = floorf(x * 1.44269504088896341f + 0.5f);
    const float r = (x - k * 0.693359375f) - k * -2.12194440e-4f;
    const float r2 = r * r;
    static const float c[6] = {1.9875691500e-4f, 1.3981999507e-3f, 8.3334519073e-3f,
                               4.1665795894e-2f, 1.6666665459e-1f, 5.0000001201e-1f};
    float p = c[0];
    for (int i = 1; i < 6; ++i) p = p * r + c[i];
    p = (p * r2 + r) + 1.0f;
    const uint32_t scale = (uint32_t)((int)k + 127) << 23;
    return p * bits_to_float(scale);
}

/* Row statistics for decoding from logits. Max over x < +inf; each finite x
 * contributes exp_nonpositive(x - max) to accumulator (v mod 256), folded in
 * increasing v from +0; the 256 accumulators are combined pairwise with
 * strides 128, 64, ..., 1; lse = max + (float) ln(sum) in double.
 * Restates src/kernels_scalar.cpp:48-66, src/kernels.hpp:197-202,
 * src/logits.hpp:79-81. */
void orc_row_stats(const float* row, int vocab, float* max_out, float* lse_out, int* invalid_out) {
    float mx = -ORC_INF;
    int invalid = 0;
    for (int v = 0; v < vocab; ++v) {
        const float x = row[v];
        if (!(x < ORC_INF)) invalid = 1;
        else if (x > mx) mx = x;
    }
    *max_out = mx;
    *invalid_out = invalid;
    if (mx == -ORC_INF) {
        *lse_out = -ORC_INF;
        return;
    }
    float acc[256];
    for (int j = 0; j < 256; ++j) acc[j] = 0.0f;
    for (int v = 0; v < vocab; ++v) {
        const float x = row[v];
        if (x < ORC_INF && x != -ORC_INF) acc[v & 255] = acc[v & 255] + orc_exp_nonpositive(x - mx);
    }
    for (int half = 128; half >= 1; half >>= 1)
        for (int j = 0; j < half; ++j) acc[j] = acc[j] + acc[j + half];
    *lse_out = mx + (float)orc_log_ge1((double)acc[0]);
}

/* softmax(x) in a row with logsumexp lse; 0 for non-finite x.
 * Restates src/logits.hpp:84-87. */
float orc_softmax_probability(float x, float lse) {
    const int finite = x < ORC_INF && x > -ORC_INF;
    return finite ? orc_exp_nonpositive(x - lse) : 0.0f;
}

/* ------------------------------------------------------------------------ */
/* Candidates and their total order                                          */
/* ------------------------------------------------------------------------ */

typedef struct Cand {
    float score;
    float raw;
    int32_t parent;
    int32_t token;
    int32_t length;
    uint8_t from_logprob;
} Cand;

/* a ranks before b: score desc, raw desc, parent asc, token asc, length asc,
 * from_logprob desc (float ==, so -0 == +0). Restates src/common.hpp:269-276. */
static int cand_before(const Cand* a, const Cand* b) {
    if (a->score != b->score) return a->score > b->score;
    if (a->raw != b->raw) return a->raw > b->raw;
    if (a->parent != b->parent) return a->parent < b->parent;
    if (a->token != b->token) return a->token < b->token;
    if (a->length != b->length) return a->length < b->length;
    return a->from_logprob > b->from_logprob;
}

/* Keeps buf[0..k) sorted best-first; a candidate that does not rank before
 * buf[k-1] is dropped (the buffer starts full of the dead sentinel). The kept
 * set is order independent (src/common.hpp:278-302 is the reference's). */
static void keep_best(Cand* buf, int k, const Cand* c) {
    if (!cand_before(c, &buf[k - 1])) return;
    int pos = k - 1;
    while (pos > 0 && cand_before(c, &buf[pos - 1])) {
        buf[pos] = buf[pos - 1];
        --pos;
    }
    buf[pos] = *c;
}

/* ------------------------------------------------------------------------ */
/* Decode                                                                    */
/* ------------------------------------------------------------------------ */

typedef struct Example {
    const OrcDecodeArgs* a;
    const void* x;     /* this example's [T, K, V] */
    int steps;
    const uint8_t* banned_a;
    const uint8_t* banned_b;
    int32_t* eos_set; /* sorted distinct */
    int eos_count;
    float log_rep;
    int penalise;
    int constrained;
} Example;

static int in_eos_set(const Example* e, int32_t token) {
    for (int i = 0; i < e->eos_count; ++i)
        if (e->eos_set[i] == token) return 1;
    return 0;
}

static int cmp_i32(const void* p, const void* q) {
    const int32_t a = *(const int32_t*)p, b = *(const int32_t*)q;
    return (a > b) - (a < b);
}

/* n-gram blocking and repetition marks of one beam's prefix.
 * Restates src/decoder.cpp:196-235 (tokens outside [0, V) are ignored). */
static void mark_prefix(const Example* e, const int32_t* prefix, int L, uint8_t* blocked, uint8_t* penal,
                        int32_t* touched, int* n_touched) {
    const int V = e->a->vocab_size;
    const int n = e->a->no_repeat_ngram_size;
    *n_touched = 0;
#define ORC_TOUCH(tok, arr)                                                     \
    do {                                                                        \
        const int32_t t_ = (tok);                                               \
        if (t_ >= 0 && t_ < V) {                                                \
            if (!blocked[t_] && !penal[t_]) touched[(*n_touched)++] = t_;       \
            arr[t_] = 1;                                                        \
        }                                                                       \
    } while (0)
    if (n == 1) {
        for (int i = 0; i < L; ++i) ORC_TOUCH(prefix[i], blocked);
    } else if (n > 1 && L >= n - 1) {
        const int tail = L - (n - 1);
        for (int i = 0; i + n <= L; ++i) {
            int same = 1;
            for (int j = 0; j < n - 1 && same; ++j) same = prefix[i + j] == prefix[tail + j];
            if (same) ORC_TOUCH(prefix[i + n - 1], blocked);
        }
    }
    if (e->penalise) {
        for (int i = 0; i < L; ++i) ORC_TOUCH(prefix[i], penal);
    }
#undef ORC_TOUCH
}

static int decode_example(Example* e, int b, const OrcDecodeOutputs* o) {
    const OrcDecodeArgs* a = e->a;
    const int T = a->steps, K = a->beam_size, V = a->vocab_size;
    const size_t elem = a->dtype == ORC_F32 ? 4 : 2;
    const int64_t trace0 = (int64_t)b * T * K;
    const float alpha = a->length_penalty_alpha;

    float* raw = malloc(sizeof(float) * K);
    float* nraw = malloc(sizeof(float) * K);
    int32_t* len = malloc(sizeof(int32_t) * K);
    int32_t* nlen = malloc(sizeof(int32_t) * K);
    uint8_t* ended = malloc(K);
    uint8_t* nended = malloc(K);
    int32_t* last = malloc(sizeof(int32_t) * K);
    Cand* top = malloc(sizeof(Cand) * K);
    float* rowbuf = malloc(sizeof(float) * V);
    int32_t* prefix = NULL;
    int32_t* nprefix = NULL;
    int32_t* plen = NULL;
    int32_t* nplen = NULL;
    uint8_t* blocked = NULL;
    uint8_t* penal = NULL;
    int32_t* touched = NULL;
    if (e->constrained) {
        prefix = malloc(sizeof(int32_t) * (size_t)K * T);
        nprefix = malloc(sizeof(int32_t) * (size_t)K * T);
        plen = calloc(K, sizeof(int32_t));
        nplen = calloc(K, sizeof(int32_t));
        blocked = calloc(V, 1);
        penal = calloc(V, 1);
        touched = malloc(sizeof(int32_t) * (size_t)(2 * T + 2));
    }

    for (int k = 0; k < K; ++k) {
        raw[k] = k == 0 ? 0.0f : -ORC_INF;
        len[k] = 0;
        ended[k] = 0;
        last[k] = -1;
    }
    /* rows not read keep lse 0; padding steps hold dead slots (c_api.cpp:759-781) */
    for (int64_t i = 0; i < (int64_t)T * K; ++i) {
        o->row_lse[trace0 + i] = 0.0f;
        if (o->row_read) o->row_read[trace0 + i] = 0;
        o->parents[trace0 + i] = -1;
        o->tokens[trace0 + i] = -1;
        o->lengths[trace0 + i] = 0;
        o->scores[trace0 + i] = -ORC_INF;
        o->raw_scores[trace0 + i] = -ORC_INF;
        o->from_logprob[trace0 + i] = 0;
    }
    int invalid = 0;

    for (int t = 0; t < e->steps; ++t) {
        const Cand dead = {-ORC_INF, -ORC_INF, -1, -1, 0, 0};
        for (int k = 0; k < K; ++k) top[k] = dead;

        /* Expansion of every live beam (src/decoder.cpp:122-172). */
        for (int k = 0; k < K; ++k) {
            const float p = raw[k];
            if (!isfinite(p)) continue;
            if (a->eos_token >= 0 && ended[k]) {
                /* carried forward: unchanged raw, ranked by raw / penalty (division) */
                const int l = len[k] > 1 ? len[k] : 1;
                Cand c = {p / orc_length_penalty(l, alpha), p, k, in_eos_set(e, last[k]) ? last[k] : a->eos_token, l, 0};
                keep_best(top, K, &c);
                continue;
            }
            const int64_t row_index = ((int64_t)t * K + k);
            const char* src = (const char*)e->x + (size_t)row_index * V * elem;
            for (int v = 0; v < V; ++v) rowbuf[v] = load_elem(src, a->dtype, v);
            if (o->row_read) o->row_read[trace0 + row_index] = 1;
            float offset = 0.0f;
            if (a->from_logits) {
                float mx, lse;
                int bad;
                orc_row_stats(rowbuf, V, &mx, &lse, &bad);
                invalid |= bad;
                o->row_lse[trace0 + row_index] = lse;
                if (lse == -ORC_INF) continue;
                offset = lse;
            }
            const int new_len = len[k] + 1;
            const float inv_pen = 1.0f / orc_length_penalty(new_len, alpha);
            const int mask_eos = new_len < a->min_length;
            int n_touched = 0;
            if (e->constrained) mark_prefix(e, prefix + (size_t)k * T, plen[k], blocked, penal, touched, &n_touched);

            for (int v = 0; v < V; ++v) {
                const float lp = a->from_logits ? rowbuf[v] - offset : rowbuf[v];
                if (!(lp < ORC_INF)) {
                    invalid = 1;
                    continue;
                }
                if (lp == -ORC_INF) continue;
                if ((e->banned_a && e->banned_a[v]) || (e->banned_b && e->banned_b[v])) continue;
                if (mask_eos && in_eos_set(e, v)) continue;
                float value = lp;
                if (e->constrained) {
                    if (blocked[v]) continue;
                    if (penal[v]) value = lp - e->log_rep;
                }
                const float r = p + value;
                const float score = r * inv_pen;
                if (score < top[K - 1].score) continue; /* cannot rank before the last kept */
                Cand c = {score, r, k, v, new_len, 1};
                keep_best(top, K, &c);
            }
            if (e->constrained) {
                for (int i = 0; i < n_touched; ++i) {
                    blocked[touched[i]] = 0;
                    penal[touched[i]] = 0;
                }
            }
        }

        /* Selection (src/decoder.cpp:314-350). */
        for (int k = 0; k < K; ++k) {
            const Cand* c = &top[k];
            const int64_t idx = trace0 + (int64_t)t * K + k;
            o->parents[idx] = c->parent;
            o->tokens[idx] = c->token;
            o->lengths[idx] = c->length;
            o->scores[idx] = c->score;
            o->raw_scores[idx] = c->raw;
            o->from_logprob[idx] = c->from_logprob;
            nraw[k] = c->raw;
            nlen[k] = c->length;
            if (c->parent >= 0) {
                nended[k] = (uint8_t)(ended[c->parent] || in_eos_set(e, c->token));
                if (e->constrained) {
                    const int L = plen[c->parent];
                    memcpy(nprefix + (size_t)k * T, prefix + (size_t)c->parent * T, sizeof(int32_t) * (size_t)L);
                    nplen[k] = L;
                    if (c->from_logprob && c->token >= 0) nprefix[(size_t)k * T + nplen[k]++] = c->token;
                }
            } else {
                nended[k] = 0;
                if (e->constrained) nplen[k] = 0;
            }
        }
        for (int k = 0; k < K; ++k) last[k] = top[k].token;
        float* tf = raw; raw = nraw; nraw = tf;
        int32_t* ti = len; len = nlen; nlen = ti;
        uint8_t* tu = ended; ended = nended; nended = tu;
        if (e->constrained) {
            ti = prefix; prefix = nprefix; nprefix = ti;
            ti = plen; plen = nplen; nplen = ti;
        }
    }

    /* Final scores divide by the penalty (src/decoder.cpp:179-187). */
    for (int k = 0; k < K; ++k) {
        const int l = len[k] > 1 ? len[k] : 1;
        o->final_scores[(int64_t)b * K + k] = raw[k] / orc_length_penalty(l, alpha);
        o->final_raw_scores[(int64_t)b * K + k] = raw[k];
        o->final_lengths[(int64_t)b * K + k] = len[k];
    }
    o->invalid[b] = (uint8_t)invalid;

    free(raw); free(nraw); free(len); free(nlen); free(ended); free(nended); free(last); free(top); free(rowbuf);
    free(prefix); free(nprefix); free(plen); free(nplen); free(blocked); free(penal); free(touched);
    return 0;
}

int orc_decode(const void* inputs, const OrcDecodeArgs* a, const OrcDecodeOutputs* o) {
    if (!inputs || !a || !o) return -1;
    const int B = a->batch_size, T = a->steps, K = a->beam_size, V = a->vocab_size;
    if (B <= 0 || T <= 0 || K <= 0 || V <= 0) return -1;
    if (a->dtype < 0 || a->dtype > 2) return -1;
    if (a->eos_token < -1 || a->eos_token >= V) return -1;
    if (a->extra_eos_count > 0 && a->eos_token < 0) return -1;
    for (int i = 0; i < a->extra_eos_count; ++i)
        if (a->extra_eos[i] < 0 || a->extra_eos[i] >= V) return -1;
    if (a->min_length < 0 || !(a->length_penalty_alpha >= 0.0f) || !isfinite(a->length_penalty_alpha)) return -1;
    if (!(a->repetition_penalty > 0.0f) || !isfinite(a->repetition_penalty)) return -1;
    if (a->steps_per_example)
        for (int b = 0; b < B; ++b)
            if (a->steps_per_example[b] < 1 || a->steps_per_example[b] > T) return -1;

    int32_t* eos_set = malloc(sizeof(int32_t) * (size_t)(a->extra_eos_count + 1));
    int eos_count = 0;
    if (a->eos_token >= 0) {
        eos_set[eos_count++] = a->eos_token;
        for (int i = 0; i < a->extra_eos_count; ++i) eos_set[eos_count++] = a->extra_eos[i];
        qsort(eos_set, (size_t)eos_count, sizeof(int32_t), cmp_i32);
        int w = 0;
        for (int i = 0; i < eos_count; ++i)
            if (w == 0 || eos_set[w - 1] != eos_set[i]) eos_set[w++] = eos_set[i];
        eos_count = w;
    }
    const int penalise = a->repetition_penalty > 1.0f;
    const float log_rep = penalise ? logf(a->repetition_penalty) : 0.0f;
    const int constrained = penalise || a->no_repeat_ngram_size > 0;
    const size_t elem = a->dtype == ORC_F32 ? 4 : 2;
    int status = 0;

#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(a->num_threads > 0 ? a->num_threads : 1) reduction(| : status)
#endif
    for (int b = 0; b < B; ++b) {
        Example e;
        e.a = a;
        e.x = (const char*)inputs + (size_t)b * T * K * V * elem;
        e.steps = a->steps_per_example ? a->steps_per_example[b] : T;
        e.banned_a = a->banned;
        e.banned_b = a->banned_per_example ? a->banned_per_example + (size_t)b * V : NULL;
        e.eos_set = eos_set;
        e.eos_count = eos_count;
        e.log_rep = log_rep;
        e.penalise = penalise;
        e.constrained = constrained;
        status |= decode_example(&e, b, o);
    }
    free(eos_set);
    return status ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* Backward                                                                  */
/* ------------------------------------------------------------------------ */

typedef struct Entry {
    int64_t index; /* (t * K + parent) * V + token within the example */
    float value;
    int64_t order; /* production order, for a stable merge */
} Entry;

static int cmp_entry(const void* p, const void* q) {
    const Entry* a = p;
    const Entry* b = q;
    if (a->index != b->index) return a->index < b->index ? -1 : 1;
    return (a->order > b->order) - (a->order < b->order);
}

/* Walks one example's trace from its last step: per slot
 *   drank = 0 (+ g_scores) (+ g_final at the last step)
 *   draw  = next[k] + drank * (1 / penalty(max(1, len))) (+ g_raw) (+ g_final_raw at the last step)
 * then a non-zero draw flows to its parent (children summed in slot order) and,
 * for an expanded slot, to the entry (t, parent, token).
 * Restates src/decoder.cpp:565-624 (the selected-beam part) and 945-988 (range checks). */
static int walk_example(const OrcBackwardArgs* a, int b, Entry** entries_out, int64_t* count_out, float* draws) {
    const int T = a->steps, K = a->beam_size, V = a->vocab_size;
    const int steps = a->steps_per_example ? a->steps_per_example[b] : T;
    const int64_t base = (int64_t)b * T * K;
    for (int64_t i = 0; i < (int64_t)steps * K; ++i) {
        const int32_t p = a->parents[base + i], tok = a->tokens[base + i], l = a->lengths[base + i];
        if (p < -1 || p >= K || tok < -1 || tok >= V || l < 0) return -1;
    }
    float* next = calloc(K, sizeof(float));
    float* prev = calloc(K, sizeof(float));
    Entry* entries = malloc(sizeof(Entry) * (size_t)((int64_t)steps * K + 1));
    int64_t n = 0;
    for (int t = steps - 1; t >= 0; --t) {
        const int last_step = t == steps - 1;
        for (int k = 0; k < K; ++k) prev[k] = 0.0f;
        for (int k = 0; k < K; ++k) {
            const int64_t slot = base + (int64_t)t * K + k;
            const int parent = a->parents[slot];
            if (parent < 0) continue;
            float drank = 0.0f;
            if (a->grad_scores) drank = drank + a->grad_scores[slot];
            if (a->grad_final_scores && last_step) drank = drank + a->grad_final_scores[(int64_t)b * K + k];
            const int l = a->lengths[slot] > 1 ? a->lengths[slot] : 1;
            const float inv_pen = 1.0f / orc_length_penalty(l, a->length_penalty_alpha);
            float draw = next[k] + drank * inv_pen;
            if (a->grad_raw_scores) draw = draw + a->grad_raw_scores[slot];
            if (a->grad_final_raw_scores && last_step) draw = draw + a->grad_final_raw_scores[(int64_t)b * K + k];
            if (draw == 0.0f) continue;
            prev[parent] = prev[parent] + draw;
            if (a->from_logprob[slot] && a->tokens[slot] >= 0) {
                entries[n].index = ((int64_t)t * K + parent) * V + a->tokens[slot];
                entries[n].value = draw;
                entries[n].order = n;
                ++n;
                if (draws) draws[slot] = draw;
            }
        }
        float* tmp = next; next = prev; prev = tmp;
    }
    free(next);
    free(prev);
    /* merge: sort by index (stable), sum each index's values in order from 0 (decoder.cpp:668-683) */
    qsort(entries, (size_t)n, sizeof(Entry), cmp_entry);
    int64_t w = 0;
    for (int64_t i = 0; i < n;) {
        int64_t j = i;
        float sum = 0.0f;
        for (; j < n && entries[j].index == entries[i].index; ++j) sum = sum + entries[j].value;
        entries[w].index = entries[i].index;
        entries[w].value = sum;
        ++w;
        i = j;
    }
    *entries_out = entries;
    *count_out = w;
    return 0;
}

/* Adds the merged entries to grad; with logits, each row r holding entries
 * receives g_v - softmax(x_v) * S in full, S = the row's entries summed in
 * token order from 0. Restates src/decoder.hpp:212-242 and
 * src/kernels_scalar.cpp:68-70. */
static void apply_entries(const OrcBackwardArgs* a, int b, const Entry* entries, int64_t n, float* grad) {
    const int T = a->steps, K = a->beam_size, V = a->vocab_size;
    float* out = grad + (size_t)b * T * K * V;
    if (!a->logits) {
        for (int64_t i = 0; i < n; ++i) out[entries[i].index] = out[entries[i].index] + entries[i].value;
        return;
    }
    const size_t elem = a->logits_dtype == ORC_F32 ? 4 : 2;
    const char* rows = (const char*)a->logits + (size_t)b * T * K * V * elem;
    const float* lse_rows = a->row_lse + (size_t)b * T * K;
    float* x = malloc(sizeof(float) * V);
    float* g = malloc(sizeof(float) * V);
    for (int64_t i = 0; i < n;) {
        const int64_t r = entries[i].index / V;
        int64_t j = i;
        float s = 0.0f;
        for (; j < n && entries[j].index / V == r; ++j) s = s + entries[j].value;
        for (int v = 0; v < V; ++v) x[v] = load_elem(rows + (size_t)r * V * elem, a->logits_dtype, v);
        const float lse = lse_rows[r];
        for (int v = 0; v < V; ++v) g[v] = 0.0f - orc_softmax_probability(x[v], lse) * s;
        for (int64_t q = i; q < j; ++q) {
            const int v = (int)(entries[q].index - r * V);
            g[v] = entries[q].value - orc_softmax_probability(x[v], lse) * s;
        }
        for (int v = 0; v < V; ++v) out[r * V + v] = out[r * V + v] + g[v];
        i = j;
    }
    free(x);
    free(g);
}

static int check_backward_args(const OrcBackwardArgs* a) {
    if (!a || a->batch_size <= 0 || a->steps <= 0 || a->beam_size <= 0 || a->vocab_size <= 0) return -1;
    if (!a->parents || !a->tokens || !a->lengths || !a->from_logprob) return -1;
    if (a->logits && (!a->row_lse || a->logits_dtype < 0 || a->logits_dtype > 2)) return -1;
    if (a->steps_per_example)
        for (int b = 0; b < a->batch_size; ++b)
            if (a->steps_per_example[b] < 1 || a->steps_per_example[b] > a->steps) return -1;
    return 0;
}

int orc_backward(const OrcBackwardArgs* a, float* grad) {
    if (check_backward_args(a) || !grad) return -1;
    int status = 0;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(a->num_threads > 0 ? a->num_threads : 1) reduction(| : status)
#endif
    for (int b = 0; b < a->batch_size; ++b) {
        Entry* entries = NULL;
        int64_t n = 0;
        if (walk_example(a, b, &entries, &n, NULL)) {
            status |= 1;
        } else {
            apply_entries(a, b, entries, n, grad);
        }
        free(entries);
    }
    return status ? -1 : 0;
}

int orc_path_gradient(const OrcBackwardArgs* a, float* draws) {
    if (check_backward_args(a) || !draws || !a->grad_final_scores) return -1;
    OrcBackwardArgs f = *a;
    f.grad_final_raw_scores = NULL;
    f.grad_scores = NULL;
    f.grad_raw_scores = NULL;
    f.logits = NULL;
    int status = 0;
    for (int64_t i = 0; i < (int64_t)a->batch_size * a->steps * a->beam_size; ++i) draws[i] = 0.0f;
    for (int b = 0; b < a->batch_size; ++b) {
        Entry* entries = NULL;
        int64_t n = 0;
        status |= walk_example(&f, b, &entries, &n, draws);
        free(entries);
    }
    return status ? -1 : 0;
}

/* Follows parent pointers from the last step; steps past an example's length
 * keep the beam index, dead beams give -1. Restates python/beamgrad/_torch.py:582-606. */
void orc_backtrack(const int32_t* tokens, const int32_t* parents, const int32_t* steps_per_example, int B, int T,
                   int K, int64_t* seq) {
    for (int b = 0; b < B; ++b) {
        const int steps = steps_per_example ? steps_per_example[b] : T;
        for (int k = 0; k < K; ++k) {
            int beam = k;
            for (int t = T - 1; t >= 0; --t) {
                int64_t* dst = seq + ((int64_t)b * K + k) * T + t;
                if (t >= steps) {
                    *dst = -1;
                    continue;
                }
                if (beam < 0) {
                    *dst = -1;
                    continue;
                }
                const int64_t slot = ((int64_t)b * T + t) * K + beam;
                *dst = tokens[slot];
                beam = parents[slot];
            }
        }
    }
}
