/*
 * uocr_oracle.c - CPU oracle (test infrastructure only; see uocr_oracle.h).
 *
 * Plain C11 + OpenMP over output rows.  Every dot accumulates in fp32 and is
 * rounded to fp16 only where the reference decode rounds.
 */
#include "uocr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "../include/uocr_format.h"

static int g_threads = 0;

void orc_set_threads(int n) {
    g_threads = n;
#ifdef _OPENMP
    if (n > 0) {
        omp_set_num_threads(n);
    }
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* fp16 / bf16 conversion (uocr_cpu_ref.c:22-100)                           */
/* ------------------------------------------------------------------------ */

static inline uint32_t fbits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float bitsf(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0u) {
        /* zero or subnormal: m * 2^-24, exact in fp32 */
        const float mag = (float)m * 5.9604644775390625e-08f;
        return bitsf(fbits(mag) | sign);
    }
    if (e == 31u) {
        return bitsf(sign | 0x7f800000u | (m << 13));
    }
    return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t orc_f32_to_f16(float value) {
    const uint32_t x = fbits(value);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: subnormal half */
        /* scaling by 2^24 is exact; rintf rounds half to even */
        const float scaled = bitsf(ax) * 16777216.0f;
        return (uint16_t)(sign | (uint16_t)rintf(scaled));
    }
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t base = (((ax >> 23) - 112u) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (base & 1u))) {
        ++base; /* a carry into the exponent field is the correct encoding */
    }
    return (uint16_t)(sign | base);
}

float orc_bf16_to_f32(uint16_t bits) {
    return bitsf((uint32_t)bits << 16);
}

int orc_f16_to_f32_array(const uint16_t *in, size_t n, float *out) {
    if (n == 0u) return 1;
    if (in == NULL || out == NULL) return 0;
    for (size_t i = 0; i < n; ++i) out[i] = orc_f16_to_f32(in[i]);
    return 1;
}

int orc_f32_to_f16_array(const float *in, size_t n, uint16_t *out) {
    if (n == 0u) return 1;
    if (in == NULL || out == NULL) return 0;
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(in[i]);
    return 1;
}

/* ------------------------------------------------------------------------ */
/* fp32 reference ops (uocr_cpu_ref.c:145-579)                              */
/* ------------------------------------------------------------------------ */

static float dot_f32(const float *a, const float *b, uint32_t n) {
    float s = 0.0f;
    for (uint32_t i = 0; i < n; ++i) s = fmaf(a[i], b[i], s);
    return s;
}

static float silu(float g) {
    return g / (1.0f + expf(-g));
}

/* uocr_cpu_ref.c:145-169 */
int orc_rmsnorm_f32(const float *in, const float *w, uint32_t rows, uint32_t cols, float eps, float *out) {
    if (!in || !w || !out || rows == 0u || cols == 0u || eps < 0.0f) return 0;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = in + (size_t)r * cols;
        const float inv = 1.0f / sqrtf(dot_f32(x, x, cols) / (float)cols + eps);
        for (uint32_t c = 0; c < cols; ++c) out[(size_t)r * cols + c] = x[c] * inv * w[c];
    }
    return 1;
}

/* uocr_cpu_ref.c:171-209: pairs (d, d + head_dim/2), inv_freq = theta^(-2d/hd) */
int orc_rope_split_half_f32(const float *q, const float *k, uint32_t n_tokens, uint32_t heads,
                            uint32_t head_dim, uint32_t start_position, float theta,
                            float *q_out, float *k_out) {
    if (!q || !k || !q_out || !k_out || n_tokens == 0u || heads == 0u || head_dim == 0u ||
        (head_dim & 1u) || theta <= 0.0f) {
        return 0;
    }
    const uint32_t half = head_dim / 2u;
    for (uint32_t t = 0; t < n_tokens; ++t) {
        const float pos = (float)(start_position + t);
        for (uint32_t h = 0; h < heads; ++h) {
            const size_t base = ((size_t)t * heads + h) * head_dim;
            for (uint32_t d = 0; d < half; ++d) {
                const float ang = pos * powf(theta, -2.0f * (float)d / (float)head_dim);
                const float c = cosf(ang), s = sinf(ang);
                const float a0 = q[base + d], a1 = q[base + half + d];
                q_out[base + d] = a0 * c - a1 * s;
                q_out[base + half + d] = a1 * c + a0 * s;
                const float b0 = k[base + d], b1 = k[base + half + d];
                k_out[base + d] = b0 * c - b1 * s;
                k_out[base + half + d] = b1 * c + b0 * s;
            }
        }
    }
    return 1;
}

/* uocr_cpu_ref.c:227-273 */
int orc_causal_sdpa_f32(const float *q, const float *k, const float *v, uint32_t n_tokens,
                        uint32_t heads, uint32_t head_dim, float scale, float *out) {
    if (!q || !k || !v || !out || n_tokens == 0u || heads == 0u || head_dim == 0u) return 0;
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf((float)head_dim);
    float *p = (float *)malloc(sizeof(float) * n_tokens);
    if (!p) return 0;
    for (uint32_t t = 0; t < n_tokens; ++t) {
        for (uint32_t h = 0; h < heads; ++h) {
            const float *qv = q + ((size_t)t * heads + h) * head_dim;
            float mx = -INFINITY;
            for (uint32_t j = 0; j <= t; ++j) {
                p[j] = dot_f32(qv, k + ((size_t)j * heads + h) * head_dim, head_dim) * sc;
                if (p[j] > mx) mx = p[j];
            }
            float den = 0.0f;
            for (uint32_t j = 0; j <= t; ++j) {
                p[j] = expf(p[j] - mx);
                den += p[j];
            }
            if (!(den > 0.0f)) {
                free(p);
                return 0;
            }
            float *o = out + ((size_t)t * heads + h) * head_dim;
            for (uint32_t d = 0; d < head_dim; ++d) {
                float acc = 0.0f;
                for (uint32_t j = 0; j <= t; ++j) acc = fmaf(p[j] / den, v[((size_t)j * heads + h) * head_dim + d], acc);
                o[d] = acc;
            }
        }
    }
    free(p);
    return 1;
}

/* uocr_cpu_ref.c:305-349 */
int orc_dense_swiglu_f32(const float *in, const float *gate, const float *up, const float *down,
                         uint32_t rows, uint32_t hidden, uint32_t inter, float *ws, float *out) {
    if (!in || !gate || !up || !down || !ws || !out || rows == 0u || hidden == 0u || inter == 0u) return 0;
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = in + (size_t)r * hidden;
        float *m = ws + (size_t)r * inter;
        for (uint32_t i = 0; i < inter; ++i) {
            m[i] = silu(dot_f32(x, gate + (size_t)i * hidden, hidden)) * dot_f32(x, up + (size_t)i * hidden, hidden);
        }
        for (uint32_t c = 0; c < hidden; ++c) out[(size_t)r * hidden + c] = dot_f32(m, down + (size_t)c * inter, inter);
    }
    return 1;
}

/* Greedy top-k over probabilities, ties to the lower id
 * (uocr_cpu_ref.c:443-463, moe.metal:12-18). */
static int greedy_topk(const float *probs, uint32_t n, uint32_t k, uint32_t *ids, float *vals) {
    for (uint32_t s = 0; s < k; ++s) {
        uint32_t best = UINT32_MAX;
        float bp = -INFINITY;
        for (uint32_t e = 0; e < n; ++e) {
            int taken = 0;
            for (uint32_t j = 0; j < s; ++j) taken |= (ids[j] == e);
            if (taken) continue;
            if (probs[e] > bp || (probs[e] == bp && e < best)) {
                bp = probs[e];
                best = e;
            }
        }
        if (best == UINT32_MAX || !(bp >= 0.0f)) return 0;
        ids[s] = best;
        vals[s] = bp;
    }
    return 1;
}

/* uocr_cpu_ref.c:388-466 */
int orc_moe_router_f32(const float *in, const float *router, uint32_t rows, uint32_t hidden,
                       uint32_t n_experts, uint32_t top_k, float scaling,
                       float *logits, float *probs, uint32_t *top_ids, float *top_weights) {
    if (!in || !router || !logits || !probs || !top_ids || !top_weights || rows == 0u || hidden == 0u ||
        n_experts == 0u || top_k == 0u || top_k > n_experts || !(scaling >= 0.0f) || !isfinite(scaling)) {
        return 0;
    }
    for (uint32_t r = 0; r < rows; ++r) {
        float *lg = logits + (size_t)r * n_experts;
        float *pr = probs + (size_t)r * n_experts;
        float mx = -INFINITY;
        for (uint32_t e = 0; e < n_experts; ++e) {
            lg[e] = dot_f32(in + (size_t)r * hidden, router + (size_t)e * hidden, hidden);
            if (lg[e] > mx) mx = lg[e];
        }
        if (!isfinite(mx)) return 0;
        float den = 0.0f;
        for (uint32_t e = 0; e < n_experts; ++e) {
            pr[e] = expf(lg[e] - mx);
            den += pr[e];
        }
        if (!(den > 0.0f) || !isfinite(den)) return 0;
        for (uint32_t e = 0; e < n_experts; ++e) pr[e] /= den;
        uint32_t *ids = top_ids + (size_t)r * top_k;
        float *w = top_weights + (size_t)r * top_k;
        if (!greedy_topk(pr, n_experts, top_k, ids, w)) return 0;
        for (uint32_t s = 0; s < top_k; ++s) w[s] *= scaling;
    }
    return 1;
}

/* uocr_cpu_ref.c:468-579 */
int orc_moe_swiglu_f32(const float *in, const float *router,
                       const float *egate, const float *eup, const float *edown,
                       const float *sgate, const float *sup, const float *sdown,
                       uint32_t rows, uint32_t hidden, uint32_t n_experts, uint32_t top_k,
                       uint32_t expert_inter, uint32_t shared_inter, float scaling,
                       float *logits, float *probs, uint32_t *top_ids, float *top_weights,
                       float *expert_ws, float *shared_ws, float *out) {
    if (!egate || !eup || !edown || !sgate || !sup || !sdown || !expert_ws || !shared_ws || !out ||
        expert_inter == 0u || shared_inter == 0u) {
        return 0;
    }
    if (!orc_moe_router_f32(in, router, rows, hidden, n_experts, top_k, scaling, logits, probs, top_ids, top_weights)) {
        return 0;
    }
    for (uint32_t r = 0; r < rows; ++r) {
        const float *x = in + (size_t)r * hidden;
        float *o = out + (size_t)r * hidden;
        for (uint32_t c = 0; c < hidden; ++c) o[c] = 0.0f;
        for (uint32_t s = 0; s < top_k; ++s) {
            const uint32_t e = top_ids[(size_t)r * top_k + s];
            const float w = top_weights[(size_t)r * top_k + s];
            if (e >= n_experts) return 0;
            float *m = expert_ws + ((size_t)r * top_k + s) * expert_inter;
            for (uint32_t i = 0; i < expert_inter; ++i) {
                const size_t off = ((size_t)e * expert_inter + i) * hidden;
                m[i] = silu(dot_f32(x, egate + off, hidden)) * dot_f32(x, eup + off, hidden);
            }
            for (uint32_t c = 0; c < hidden; ++c) {
                const float d = dot_f32(m, edown + ((size_t)e * hidden + c) * expert_inter, expert_inter);
                o[c] = fmaf(w, d, o[c]);
            }
        }
        float *sm = shared_ws + (size_t)r * shared_inter;
        for (uint32_t i = 0; i < shared_inter; ++i) {
            sm[i] = silu(dot_f32(x, sgate + (size_t)i * hidden, hidden)) * dot_f32(x, sup + (size_t)i * hidden, hidden);
        }
        for (uint32_t c = 0; c < hidden; ++c) o[c] += dot_f32(sm, sdown + (size_t)c * shared_inter, shared_inter);
    }
    return 1;
}

/* uocr_cpu_ref.c:616-637 */
int orc_kv_cache_token_for_position(uint32_t prompt_length, uint32_t prompt_capacity, uint32_t ring,
                                    uint32_t position, uint32_t *out) {
    if (!out || prompt_length == 0u || prompt_length > prompt_capacity || ring == 0u) return 0;
    if (position < prompt_length) {
        *out = position;
        return 1;
    }
    *out = prompt_length + (position - prompt_length) % ring;
    return 1;
}

/* uocr_cpu_ref.c:694-729 */
int orc_decode_attention_plan(uint32_t prompt_length, uint32_t prompt_capacity, uint32_t ring,
                              uint32_t generated_count, orc_attention_plan *p) {
    if (!p || prompt_length == 0u || prompt_length > prompt_capacity || ring == 0u ||
        generated_count > UINT32_MAX - prompt_length) {
        return 0;
    }
    const uint32_t live = generated_count < ring ? generated_count : ring;
    p->prompt_length = prompt_length;
    p->generated_count = generated_count;
    p->live_generated = live;
    p->first_generated_index = generated_count - live;
    p->query_position = generated_count == 0u ? prompt_length : prompt_length + generated_count - 1u;
    p->attention_length = prompt_length + live;
    p->ring_window = ring;
    return 1;
}

/* uocr_cpu_ref.c:731-755 */
int orc_attention_index_to_token(const orc_attention_plan *p, uint32_t index, uint32_t *out) {
    if (!p || !out || p->prompt_length == 0u || p->ring_window == 0u || index >= p->attention_length) return 0;
    if (index < p->prompt_length) {
        *out = index;
        return 1;
    }
    const uint32_t g = index - p->prompt_length;
    if (g >= p->live_generated) return 0;
    *out = p->prompt_length + (p->first_generated_index + g) % p->ring_window;
    return 1;
}

/* ------------------------------------------------------------------------ */
/* quantised decode ops                                                     */
/* ------------------------------------------------------------------------ */

float orc_weight_at(uint32_t qtype, const void *W, const uint16_t *S, uint32_t K, uint32_t row, uint32_t col) {
    const uint32_t g = col / UOCR_QGROUP;
    if (qtype == UOCR_TENSOR_F16) {
        return orc_f16_to_f32(((const uint16_t *)W)[(size_t)row * K + col]);
    }
    const float sc = orc_f16_to_f32(S[(size_t)row * (K / UOCR_QGROUP) + g]);
    if (qtype == UOCR_TENSOR_Q8_0) {
        return (float)((const int8_t *)W)[(size_t)row * K + col] * sc;
    }
    /* Q4_0 group-half split: byte j of group g holds col g*64+j (low nibble)
     * and g*64+32+j (high nibble).  convert.py:2266-2274. */
    const uint32_t j = col % UOCR_QGROUP;
    const uint8_t b = ((const uint8_t *)W)[(size_t)row * (K / 2u) + g * 32u + (j & 31u)];
    const int nib = j < 32u ? (b & 0x0f) : (b >> 4);
    return (float)(nib - 8) * sc;
}

/* Row dot with the activation already widened to fp32 (same values and
 * summation order as orc_row_dot). */
static float row_dot_f(uint32_t qtype, const void *W, const uint16_t *S, uint32_t K, uint32_t row, const float *x) {
    float acc = 0.0f;
    if (qtype == UOCR_TENSOR_F16) {
        const uint16_t *w = (const uint16_t *)W + (size_t)row * K;
        for (uint32_t c = 0; c < K; ++c) acc = fmaf(orc_f16_to_f32(w[c]), x[c], acc);
        return acc;
    }
    const uint32_t groups = K / UOCR_QGROUP;
    const uint16_t *s = S + (size_t)row * groups;
    if (qtype == UOCR_TENSOR_Q8_0) {
        const int8_t *w = (const int8_t *)W + (size_t)row * K;
        for (uint32_t g = 0; g < groups; ++g) {
            float gs = 0.0f;
            for (uint32_t j = 0; j < UOCR_QGROUP; ++j) gs = fmaf((float)w[g * UOCR_QGROUP + j], x[g * UOCR_QGROUP + j], gs);
            acc = fmaf(gs, orc_f16_to_f32(s[g]), acc);
        }
        return acc;
    }
    const uint8_t *w = (const uint8_t *)W + (size_t)row * (K / 2u);
    for (uint32_t g = 0; g < groups; ++g) {
        const uint8_t *gb = w + g * 32u;
        const float *gx = x + g * UOCR_QGROUP;
        float gs = 0.0f;
        for (uint32_t j = 0; j < 32u; ++j) {
            gs = fmaf((float)((int)(gb[j] & 0x0f) - 8), gx[j], gs);
            gs = fmaf((float)((int)(gb[j] >> 4) - 8), gx[32u + j], gs);
        }
        acc = fmaf(gs, orc_f16_to_f32(s[g]), acc);
    }
    return acc;
}

static float *widen(const uint16_t *x, uint32_t n) {
    float *f = (float *)malloc(sizeof(float) * (n ? n : 1u));
    if (f) {
        for (uint32_t i = 0; i < n; ++i) f[i] = orc_f16_to_f32(x[i]);
    }
    return f;
}

float orc_row_dot(uint32_t qtype, const void *W, const uint16_t *S, uint32_t K, uint32_t row, const uint16_t *x) {
    float *xf = widen(x, K);
    if (!xf) return NAN;
    const float r = row_dot_f(qtype, W, S, K, row, xf);
    free(xf);
    return r;
}

static int qtype_ok(uint32_t q) {
    return q == UOCR_TENSOR_F16 || q == UOCR_TENSOR_Q8_0 || q == UOCR_TENSOR_Q4_0;
}

int orc_gemv(uint32_t qtype, const void *W, const uint16_t *S, uint32_t rows, uint32_t K,
             const uint16_t *x, const uint16_t *residual, uint16_t *y) {
    if (!qtype_ok(qtype) || !W || !x || !y || rows == 0u || K == 0u || (K % UOCR_QGROUP)) return 0;
    if (qtype != UOCR_TENSOR_F16 && !S) return 0;
    float *xf = widen(x, K);
    if (!xf) return 0;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        float v = row_dot_f(qtype, W, S, K, (uint32_t)r, xf);
        if (residual) v += orc_f16_to_f32(residual[r]);
        y[r] = orc_f32_to_f16(v);
    }
    free(xf);
    return 1;
}

int orc_swiglu_mid(uint32_t qtype, const void *G, const uint16_t *Gs, const void *U, const uint16_t *Us,
                   uint32_t rows, uint32_t K, const uint16_t *x, uint16_t *mid) {
    if (!qtype_ok(qtype) || !G || !U || !x || !mid || rows == 0u || (K % UOCR_QGROUP)) return 0;
    float *xf = widen(x, K);
    if (!xf) return 0;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        const float g = row_dot_f(qtype, G, Gs, K, (uint32_t)r, xf);
        const float u = row_dot_f(qtype, U, Us, K, (uint32_t)r, xf);
        mid[r] = orc_f32_to_f16(silu(g) * u);
    }
    free(xf);
    return 1;
}

int orc_rmsnorm_f16(const uint16_t *x, const uint16_t *w, uint32_t n, float eps, uint16_t *out) {
    if (!x || !w || !out || n == 0u) return 0;
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        const float v = orc_f16_to_f32(x[i]);
        ss = fmaf(v, v, ss);
    }
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint32_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16(orc_f16_to_f32(x[i]) * inv * orc_f16_to_f32(w[i]));
    return 1;
}

int orc_rope_f16(uint16_t *q, uint16_t *k, uint32_t heads, uint32_t head_dim, uint32_t position, float theta) {
    if (!q || !k || heads == 0u || head_dim == 0u || (head_dim & 1u) || !(theta > 0.0f)) return 0;
    const uint32_t half = head_dim / 2u;
    const float freq_scale = -2.0f * log2f(theta) / (float)head_dim;
    for (uint32_t d = 0; d < half; ++d) {
        const float ang = (float)position * exp2f((float)d * freq_scale);
        const float c = cosf(ang), s = sinf(ang);
        for (uint32_t h = 0; h < heads; ++h) {
            const size_t b = (size_t)h * head_dim;
            const float q0 = orc_f16_to_f32(q[b + d]), q1 = orc_f16_to_f32(q[b + half + d]);
            const float k0 = orc_f16_to_f32(k[b + d]), k1 = orc_f16_to_f32(k[b + half + d]);
            q[b + d] = orc_f32_to_f16(q0 * c - q1 * s);
            q[b + half + d] = orc_f32_to_f16(q0 * s + q1 * c);
            k[b + d] = orc_f32_to_f16(k0 * c - k1 * s);
            k[b + half + d] = orc_f32_to_f16(k0 * s + k1 * c);
        }
    }
    return 1;
}

typedef struct best2 {
    float s1, s2;
    int32_t id1;
} best2;

static void best2_push(best2 *b, float s, int32_t id) {
    if (b->id1 < 0 || s > b->s1 || (s == b->s1 && id < b->id1)) {
        if (b->id1 >= 0) b->s2 = b->s1 > b->s2 ? b->s1 : b->s2;
        b->s1 = s;
        b->id1 = id;
    } else if (s > b->s2) {
        b->s2 = s;
    }
}

int orc_lm_head_argmax(uint32_t qtype, const void *W, const uint16_t *S, uint32_t vocab, uint32_t K,
                       const uint16_t *x, int32_t *out_id, float *out_score, float *out_second) {
    if (!qtype_ok(qtype) || !W || !x || !out_id || vocab == 0u || (K % UOCR_QGROUP)) return 0;
    best2 all = {-INFINITY, -INFINITY, -1};
    float *xf = widen(x, K);
    if (!xf) return 0;
#pragma omp parallel
    {
        best2 mine = {-INFINITY, -INFINITY, -1};
#pragma omp for schedule(static)
        for (int64_t v = 0; v < (int64_t)vocab; ++v) {
            const float s = row_dot_f(qtype, W, S, K, (uint32_t)v, xf);
            if (!isnan(s)) best2_push(&mine, s, (int32_t)v);
        }
#pragma omp critical
        {
            if (mine.id1 >= 0) {
                best2_push(&all, mine.s1, mine.id1);
                best2_push(&all, mine.s2, INT32_MAX);
            }
        }
    }
    free(xf);
    *out_id = all.id1 < 0 ? 0 : all.id1;
    if (out_score) *out_score = all.id1 < 0 ? -INFINITY : all.s1;
    if (out_second) *out_second = all.s2;
    return 1;
}

int orc_router_topk(const uint16_t *x, const uint16_t *R, uint32_t n_experts, uint32_t K, uint32_t top_k,
                    int norm_topk, uint32_t *ids, float *weights, float *probs_out, float *margin_out) {
    if (!x || !R || !ids || !weights || n_experts == 0u || n_experts > 256u || top_k == 0u || top_k > n_experts) return 0;
    float logits[256], probs[256];
    float mx = -INFINITY;
    for (uint32_t e = 0; e < n_experts; ++e) {
        float s = 0.0f;
        for (uint32_t c = 0; c < K; ++c) s = fmaf(orc_f16_to_f32(x[c]), orc_f16_to_f32(R[(size_t)e * K + c]), s);
        logits[e] = s;
        if (s > mx) mx = s;
    }
    if (!isfinite(mx)) return 0;
    float den = 0.0f;
    for (uint32_t e = 0; e < n_experts; ++e) {
        probs[e] = expf(logits[e] - mx);
        den += probs[e];
    }
    for (uint32_t e = 0; e < n_experts; ++e) probs[e] /= den;
    if (!greedy_topk(probs, n_experts, top_k, ids, weights)) return 0;
    if (margin_out) {
        /* selection margin in logit space: the smallest gap between
         * consecutive ranks, including rank k against the best unselected */
        float next = -INFINITY;
        for (uint32_t e = 0; e < n_experts; ++e) {
            int taken = 0;
            for (uint32_t j = 0; j < top_k; ++j) taken |= (ids[j] == e);
            if (!taken && logits[e] > next) next = logits[e];
        }
        float m = n_experts > top_k ? logits[ids[top_k - 1]] - next : INFINITY;
        for (uint32_t j = 1; j < top_k; ++j) {
            const float d = logits[ids[j - 1]] - logits[ids[j]];
            if (d < m) m = d;
        }
        *margin_out = m;
    }
    if (norm_topk) {
        float s = 0.0f;
        for (uint32_t j = 0; j < top_k; ++j) s += weights[j];
        for (uint32_t j = 0; j < top_k; ++j) weights[j] /= s;
    }
    if (probs_out) memcpy(probs_out, probs, sizeof(float) * n_experts);
    return 1;
}

int orc_moe_ffn(const uint16_t *x, const uint16_t *residual, const uint16_t *router,
                uint32_t n_experts, uint32_t top_k, int norm_topk,
                const orc_expert_view *ev, uint32_t expert_inter,
                uint32_t shared_qtype, const void *sg, const uint16_t *sgs, const void *su, const uint16_t *sus,
                const void *sd, const uint16_t *sds, uint32_t shared_inter,
                uint16_t *out, uint32_t *ids_out, float *weights_out, float *margin_out) {
    const uint32_t H = UOCR_HIDDEN_SIZE;
    if (!x || !router || !ev || !out || top_k > 16u) return 0;
    uint32_t ids[16];
    float w[16];
    if (!orc_router_topk(x, router, n_experts, H, top_k, norm_topk, ids, w, NULL, margin_out)) return 0;
    uint16_t *smid = (uint16_t *)malloc(sizeof(uint16_t) * shared_inter);
    uint16_t *shared = (uint16_t *)malloc(sizeof(uint16_t) * H);
    uint16_t *mid = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)top_k * expert_inter);
    if (!smid || !shared || !mid) {
        free(smid); free(shared); free(mid);
        return 0;
    }
    int ok = orc_swiglu_mid(shared_qtype, sg, sgs, su, sus, shared_inter, H, x, smid) &&
             orc_gemv(shared_qtype, sd, sds, H, shared_inter, smid, NULL, shared);
    const uint32_t q = ev->qtype;
    for (uint32_t r = 0; ok && r < top_k; ++r) {
        const uint32_t e = ids[r];
        ok = orc_swiglu_mid(q, ev->gate_w + e * ev->w_stride, ev->gate_s ? ev->gate_s + e * ev->s_stride : NULL,
                            ev->up_w + e * ev->w_stride, ev->up_s ? ev->up_s + e * ev->s_stride : NULL,
                            expert_inter, H, x, mid + (size_t)r * expert_inter);
    }
    float *midf = ok ? widen(mid, top_k * expert_inter) : NULL;
    if (ok && !midf) ok = 0;
    if (ok) {
#pragma omp parallel for schedule(static)
        for (int64_t c = 0; c < (int64_t)H; ++c) {
            float acc = 0.0f;
            for (uint32_t r = 0; r < top_k; ++r) {
                const uint32_t e = ids[r];
                const float d = row_dot_f(q, ev->down_w + e * ev->w_stride,
                                          ev->down_s ? ev->down_s + e * ev->s_stride : NULL,
                                          expert_inter, (uint32_t)c, midf + (size_t)r * expert_inter);
                acc = fmaf(w[r], d, acc);
            }
            float v = acc + orc_f16_to_f32(shared[c]);
            if (residual) v += orc_f16_to_f32(residual[c]);
            out[c] = orc_f32_to_f16(v);
        }
    }
    if (ok && ids_out) memcpy(ids_out, ids, sizeof(uint32_t) * top_k);
    if (ok && weights_out) memcpy(weights_out, w, sizeof(float) * top_k);
    free(midf);
    free(smid);
    free(shared);
    free(mid);
    return ok;
}

int orc_attention_decode(const uint16_t *q, const uint16_t *kc, const uint16_t *vc,
                         uint32_t heads, uint32_t hd, const orc_attention_plan *plan, uint16_t *out) {
    if (!q || !kc || !vc || !plan || !out || plan->attention_length == 0u || hd > 512u) return 0;
    const uint32_t L = plan->attention_length;
    uint32_t *tok = (uint32_t *)malloc(sizeof(uint32_t) * L);
    if (!tok) return 0;
    for (uint32_t i = 0; i < L; ++i) {
        if (!orc_attention_index_to_token(plan, i, &tok[i])) {
            free(tok);
            return 0;
        }
    }
    const float scale = 1.0f / sqrtf((float)hd);
    int ok = 1;
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < (int64_t)heads; ++h) {
        float *p = (float *)malloc(sizeof(float) * L);
        float qf[512], acc[512];
        if (!p) {
            ok = 0;
            continue;
        }
        for (uint32_t d = 0; d < hd; ++d) {
            qf[d] = orc_f16_to_f32(q[(size_t)h * hd + d]);
            acc[d] = 0.0f;
        }
        float mx = -INFINITY;
        for (uint32_t i = 0; i < L; ++i) {
            const uint16_t *kr = kc + ((size_t)tok[i] * heads + (size_t)h) * hd;
            float s = 0.0f;
            for (uint32_t d = 0; d < hd; ++d) s = fmaf(qf[d], orc_f16_to_f32(kr[d]), s);
            p[i] = s * scale;
            if (p[i] > mx) mx = p[i];
        }
        float den = 0.0f;
        for (uint32_t i = 0; i < L; ++i) {
            p[i] = expf(p[i] - mx);
            den += p[i];
        }
        for (uint32_t i = 0; i < L; ++i) {
            const uint16_t *vr = vc + ((size_t)tok[i] * heads + (size_t)h) * hd;
            for (uint32_t d = 0; d < hd; ++d) acc[d] = fmaf(p[i], orc_f16_to_f32(vr[d]), acc[d]);
        }
        for (uint32_t d = 0; d < hd; ++d) out[(size_t)h * hd + d] = orc_f32_to_f16(acc[d] / den);
        free(p);
    }
    free(tok);
    return ok;
}

int orc_embed_row(uint32_t qtype, const void *W, const uint16_t *S, uint32_t rows, uint32_t K,
                  int32_t token, uint16_t *out) {
    if (!qtype_ok(qtype) || !W || !out) return 0;
    if (token < 0 || (uint32_t)token >= rows) {
        memset(out, 0, sizeof(uint16_t) * K); /* embedding_q4.metal:44-49 */
        return 1;
    }
    for (uint32_t c = 0; c < K; ++c) out[c] = orc_f32_to_f16(orc_weight_at(qtype, W, S, K, (uint32_t)token, c));
    return 1;
}

/* ------------------------------------------------------------------------ */
/* vision linear                                                            */
/* ------------------------------------------------------------------------ */

/* Abramowitz & Stegun 7.1.26, as sam.metal:78-87 evaluates it. */
static float erf_as(float x) {
    const float sign = x < 0.0f ? -1.0f : 1.0f;
    const float ax = fabsf(x);
    const float t = 1.0f / (1.0f + 0.3275911f * ax);
    const float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                            0.254829592f) * t * expf(-(ax * ax));
    return sign * y;
}

static float vision_act(uint32_t act, float v) {
    if (act == 1u) return v / (1.0f + expf(-1.702f * v));
    if (act == 2u) return 0.5f * v * (1.0f + erf_as(v * 0.70710678118654752440f));
    return v;
}

int orc_vision_linear(uint32_t qtype, const void *W, const uint16_t *S, const uint16_t *bias, uint32_t m,
                      uint32_t K, uint32_t N, uint32_t act, uint32_t split, const uint16_t *x, uint16_t *dst0,
                      uint16_t *dst1, uint16_t *dst2) {
    if (!qtype_ok(qtype) || !W || !bias || !x || !dst0 || m == 0u || N == 0u || K == 0u || (K % UOCR_QGROUP) ||
        act > 2u || (qtype != UOCR_TENSOR_F16 && !S) || (split && (N != 3u * split || !dst1 || !dst2))) {
        return 0;
    }
    /* the fp16 weight tile as the GEMM stages it */
    float *wf = (float *)malloc((size_t)N * K * sizeof(float));
    float *xf = widen(x, (uint32_t)((size_t)m * K));
    if (!wf || !xf) {
        free(wf);
        free(xf);
        return 0;
    }
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < (int64_t)N; ++n) {
        for (uint32_t c = 0; c < K; ++c) {
            wf[(size_t)n * K + c] = orc_f16_to_f32(orc_f32_to_f16(orc_weight_at(qtype, W, S, K, (uint32_t)n, c)));
        }
    }
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)m; ++r) {
        const float *xr = xf + (size_t)r * K;
        for (uint32_t n = 0; n < N; ++n) {
            const float *wr = wf + (size_t)n * K;
            float acc = 0.0f;
            for (uint32_t c = 0; c < K; ++c) acc = fmaf(xr[c], wr[c], acc);
            if (qtype == UOCR_TENSOR_F16) acc = orc_f16_to_f32(orc_f32_to_f16(acc));
            const uint16_t v = orc_f32_to_f16(vision_act(act, acc + orc_f16_to_f32(bias[n])));
            if (split == 0u) {
                dst0[(size_t)r * N + n] = v;
            } else {
                const uint32_t pj = n / split;
                uint16_t *d = pj == 0u ? dst0 : (pj == 1u ? dst1 : dst2);
                d[(size_t)r * split + (n - pj * split)] = v;
            }
        }
    }
    free(wf);
    free(xf);
    return 1;
}

/* ------------------------------------------------------------------------ */
/* model over a .uocr image                                                 */
/* ------------------------------------------------------------------------ */

typedef struct orc_tensor {
    uint32_t qtype;
    uint32_t rows, cols;
    const uint8_t *w;
    const uint16_t *s;
} orc_tensor;

typedef struct orc_layer {
    orc_tensor in_norm, post_norm, q, k, v, o;
    orc_tensor gate, up, down;          /* dense (layer 0) */
    orc_tensor router, sgate, sup, sdown;
    orc_tensor egate[UOCR_ROUTED_EXPERTS], eup[UOCR_ROUTED_EXPERTS], edown[UOCR_ROUTED_EXPERTS];
} orc_layer;

struct orc_model {
    orc_tensor embed, lm_head, final_norm;
    orc_layer layers[UOCR_DECODER_LAYERS];
};

static const uocr_tensor_entry *find_entry(const uocr_tensor_entry *e, uint32_t n, uint32_t id) {
    uint32_t lo = 0, hi = n;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) / 2u;
        if (e[mid].id == id) return &e[mid];
        if (e[mid].id < id) lo = mid + 1u; else hi = mid;
    }
    return NULL;
}

static int bind(const uint8_t *b, size_t size, const uocr_tensor_entry *e, uint32_t n, uint32_t id,
                uint32_t rows, uint32_t cols, orc_tensor *t) {
    const uocr_tensor_entry *te = find_entry(e, n, id);
    if (!te) return 0;
    const uint32_t r = te->rank == 1u ? 1u : te->logical_shape[0];
    const uint32_t c = te->rank == 1u ? te->logical_shape[0] : te->logical_shape[1];
    if (r != rows || c != cols) return 0;
    if (te->payload_offset + te->payload_size > size) return 0;
    t->qtype = te->qtype;
    t->rows = rows;
    t->cols = cols;
    t->w = b + te->payload_offset;
    t->s = te->scale_size ? (const uint16_t *)(const void *)(b + te->scale_offset) : NULL;
    return qtype_ok(te->qtype) && (te->qtype == UOCR_TENSOR_F16 || t->s != NULL);
}

orc_model *orc_model_open(const uint8_t *bytes, size_t size, char *err, size_t err_size) {
#define ORC_FAIL(msg)                                              \
    do {                                                           \
        if (err && err_size) {                                     \
            strncpy(err, (msg), err_size - 1u);                    \
            err[err_size - 1u] = '\0';                             \
        }                                                          \
        free(m);                                                   \
        return NULL;                                               \
    } while (0)
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    if (!m) ORC_FAIL("oom");
    if (!bytes || size < sizeof(uocr_file_header)) ORC_FAIL("short file");
    const uocr_file_header *h = (const uocr_file_header *)(const void *)bytes;
    if (memcmp(h->magic, UOCR_FILE_MAGIC, 4) != 0) ORC_FAIL("bad magic");
    const uocr_section_entry *sec = (const uocr_section_entry *)(const void *)(bytes + h->section_dir_offset);
    const uocr_tensor_entry *ents = NULL;
    uint32_t count = 0;
    for (uint32_t i = 0; i < h->section_count; ++i) {
        if (sec[i].type == UOCR_SECTION_TENSOR_DIRECTORY) {
            const uocr_tensor_directory_header *dh = (const uocr_tensor_directory_header *)(const void *)(bytes + sec[i].offset);
            ents = (const uocr_tensor_entry *)(const void *)(bytes + sec[i].offset + sizeof(*dh));
            count = dh->tensor_count;
        }
    }
    if (!ents) ORC_FAIL("no tensor directory");
    const uint32_t H = UOCR_HIDDEN_SIZE, V = UOCR_VOCAB_SIZE;
    if (!bind(bytes, size, ents, count, UOCR_TID_TOK_EMBED, V, H, &m->embed)) ORC_FAIL("token embedding");
    if (!bind(bytes, size, ents, count, UOCR_TID_LM_HEAD, V, H, &m->lm_head)) ORC_FAIL("lm head");
    if (!bind(bytes, size, ents, count, UOCR_TID_FINAL_NORM, 1, H, &m->final_norm)) ORC_FAIL("final norm");
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        orc_layer *L = &m->layers[l];
        int ok = bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_INPUT_NORM), 1, H, &L->in_norm) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_POST_ATTN_NORM), 1, H, &L->post_norm) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_ATTN_Q), H, H, &L->q) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_ATTN_K), H, H, &L->k) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_ATTN_V), H, H, &L->v) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_ATTN_O), H, H, &L->o);
        if (!ok) ORC_FAIL("attention tensors");
        if (l == 0u) {
            const uint32_t I = UOCR_DENSE_LAYER0_INTERMEDIATE;
            ok = bind(bytes, size, ents, count, uocr_tid_layer(0, UOCR_TID_L_DENSE_GATE), I, H, &L->gate) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(0, UOCR_TID_L_DENSE_UP), I, H, &L->up) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(0, UOCR_TID_L_DENSE_DOWN), H, I, &L->down);
            if (!ok) ORC_FAIL("dense mlp tensors");
        } else {
            const uint32_t SI = UOCR_MOE_SHARED_INTERMEDIATE, EI = UOCR_MOE_EXPERT_INTERMEDIATE;
            ok = bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_MOE_ROUTER), UOCR_ROUTED_EXPERTS, H, &L->router) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_SHARED_GATE), SI, H, &L->sgate) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_SHARED_UP), SI, H, &L->sup) &&
                 bind(bytes, size, ents, count, uocr_tid_layer(l, UOCR_TID_L_SHARED_DOWN), H, SI, &L->sdown);
            if (!ok || L->router.qtype != UOCR_TENSOR_F16) ORC_FAIL("moe router/shared tensors");
            for (uint32_t e = 0; e < UOCR_ROUTED_EXPERTS; ++e) {
                ok = bind(bytes, size, ents, count, uocr_tid_expert(l, e, 0), EI, H, &L->egate[e]) &&
                     bind(bytes, size, ents, count, uocr_tid_expert(l, e, 1), EI, H, &L->eup[e]) &&
                     bind(bytes, size, ents, count, uocr_tid_expert(l, e, 2), H, EI, &L->edown[e]);
                if (!ok) ORC_FAIL("expert tensors");
            }
        }
    }
    return m;
#undef ORC_FAIL
}

void orc_model_close(orc_model *m) {
    free(m);
}

struct orc_session {
    const orc_model *m;
    uint32_t prompt_capacity;
    uint32_t cache_tokens;
    uint32_t prompt_length;
    uint16_t *k[UOCR_DECODER_LAYERS];
    uint16_t *v[UOCR_DECODER_LAYERS];
};

orc_session *orc_session_create(const orc_model *m, uint32_t prompt_capacity) {
    if (!m || prompt_capacity == 0u) return NULL;
    orc_session *s = (orc_session *)calloc(1, sizeof(orc_session));
    if (!s) return NULL;
    s->m = m;
    s->prompt_capacity = prompt_capacity;
    s->cache_tokens = prompt_capacity + UOCR_GENERATED_RING_WINDOW;
    const size_t n = (size_t)s->cache_tokens * UOCR_HIDDEN_SIZE;
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        s->k[l] = (uint16_t *)calloc(n, sizeof(uint16_t));
        s->v[l] = (uint16_t *)calloc(n, sizeof(uint16_t));
        if (!s->k[l] || !s->v[l]) {
            orc_session_destroy(s);
            return NULL;
        }
    }
    return s;
}

void orc_session_destroy(orc_session *s) {
    if (!s) return;
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        free(s->k[l]);
        free(s->v[l]);
    }
    free(s);
}

int orc_session_reset(orc_session *s, uint32_t prompt_length) {
    if (!s || prompt_length == 0u || prompt_length > s->prompt_capacity) return 0;
    s->prompt_length = prompt_length;
    return 1;
}

static uint64_t splitmix(uint64_t *st) {
    uint64_t z = (*st += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

int orc_session_fill_kv(orc_session *s, uint32_t n, uint64_t seed) {
    if (!s || n > s->cache_tokens) return 0;
    uint64_t st = seed;
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        for (size_t i = 0; i < (size_t)n * UOCR_HIDDEN_SIZE; ++i) {
            const double u1 = ((double)(splitmix(&st) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
            const double u2 = (double)(splitmix(&st) >> 11) * (1.0 / 9007199254740992.0);
            const double r = sqrt(-2.0 * log(u1));
            s->k[l][i] = orc_f32_to_f16((float)(r * cos(6.283185307179586 * u2)));
            s->v[l][i] = orc_f32_to_f16((float)(r * sin(6.283185307179586 * u2)));
        }
    }
    return 1;
}

/* One decoder token, uocr_metal.m:14299-14518 op order, golden.py rounding. */
static int forward_token(orc_session *s, uint16_t *hidden, uint32_t position, uint32_t *trace_ids,
                         float *trace_margins, float *trace_weights) {
    const uint32_t H = UOCR_HIDDEN_SIZE, NH = UOCR_ATTENTION_HEADS, HD = UOCR_HEAD_DIM;
    if (!s || !hidden || s->prompt_length == 0u) return 0;
    const uint32_t P = s->prompt_length, R = UOCR_GENERATED_RING_WINDOW;
    orc_attention_plan plan;
    memset(&plan, 0, sizeof(plan));
    if (position < P) {
        /* prompt token: causal attention over positions 0..position */
        plan.prompt_length = position + 1u;
        plan.attention_length = position + 1u;
        plan.ring_window = R;
        plan.query_position = position;
    } else if (!orc_decode_attention_plan(P, s->prompt_capacity, R, position - P + 1u, &plan)) {
        return 0;
    }
    uint32_t cache_tok = 0;
    if (!orc_kv_cache_token_for_position(P, s->prompt_capacity, R, position, &cache_tok)) return 0;

    uint16_t n[UOCR_HIDDEN_SIZE], q[UOCR_HIDDEN_SIZE], k[UOCR_HIDDEN_SIZE], v[UOCR_HIDDEN_SIZE];
    uint16_t ctx[UOCR_HIDDEN_SIZE], a[UOCR_HIDDEN_SIZE], n2[UOCR_HIDDEN_SIZE];
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const orc_layer *L = &s->m->layers[l];
        int ok = orc_rmsnorm_f16(hidden, (const uint16_t *)L->in_norm.w, H, UOCR_RMS_NORM_EPS, n) &&
                 orc_gemv(L->q.qtype, L->q.w, L->q.s, H, H, n, NULL, q) &&
                 orc_gemv(L->k.qtype, L->k.w, L->k.s, H, H, n, NULL, k) &&
                 orc_gemv(L->v.qtype, L->v.w, L->v.s, H, H, n, NULL, v) &&
                 orc_rope_f16(q, k, NH, HD, position, (float)UOCR_ROPE_THETA);
        if (!ok) return 0;
        memcpy(s->k[l] + (size_t)cache_tok * H, k, sizeof(k));
        memcpy(s->v[l] + (size_t)cache_tok * H, v, sizeof(v));
        ok = orc_attention_decode(q, s->k[l], s->v[l], NH, HD, &plan, ctx) &&
             orc_gemv(L->o.qtype, L->o.w, L->o.s, H, H, ctx, hidden, a) &&
             orc_rmsnorm_f16(a, (const uint16_t *)L->post_norm.w, H, UOCR_RMS_NORM_EPS, n2);
        if (!ok) return 0;
        if (l == 0u) {
            const uint32_t I = UOCR_DENSE_LAYER0_INTERMEDIATE;
            uint16_t *mid = (uint16_t *)malloc(sizeof(uint16_t) * I);
            if (!mid) return 0;
            ok = orc_swiglu_mid(L->gate.qtype, L->gate.w, L->gate.s, L->up.w, L->up.s, I, H, n2, mid) &&
                 orc_gemv(L->down.qtype, L->down.w, L->down.s, H, I, mid, a, hidden);
            free(mid);
            if (!ok) return 0;
        } else {
            uint32_t ids[UOCR_MOE_TOP_K];
            float w[UOCR_MOE_TOP_K];
            float probs[UOCR_ROUTED_EXPERTS];
            if (!orc_router_topk(n2, (const uint16_t *)L->router.w, UOCR_ROUTED_EXPERTS, H, UOCR_MOE_TOP_K, 0, ids, w,
                                 probs, NULL)) {
                return 0;
            }
            if (trace_ids) memcpy(trace_ids + (size_t)(l - 1u) * UOCR_MOE_TOP_K, ids, sizeof(ids));
            if (trace_weights) memcpy(trace_weights + (size_t)(l - 1u) * UOCR_MOE_TOP_K, w, sizeof(w));
            if (trace_margins) {
                /* set margin in logit space: log p of the 6th choice over the
                 * best unselected expert (softmax keeps logit differences) */
                float next = 0.0f;
                for (uint32_t e = 0; e < UOCR_ROUTED_EXPERTS; ++e) {
                    int taken = 0;
                    for (uint32_t j = 0; j < UOCR_MOE_TOP_K; ++j) taken |= ids[j] == e;
                    if (!taken && probs[e] > next) next = probs[e];
                }
                trace_margins[l - 1u] = logf(probs[ids[UOCR_MOE_TOP_K - 1u]]) - logf(next);
            }
            const uint32_t SI = UOCR_MOE_SHARED_INTERMEDIATE, EI = UOCR_MOE_EXPERT_INTERMEDIATE;
            uint16_t smid[UOCR_MOE_SHARED_INTERMEDIATE], shared[UOCR_HIDDEN_SIZE];
            uint16_t mid[UOCR_MOE_TOP_K * UOCR_MOE_EXPERT_INTERMEDIATE];
            ok = orc_swiglu_mid(L->sgate.qtype, L->sgate.w, L->sgate.s, L->sup.w, L->sup.s, SI, H, n2, smid) &&
                 orc_gemv(L->sdown.qtype, L->sdown.w, L->sdown.s, H, SI, smid, NULL, shared);
            for (uint32_t r = 0; ok && r < UOCR_MOE_TOP_K; ++r) {
                const orc_tensor *G = &L->egate[ids[r]], *U = &L->eup[ids[r]];
                ok = orc_swiglu_mid(G->qtype, G->w, G->s, U->w, U->s, EI, H, n2, mid + (size_t)r * EI);
            }
            if (!ok) return 0;
            float *midf = widen(mid, UOCR_MOE_TOP_K * EI);
            if (!midf) return 0;
#pragma omp parallel for schedule(static)
            for (int64_t c = 0; c < (int64_t)H; ++c) {
                float acc = 0.0f;
                for (uint32_t r = 0; r < UOCR_MOE_TOP_K; ++r) {
                    const orc_tensor *D = &L->edown[ids[r]];
                    acc = fmaf(w[r], row_dot_f(D->qtype, D->w, D->s, EI, (uint32_t)c, midf + (size_t)r * EI), acc);
                }
                hidden[c] = orc_f32_to_f16(acc + orc_f16_to_f32(shared[c]) + orc_f16_to_f32(a[c]));
            }
            free(midf);
        }
    }
    return 1;
}

int orc_forward_token(orc_session *s, uint16_t *hidden, uint32_t position, uint32_t *trace_ids) {
    return forward_token(s, hidden, position, trace_ids, NULL, NULL);
}

int orc_forward_token_traced(orc_session *s, uint16_t *hidden, uint32_t position, uint32_t *trace_ids,
                             float *trace_margins, float *trace_weights) {
    return forward_token(s, hidden, position, trace_ids, trace_margins, trace_weights);
}

int orc_select(orc_session *s, const uint16_t *hidden, int32_t *id, float *score, float *second) {
    uint16_t n[UOCR_HIDDEN_SIZE];
    const orc_model *m = s->m;
    if (!orc_rmsnorm_f16(hidden, (const uint16_t *)m->final_norm.w, UOCR_HIDDEN_SIZE, UOCR_RMS_NORM_EPS, n)) return 0;
    return orc_lm_head_argmax(m->lm_head.qtype, m->lm_head.w, m->lm_head.s, UOCR_VOCAB_SIZE, UOCR_HIDDEN_SIZE, n, id,
                              score, second);
}

int orc_session_embed(orc_session *s, int32_t token, uint16_t *out) {
    if (!s || !out) return 0;
    const orc_model *m = s->m;
    return orc_embed_row(m->embed.qtype, m->embed.w, m->embed.s, UOCR_VOCAB_SIZE, UOCR_HIDDEN_SIZE, token, out);
}

int orc_generate(orc_session *s, const int32_t *ids, const uint8_t *image_mask, const uint16_t *image_rows,
                 uint32_t n_tokens, uint32_t max_new_tokens, int ignore_eos, int32_t *out_ids, float *out_margins) {
    const uint32_t H = UOCR_HIDDEN_SIZE;
    if (!s || !ids || n_tokens == 0u || !orc_session_reset(s, n_tokens)) return -1;
    const orc_model *m = s->m;
    uint16_t h[UOCR_HIDDEN_SIZE];
    uint32_t image_row = 0;
    for (uint32_t i = 0; i < n_tokens; ++i) {
        if (image_mask && image_mask[i]) {
            if (!image_rows) return -1;
            memcpy(h, image_rows + (size_t)image_row * H, sizeof(h));
            ++image_row;
        } else if (!orc_embed_row(m->embed.qtype, m->embed.w, m->embed.s, UOCR_VOCAB_SIZE, H, ids[i], h)) {
            return -1;
        }
        if (!orc_forward_token(s, h, i, NULL)) return -1;
    }
    uint32_t count = 0;
    for (uint32_t t = 0; t < max_new_tokens; ++t) {
        int32_t id = 0;
        float s1 = 0.0f, s2 = 0.0f;
        if (!orc_select(s, h, &id, &s1, &s2)) return -1;
        out_ids[t] = id;
        if (out_margins) out_margins[t] = s1 - s2;
        count = t + 1u;
        if (id == UOCR_TOKEN_EOS && !ignore_eos) break;
        if (t + 1u == max_new_tokens) break;
        if (!orc_embed_row(m->embed.qtype, m->embed.w, m->embed.s, UOCR_VOCAB_SIZE, H, id, h)) return -1;
        if (!orc_forward_token(s, h, n_tokens + t, NULL)) return -1;
    }
    return (int)count;
}
