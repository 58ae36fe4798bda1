/* uocr_convert.c - quantisers of the .uocr writer (see uocr_convert.h). */
#include "uocr_convert.h"

#include <math.h>
#include <string.h>

#include "uocr_format.h"
#include "uocr_half.h"

uint16_t uocr_half_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds past 65504 */
    if (ax < 0x38800000u) {                                    /* fp16 subnormal range */
        float a;
        memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint16_t)rintf(a * 16777216.0f));
    }
    const uint32_t m = ax & 0x7fffffu;
    uint32_t h = (((ax >> 23) - 112u) << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static float half_value(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0u) {
        const float v = (float)m * (1.0f / 16777216.0f);
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31u) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static float clampf(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* one row of cols values; returns 0 on a non-finite input */
static int quantize_row(uint32_t qtype, const float *x, uint32_t cols, uint8_t *w, uint16_t *sc) {
    for (uint32_t c = 0; c < cols; ++c) {
        if (!isfinite(x[c])) return 0;
    }
    if (qtype == UOCR_TENSOR_F16) {
        uint16_t *h = (uint16_t *)(void *)w;
        for (uint32_t c = 0; c < cols; ++c) h[c] = uocr_half_bits(x[c]);
        return 1;
    }
    for (uint32_t g = 0; g < cols / UOCR_QGROUP; ++g) {
        const float *v = x + g * UOCR_QGROUP;
        if (qtype == UOCR_TENSOR_Q8_0) {
            /* convert.py:2058-2063 */
            float mx = 0.0f;
            for (uint32_t k = 0; k < UOCR_QGROUP; ++k) mx = fmaxf(mx, fabsf(v[k]));
            const float s = mx == 0.0f ? 1.0f : mx / 127.0f;
            int8_t *q = (int8_t *)(void *)(w + g * UOCR_QGROUP);
            for (uint32_t k = 0; k < UOCR_QGROUP; ++k) q[k] = (int8_t)clampf(rintf(v[k] / s), -127.0f, 127.0f);
            sc[g] = uocr_half_bits(s);
        } else {
            /* convert.py:2249-2276: the first element of largest magnitude
             * sets the scale (it maps to -8); nibbles q + 8, byte j holding
             * columns j (low) and j + 32 (high) of the group */
            uint32_t idx = 0;
            float best = fabsf(v[0]);
            for (uint32_t k = 1; k < UOCR_QGROUP; ++k) {
                if (fabsf(v[k]) > best) {
                    best = fabsf(v[k]);
                    idx = k;
                }
            }
            const uint16_t hb = uocr_half_bits(v[idx] / -8.0f);
            const float h = half_value(hb);
            const float safe = h == 0.0f ? 1.0f : h;
            uint8_t nib[UOCR_QGROUP];
            for (uint32_t k = 0; k < UOCR_QGROUP; ++k) nib[k] = (uint8_t)((int)clampf(rintf(v[k] / safe), -8.0f, 7.0f) + 8);
            uint8_t *p = w + g * (UOCR_QGROUP / 2u);
            for (uint32_t j = 0; j < UOCR_QGROUP / 2u; ++j) p[j] = (uint8_t)(nib[j] | (nib[j + UOCR_QGROUP / 2u] << 4));
            sc[g] = hb;
        }
    }
    return 1;
}

int uocr_quantize_rows(uint32_t qtype, const float *src, uint32_t rows, uint32_t cols, void *payload,
                       uint16_t *scales) {
    if (src == NULL || payload == NULL || rows == 0u || cols == 0u) return UOCR_ERROR_INVALID_ARGUMENT;
    if (qtype != UOCR_TENSOR_F16 && qtype != UOCR_TENSOR_Q8_0 && qtype != UOCR_TENSOR_Q4_0) {
        return UOCR_ERROR_INVALID_ARGUMENT;
    }
    if (qtype != UOCR_TENSOR_F16 && (scales == NULL || cols % UOCR_QGROUP != 0u)) return UOCR_ERROR_INVALID_ARGUMENT;
    const size_t row_bytes = qtype == UOCR_TENSOR_F16 ? (size_t)cols * 2u : (qtype == UOCR_TENSOR_Q8_0 ? cols : cols / 2u);
    const uint32_t G = cols / UOCR_QGROUP;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(| : bad)
    for (int64_t r = 0; r < (int64_t)rows; ++r) {
        if (!quantize_row(qtype, src + (size_t)r * cols, cols, (uint8_t *)payload + (size_t)r * row_bytes,
                          qtype == UOCR_TENSOR_F16 ? NULL : scales + (size_t)r * G)) {
            bad = 1;
        }
    }
    return bad ? UOCR_ERROR_INVALID_ARGUMENT : UOCR_OK;
}
