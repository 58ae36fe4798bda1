/* uocr_runtime.c - results, profile events and memory accounting. */
#include "uocr_runtime.h"

#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---- results (reference: src/core/uocr_result.c) ------------------------ */

int uocr_result_create(uint32_t count, const int32_t *const *lists, const uint32_t *lengths, uocr_result **out) {
    if (out == NULL) return UOCR_ERROR_INVALID_ARGUMENT;
    *out = NULL;
    uocr_result *r = (uocr_result *)calloc(1, sizeof(*r));
    if (r == NULL) return UOCR_ERROR_OUT_OF_MEMORY;
    r->count = count;
    if (count != 0u) {
        r->lengths = (uint32_t *)calloc(count, sizeof(uint32_t));
        r->tokens = (int32_t **)calloc(count, sizeof(int32_t *));
        if (r->lengths == NULL || r->tokens == NULL) {
            uocr_result_free(r);
            return UOCR_ERROR_OUT_OF_MEMORY;
        }
        for (uint32_t i = 0; i < count; ++i) {
            const uint32_t n = lengths != NULL ? lengths[i] : 0u;
            r->lengths[i] = n;
            if (n != 0u) {
                r->tokens[i] = (int32_t *)malloc(sizeof(int32_t) * n);
                if (r->tokens[i] == NULL) {
                    uocr_result_free(r);
                    return UOCR_ERROR_OUT_OF_MEMORY;
                }
                memcpy(r->tokens[i], lists[i], sizeof(int32_t) * n);
            }
        }
    }
    *out = r;
    return UOCR_OK;
}

uint32_t uocr_result_count(const uocr_result *result) {
    return result != NULL ? result->count : 0u;
}

const int32_t *uocr_result_tokens(const uocr_result *result, uint32_t index, uint32_t *n_tokens) {
    if (n_tokens != NULL) *n_tokens = 0u;
    if (result == NULL || index >= result->count) return NULL;
    if (n_tokens != NULL) *n_tokens = result->lengths[index];
    return result->tokens[index];
}

void uocr_result_free(uocr_result *result) {
    if (result == NULL) return;
    if (result->tokens != NULL) {
        for (uint32_t i = 0; i < result->count; ++i) free(result->tokens[i]);
    }
    free(result->tokens);
    free(result->lengths);
    free(result);
}

/* ---- profile ------------------------------------------------------------ */

uint64_t uocr_now_ns(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

void uocr_profile_init(uocr_profile_state *p, int enabled) {
    memset(p, 0, sizeof(*p));
    p->report.enabled = enabled ? 1u : 0u;
}

int uocr_profile_env_enabled(void) {
    const char *v = getenv("UOCR_PROFILE");
    return v != NULL && v[0] != '\0' && strcmp(v, "0") != 0;
}

void uocr_profile_add_ms(uocr_profile_state *p, const char *name, double ms) {
    if (p == NULL || !p->report.enabled || name == NULL) return;
    uocr_profile_report *r = &p->report;
    for (uint32_t i = 0; i < r->event_count; ++i) {
        uocr_profile_event *e = &r->events[i];
        if (strncmp(e->name, name, UOCR_PROFILE_EVENT_NAME_SIZE) == 0) {
            e->calls += 1u;
            e->total_ms += ms;
            if (ms < e->min_ms) e->min_ms = ms;
            if (ms > e->max_ms) e->max_ms = ms;
            return;
        }
    }
    if (r->event_count >= UOCR_PROFILE_MAX_EVENTS) {
        r->dropped_event_count += 1u;
        return;
    }
    uocr_profile_event *e = &r->events[r->event_count++];
    memset(e, 0, sizeof(*e));
    strncpy(e->name, name, UOCR_PROFILE_EVENT_NAME_SIZE - 1u);
    e->calls = 1u;
    e->total_ms = ms;
    e->min_ms = ms;
    e->max_ms = ms;
}

void uocr_profile_add_since(uocr_profile_state *p, const char *name, uint64_t start_ns) {
    if (p == NULL || !p->report.enabled) return;
    uocr_profile_add_ms(p, name, (double)(uocr_now_ns() - start_ns) / 1.0e6);
}

void uocr_profile_reset(uocr_profile_state *p) {
    const uint32_t enabled = p->report.enabled;
    const uint64_t gen = p->report.generation_index;
    memset(&p->report, 0, sizeof(p->report));
    p->report.enabled = enabled;
    p->report.generation_index = gen;
}

void uocr_profile_begin_request(uocr_profile_state *p) {
    p->report.generation_index += 1u;
}

/* ---- memory ------------------------------------------------------------- */

void uocr_memory_init(uocr_memory_tracker *m) {
    memset(m, 0, sizeof(*m));
}

int uocr_memory_reserve(uocr_memory_tracker *m, uint32_t category, uint64_t bytes) {
    if (m == NULL || category >= UOCR_MEMORY_CATEGORY_COUNT) return UOCR_ERROR_INVALID_ARGUMENT;
    if (UINT64_MAX - m->live[category] < bytes || UINT64_MAX - m->total_live < bytes) return UOCR_ERROR_OUT_OF_MEMORY;
    m->live[category] += bytes;
    m->total_live += bytes;
    if (m->live[category] > m->peak[category]) m->peak[category] = m->live[category];
    if (m->total_live > m->total_peak) m->total_peak = m->total_live;
    return UOCR_OK;
}

void uocr_memory_release(uocr_memory_tracker *m, uint32_t category, uint64_t bytes) {
    if (m == NULL || category >= UOCR_MEMORY_CATEGORY_COUNT) return;
    const uint64_t b = bytes > m->live[category] ? m->live[category] : bytes;
    m->live[category] -= b;
    m->total_live -= b > m->total_live ? m->total_live : b;
}

void uocr_memory_reset_peaks(uocr_memory_tracker *m) {
    for (uint32_t i = 0; i < UOCR_MEMORY_CATEGORY_COUNT; ++i) m->peak[i] = m->live[i];
    m->total_peak = m->total_live;
}
