/*
 * uocr_runtime.h - host runtime pieces behind the public ABI: result objects,
 * profile events, memory accounting, sequence/EOS state, error text.
 *
 * Behaviour follows the reference runtime: results own generated ids
 * (src/core/uocr_result.c), profile events keep calls/total/min/max ms with
 * at most 256 named events (src/runtime/uocr_profile.c:95-170), memory is
 * tracked per category with live/peak bytes (src/runtime/uocr_memory.c:50-108),
 * and generation stops on EOS (token 1, kept) or max_new_tokens
 * (src/runtime/uocr_sequence.c:120-166).
 */
#ifndef UOCR_RUNTIME_H
#define UOCR_RUNTIME_H

#include <stddef.h>
#include <stdint.h>

#include "unlimitedocr.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- results ------------------------------------------------------------ */
struct uocr_result {
    uint32_t count;
    uint32_t *lengths;
    int32_t **tokens;
};

int uocr_result_create(uint32_t count, const int32_t *const *lists, const uint32_t *lengths, uocr_result **out);

/* ---- profile ------------------------------------------------------------ */
typedef struct uocr_profile_state {
    uocr_profile_report report;
} uocr_profile_state;

uint64_t uocr_now_ns(void);
void uocr_profile_init(uocr_profile_state *p, int enabled);
int uocr_profile_env_enabled(void);
void uocr_profile_add_ms(uocr_profile_state *p, const char *name, double ms);
void uocr_profile_add_since(uocr_profile_state *p, const char *name, uint64_t start_ns);
void uocr_profile_reset(uocr_profile_state *p);
void uocr_profile_begin_request(uocr_profile_state *p);

/* ---- memory ------------------------------------------------------------- */
typedef struct uocr_memory_tracker {
    uint64_t live[UOCR_MEMORY_CATEGORY_COUNT];
    uint64_t peak[UOCR_MEMORY_CATEGORY_COUNT];
    uint64_t total_live;
    uint64_t total_peak;
} uocr_memory_tracker;

void uocr_memory_init(uocr_memory_tracker *m);
int uocr_memory_reserve(uocr_memory_tracker *m, uint32_t category, uint64_t bytes);
void uocr_memory_release(uocr_memory_tracker *m, uint32_t category, uint64_t bytes);
void uocr_memory_reset_peaks(uocr_memory_tracker *m);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_RUNTIME_H */
