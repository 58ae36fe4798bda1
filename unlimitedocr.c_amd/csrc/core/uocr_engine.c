/*
 * uocr_engine.c - public C ABI (include/unlimitedocr.h) of the MI355X build.
 *
 * Mirrors the reference engine core (src/core/uocr_api.c): backend
 * resolution (:794-849), engine limits and model open (:832-974), per-engine
 * and thread-local error text (:55-92), memory and profile reports
 * (:1003-1030), request validation and admission (:1032-1197) and generation
 * dispatch (:1199-1231).  The "hip" backend replaces "metal"; "cpu-ref"
 * validates requests but does not generate, exactly as in the reference
 * (tests/test_ffi.py:176).
 */
#define _GNU_SOURCE
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "unlimitedocr.h"
#include "uocr_hip.h"
#include "uocr_model.h"
#include "uocr_runtime.h"
#include "../hip/uocr_backend.h"

#define ERR_SIZE 1024u

struct uocr_engine {
    char *model_path;
    char *backend;
    uint32_t max_batch, max_prompt_tokens, max_gen_tokens;
    uint64_t memory_budget_bytes;
    uint64_t model_view_bytes;
    int has_model;
    uocr_model_file model;
    uocr_memory_tracker memory;
    uocr_profile_state profile;
    uocr_memory_report estimate;
    uocr_hip_ctx *hip;
    int decoder_ready;
    char bind_error[512];
    char last_error[ERR_SIZE];
};

static _Thread_local char g_last_error[ERR_SIZE] = "OK";

static int set_error(uocr_engine *e, int status, const char *fmt, ...) {
    char buf[ERR_SIZE];
    va_list ap;
    va_start(ap, fmt);
    (void)vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (e != NULL) snprintf(e->last_error, sizeof(e->last_error), "%s", buf);
    snprintf(g_last_error, sizeof(g_last_error), "%s", buf);
    return status;
}

static void clear_error(uocr_engine *e) {
    if (e != NULL) snprintf(e->last_error, sizeof(e->last_error), "OK");
    snprintf(g_last_error, sizeof(g_last_error), "OK");
}

static char *dup_or_null(const char *s) {
    return s != NULL ? strdup(s) : NULL;
}

uint32_t uocr_abi_version(void) {
    return UOCR_ABI_VERSION;
}

const char *uocr_status_string(int status) {
    switch (status) {
        case UOCR_OK: return "OK";
        case UOCR_ERROR_INVALID_ARGUMENT: return "invalid argument";
        case UOCR_ERROR_UNSUPPORTED: return "unsupported";
        case UOCR_ERROR_OUT_OF_MEMORY: return "out of memory";
        case UOCR_ERROR_NOT_IMPLEMENTED: return "not implemented";
        case UOCR_ERROR_INTERNAL: return "internal error";
        default: return "unknown status";
    }
}

const char *uocr_memory_category_name(uocr_memory_category c) {
    switch (c) {
        case UOCR_MEMORY_MODEL_VIEWS: return "model-views";
        case UOCR_MEMORY_KV_CACHE: return "kv-cache";
        case UOCR_MEMORY_PROMPT_EMBEDDINGS: return "prompt-embeddings";
        case UOCR_MEMORY_VISION_GPU_WORKSPACE: return "vision-gpu-workspace";
        case UOCR_MEMORY_VISION_FINAL_FEATURES: return "vision-final-features";
        case UOCR_MEMORY_VISION_HOST_STAGING: return "vision-host-staging";
        case UOCR_MEMORY_DECODER_SCRATCH: return "decoder-scratch";
        case UOCR_MEMORY_MOE_SCRATCH: return "moe-scratch";
        case UOCR_MEMORY_LOGITS_READBACK: return "logits-readback";
        case UOCR_MEMORY_TRANSIENT_BUFFERS: return "transient-buffers";
        default: return "unknown";
    }
}

/* ---- memory estimate (uocr_memory.c role, for admission) ------------------ */

static void estimate_memory(uint32_t batch, uint32_t prompt, uint64_t model_bytes, uocr_memory_report *r) {
    memset(r, 0, sizeof(*r));
    const uint64_t cache = (uint64_t)prompt + UOCR_GENERATED_RING_WINDOW;
    r->estimated_model_views_bytes = model_bytes;
    r->estimated_kv_cache_bytes = (uint64_t)batch * UOCR_DECODER_LAYERS * 2u * cache * UOCR_HIDDEN_SIZE * 2u;
    r->estimated_prompt_embeddings_bytes = (uint64_t)batch * prompt * UOCR_HIDDEN_SIZE * 2u;
    r->estimated_decoder_scratch_bytes = (uint64_t)batch * (8u * UOCR_HIDDEN_SIZE * 2u + 64u * 1024u);
    r->estimated_moe_scratch_bytes = (uint64_t)batch * (UOCR_DENSE_LAYER0_INTERMEDIATE + UOCR_MOE_SHARED_INTERMEDIATE) * 2u;
    r->estimated_logits_readback_bytes = (uint64_t)batch * 16u * 1024u;
    r->estimated_transient_bytes = (uint64_t)batch * UOCR_DEFAULT_MAX_GEN_TOKENS * 8u;
    r->estimated_safety_margin_bytes = 64u * 1024u * 1024u;
    r->estimated_total_bytes = r->estimated_model_views_bytes + r->estimated_kv_cache_bytes +
                               r->estimated_prompt_embeddings_bytes + r->estimated_decoder_scratch_bytes +
                               r->estimated_moe_scratch_bytes + r->estimated_logits_readback_bytes +
                               r->estimated_transient_bytes + r->estimated_safety_margin_bytes;
}

static const char *default_backend(void) {
    return uocr_hip_is_available(NULL, 0) ? "hip" : "cpu-ref";
}

static int backend_supported(const char *b, char *why, size_t n) {
    if (strcmp(b, "cpu-ref") == 0) return 1;
    if (strcmp(b, "hip") == 0) {
        if (uocr_hip_is_available(why, n)) return 1;
        return 0;
    }
    if (strcmp(b, "metal") == 0) {
        snprintf(why, n, "Metal backend was not compiled for this build");
        return 0;
    }
    snprintf(why, n, "unsupported backend '%s'", b);
    return 0;
}

static uocr_engine *open_common(const uocr_engine_opts *opts, const void *mem, size_t mem_size) {
    const char *backend = opts != NULL ? opts->backend : NULL;
    if (backend == NULL || backend[0] == '\0' || strcmp(backend, "auto") == 0) backend = default_backend();
    char why[256] = {0};
    if (!backend_supported(backend, why, sizeof(why))) {
        set_error(NULL, UOCR_ERROR_UNSUPPORTED, "%s", why);
        return NULL;
    }
    uocr_engine *e = (uocr_engine *)calloc(1, sizeof(*e));
    if (e == NULL) {
        set_error(NULL, UOCR_ERROR_OUT_OF_MEMORY, "failed to allocate engine");
        return NULL;
    }
    e->max_batch = (opts != NULL && opts->max_batch) ? opts->max_batch : UOCR_DEFAULT_MAX_BATCH;
    e->max_prompt_tokens = (opts != NULL && opts->max_prompt_tokens) ? opts->max_prompt_tokens : UOCR_DEFAULT_MAX_PROMPT_TOKENS;
    e->max_gen_tokens = (opts != NULL && opts->max_gen_tokens) ? opts->max_gen_tokens : UOCR_DEFAULT_MAX_GEN_TOKENS;
    e->memory_budget_bytes = opts != NULL ? opts->memory_budget_bytes : 0u;
    uocr_profile_init(&e->profile, (opts != NULL && opts->profile != 0u) || uocr_profile_env_enabled());
    uocr_memory_init(&e->memory);
    e->backend = dup_or_null(backend);
    if (e->backend == NULL) {
        set_error(e, UOCR_ERROR_OUT_OF_MEMORY, "failed to copy engine option strings");
        uocr_engine_close(e);
        return NULL;
    }
    if (e->max_prompt_tokens > UOCR_MAX_POSITIONS) {
        set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "max_prompt_tokens %u exceeds the position limit %u", e->max_prompt_tokens,
                  UOCR_MAX_POSITIONS);
        uocr_engine_close(e);
        return NULL;
    }
    const char *path = opts != NULL ? opts->model_path : NULL;
    char merr[512] = {0};
    int have = 0;
    if (mem != NULL) {
        if (uocr_model_open_memory(mem, mem_size, &e->model, merr, sizeof(merr)) != 0) {
            set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "failed to open in-memory model: %s", merr);
            uocr_engine_close(e);
            return NULL;
        }
        have = 1;
    } else if (path != NULL && path[0] != '\0') {
        if (uocr_model_open_path(path, &e->model, merr, sizeof(merr)) != 0) {
            set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "failed to open model file '%s': %s", path, merr);
            uocr_engine_close(e);
            return NULL;
        }
        e->model_path = dup_or_null(path);
        have = 1;
    }
    if (have) {
        e->has_model = 1;
        e->model_view_bytes = e->model.tensor_data_bytes;
        if (e->memory_budget_bytes != 0u && e->model_view_bytes > e->memory_budget_bytes) {
            estimate_memory(e->max_batch, e->max_prompt_tokens, e->model_view_bytes, &e->estimate);
            set_error(e, UOCR_ERROR_OUT_OF_MEMORY,
                      "engine admission rejected: model tensor-data view estimate %llu bytes exceeds budget %llu bytes",
                      (unsigned long long)e->model_view_bytes, (unsigned long long)e->memory_budget_bytes);
            uocr_engine_close(e);
            return NULL;
        }
        uocr_memory_reserve(&e->memory, UOCR_MEMORY_MODEL_VIEWS, e->model_view_bytes);
    }
    estimate_memory(e->max_batch, e->max_prompt_tokens, e->model_view_bytes, &e->estimate);
    if (strcmp(e->backend, "hip") == 0) {
        char herr[512] = {0};
        e->hip = uocr_hip_context_create(herr, sizeof(herr));
        if (e->hip == NULL) {
            set_error(e, UOCR_ERROR_INTERNAL, "failed to initialize HIP backend: %s", herr);
            uocr_engine_close(e);
            return NULL;
        }
        uocr_hip_context_set_profile(e->hip, &e->profile);
        uocr_hip_context_set_memory_tracker(e->hip, &e->memory);
        if (e->has_model) {
            uocr_decoder_bindings *b = (uocr_decoder_bindings *)malloc(sizeof(*b));
            if (b == NULL) {
                set_error(e, UOCR_ERROR_OUT_OF_MEMORY, "failed to allocate decoder bindings");
                uocr_engine_close(e);
                return NULL;
            }
            if (uocr_bind_decoder(&e->model, b, e->bind_error, sizeof(e->bind_error)) == 0) {
                const uint64_t start = uocr_now_ns();
                if (!uocr_hip_context_map_model(e->hip, b, herr, sizeof(herr)) ||
                    !uocr_hip_context_allocate_runtime(e->hip, e->max_prompt_tokens, e->max_gen_tokens, herr, sizeof(herr))) {
                    free(b);
                    set_error(e, UOCR_ERROR_INTERNAL, "failed to map model into HBM: %s", herr);
                    uocr_engine_close(e);
                    return NULL;
                }
                uocr_profile_add_since(&e->profile, "hip.map_model", start);
                e->decoder_ready = 1;
            }
            free(b);
        }
    }
    clear_error(e);
    return e;
}

uocr_engine *uocr_engine_open(const uocr_engine_opts *opts) {
    return open_common(opts, NULL, 0u);
}

uocr_engine *uocr_engine_open_memory(const uocr_engine_opts *opts, const void *data, size_t size) {
    if (data == NULL || size == 0u) {
        set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "model image is empty");
        return NULL;
    }
    return open_common(opts, data, size);
}

void uocr_engine_close(uocr_engine *e) {
    if (e == NULL) return;
    if (e->hip != NULL) uocr_hip_context_destroy(e->hip);
    if (e->has_model) uocr_model_close(&e->model);
    free(e->model_path);
    free(e->backend);
    free(e);
}

const char *uocr_last_error(const uocr_engine *e) {
    if (e != NULL) return e->last_error[0] != '\0' ? e->last_error : "OK";
    return g_last_error[0] != '\0' ? g_last_error : "OK";
}

const char *uocr_engine_backend(const uocr_engine *e) {
    if (e == NULL) {
        set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine is null");
        return NULL;
    }
    return e->backend;
}

static void fill_memory(const uocr_engine *e, uocr_memory_report *r) {
    *r = e->estimate;
    for (uint32_t i = 0; i < UOCR_MEMORY_CATEGORY_COUNT; ++i) {
        r->category_live_bytes[i] = e->memory.live[i];
        r->category_peak_bytes[i] = e->memory.peak[i];
    }
    r->total_live_bytes = e->memory.total_live;
    r->total_peak_bytes = e->memory.total_peak;
    r->memory_budget_bytes = e->memory_budget_bytes;
}

int uocr_engine_memory_report(const uocr_engine *e, uocr_memory_report *out) {
    if (e == NULL || out == NULL) return set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine and out_report must be non-null");
    fill_memory(e, out);
    return UOCR_OK;
}

int uocr_engine_profile_report(const uocr_engine *e, uocr_profile_report *out) {
    if (e == NULL || out == NULL) return set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine and out_report must be non-null");
    *out = e->profile.report;
    fill_memory(e, &out->memory);
    return UOCR_OK;
}

int uocr_engine_profile_reset(uocr_engine *e) {
    if (e == NULL) return set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine is null");
    uocr_profile_reset(&e->profile);
    uocr_memory_reset_peaks(&e->memory);
    return UOCR_OK;
}

/* ---- request validation (uocr_request_validation.c rules) ------------------ */

static int validate_request(const uocr_engine *e, const uocr_prepared_request *r, char *err, size_t n) {
#define BAD(...) (snprintf(err, n, __VA_ARGS__), UOCR_ERROR_INVALID_ARGUMENT)
    if (r->n_tokens == 0u) return BAD("prepared request must contain at least BOS");
    if (r->input_ids == NULL) return BAD("input_ids pointer is null");
    if (r->image_mask == NULL) return BAD("image_mask pointer is null");
    if (r->n_tokens > e->max_prompt_tokens) return BAD("prompt has %u tokens, engine limit is %u", r->n_tokens, e->max_prompt_tokens);
    if (r->max_new_tokens > e->max_gen_tokens) {
        return BAD("request asks for %u new tokens, engine limit is %u", r->max_new_tokens, e->max_gen_tokens);
    }
    if (r->n_tokens > UOCR_MAX_POSITIONS || r->max_new_tokens > UOCR_MAX_POSITIONS - r->n_tokens) {
        return BAD("sequence length exceeds model position budget: prompt %u + max_new_tokens %u > %u", r->n_tokens,
                   r->max_new_tokens, UOCR_MAX_POSITIONS);
    }
    if (r->input_ids[0] != UOCR_TOKEN_BOS) return BAD("first token must be BOS id %d, got %d", UOCR_TOKEN_BOS, r->input_ids[0]);
    uint32_t first = r->n_tokens, last = 0, count = 0;
    for (uint32_t i = 0; i < r->n_tokens; ++i) {
        const int32_t t = r->input_ids[i];
        if (t < 0 || t >= (int32_t)UOCR_VOCAB_SIZE) return BAD("token %u is out of vocabulary: %d", i, t);
        if (r->image_mask[i] > 1u) return BAD("image_mask[%u] must be 0 or 1, got %u", i, (unsigned)r->image_mask[i]);
        if (r->image_mask[i] == 1u) {
            if (t != UOCR_TOKEN_IMAGE) return BAD("image_mask[%u] is set but token id is %d, expected image token %d", i, t, UOCR_TOKEN_IMAGE);
            if (first == r->n_tokens) first = i;
            last = i;
            ++count;
        } else if (t == UOCR_TOKEN_IMAGE) {
            return BAD("token %u is image token %d but image_mask is 0", i, UOCR_TOKEN_IMAGE);
        }
    }
    if (count != 0u && last - first + 1u != count) return BAD("image placeholders must form one contiguous span");
    if (r->n_views != 0u && r->views == NULL) return BAD("n_views is %u but views pointer is null", r->n_views);
    if (count != 0u && r->n_views == 0u) return BAD("image placeholders require image views");
    return UOCR_OK;
#undef BAD
}

static uint32_t count_image(const uocr_prepared_request *r) {
    uint32_t c = 0;
    for (uint32_t i = 0; i < r->n_tokens; ++i) c += r->image_mask[i] == 1u;
    return c;
}

static int run_hip(uocr_engine *e, const int32_t *ids, const uint8_t *mask, const uint16_t *rows, uint32_t n_rows,
                   uint32_t n_tokens, uint32_t max_new, uint32_t flags, int32_t *out, float *scores, uint32_t *count,
                   double *prefill_ms, double *decode_ms) {
    if (e->hip == NULL) return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED, "backend '%s' does not generate", e->backend);
    if (!e->has_model) return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED, "HIP text generation requires a mapped .uocr model");
    if (!e->decoder_ready) {
        return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED, "HIP generation requires complete validated decoder tensor bindings: %s",
                         e->bind_error);
    }
    uocr_hip_decoder_request req;
    memset(&req, 0, sizeof(req));
    req.input_ids = ids;
    req.image_mask = mask;
    req.image_rows = rows;
    req.n_image_rows = n_rows;
    req.n_tokens = n_tokens;
    req.max_new_tokens = max_new;
    req.flags = flags;
    uocr_hip_decoder_result res;
    memset(&res, 0, sizeof(res));
    res.generated_ids = out;
    res.generated_scores = scores;
    res.generated_capacity = max_new;
    char herr[512] = {0};
    const uint64_t start = uocr_now_ns();
    if (!uocr_hip_context_generate(e->hip, &req, &res, herr, sizeof(herr))) {
        return set_error(e, UOCR_ERROR_INTERNAL, "HIP generation failed: %s", herr[0] ? herr : "unknown error");
    }
    uocr_profile_add_since(&e->profile, "hip.text_generate", start);
    *count = res.generated_count;
    if (prefill_ms != NULL) *prefill_ms = res.prefill_ms;
    if (decode_ms != NULL) *decode_ms = res.decode_ms;
    return UOCR_OK;
}

int uocr_generate_prepared(uocr_engine *e, const uocr_prepared_request *requests, uint32_t n_requests,
                           uocr_result **out_result) {
    if (out_result != NULL) *out_result = NULL;
    if (e == NULL) return set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine is null");
    clear_error(e);
    if (out_result == NULL) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "out_result pointer is null");
    if (requests == NULL) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "requests pointer is null");
    if (n_requests == 0u) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "n_requests must be non-zero");
    if (n_requests > e->max_batch) {
        return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "batch size %u exceeds engine limit %u", n_requests, e->max_batch);
    }
    uocr_profile_begin_request(&e->profile);
    const uint64_t vstart = uocr_now_ns();
    uint32_t max_prompt = 0;
    int any_gen = 0;
    for (uint32_t i = 0; i < n_requests; ++i) {
        char verr[512] = {0};
        const int st = validate_request(e, &requests[i], verr, sizeof(verr));
        if (st != UOCR_OK) return set_error(e, st, "request %u invalid: %s", i, verr);
        if (requests[i].n_tokens > max_prompt) max_prompt = requests[i].n_tokens;
        if (requests[i].max_new_tokens > 0u) any_gen = 1;
    }
    uocr_profile_add_since(&e->profile, "request.validation", vstart);
    estimate_memory(n_requests, max_prompt, e->model_view_bytes, &e->estimate);
    if (e->memory_budget_bytes != 0u && e->estimate.estimated_total_bytes > e->memory_budget_bytes) {
        return set_error(e, UOCR_ERROR_OUT_OF_MEMORY,
                         "request admission rejected: estimated %llu bytes exceeds budget %llu bytes",
                         (unsigned long long)e->estimate.estimated_total_bytes, (unsigned long long)e->memory_budget_bytes);
    }
    if (!any_gen) {
        const int st = uocr_result_create(n_requests, NULL, NULL, out_result);
        if (st != UOCR_OK) return set_error(e, st, "failed to allocate result");
        clear_error(e);
        return UOCR_OK;
    }
    if (strcmp(e->backend, "hip") != 0) {
        return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED,
                         "inference kernels are not implemented yet; use max_new_tokens=0 for ABI smoke tests");
    }
    if (n_requests != 1u) return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED, "HIP generation currently supports exactly one request");
    const uocr_prepared_request *r = &requests[0];
    if (r->n_views != 0u || count_image(r) != 0u) {
        return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED,
                         "HIP image generation needs precomputed visual features (uocr_generate_embeddings); "
                         "the vision encoder is not part of this build");
    }
    int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * r->max_new_tokens);
    if (ids == NULL) return set_error(e, UOCR_ERROR_OUT_OF_MEMORY, "failed to allocate generated-token buffer");
    uocr_memory_reserve(&e->memory, UOCR_MEMORY_TRANSIENT_BUFFERS, sizeof(int32_t) * r->max_new_tokens);
    uint32_t count = 0;
    int st = run_hip(e, r->input_ids, NULL, NULL, 0u, r->n_tokens, r->max_new_tokens, 0u, ids, NULL, &count, NULL, NULL);
    if (st == UOCR_OK) {
        const int32_t *lists[1] = {ids};
        st = uocr_result_create(1u, lists, &count, out_result);
        if (st != UOCR_OK) set_error(e, st, "failed to allocate generated-token result");
    }
    free(ids);
    uocr_memory_release(&e->memory, UOCR_MEMORY_TRANSIENT_BUFFERS, sizeof(int32_t) * r->max_new_tokens);
    if (st == UOCR_OK) clear_error(e);
    return st;
}

int uocr_generate_embeddings(uocr_engine *e, const int32_t *input_ids, const uint8_t *image_mask,
                             const uint16_t *image_rows_f16, uint32_t n_image_rows, uint32_t n_tokens,
                             uint32_t max_new_tokens, uint32_t flags, int32_t *out_ids, float *out_scores,
                             uint32_t *out_count, double *out_prefill_ms, double *out_decode_ms) {
    if (e == NULL) return set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine is null");
    clear_error(e);
    if (input_ids == NULL || out_ids == NULL || out_count == NULL || n_tokens == 0u || max_new_tokens == 0u) {
        return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "invalid embeddings generation request");
    }
    *out_count = 0u;
    if (n_tokens > e->max_prompt_tokens || max_new_tokens > e->max_gen_tokens) {
        return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "request exceeds engine limits (%u/%u prompt, %u/%u new)", n_tokens,
                         e->max_prompt_tokens, max_new_tokens, e->max_gen_tokens);
    }
    uint32_t masked = 0;
    for (uint32_t i = 0; i < n_tokens; ++i) {
        if (input_ids[i] < 0 || input_ids[i] >= (int32_t)UOCR_VOCAB_SIZE) {
            return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "token %u is out of vocabulary: %d", i, input_ids[i]);
        }
        if (image_mask != NULL) {
            if (image_mask[i] > 1u) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "image_mask[%u] must be 0 or 1", i);
            masked += image_mask[i];
        }
    }
    if (masked != n_image_rows || (masked != 0u && image_rows_f16 == NULL)) {
        return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "image mask selects %u rows but %u feature rows were given", masked,
                         n_image_rows);
    }
    uocr_profile_begin_request(&e->profile);
    const int st = run_hip(e, input_ids, image_mask, image_rows_f16, n_image_rows, n_tokens, max_new_tokens, flags, out_ids,
                           out_scores, out_count, out_prefill_ms, out_decode_ms);
    if (st == UOCR_OK) clear_error(e);
    return st;
}

static int hip_ready(uocr_engine *e) {
    if (e == NULL) return set_error(NULL, UOCR_ERROR_INVALID_ARGUMENT, "engine is null");
    clear_error(e);
    if (e->hip == NULL || !e->decoder_ready) {
        return set_error(e, UOCR_ERROR_NOT_IMPLEMENTED, "decode trace requires the HIP backend with a bound decoder");
    }
    return UOCR_OK;
}

int uocr_engine_trace_enable(uocr_engine *e, uint32_t steps) {
    const int st = hip_ready(e);
    if (st != UOCR_OK) return st;
    if (steps > e->max_gen_tokens) {
        return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "trace of %u steps exceeds max_gen_tokens %u", steps, e->max_gen_tokens);
    }
    char herr[512] = {0};
    if (!uocr_hip_context_trace_enable(e->hip, steps, herr, sizeof(herr))) {
        return set_error(e, UOCR_ERROR_INTERNAL, "decode trace setup failed: %s", herr);
    }
    return UOCR_OK;
}

int uocr_engine_trace_read(uocr_engine *e, uint32_t *expert_ids, uint16_t *hidden) {
    const int st = hip_ready(e);
    if (st != UOCR_OK) return st;
    char herr[512] = {0};
    if (!uocr_hip_context_trace_read(e->hip, expert_ids, hidden, herr, sizeof(herr))) {
        return set_error(e, UOCR_ERROR_INTERNAL, "decode trace readback failed: %s", herr);
    }
    return UOCR_OK;
}

int uocr_engine_trace_read_weights(uocr_engine *e, float *weights) {
    const int st = hip_ready(e);
    if (st != UOCR_OK) return st;
    if (weights == NULL) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "weights is null");
    char herr[512] = {0};
    if (!uocr_hip_context_trace_read2(e->hip, NULL, weights, NULL, herr, sizeof(herr))) {
        return set_error(e, UOCR_ERROR_INTERNAL, "decode trace readback failed: %s", herr);
    }
    return UOCR_OK;
}

int uocr_engine_trace_read_router_inputs(uocr_engine *e, uint16_t *inputs) {
    const int st = hip_ready(e);
    if (st != UOCR_OK) return st;
    if (inputs == NULL) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "inputs is null");
    char herr[512] = {0};
    if (!uocr_hip_context_trace_read_inputs(e->hip, inputs, herr, sizeof(herr))) {
        return set_error(e, UOCR_ERROR_INTERNAL, "decode trace readback failed: %s", herr);
    }
    return UOCR_OK;
}

int uocr_engine_decode_path(uocr_engine *e) {
    if (e == NULL || e->hip == NULL) return -1;
    return uocr_hip_context_decode_path(e->hip);
}

int uocr_engine_trace_force(uocr_engine *e, const int32_t *ids, uint32_t n) {
    const int st = hip_ready(e);
    if (st != UOCR_OK) return st;
    if (n > e->max_gen_tokens) return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "forcing %u ids exceeds max_gen_tokens", n);
    char herr[512] = {0};
    if (!uocr_hip_context_trace_force(e->hip, ids, n, herr, sizeof(herr))) {
        return set_error(e, UOCR_ERROR_INVALID_ARGUMENT, "teacher forcing setup failed: %s", herr);
    }
    return UOCR_OK;
}
