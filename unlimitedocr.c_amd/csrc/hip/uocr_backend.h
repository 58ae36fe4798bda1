/*
 * uocr_backend.h - HIP backend behind the engine core.
 *
 * Replaces the reference's Metal backend interface
 * (src/backend/metal/uocr_metal.h:170-299: context create/destroy, profile
 * and memory-tracker hooks, map_model, runtime arenas, generate_f16 with the
 * decoder request/result of :107-128).  One context owns one HIP stream on
 * one device, the weights copied into HBM, the KV cache and all scratch.
 * Every entry returns 1 on success, 0 with a message in err on failure.
 */
#ifndef UOCR_BACKEND_H
#define UOCR_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#include "../core/uocr_model.h"
#include "../core/uocr_runtime.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct uocr_hip_ctx uocr_hip_ctx;

/* flags of uocr_hip_decoder_request */
#define UOCR_GEN_IGNORE_EOS 1u   /* keep decoding past token 1 (benchmarks) */
#define UOCR_GEN_NO_GRAPH 2u     /* enqueue kernels directly instead of replaying captured graphs */
#define UOCR_GEN_TOKEN_PREFILL 4u /* prefill by replaying the decode layer kernels per prompt position */
#define UOCR_GEN_NO_RUN 8u        /* decode with per-step graphs instead of the persistent run */

typedef struct uocr_hip_decoder_request {
    const int32_t *input_ids;
    const uint8_t *image_mask;      /* may be NULL: no image rows */
    const uint16_t *image_rows;     /* fp16 [n_image_rows][1280], in mask order */
    uint32_t n_image_rows;
    uint32_t n_tokens;
    uint32_t max_new_tokens;
    uint32_t flags;
} uocr_hip_decoder_request;

typedef struct uocr_hip_decoder_result {
    int32_t *generated_ids;
    float *generated_scores;        /* may be NULL */
    uint32_t generated_capacity;
    uint32_t generated_count;
    uint32_t stopped_on_eos;
    double prefill_ms;
    double decode_ms;
} uocr_hip_decoder_result;

int uocr_hip_is_available(char *why, size_t why_size);
uocr_hip_ctx *uocr_hip_context_create(char *err, size_t err_size);
void uocr_hip_context_destroy(uocr_hip_ctx *ctx);
void uocr_hip_context_set_profile(uocr_hip_ctx *ctx, uocr_profile_state *profile);
void uocr_hip_context_set_memory_tracker(uocr_hip_ctx *ctx, uocr_memory_tracker *tracker);
/* Copies the bound decoder tensors into HBM (weights + expert slabs). */
int uocr_hip_context_map_model(uocr_hip_ctx *ctx, const uocr_decoder_bindings *b, char *err, size_t err_size);
/* Allocates KV cache and scratch for prompts up to prompt_capacity tokens and
 * up to max_gen generated tokens. */
int uocr_hip_context_allocate_runtime(uocr_hip_ctx *ctx, uint32_t prompt_capacity, uint32_t max_gen, char *err,
                                      size_t err_size);
int uocr_hip_context_generate(uocr_hip_ctx *ctx, const uocr_hip_decoder_request *req, uocr_hip_decoder_result *res,
                              char *err, size_t err_size);
uint64_t uocr_hip_context_weight_bytes(const uocr_hip_ctx *ctx);
/* Decode trace for parity tests: the following generations record, for
 * decode steps t < steps, the expert ids of layers 1-11 ([steps][11][6])
 * and their routing weights,
 * and the final hidden state (the last step's LM-head input, fp16 [1280]).
 * steps = 0 turns it off.  The graph path records through its eager per-step
 * loop; the persistent run records in place. */
int uocr_hip_context_trace_enable(uocr_hip_ctx *ctx, uint32_t steps, char *err, size_t err_size);
/* Teacher forcing for parity tests: the following generations embed ids[t]
 * after decode step t < n instead of the token they select (which they still
 * report); n = 0 turns it off. */
int uocr_hip_context_trace_force(uocr_hip_ctx *ctx, const int32_t *ids, uint32_t n, char *err, size_t err_size);
int uocr_hip_context_trace_read(uocr_hip_ctx *ctx, uint32_t *expert_ids, uint16_t *hidden, char *err, size_t err_size);
/* trace_read that also copies the routing weights of the traced selections
 * ([steps][11][6] fp32, selection order; NaN bits for steps not reached) */
int uocr_hip_context_trace_read2(uocr_hip_ctx *ctx, uint32_t *expert_ids, float *weights, uint16_t *hidden, char *err,
                                 size_t err_size);
/* The router inputs of the traced selections: a = h + O ctx (fp16
 * [steps][11][1280], the pre-norm input of each MoE layer's router; 0xffff
 * bits for steps not reached). */
int uocr_hip_context_trace_read_inputs(uocr_hip_ctx *ctx, uint16_t *inputs, char *err, size_t err_size);
/* Decode path of the last generation: 1 the persistent run, 0 the per-step
 * kernels, 2 the per-step kernels after the run gave up waiting, -1 none. */
int uocr_hip_context_decode_path(const uocr_hip_ctx *ctx);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_BACKEND_H */
