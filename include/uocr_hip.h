/*
 * uocr_hip.h - MI355X extensions of libunlimitedocr.so.
 *
 * Three groups of extern "C" entry points, all plain pointers and sizes:
 *
 *  1. Engine extensions.  The reference feeds precomputed visual rows into
 *     the decoder through an internal image_features_f16 span
 *     (src/backend/metal/uocr_metal.m:14988-15017); uocr_generate_embeddings
 *     exposes that path so a prompt of image-embedding rows plus text ids
 *     can be generated without the vision encoder.
 *     uocr_engine_open_memory opens a .uocr image already in host memory.
 *
 *  2. Hot-path operators.  Each runs one kernel (or fusion) of the decode
 *     step on device buffers and replaces one reference Metal kernel, cited
 *     per function.  Operands use the .uocr storage layout: row-major payload
 *     plus a separate [rows][K/64] fp16 scale array (NULL for f16); all
 *     activations are fp16 bit patterns (uint16), dots accumulate in fp32.
 *     Operators are enqueued on one library stream on device 0 and return
 *     before completion; uocr_hip_sync() waits.  They return 0 on success
 *     and a negative uocr_status on error (text in uocr_hip_op_error()).
 *
 *  3. Device-memory plumbing (alloc/copy/sync/timers) so callers with no HIP
 *     binding (ctypes, tests, benchmarks) can drive the operators.
 *
 * The synthetic .uocr builder used by the tests and benchmarks is declared
 * in uocr_synth.h.
 */
#ifndef UOCR_HIP_H
#define UOCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "unlimitedocr.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- 1. engine extensions ------------------------------------------------ */

/* Like uocr_engine_open but validates and maps a .uocr image in memory.  The
 * caller keeps `data` alive until uocr_engine_close. */
UOCR_API uocr_engine *uocr_engine_open_memory(const uocr_engine_opts *opts, const void *data, size_t size);

#define UOCR_GEN_FLAG_IGNORE_EOS 1u  /* decode past EOS (benchmarks) */
#define UOCR_GEN_FLAG_NO_GRAPH 2u    /* enqueue kernels directly, no hipGraph replay */
#define UOCR_GEN_FLAG_TOKEN_PREFILL 4u /* prefill through the decode kernels, one prompt position at a time */
#define UOCR_GEN_FLAG_NO_RUN 8u      /* decode with per-step kernel graphs instead of the persistent run */

/* Greedy generation from a prompt whose image positions (image_mask[i] == 1)
 * take the next row of image_rows_f16 ([n_image_rows][1280] fp16) instead of
 * the token embedding.  Replaces the Metal image_features_f16 span path
 * (uocr_metal.m:14988-15017) followed by uocr_metal.m:14909-15382.
 * Writes up to max_new_tokens ids (EOS included when it stops generation)
 * and optionally the argmax score of each; reports prefill and decode wall
 * time in ms.  Returns a uocr_status. */
UOCR_API int uocr_generate_embeddings(uocr_engine *engine, const int32_t *input_ids, const uint8_t *image_mask,
                                      const uint16_t *image_rows_f16, uint32_t n_image_rows, uint32_t n_tokens,
                                      uint32_t max_new_tokens, uint32_t flags, int32_t *out_ids, float *out_scores,
                                      uint32_t *out_count, double *out_prefill_ms, double *out_decode_ms);

/* Decode trace, for parity tests against a CPU restatement of the decoder
 * (no counterpart in the reference; it reads the router selection of
 * uocr_metal.m:14227-14548 and the hidden state fed to the LM head).  After
 * uocr_engine_trace_enable(engine, steps), each generation records the
 * expert ids the router selects in layers 1-11 while computing the hidden
 * state of decode steps t < steps.  uocr_engine_trace_read copies them to
 * expert_ids ([steps][11][6], 0xffffffff for steps the last generation did
 * not reach; may be NULL)
 * and the final hidden state of the last generation (the fp16 [1280] input
 * of its last token's final norm; may be NULL).  steps = 0 turns tracing off.
 * Tracing switches the per-step graph path to eager launches. */
UOCR_API int uocr_engine_trace_enable(uocr_engine *engine, uint32_t steps);
UOCR_API int uocr_engine_trace_read(uocr_engine *engine, uint32_t *expert_ids, uint16_t *hidden);
/* The routing weights of the traced selections ([steps][11][6] fp32, the raw
 * softmax probabilities in the order of the ids uocr_engine_trace_read
 * returns; NaN bits for steps the last generation did not reach). */
UOCR_API int uocr_engine_trace_read_weights(uocr_engine *engine, float *weights);
/* The router input of each traced selection: a = h + O ctx, the fp16
 * [steps][11][1280] pre-norm input of the layer's router (0xffff bits for
 * steps not reached), so a test can recompute the reference router on the
 * engine's own input. */
UOCR_API int uocr_engine_trace_read_router_inputs(uocr_engine *engine, uint16_t *inputs);
/* Which decode loop served the engine's last generation (no counterpart in
 * the reference; for tests and diagnostics): 1 the persistent
 * run, 0 the per-step kernels, 2 the per-step kernels after the run gave up
 * waiting on a workgroup and the request was served again, -1 none yet or
 * not a HIP engine. */
UOCR_API int uocr_engine_decode_path(uocr_engine *engine);
/* Teacher forcing, also for parity tests (no counterpart in the reference):
 * after uocr_engine_trace_force(engine, ids, n) each generation embeds ids[t]
 * after decode step t < n instead of the token it selected, and still
 * reports its own selection in out_ids.  Each step is then a function of the
 * forced prefix alone, so a CPU restatement can be compared step by step
 * over a whole generation.  n = 0 turns it off.  Forcing switches the
 * per-step graph path to eager launches. */
UOCR_API int uocr_engine_trace_force(uocr_engine *engine, const int32_t *ids, uint32_t n);

/* ---- 2. hot-path operators ----------------------------------------------- */

/* Bytes of the device workspace every operator below takes (partials,
 * counters, routing ids, intermediates, step state).  A workspace must be
 * zero before its first use (uocr_hip_alloc returns zeroed memory); the
 * operators leave their counters at zero. */
UOCR_API size_t uocr_op_workspace_bytes(void);

/* y[r] = fp16(sum_k W[r][k] * x[k] (+ residual[r])), r < rows, K % 64 == 0,
 * K <= 6848.  Replaces uocr_decode_linear_residual_gemv_q8_0_to_f16
 * (kernels/decode_gemv_q8.metal:97-126) and its Q4 twin
 * (kernels/decode_gemv_q4.metal:69-98); BASELINE config 1. */
UOCR_API int uocr_op_gemv(uint32_t qtype, const void *w, const void *s, uint32_t rows, uint32_t k, const void *x,
                          const void *residual, void *y);

/* mid[r] = fp16(silu(G[r].xin) * (U[r].xin)), xin = x or rmsnorm(x, norm_w).
 * Replaces uocr_decode_swiglu_gate_up_gemv_q4_0_to_f16
 * (kernels/decode_gemv_q4.metal:101-135). */
UOCR_API int uocr_op_swiglu(uint32_t qtype, const void *gw, const void *gs, const void *uw, const void *us,
                            uint32_t rows, uint32_t k, const void *x, const void *norm_w, void *mid);

/* y = fp16(x * 1/sqrt(mean(x^2) + 1e-6) * w).  Replaces uocr_rmsnorm_f16_to_f16
 * (kernels/norm.metal:12-40). */
UOCR_API int uocr_op_rmsnorm(const void *x, const void *w, uint32_t n, void *y);

/* Fused [optional final RMSNorm] + LM-head GEMV + argmax over vocab rows of
 * K = 1280 (NaN rows skipped, ties to the lowest id, none valid -> id 0).
 * Writes the token id and its score to device memory.  Replaces
 * uocr_lm_head_argmax_q4_0_to_f16 + uocr_argmax_pairs_f32
 * (kernels/lm_head_q4.metal:25-98, kernels/sampling.metal:173-200);
 * BASELINE config 2. */
UOCR_API int uocr_op_lm_head_argmax(uint32_t qtype, const void *w, const void *s, uint32_t vocab, const void *x,
                                    const void *norm_w, void *workspace, int32_t *token, float *score);

/* The streaming part of uocr_op_lm_head_argmax alone (its first launch):
 * [final RMSNorm +] LM-head GEMV + per-block argmax, each block adding its
 * best (score, row) as a 64-bit key, (order(score) << 32) | (0xffffffff -
 * row), by atomic max into keys[block % 16] (16 uint64 on the device; start
 * them at zero; the largest key is the winner, 0: no valid row).  The
 * decode loop chooses the token from these keys in its next launch.  No
 * reference counterpart: it exposes the LM head's dominant kernel for
 * measurement. */
UOCR_API int uocr_op_lm_head_keys(uint32_t qtype, const void *w, const void *s, uint32_t vocab, const void *x,
                                  const void *norm_w, uint64_t *keys);

/* MoE router over 64 fp16 rows of K = 1280: softmax, greedy top-6 with ties
 * to the lower id, raw probabilities (renormalised when norm_topk != 0).
 * Replaces uocr_moe_router_decode_fused_f16 (kernels/moe.metal:53-189). */
UOCR_API int uocr_op_router(const void *router_w, const void *x, const void *norm_w, int norm_topk, void *workspace,
                            uint32_t *ids, float *weights);

/* Weights of one MoE FFN.  Expert projections are slabs of 64 experts:
 * projection p of expert e at p_w + e * *_w_stride bytes and p_s + e *
 * *_s_stride fp16 values.  Shared experts (merged, intermediate 1792) use
 * shared_qtype; routed experts use expert_qtype. */
typedef struct uocr_op_moe_weights {
    const void *router;                   /* fp16 [64][1280] */
    uint32_t expert_qtype;
    const void *gate_w, *gate_s, *up_w, *up_s; /* [64] x [896][1280] */
    uint64_t gu_w_stride, gu_s_stride;
    const void *down_w, *down_s;          /* [64] x [1280][896] */
    uint64_t dn_w_stride, dn_s_stride;
    uint32_t shared_qtype;
    const void *sgate_w, *sgate_s, *sup_w, *sup_s; /* [1792][1280] */
    const void *sdown_w, *sdown_s;        /* [1280][1792] */
} uocr_op_moe_weights;

/* out = fp16(sum_r w_r D_e(mid_r) + fp16(SD(smid)) + residual) with
 * mid_r = fp16(silu(G_e xin) * U_e xin), smid likewise for the shared
 * experts, xin = x or rmsnorm(x, norm_w); the chosen ids and weights are
 * also written (device).  Replaces the decode MoE sequence of
 * uocr_metal.m:14433-14497 (router, shared SwiGLU, routed gate/up
 * decode_gemv_q4.metal:138-180, down-combine :185-224); BASELINE config 3. */
UOCR_API int uocr_op_moe_ffn(const uocr_op_moe_weights *m, const void *x, const void *norm_w, const void *residual,
                             int norm_topk, void *workspace, void *out, uint32_t *ids, float *weights);

/* The gate/up stage of uocr_op_moe_ffn alone: from router logits (fp32[64],
 * device) the top-6 experts and their softmax weights (renormalised when
 * norm_topk), then mid[r] = fp16(silu(G_e xin) * U_e xin) for each selected
 * expert e = ids[r] (mid: [6][896] fp16) and smid likewise for the merged
 * shared experts ([1792] fp16), xin = x or rmsnorm(x, norm_w); all pointers
 * device.  One kernel launch.  Replaces uocr_moe_router_softmax_topk_f32
 * (kernels/moe.metal:194) followed by uocr_moe_decode_gate_up_gemv_q4_0_to_f16
 * (kernels/decode_gemv_q4.metal:138-180) and the shared SwiGLU of
 * uocr_metal.m:14433-14497. */
UOCR_API int uocr_op_moe_gate_up(const uocr_op_moe_weights *m, const float *logits, const void *x, const void *norm_w,
                                 int norm_topk, void *mid, void *smid, uint32_t *ids, float *weights);

/* Decode attention of one query (fp16 [10][128]) over a KV cache laid out
 * [10 heads][cache_capacity][128] fp16, for prompt_length prompt slots plus
 * generated_count generated tokens in the 128-token ring (generated_count
 * counts the token just written; 0 means prompt-only).  fp32 softmax scaled
 * by 1/sqrt(128); output fp16 [10][128].  Replaces
 * uocr_decode_attention_flash_f16_to_f16 (kernels/attention_decode.metal:
 * 25-131); BASELINE config 4. */
UOCR_API int uocr_op_attention_decode(const void *q, const void *k_cache, const void *v_cache,
                                      uint32_t cache_capacity, uint32_t prompt_length, uint32_t generated_count,
                                      void *workspace, void *out);

/* Full attention half of a decoder layer at one decode position:
 * rmsnorm(hidden, norm_w) -> q/k/v GEMVs (qtype, K = 1280) -> split-half RoPE
 * (theta 10000) at position prompt_length + generated_count - 1 -> K/V write
 * into the ring slot -> decode attention -> out = fp16(O ctx + hidden).
 * Replaces uocr_metal.m:14338-14393 (norm, QKV :11614, rope.metal:39-70,
 * kv_cache.metal:20-62, attention, decode_gemv_q8.metal:97-126); BASELINE
 * config 4 with projections. */
UOCR_API int uocr_op_attention_block(uint32_t qtype, const void *wq, const void *sq, const void *wk, const void *sk,
                                     const void *wv, const void *sv, const void *wo, const void *so,
                                     const void *hidden, const void *norm_w, void *k_cache, void *v_cache,
                                     uint32_t cache_capacity, uint32_t prompt_length, uint32_t generated_count,
                                     void *workspace, void *out);

/* Embedding row of `token` (device int32) dequantised to fp16 [1280];
 * out-of-range ids give zeros.  Replaces uocr_get_rows_q4_0_to_f16_h1280_g64
 * (kernels/embedding_q4.metal:21-56) and its Q8/f16 twins. */
UOCR_API int uocr_op_embed(uint32_t qtype, const void *w, const void *s, uint32_t vocab, const int32_t *token,
                           void *out);

/* ---- prefill operators (MFMA) ------------------------------------------- */

/* y = f16(x . W^T (+ residual)) for m rows: x fp16 [m][k], W [n][k] in the
 * .uocr layout (k % 64 == 0), residual/y fp16 [m][n].  The tiled MFMA GEMM of
 * the prompt prefill.  Replaces uocr_decoder_gemm_residual_q4_0_to_f16
 * (kernels/gemm_q4.metal:135-195) and its Q8 twin (kernels/gemm_q8.metal). */
UOCR_API int uocr_op_gemm(uint32_t qtype, const void *w, const void *s, uint32_t m, uint32_t n, uint32_t k,
                          const void *x, const void *residual, void *y);

/* ---- vision linear (MFMA) ------------------------------------------------ */

#ifndef UOCR_VISION_ACT_NONE
#define UOCR_VISION_ACT_NONE 0u      /* identity */
#define UOCR_VISION_ACT_QUICKGELU 1u /* x * sigmoid(1.702 x), CLIP MLP fc1 */
#define UOCR_VISION_ACT_GELU_ERF 2u  /* 0.5 x (1 + erf(x / sqrt 2)), SAM MLP lin1 */
#endif

/* dst = f16(act(x . W^T + bias)) for m rows: x fp16 [m][k], W [n][k] in the
 * .uocr layout (qtype f16, Q8_0 or Q4_0; k % 64 == 0), bias fp16 [n].
 * split == 0: dst0 fp16 [m][n] (dst1, dst2 ignored).  split != 0 (fused QKV):
 * n == 3 * split and column c goes to (dst0, dst1, dst2)[c / split] at
 * [row][c % split].  erf is Abramowitz & Stegun 7.1.26, as the reference's.
 * Replaces metal_run_vision_gemm_q8_0 (src/backend/metal/uocr_metal.m:6321-
 * 6396) with its kernels uocr_vision_gemm_q8_0_to_f16 (kernels/gemm_q8.metal:
 * 161-221) and uocr_vision_gemm_q4_0_to_f16 (kernels/gemm_q4.metal:63-131),
 * and the fp16 path MPS matmul + bias/activation (uocr_metal.m:17232-17250,
 * kernels/dense.metal:68-79, kernels/sam.metal:93-104), which is fused here
 * (one fp16 rounding instead of two).  GEMMs with k >= 2048 on grids of
 * fewer than 128 output tiles split K over up to 8 blocks per tile through an fp32 partials buffer that
 * the library allocates on first need (outside graph capture; under capture
 * without room the unsplit kernel runs) and keeps: calls must not overlap.
 * Errors: UOCR_ERROR_INVALID_ARGUMENT for
 * a bad qtype, act, shape or split, or a missing bias, scales or output. */
UOCR_API int uocr_op_vision_linear(uint32_t qtype, const void *w, const void *s, const void *bias, uint32_t m,
                                   uint32_t k, uint32_t n, uint32_t act, uint32_t split, const void *x, void *dst0,
                                   void *dst1, void *dst2);

/* Causal attention of P prompt queries (fp16 [P][1280], RoPE applied) over
 * cache slots 0..P-1 of caches laid out [10][cache_capacity][128]; ctx fp16
 * [P][1280].  Long causal key ranges are split over several blocks and
 * merged by a second kernel, through a 17 MB partials buffer the library
 * allocates on the first call made outside graph capture and keeps (without
 * it the unsplit kernel runs; calls must not overlap).  Replaces
 * uocr_prefill_attention_flash_staged_f16_to_f16
 * (kernels/attention_prefill.metal:105). */
UOCR_API int uocr_op_prefill_attention(const void *q, const void *k_cache, const void *v_cache,
                                       uint32_t cache_capacity, uint32_t prompt_length, void *ctx);

/* Bytes of the workspace uocr_op_moe_ffn_rows needs for P rows (any
 * contents: the expert buckets are built in LDS on every call). */
UOCR_API size_t uocr_op_moe_rows_workspace_bytes(uint32_t rows);

/* The MoE FFN of uocr_op_moe_ffn for P rows at once (x, residual, out fp16
 * [P][1280]): router GEMM, per-row top-6, expert buckets, shared and
 * expert-grouped SwiGLU GEMMs, combine.  Replaces the bucketed prefill MoE
 * (kernels/gemm_q8.metal:462-919, gemm_q4.metal:260-339). */
UOCR_API int uocr_op_moe_ffn_rows(const uocr_op_moe_weights *m, const void *x, const void *norm_w,
                                  const void *residual, uint32_t rows, int norm_topk, void *workspace, void *out);

/* Maximum rows of uocr_op_moe_ffn_rows_static. */
#define UOCR_OP_STATIC_MAX_ROWS 64u

/* uocr_op_moe_ffn_rows without a workspace argument and without any device
 * allocation: the workspace is a file-scope device array of the library
 * (3,235,840 bytes: UOCR_OP_STATIC_MAX_ROWS rows), which every GPU the
 * library runs on holds until the process ends.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Rejects
 * rows > UOCR_OP_STATIC_MAX_ROWS with UOCR_ERROR_INVALID_ARGUMENT.  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU
 * race.  The array needs no clearing (the expert buckets are rebuilt on
 * every call) and keeps the last call's contents. */
UOCR_API int uocr_op_moe_ffn_rows_static(const uocr_op_moe_weights *m, const void *x, const void *norm_w,
                                         const void *residual, uint32_t rows, int norm_topk, void *out);

/* ---- 3. device plumbing ---------------------------------------------------- */
UOCR_API int uocr_hip_device_count(void);
/* Device memory on the library's device, zero-filled (a fresh operator
 * workspace must start at zero). */
UOCR_API void *uocr_hip_alloc(size_t bytes);
UOCR_API int uocr_hip_free(void *p);
UOCR_API int uocr_hip_upload(void *dst, const void *src, size_t bytes);
UOCR_API int uocr_hip_download(void *dst, const void *src, size_t bytes);
UOCR_API int uocr_hip_memset(void *dst, int value, size_t bytes); /* refused (INVALID_ARGUMENT) while capturing */
UOCR_API int uocr_hip_copy(void *dst, const void *src, size_t bytes); /* device to device, on the operator stream */
UOCR_API int uocr_hip_sync(void);
UOCR_API const char *uocr_hip_op_error(void);
/* hipEvent timer on the operator stream: begin records the start event, end
 * records the stop event, waits for it and returns the elapsed ms (< 0 on
 * error). */
UOCR_API int uocr_hip_timer_begin(void);
UOCR_API float uocr_hip_timer_end_ms(void);
/* One hipGraph of operator calls, for callers that replay a fixed sequence
 * (benchmarks): begin starts capturing the operator stream, the operator
 * calls that follow are recorded instead of run, end instantiates the
 * recording, replay launches it `times` times on the operator stream, release
 * frees it.  One graph is held at a time; operators that synchronise cannot be
 * captured. */
UOCR_API int uocr_hip_capture_begin(void);
UOCR_API int uocr_hip_capture_end(void);
UOCR_API int uocr_hip_graph_replay(uint32_t times);
UOCR_API int uocr_hip_graph_release(void);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_HIP_H */
