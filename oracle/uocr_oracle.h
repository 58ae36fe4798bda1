/*
 * uocr_oracle.h - CPU oracle for the UnlimitedOCR language-model token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP backend:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it.  The product (libunlimitedocr.so) never links or calls it.
 *
 * It restates, in plain C, the reference's CPU path and the arithmetic the
 * reference's GPU decode performs:
 *   - fp32 reference ops of src/backend/cpu_ref/uocr_cpu_ref.c (conversions
 *     :22-139, rmsnorm :145, rope :171, causal sdpa :227, dense swiglu :305,
 *     router :388, moe swiglu :468, KV ring :581-755);
 *   - Q8_0 / Q4_0 group-64 dequantised dots as the converter writes them
 *     (src/unlimitedocr_c/convert.py:2058-2063, :2249-2276) and the decode
 *     GEMVs read them (kernels/decode_gemv_q4.metal:34-57);
 *   - the LM-head argmax tie/NaN rules (kernels/lm_head_q4.metal:48-97,
 *     kernels/sampling.metal:173-200);
 *   - the decode-step op order (src/backend/metal/uocr_metal.m:14299-14518,
 *     selection :11360-11462, chunk loop :11487-11576) with fp16 rounding at
 *     the points of src/unlimitedocr_c/golden.py:381-666.
 * Each function cites the reference lines it follows.  How each one is
 * pinned (golden vectors, closed forms, brute force, the reference's own
 * compiled CPU ops) is listed in the test files that exercise it
 * (tests/test_oracle.py, tests/test_oracle_compose.py for the decode-step
 * and MoE compositions); functions with no independent pin would be marked
 * "parity unpinned" at their declaration (none is).
 */
#ifndef UOCR_ORACLE_H
#define UOCR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 conversion (uocr_cpu_ref.c:26-100) ---------------------------- */
float orc_f16_to_f32(uint16_t bits);
uint16_t orc_f32_to_f16(float value);   /* round-to-nearest-even */
float orc_bf16_to_f32(uint16_t bits);
int orc_f16_to_f32_array(const uint16_t *in, size_t n, float *out);
int orc_f32_to_f16_array(const float *in, size_t n, uint16_t *out);

/* ---- fp32 reference ops (uocr_cpu_ref.c) -------------------------------- */
int orc_rmsnorm_f32(const float *in, const float *w, uint32_t rows, uint32_t cols, float eps, float *out);
int orc_rope_split_half_f32(const float *q, const float *k, uint32_t n_tokens, uint32_t heads,
                            uint32_t head_dim, uint32_t start_position, float theta,
                            float *q_out, float *k_out);
int orc_causal_sdpa_f32(const float *q, const float *k, const float *v, uint32_t n_tokens,
                        uint32_t heads, uint32_t head_dim, float scale, float *out);
int orc_dense_swiglu_f32(const float *in, const float *gate, const float *up, const float *down,
                         uint32_t rows, uint32_t hidden, uint32_t inter, float *workspace, float *out);
int orc_moe_router_f32(const float *in, const float *router, uint32_t rows, uint32_t hidden,
                       uint32_t n_experts, uint32_t top_k, float scaling,
                       float *logits, float *probs, uint32_t *top_ids, float *top_weights);
int orc_moe_swiglu_f32(const float *in, const float *router,
                       const float *egate, const float *eup, const float *edown,
                       const float *sgate, const float *sup, const float *sdown,
                       uint32_t rows, uint32_t hidden, uint32_t n_experts, uint32_t top_k,
                       uint32_t expert_inter, uint32_t shared_inter, float scaling,
                       float *logits, float *probs, uint32_t *top_ids, float *top_weights,
                       float *expert_ws, float *shared_ws, float *out);

/* KV ring arithmetic (uocr_cpu_ref.c:616-755). */
typedef struct orc_attention_plan {
    uint32_t prompt_length;
    uint32_t generated_count;
    uint32_t live_generated;
    uint32_t first_generated_index;
    uint32_t query_position;
    uint32_t attention_length;
    uint32_t ring_window;
} orc_attention_plan;

int orc_kv_cache_token_for_position(uint32_t prompt_length, uint32_t prompt_capacity, uint32_t ring,
                                    uint32_t position, uint32_t *out_cache_token);
int orc_decode_attention_plan(uint32_t prompt_length, uint32_t prompt_capacity, uint32_t ring,
                              uint32_t generated_count, orc_attention_plan *out);
int orc_attention_index_to_token(const orc_attention_plan *plan, uint32_t index, uint32_t *out_cache_token);

/* ---- quantised decode ops (fp16 activations, fp32 accumulation) --------- */
/* qtype uses the .uocr values: 1 = f16, 3 = q8_0, 4 = q4_0.
 * W is the row-major payload, S the [rows][K/64] fp16 scales (NULL for f16).
 * Dots accumulate each 64-column group in fp32, then scale, then sum groups. */
float orc_row_dot(uint32_t qtype, const void *W, const uint16_t *S, uint32_t K,
                  uint32_t row, const uint16_t *x);
/* Dequantised weight w[row][col] as fp32 (closed form of the storage format). */
float orc_weight_at(uint32_t qtype, const void *W, const uint16_t *S, uint32_t K,
                    uint32_t row, uint32_t col);

/* y[r] = f16(dot(W_r, x) + residual[r]) for r < rows (residual may be NULL).
 * kernels/decode_gemv_q8.metal:97-126, decode_gemv_q4.metal:69-98. */
int orc_gemv(uint32_t qtype, const void *W, const uint16_t *S, uint32_t rows, uint32_t K,
             const uint16_t *x, const uint16_t *residual, uint16_t *y);
/* mid[r] = f16(silu(G_r.x) * (U_r.x)).  decode_gemv_q4.metal:101-135. */
int orc_swiglu_mid(uint32_t qtype, const void *G, const uint16_t *Gs, const void *U, const uint16_t *Us,
                   uint32_t rows, uint32_t K, const uint16_t *x, uint16_t *mid);
/* out = f16(x * 1/sqrt(mean(x^2)+eps) * w), fp32 math.  norm.metal:12-40. */
int orc_rmsnorm_f16(const uint16_t *x, const uint16_t *w, uint32_t n, float eps, uint16_t *out);
/* Split-half RoPE on fp16 q,k [heads][128] at one position, exp2 frequency
 * form of golden.py:402-426 / rope.metal:16-70; outputs rounded to fp16. */
int orc_rope_f16(uint16_t *q, uint16_t *k, uint32_t heads, uint32_t head_dim, uint32_t position, float theta);
/* Fused LM-head argmax: id = argmax_v dot(W_v, x); NaN rows skipped; ties to
 * the lowest id; no valid row -> id 0, score -inf.  Also returns the second
 * best score so callers can apply the 1e-2 top-2 margin rule.
 * lm_head_q4.metal:25-98, sampling.metal:173-200. */
int orc_lm_head_argmax(uint32_t qtype, const void *W, const uint16_t *S, uint32_t vocab, uint32_t K,
                       const uint16_t *x, int32_t *out_id, float *out_score, float *out_second);
/* Router: logits = x.R^T (fp16 R, fp32 acc), max-subtracted softmax, greedy
 * top-k with ties to the lower id; weights are the raw probabilities unless
 * norm_topk is set (then divided by their sum).  uocr_cpu_ref.c:388-466,
 * moe.metal:53-189, golden.py:544-562.  margin_out (may be NULL) receives
 * the selection margin: the smallest logit gap between consecutive ranks,
 * including the k-th selected expert against the best unselected one. */
int orc_router_topk(const uint16_t *x, const uint16_t *R, uint32_t n_experts, uint32_t K, uint32_t top_k,
                    int norm_topk, uint32_t *ids, float *weights, float *probs_out, float *margin_out);

/* One MoE FFN at batch 1 (uocr_metal.m:14433-14497, decode_gemv_q4.metal:
 * 138-224): shared = f16(SD . f16(silu(SG x) * (SU x))); mid_r =
 * f16(silu(G_e x) * (U_e x)); out = f16(sum_r w_r (D_e mid_r) + shared +
 * residual).  Expert e's gate/up/down live at egate + e*expert_stride_* etc.
 * (strides in bytes for weights, in fp16 values for scales). */
typedef struct orc_expert_view {
    uint32_t qtype;
    const uint8_t *gate_w; const uint16_t *gate_s;
    const uint8_t *up_w;   const uint16_t *up_s;
    const uint8_t *down_w; const uint16_t *down_s;
    uint64_t w_stride;     /* bytes between expert e and e+1 for each projection */
    uint64_t s_stride;     /* fp16 values between experts for each projection's scales */
} orc_expert_view;

int orc_moe_ffn(const uint16_t *x, const uint16_t *residual, const uint16_t *router,
                uint32_t n_experts, uint32_t top_k, int norm_topk,
                const orc_expert_view *experts, uint32_t expert_inter,
                uint32_t shared_qtype, const void *sg, const uint16_t *sgs, const void *su, const uint16_t *sus,
                const void *sd, const uint16_t *sds, uint32_t shared_inter,
                uint16_t *out, uint32_t *ids_out, float *weights_out, float *margin_out);

/* Decode attention for one query over the cache tokens of a plan.
 * q f16[heads*head_dim]; caches in the reference layout
 * [cache_token][heads][head_dim] (kv_cache.metal:50-52, one layer/slot);
 * fp32 scores scaled by 1/sqrt(head_dim), max-subtracted softmax, output
 * rounded to fp16.  attention_decode.metal:49-131, uocr_cpu_ref.c:694-755. */
int orc_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                         uint32_t heads, uint32_t head_dim, const orc_attention_plan *plan, uint16_t *out);

/* Embedding row gather + dequant to fp16 (embedding_q4.metal:21-56). */
int orc_embed_row(uint32_t qtype, const void *W, const uint16_t *S, uint32_t rows, uint32_t K,
                  int32_t token, uint16_t *out);

/* ---- vision linear ------------------------------------------------------ */

/* dst = f16(act(x . W^T + bias)) per row (kernels/gemm_q8.metal:161-221,
 * gemm_q4.metal:63-131): each quantised weight is first rounded to fp16 as
 * half(float(q) * scale) (gemm_q8.metal:58, the B-tile staging), products
 * accumulate in fp32 over k in order, then bias, activation (act 1:
 * x / (1 + exp(-1.702 x)), dense.metal:64-66; act 2: 0.5 x (1 + erf(x /
 * sqrt 2)) with the Abramowitz & Stegun 7.1.26 erf, sam.metal:78-91) and one
 * fp16 rounding.  qtype f16 follows the reference's MPS path
 * (uocr_metal.m:17232-17250): the product is rounded to fp16, then bias and
 * activation are applied in fp32 and rounded again (dense.metal:68-79).
 * split != 0: n == 3 * split, column c to (dst0, dst1, dst2)[c / split] at
 * [row][c % split] (gemm_q8.metal:208-219).  Pinned by brute-force fp64
 * products and the closed forms of both activations (tests/test_oracle.py). */
int orc_vision_linear(uint32_t qtype, const void *W, const uint16_t *S, const uint16_t *bias, uint32_t m,
                      uint32_t K, uint32_t N, uint32_t act, uint32_t split, const uint16_t *x, uint16_t *dst0,
                      uint16_t *dst1, uint16_t *dst2);

/* ---- full model over a .uocr image in memory ---------------------------- */
typedef struct orc_model orc_model;
orc_model *orc_model_open(const uint8_t *bytes, size_t size, char *err, size_t err_size);
void orc_model_close(orc_model *m);

typedef struct orc_session orc_session;
orc_session *orc_session_create(const orc_model *m, uint32_t prompt_capacity);
void orc_session_destroy(orc_session *s);

/* Greedy generation (uocr_metal.m:14909-15382 semantics): prefill the prompt
 * token by token through the decode-step math (causal attention over the
 * prefix), then repeat selection -> embed -> decode.  Prompt rows come from
 * the token embedding, except positions with image_mask[i] != 0, which take
 * the next row of image_rows (fp16 [n_image][1280]).  Stops after
 * max_new_tokens or on EOS (token 1, included) unless ignore_eos.
 * Writes generated ids and each step's top-2 margin; returns the count,
 * or -1 on error. */
int orc_generate(orc_session *s, const int32_t *ids, const uint8_t *image_mask, const uint16_t *image_rows,
                 uint32_t n_tokens, uint32_t max_new_tokens, int ignore_eos,
                 int32_t *out_ids, float *out_margins);

/* Lower-level step API used by tests and the CPU baseline timing. */
int orc_session_reset(orc_session *s, uint32_t prompt_length);
/* Runs the 12 decoder layers on hidden (in place) at position, writing K/V
 * for that position; attention covers the plan implied by (prompt_length,
 * position).  Optional trace_ids receives the router ids [11][6]. */
int orc_forward_token(orc_session *s, uint16_t *hidden, uint32_t position, uint32_t *trace_ids);
/* orc_forward_token that also writes, per MoE layer, the router's set
 * margin ([11] floats): the logit gap between the 6th selected expert and
 * the best unselected one (how far the selection, as a set, is from a
 * tie); and (trace_weights, optional, [11][6]) the routing weights of the
 * selected experts in selection order (raw softmax probabilities). */
int orc_forward_token_traced(orc_session *s, uint16_t *hidden, uint32_t position, uint32_t *trace_ids,
                             float *trace_margins, float *trace_weights);
int orc_select(orc_session *s, const uint16_t *hidden, int32_t *id, float *score, float *second);
/* The model's embedding row of token (fp16 bits), as orc_generate stages it. */
int orc_session_embed(orc_session *s, int32_t token, uint16_t *out);
/* Fills the KV cache prefix [0, n) of every layer with fp16 values from a
 * seeded N(0,1) stream (for timing decode at a given context length). */
int orc_session_fill_kv(orc_session *s, uint32_t n, uint64_t seed);
/* Sets the OpenMP thread count used by row-parallel loops (0 = default). */
void orc_set_threads(int n);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_ORACLE_H */
