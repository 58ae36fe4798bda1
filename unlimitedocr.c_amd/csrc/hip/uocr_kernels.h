/*
 * uocr_kernels.h - launch interface of the gfx950 decode kernels.
 *
 * Internal to libunlimitedocr.so.  Every launcher validates the shapes its
 * kernel and grid assume before launching and returns hipErrorInvalidValue
 * instead of launching on a mismatch.
 *
 * Tensor storage is the .uocr layout: row-major payload (f16, int8, or Q4_0
 * group-half-split nibbles) plus a separate [rows][K/64] fp16 scale array.
 * Activations are fp16; all dots accumulate in fp32.
 */
#ifndef UOCR_KERNELS_H
#define UOCR_KERNELS_H

#include <hip/hip_runtime.h>
#include <stdint.h>

/* qtype values follow the .uocr tensor qtype enum */
#define UOCR_QT_F16 1u
#define UOCR_QT_Q8 3u
#define UOCR_QT_Q4 4u

#define UOCR_K_HIDDEN 1280
#define UOCR_K_HEADS 10
#define UOCR_K_HEAD_DIM 128
#define UOCR_K_EXPERTS 64
#define UOCR_K_TOPK 6
#define UOCR_K_RING 128
#define UOCR_K_MAX_K 6848          /* largest GEMV reduction length */
#ifndef UOCR_K_ATTN_SPLITS
#define UOCR_K_ATTN_SPLITS 16      /* split-K blocks per head in decode attention */
#endif
#define UOCR_K_ATTN_SPLITS_WIDE 32 /* partials layout of the operator API's wide split (long contexts) */
#define UOCR_K_LM_BLOCKS 1024      /* upper bound on LM-head blocks */
#define UOCR_K_ROUTER_FIX_SHIFT 32 /* router fold accumulator: round(z * 2^32) in int64 */
#define UOCR_K_ROUTER_ACC_COPIES 4 /* accumulator copies (block b adds into copy b % 4) */
#define UOCR_ROUTER_ACC_WORDS (UOCR_K_ROUTER_ACC_COPIES * UOCR_K_EXPERTS) /* int64 words */

/* Per-step decode state kept in device memory so one captured graph can be
 * replayed for every token.  Positions follow uocr_metal.m:14239 and the ring
 * plan of attention_decode.metal:25-33. */
typedef struct uocr_step_state {
    int32_t t;            /* generated tokens selected so far */
    int32_t prompt_len;   /* P */
    int32_t pos;          /* position of the token being decoded */
    int32_t cache_token;  /* KV slot written for pos */
    int32_t attn_prompt;  /* attention indices below this map 1:1 to slots */
    int32_t attn_len;     /* attention length */
    int32_t first_gen;    /* logical index of the first live ring token */
    int32_t cur_token;    /* token id embedded this step */
    float rope_cos[UOCR_K_HEAD_DIM / 2]; /* cos/sin(pos * inv_freq[d]) of this step's position */
    float rope_sin[UOCR_K_HEAD_DIM / 2];
} uocr_step_state;

typedef struct uocr_qmat {
    const void *w;        /* payload */
    const uint16_t *s;    /* scales (NULL for f16) */
    uint32_t qtype;
} uocr_qmat;

/* Expert slab of one layer: projection p of expert e at w + e * w_stride
 * (bytes) and s + e * s_stride (fp16 values). */
typedef struct uocr_expert_slab {
    uocr_qmat gate, up, down;
    uint64_t gu_w_stride, gu_s_stride;   /* gate/up: [896][1280] per expert */
    uint64_t dn_w_stride, dn_s_stride;   /* down:    [1280][896] per expert */
} uocr_expert_slab;

/* Scratch sizes (bytes) the launchers expect. */
#define UOCR_ATTN_PARTIAL_FLOATS (UOCR_K_HEADS * UOCR_K_ATTN_SPLITS * (UOCR_K_HEAD_DIM + 2))
#define UOCR_ATTN_PARTIAL_FLOATS_WIDE (UOCR_K_HEADS * UOCR_K_ATTN_SPLITS_WIDE * (UOCR_K_HEAD_DIM + 2))
#define UOCR_LM_KEYS 16 /* LM-head argmax key copies (block b -> copy b % 16) */
#define UOCR_LM_PARTIAL_WORDS (2 * UOCR_LM_KEYS) /* the 64-bit argmax keys, in 32-bit words */

#ifdef __cplusplus
extern "C" {
#endif

/* y[r] = f16(dot(W_r, xin) [+ res[r]]); xin = x, or rmsnorm(x, nw) when nw. */
hipError_t uocr_launch_gemv(hipStream_t st, uocr_qmat W, uint32_t rows, uint32_t K, const uint16_t *x,
                            const uint16_t *nw, const uint16_t *res, uint16_t *y);
/* mid[r] = f16(silu(G_r.xin) * (U_r.xin)); xin as above. */
hipError_t uocr_launch_swiglu(hipStream_t st, uocr_qmat G, uocr_qmat U, uint32_t rows, uint32_t K,
                              const uint16_t *x, const uint16_t *nw, uint16_t *mid);
/* RMSNorm of x (fp16 [n]) with weight nw -> y (fp16). */
hipError_t uocr_launch_rmsnorm(hipStream_t st, const uint16_t *x, const uint16_t *nw, uint32_t n, uint16_t *y);
/* Fused attention input: rmsnorm(h) -> q,k,v GEMVs -> f16 -> split-half RoPE
 * at st->pos -> q to qout, k/v into the caches at st->cache_token.
 * Caches are [heads][cache_capacity][128] fp16 for one layer. */
hipError_t uocr_launch_qkv_rope(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                                const uint16_t *nw, const uocr_step_state *state, uint16_t *qout, uint16_t *kcache,
                                uint16_t *vcache, uint32_t cache_capacity);
/* uocr_launch_qkv_rope for decode step t after a prompt_len-token prompt
 * without a step state prepared beforehand: the launch computes the KV slot
 * and RoPE of that step itself (uocr_launch_decode_state's arithmetic, with
 * inv_freq [64]) and writes the step state for the attention launch after it. */
hipError_t uocr_launch_qkv_rope_plan(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                                     const uint16_t *nw, uocr_step_state *state, uint16_t *qout, uint16_t *kcache,
                                     uint16_t *vcache, uint32_t cache_capacity, int32_t prompt_len, int32_t t,
                                     const float *inv_freq);
/* Split-K decode attention over the live slots [0, state->attn_len) of one
 * layer's caches (UOCR_K_ATTN_SPLITS blocks per head, slots partitioned by
 * cache_capacity): writes UOCR_ATTN_PARTIAL_FLOATS of per-split partials.
 * router_acc (may be NULL) is cleared for the following attn_out, and the
 * UOCR_LM_KEYS LM-head keys at clear_keys (may be NULL) for the next step. */
hipError_t uocr_launch_attention(hipStream_t st, const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                                 uint32_t cache_capacity, const uocr_step_state *state, float *partials,
                                 int64_t *router_acc, uint64_t *clear_keys);
/* O projection with the attention merge in its prologue:
 * out = f16(O . ctx + res), ctx = f16(merge(partials)); ctx_out (may be
 * NULL) receives ctx.  With router_fold (fp32 [1280][64], entry [i][e] =
 * R[e][i] * post_norm[i]) each block also adds its rows' share of the
 * un-normalised router logits z[e] = sum_i fold[i][e] * out[i] into
 * router_acc (UOCR_ROUTER_ACC_WORDS, cleared beforehand) as fixed point,
 * round(x * 2^32), so the sum is independent of the order of the
 * additions. */
hipError_t uocr_launch_attn_out(hipStream_t st, uocr_qmat O, const float *partials, const uint16_t *res,
                                uint16_t *out, uint16_t *ctx_out, const float *router_fold, int64_t *router_acc);
/* The merge alone: ctx = f16(merge(partials)). */
hipError_t uocr_launch_attn_merge(hipStream_t st, const float *partials, uint16_t *ctx);
/* The same three over the wide partials layout (UOCR_K_ATTN_SPLITS_WIDE
 * splits, UOCR_ATTN_PARTIAL_FLOATS_WIDE floats): `splits` <= 32 blocks per
 * head run, the layout's other splits are marked empty, so the merge is the
 * same function of the live slots at any split count. */
hipError_t uocr_launch_attention_wide(hipStream_t st, const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                                      uint32_t cache_capacity, const uocr_step_state *state, float *partials,
                                      uint32_t splits);
hipError_t uocr_launch_attn_out_wide(hipStream_t st, uocr_qmat O, const float *partials, const uint16_t *res,
                                     uint16_t *out, uint16_t *ctx_out);
hipError_t uocr_launch_attn_merge_wide(hipStream_t st, const float *partials, uint16_t *ctx);
/* Router logits: logits[e] = R_e . rmsnorm(x) (fp16 R [64][1280], fp32 dot),
 * one wavefront per expert row. */
hipError_t uocr_launch_router_logits(hipStream_t st, const uint16_t *R, const uint16_t *x, const uint16_t *nw,
                                     float *logits);
/* Router logits + softmax + greedy top-6 (ties to the lower id; raw
 * probabilities unless norm_topk) into ids/weights. */
hipError_t uocr_launch_router(hipStream_t st, const uint16_t *R, const uint16_t *x, const uint16_t *nw, int norm_topk,
                              float *logits, uint32_t *ids, float *weights);
/* Gate/up of the routed experts (top-6 recomputed from logits per
 * wavefront) and of the shared experts in one launch:
 *   mid[r*896 + c] = f16(silu(G_e[c].xin) * (U_e[c].xin)), e = rank-r expert,
 *   smid[c]        = f16(silu(SG[c].xin) * (SU[c].xin)),  c < 1792,
 * xin = x or rmsnorm(x, nw); ids receive the selection.  Exactly one of
 * logits (the router logits; weights receive the selection's
 * probabilities) and router_acc (the fixed-point un-normalised logits of
 * attn_out, z = logits / inv_rms(x), which order the experts) is set.  With
 * router_acc, router (the fp16 [64][1280] router) and lg_part (256 floats)
 * give the exact logits: lg_part[4e + q] = the sum over columns [320 q,
 * + 320) of router[e] times the normalised row, for uocr_launch_moe_down. */
hipError_t uocr_launch_moe_gate_up(hipStream_t st, const uocr_expert_slab *slab, uocr_qmat SG, uocr_qmat SU,
                                   const float *logits, const int64_t *router_acc, int norm_topk, const uint16_t *x,
                                   const uint16_t *nw, uint16_t *mid, uint16_t *smid, uint32_t *ids, float *weights,
                                   const uint16_t *router, float *lg_part);
/* Routed down + weighted combine + shared down + residual:
 * out[c] = f16(sum_r w_r * D_e[c].mid_r + f16(SD[c].smid) + res[c]).  The
 * weights w_r come from weights, or (lg_part non-NULL) are the softmax
 * probabilities of the exact logits sum_q lg_part[4e + q] of the selected
 * experts, also written to w_out when it is non-NULL. */
hipError_t uocr_launch_moe_down(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids,
                                const float *weights, const uint16_t *mid, uocr_qmat SD, const uint16_t *smid,
                                const uint16_t *res, uint16_t *out, const float *lg_part, float *w_out);
/* Final norm + LM-head GEMV + argmax keys (k_lm_keys): every block adds its
 * best (score, row) as a 64-bit key by atomic max into keys[block % 16]
 * (UOCR_LM_KEYS words, zero on entry); with advance, block 0 advances the
 * step state (position, KV slot, attention length, t + 1, RoPE table). */
hipError_t uocr_launch_lm_keys(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x, const uint16_t *nw,
                               uint64_t *keys, uocr_step_state *state, int advance, const float *inv_freq);
/* The selection from the keys (one wavefront): token and score at
 * tokens[state->t - 1] with advance (the keys launch advanced t), else
 * tokens[0]; state->cur_token; with E.w the token's embedding row into
 * hout.  Leaves the keys zero. */
hipError_t uocr_launch_lm_finalize(hipStream_t st, uint64_t *keys, uocr_step_state *state, int advance,
                                   int32_t *tokens, float *scores, uocr_qmat E, uint32_t vocab, uint16_t *hout);
/* Layer 0's QKV launch of a decode step with the selection folded in: the
 * token is chosen from the keys, its embedding row (E) is the activation and
 * is stored to hout (the hidden state), the token and score go to
 * tokens[state->t - 1] and state->cur_token.  The keys are left for
 * uocr_launch_attention's clear_keys. */
hipError_t uocr_launch_qkv_rope_select(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *nw,
                                       uocr_step_state *state, uint16_t *qout, uint16_t *kcache, uint16_t *vcache,
                                       uint32_t cache_capacity, const uint64_t *keys, uocr_qmat E, uint32_t vocab,
                                       int32_t *tokens, float *scores, uint16_t *hout);
/* Keys launch followed by the finalize launch (the operator API's LM head).
 * partials: UOCR_LM_PARTIAL_WORDS words, zero before the first call; every
 * call leaves them zero. */
hipError_t uocr_launch_lm_head(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x, const uint16_t *nw,
                               uint32_t *partials, uocr_step_state *state, int advance, int32_t *tokens,
                               float *scores, uocr_qmat E, uint16_t *hout, const float *inv_freq);
/* Embedding gather of tokens[0] (token == NULL: state->cur_token) -> fp16 row. */
hipError_t uocr_launch_embed(hipStream_t st, uocr_qmat E, uint32_t vocab, const int32_t *token,
                             const uocr_step_state *state, uint16_t *out);
/* Prompt rows: out[b] = embedding of ids[b] for every b with !mask[b]. */
hipError_t uocr_launch_embed_rows(hipStream_t st, uocr_qmat E, uint32_t vocab, const int32_t *ids,
                                  const uint8_t *mask, uint32_t n, uint16_t *out);
/* Replayable prefill step: copies prompt row state->t into h, sets the
 * causal-prefix plan for that position and increments state->t. */
hipError_t uocr_launch_prefill_next(hipStream_t st, uocr_step_state *state, const uint16_t *prompt, uint16_t *h,
                                    const float *inv_freq);
/* Sets *state for prompt position i (prefill through the decode kernels). */
hipError_t uocr_launch_prefill_state(hipStream_t st, uocr_step_state *state, int32_t i, const float *inv_freq);
/* Sets *state for decode with explicit (prompt_len, gen_after_write). */
hipError_t uocr_launch_decode_state(hipStream_t st, uocr_step_state *state, int32_t prompt_len, int32_t t,
                                    const float *inv_freq);

/* ---- prefill (MFMA) ------------------------------------------------------ */

#define UOCR_GEMM_F16 0    /* out = f16(acc (+ res)) */
#define UOCR_GEMM_F32 1    /* out = acc (fp32) */
#define UOCR_GEMM_SWIGLU 2 /* out = f16(silu(acc(W[0])) * acc(W[1])) */
#define UOCR_GEMM_VISION 3 /* out = f16(act(acc + bias)), optionally split into three outputs */

#ifndef UOCR_VISION_ACT_NONE
#define UOCR_VISION_ACT_NONE 0u      /* identity */
#define UOCR_VISION_ACT_QUICKGELU 1u /* x * sigmoid(1.702 x), CLIP MLP */
#define UOCR_VISION_ACT_GELU_ERF 2u  /* 0.5 x (1 + erf(x / sqrt 2)), SAM MLP */
#endif

/* C[m][n] = sum_k A[m][k] W[n][k]: fp16 activations A (row stride lda,
 * multiple of 8), weights in the .uocr layout ([N][K], K % 64 == 0).
 * Dense: rows 0..M-1 of A to rows 0..M-1 of out.  Grouped (tile_e set): a
 * device tile table (tile_e, tile_s0, tile_s1, *ntiles <= max_tiles) maps
 * launch tile i to expert tile_e[i] and slots [tile_s0[i], tile_s1[i]); slot
 * s reads A row a_idx[s] and writes out row o_idx[s]; expert e's weights are
 * at W.w + e * w_stride bytes and W.s + e * s_stride halves.  nseg != 0:
 * columns [s*nseg, (s+1)*nseg) use W[s] (nseg a multiple of 128). */
typedef struct uocr_gemm_desc {
    const uint16_t *A;
    uint32_t lda;
    const int32_t *a_idx, *o_idx;
    uint32_t M, N, K;
    uocr_qmat W[3];
    uint32_t nseg;
    uint64_t w_stride, s_stride;
    const int32_t *tile_e, *tile_s0, *tile_s1, *ntiles;
    uint32_t max_tiles;
    void *out;
    uint32_t ldo;
    const uint16_t *res;
    uint32_t ldr;
    /* UOCR_GEMM_VISION only: bias [N] (required), activation, and split: 0
     * writes out [M][ldo]; else N == 3 * split and column c goes to
     * (out, out1, out2)[c / split] at [row][c % split], row stride split */
    const uint16_t *bias;
    uint32_t act, split;
    void *out1, *out2;
    /* UOCR_GEMM_VISION, F16 and F32 (not grouped): ksplit > 1 splits K over
     * that many blocks per tile, each writing fp32 partials into part
     * ([ksplit][M][N] floats), reduced in order by a second kernel that
     * applies the epilogue; ksplit <= 1 or part NULL: no split */
    uint32_t ksplit;
    float *part;
    /* Q4/Q8 weights: W[i].w (and each expert of a slab) holds the GEMM-packed
     * copy of uocr_launch_pack_gemm_rows instead of the row-major payload */
    uint32_t packed;
    /* UOCR_GEMM_F16, not grouped, N == ldo == 1280: norm_w set also writes
     * norm_out = f16(rmsnorm(out) * norm_w) (fused into the split-K reduce) */
    const uint16_t *norm_w;
    uint16_t *norm_out;
} uocr_gemm_desc;

hipError_t uocr_launch_gemm(hipStream_t st, int epi, const uocr_gemm_desc *d);
/* Two independent GEMMs in one launch (blocks split between their tile
 * grids): A plain SwiGLU with B the fp16 router (F32), or A plain F16 with B
 * grouped SwiGLU or grouped F32 of the same qtype; neither split-K, fused
 * norm nor nseg.
 * Other pairs, or UOCR_HIP_GEMM_PAIR=0, run as two launches. */
hipError_t uocr_launch_gemm_pair(hipStream_t st, int epi_a, const uocr_gemm_desc *da, int epi_b,
                                 const uocr_gemm_desc *db);
/* GEMM-packed copy of a Q4_0 / Q8_0 payload of `rows` x K (rows % 32 == 0,
 * K % 64 == 0), `count` matrices `stride` bytes apart (an expert slab; the
 * copy keeps the stride).  Per 32-row block and 64-column step the block's
 * bytes are stored as [half h][row r][RB/2], RB = 32 (Q4) or 64 (Q8) bytes
 * per row and step, so the wavefront that owns the 32 rows reads one
 * contiguous run per step (lane 32h + r takes row r's half h). */
hipError_t uocr_launch_pack_gemm_rows(hipStream_t st, uint32_t qtype, const void *src, void *dst, uint32_t rows,
                                      uint32_t K, uint32_t count, uint64_t stride);
/* K splits (1: none) for a plain GEMM of M x N x K whose tile grid is under
 * one block per CU; UOCR_GEMM_F16 / F32 / VISION honour desc ksplit + part. */
uint32_t uocr_gemm_ksplit(uint32_t M, uint32_t N, uint32_t K);
/* y[t] = rmsnorm(x[t], w) for P rows of 1280. */
hipError_t uocr_launch_rows_rmsnorm(hipStream_t st, const uint16_t *x, const uint16_t *w, uint32_t P, uint16_t *y);
/* cs [P][64][2] = (cos, sin) of t * inv_freq[d] for tokens t < P (inv_freq:
 * 64 host floats). */
hipError_t uocr_launch_rope_table(hipStream_t st, const float *inv_freq, uint32_t P, float *cs);
/* The Q | K | V projection (d: UOCR_GEMM_F16 shape, N = 3840, nseg = 1280,
 * not grouped, M <= cap; d->out unused) with RoPE and the cache scatter as
 * its epilogue: RoPE'd q -> qout [M][1280], RoPE'd k and v -> cache slots
 * 0..M-1 ([head][cap][128]); cs is uocr_launch_rope_table's table for M. */
hipError_t uocr_launch_gemm_qkv_rope(hipStream_t st, const uocr_gemm_desc *d, const float *cs, uint16_t *qout,
                                     uint16_t *kcache, uint16_t *vcache, uint32_t cap);
/* Causal attention of P prompt queries over cache slots 0..P-1 -> ctx [P][1280]. */
hipError_t uocr_launch_flash_attn(hipStream_t st, const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                                  uint32_t cap, uint32_t P, uint16_t *ctx, float *ws);
/* Workspace of uocr_launch_flash_attn's key split (partials of up to 512
 * blocks); with ws NULL every query tile is one block (no split). */
size_t uocr_flash_attn_ws_bytes(void);
/* Per-token top-6 over logits [P][64] -> ids/wts [P][6]; expert buckets:
 * offsets (64), grouped-GEMM tile table (up to P*6/64 + 64 entries) and the
 * (token, pair) slot lists [P*6], built in LDS by one block (no global
 * counters, nothing to clear between calls, so the call can be captured
 * into a graph). */
hipError_t uocr_launch_route_rows(hipStream_t st, const float *logits, uint32_t P, int norm_topk, int32_t *ids,
                                  float *wts, int32_t *offsets, int32_t *tile_e,
                                  int32_t *tile_s0, int32_t *tile_s1, int32_t *ntiles, int32_t *list_tok,
                                  int32_t *list_pair);
/* out[t] = f16(sum_r wts[t][r] * Y[t*6+r] + shared[t] + res[t]). */
/* uocr_launch_moe_combine, then norm_out = f16(rmsnorm(out) * norm_w) of each
 * row (the next layer's input norm), in one launch. */
hipError_t uocr_launch_moe_combine_norm(hipStream_t st, const float *Y, const float *wts, const uint16_t *shared,
                                        const uint16_t *res, uint32_t P, uint16_t *out, const uint16_t *norm_w,
                                        uint16_t *norm_out);
hipError_t uocr_launch_moe_combine(hipStream_t st, const float *Y, const float *wts, const uint16_t *shared,
                                   const uint16_t *res, uint32_t P, uint16_t *out);
/* The same two with fp16 per-pair outputs Y. */
hipError_t uocr_launch_moe_combine_norm_h(hipStream_t st, const uint16_t *Y, const float *wts, const uint16_t *shared,
                                          const uint16_t *res, uint32_t P, uint16_t *out, const uint16_t *norm_w,
                                          uint16_t *norm_out);
hipError_t uocr_launch_moe_combine_h(hipStream_t st, const uint16_t *Y, const float *wts, const uint16_t *shared,
                                     const uint16_t *res, uint32_t P, uint16_t *out);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_KERNELS_H */
