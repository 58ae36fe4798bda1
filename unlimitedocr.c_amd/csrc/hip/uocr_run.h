/*
 * uocr_run.h - the persistent decode run: one launch of 256 resident workgroups that
 * carries several greedy decode steps (LM head + selection + 12 decoder
 * layers per step) through the whole GPU.
 *
 * Internal to libunlimitedocr.so.  The run replaces the per-step graph of
 * ~61 kernels (uocr_metal.m:14227-14548 op order, 8-step chunks as in
 * :11487-11576) with 256 resident workgroups, one per CU, that hand each
 * stage's outputs to the next through tagged packets in device memory:
 *   - a packet is 16 bytes, {tag, 3 payload words}, written with one
 *     device-coherent 16-byte store, so a reader that sees the current tag
 *     sees the payload written with it;
 *   - readers poll with device-coherent loads (they never hit a stale L2
 *     line) until every packet they need carries the step's tag;
 *   - every packet is written in UOCR_RUN_REPL copies and a block reads copy
 *     (its XCD) % UOCR_RUN_REPL, so no line is polled by more than the CUs of
 *     8 / UOCR_RUN_REPL XCDs (4 copies measured faster than 8, 2 or 1).
 * A block issues the weight loads of its next stage before it polls for
 * that stage's inputs, so the weights stream while the hand-off completes.
 */
#ifndef UOCR_RUN_H
#define UOCR_RUN_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "uocr_kernels.h"

#define UOCR_RUN_BLOCKS 256u  /* one workgroup per CU of an MI355X */
#define UOCR_RUN_THREADS 512u
#ifndef UOCR_RUN_REPL
#define UOCR_RUN_REPL 4u /* packet copies: XCD x polls copy x % 4 */
#endif
#define UOCR_RUN_LAYERS 12u
#define UOCR_RUN_MAX_STEPS 64u

/* Device pointers of one decoder layer (weights in the HBM arena). */
typedef struct uocr_run_layer {
    const void *q, *k, *v, *o;
    const uint16_t *qs, *ks, *vs, *os;
    const uint16_t *in_norm, *post_norm;
    const float *fold;              /* [1280][64] router * post_norm (MoE layers) */
    const float *fold_o;            /* [1280][64] O^T fold: z's weights on the attention context */
    const uint16_t *router;         /* [64][1280] fp16 router rows (exact logits for the routing weights) */
    const void *gate, *up, *down;   /* layer 0 dense SwiGLU */
    const uint16_t *gs, *us, *ds;
    const void *sg, *su, *sd;       /* shared experts (merged 1792) */
    const uint16_t *sgs, *sus, *sds;
    const void *eg, *eu, *ed;       /* routed expert slabs */
    const uint16_t *egs, *eus, *eds;
    uint64_t gu_w_stride, gu_s_stride, dn_w_stride, dn_s_stride;
} uocr_run_layer;

typedef struct uocr_run_model {
    uocr_run_layer L[UOCR_RUN_LAYERS];
    const void *lm, *emb;
    const uint16_t *lms, *embs, *final_norm;
    float invf[UOCR_K_HEAD_DIM / 2];
    uint32_t qa, qf, ql, qe;        /* qtypes: attention, FFN, LM head, embedding */
    uint64_t limit_ticks;           /* longest wait for a packet (s_memrealtime ticks, 100 MHz) */
} uocr_run_model;

/* Run-control words at the start of the packet arena. */
#define UOCR_RUN_CTL_ABORT 0u   /* nonzero once any block gave up waiting */
#define UOCR_RUN_CTL_WHERE 1u   /* stage code of the first timeout */
#define UOCR_RUN_CTL_STEP 2u
#define UOCR_RUN_CTL_BLOCK 3u

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the packet arena (control words + every stage's packets). */
uint64_t uocr_run_arena_bytes(void);
/* 1 when the model's qtype mix has a persistent-run kernel. */
int uocr_run_supported(const uocr_run_model *m);
/* Publishes the hidden state h (fp16[1280]) as layer 11's output with the
 * given tag, so a run whose first step carries tag + 1 starts from it. */
hipError_t uocr_run_seed(hipStream_t st, void *arena, const uint16_t *h, uint32_t tag);
/* out[c][e] = sum_r fold[r][e] * O[r][c] over the 1280 rows r of the O
 * projection (qtype f16, q8_0 or q4_0; fp32, summed in row order), so the
 * router's pre-norm logits are fold^T h + out^T ctx for a = h + O ctx. */
hipError_t uocr_run_fold_o(hipStream_t st, uint32_t qtype, const void *ow, const uint16_t *os, const float *fold,
                           float *out);
/* Clears the control words (abort flag). */
hipError_t uocr_run_reset(hipStream_t st, void *arena);
/* Steps t0 .. t0+n-1 of a request with prompt length P: step t selects
 * token t (tokens[t], scores[t]) from the LM head over the current hidden
 * state and, unless last and t is the final step, runs the 12 layers at
 * position P + t.  Step t0+i uses tag tag0+i.  model points to a device copy
 * of host_model.  kc/vc: [12][10][cap][128] fp16 caches.  hidden receives
 * each step's final hidden state (layer 11's output); trace (may be NULL)
 * the expert ids of layers 1-11 for steps t < trace_steps ([t][11][6]),
 * followed by their routing weights (fp32, [trace_steps][11][6]) and the
 * router inputs a (fp16, [trace_steps][11][1280]).
 * force (may be NULL): step t < force_n embeds force[t] instead of the token
 * it selects (teacher forcing for parity tests). */
hipError_t uocr_run_launch(hipStream_t st, const uocr_run_model *model, const uocr_run_model *host_model,
                           void *arena, uint16_t *kc, uint16_t *vc, uint32_t cap, int32_t P, int32_t t0, int32_t n,
                           int last, uint32_t tag0, int32_t *tokens, float *scores, uint16_t *hidden,
                           uint32_t *trace, uint32_t trace_steps, const int32_t *force, uint32_t force_n);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_RUN_H */
