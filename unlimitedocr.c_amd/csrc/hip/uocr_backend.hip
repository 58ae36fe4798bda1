/*
 * uocr_backend.hip - HIP backend: weight residency in HBM, KV cache and
 * scratch arenas, prompt assembly, prefill and the greedy decode token loop.
 *
 * Per token the decode step is one captured hipGraph:
 *   [final RMSNorm + LM-head argmax partials] -> [argmax finalize + step-state
 *   advance + embedding gather of the selected token] -> 12 x decoder layer
 * and is replayed once per generated token.  All position-dependent values
 * (position, KV slot, ring attention plan, selected token) live in device
 * memory (uocr_step_state), written by the LM-head finalize block, so the
 * graph is captured once per context.  The host reads token ids back per
 * chunk of 8 steps, one chunk behind the GPU, and stops on EOS
 * (uocr_metal.m:15248-15358 semantics, without stalling the device).
 *
 * Prompt processing (prefill) runs all P prompt rows through each layer at
 * once on MFMA GEMMs (uocr_prefill.hip): QKV GEMM -> RoPE + KV scatter ->
 * causal flash attention -> O GEMM + residual -> dense SwiGLU GEMMs (layer 0)
 * or router GEMM -> per-token top-6 -> expert buckets -> shared and
 * expert-grouped SwiGLU GEMMs -> combine.  The last row's hidden state seeds
 * the decode loop.  UOCR_GEN_TOKEN_PREFILL instead replays the decode layer
 * kernels once per prompt position (a replayable prefill graph).
 */
#include "uocr_backend.h"

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <mutex>
#include <vector>

#include "uocr_kernels.h"
#include "uocr_run.h"

#define H_SIZE 1280u
#define DECODE_CHUNK 8u

namespace {

#ifndef UOCR_PREFILL_KSPLIT_MAX
#define UOCR_PREFILL_KSPLIT_MAX 4u /* K splits (P x 1280 fp32 planes) the prefill's partial buffer holds */
#endif

struct dev_layer {
    uocr_qmat q, k, v, o, gate, up, down, sgate, sup, sdown;
    const uint16_t *in_norm, *post_norm, *router;
    const float *rfold; /* [1280][64] router * post_norm, or NULL (router kernel) */
    const float *rfold_all; /* the same fold whatever its range (the persistent run sums it in fp32) */
    const float *rfold_o;   /* [1280][64] O^T rfold_all (persistent run) */
    uocr_expert_slab slab;
    /* GEMM-packed payload copies for the MFMA prefill (Q4/Q8; NULL for fp16) */
    const void *pq, *pk, *pv, *po, *pgate, *pup, *pdown, *psg, *psu, *psd, *peg, *peu, *ped;
};

int bfail(char *err, size_t n, const char *fmt, ...) {
    if (err != nullptr && n > 0u) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(err, n, fmt, ap);
        va_end(ap);
    }
    return 0;
}

uint64_t align256(uint64_t v) {
    return (v + 255u) & ~(uint64_t)255u;
}

}  // namespace

struct uocr_hip_ctx {
    int device;
    hipStream_t stream;
    uocr_profile_state *profile;
    uocr_memory_tracker *mem;

    uint8_t *warena;
    uint64_t warena_bytes;
    int mapped;
    uocr_qmat embed, lm_head;
    const uint16_t *final_norm;
    dev_layer L[UOCR_DECODER_LAYERS];

    int runtime_ready;
    uint32_t prompt_cap, cache_cap, max_gen;
    uint8_t *rarena;
    uint64_t rarena_bytes;
    uint64_t kv_bytes, scratch_bytes, moe_bytes, logits_bytes, prompt_bytes, prefill_bytes;
    uint16_t *kc, *vc, *h, *a, *q, *ctxv, *mid, *smid, *prompt;
    float *attn_part, *logits, *route_w;
    float *lg_part; /* [4 x 64] quarters of the exact router logits (folded router) */
    int64_t *racc; /* un-normalised router logits, fixed point (k_attn_out -> k_moe_gate_up) */
    int fold_select; /* the token is chosen in layer 0's QKV launch (not a finalize launch) */
    int prefill_ksplit; /* small-grid prefill GEMMs split K */
    uint32_t *route_ids;
    /* MFMA prefill scratch, sized for prompt_cap rows */
    uint16_t *p_xn, *p_q, *p_ctx, *p_a, *p_mid, *p_smid, *p_sout, *p_rmid;
    float *p_fa_ws; /* prefill attention key-split partials */
    float *p_rope;  /* prefill RoPE (cos, sin) per token and pair */
    float *p_kpart; /* prefill GEMM split-K partials */
    float *p_logits, *p_wts;
    uint16_t *p_y; /* per-pair routed expert outputs, fp16 */
    int32_t *p_ids, *p_offsets, *p_tile_e, *p_tile_s0, *p_tile_s1, *p_ntiles, *p_list_tok,
        *p_list_pair;
    uint32_t p_max_tiles;
    uint32_t *lm_part;
    uocr_step_state *state;
    int32_t *tokens;
    float *scores;
    int32_t *d_ids;
    uint8_t *d_mask;
    int32_t *h_tokens;
    float *h_scores;
    uint16_t *h_prompt;

    float invf[UOCR_K_HEAD_DIM / 2];
    hipGraphExec_t g_decode, g_decode_chunk, g_prefill; /* one step, DECODE_CHUNK steps, one prompt position */
    int graphs_ready;
    /* MFMA prefill of one prompt length, captured when the same length comes
     * twice in a row (its grids depend on the length) */
    hipGraphExec_t g_mfma;
    uint32_t g_mfma_P, last_mfma_P, cap_P;
    /* persistent decode run (uocr_decode_run.hip) */
    uocr_run_model run_model;
    uocr_run_model *d_run_model; /* device copy, in the weight arena */
    int run_ok;                  /* the model, device and environment allow the run */
    int last_path;               /* decode path of the last generation (uocr_hip_context_decode_path) */
    int run_aborted;             /* the last decode_run ended on a run timeout */
    uint8_t *run_arena;          /* packet arena, in the runtime arena */
    uint32_t run_tag;            /* next unused packet tag */
    /* hot-path allocation guard (uocr_metal.m:8447-8486): every device and
     * pinned allocation of the backend is counted */
    uint64_t alloc_count, alloc_bytes;
    int fault_alloc;             /* test hook (UOCR_HIP_FAULT_ALLOC): 1 prefill, 2 decode */
    /* opt-in per-op decode timing (UOCR_HIP_DECODER_PROFILE_DETAIL >= 3 with
     * profiling on): event pairs around every decode launch */
    int profile_detail;
    int run_events;              /* UOCR_HIP_RUN_EVENTS=1: time each persistent-run launch (profiling on) */
    struct op_timer *tm;         /* active only inside the timed decode loop */
    /* decode trace (uocr_hip_context_trace_enable) */
    uint32_t trace_steps;
    uint32_t *d_trace;           /* [trace_steps][11][6] expert ids, as many fp32 routing weights, then the
                                  * router inputs a (fp16 [trace_steps][11][1280]) */
    int32_t trace_step;          /* step being enqueued by the eager loop (-1: none) */
    int32_t *d_force;            /* teacher-forced token ids (uocr_hip_context_trace_force) */
    uint32_t force_n;
};

#define OP_TIMER_MAX 96
struct op_timer {
    hipEvent_t ev[2 * OP_TIMER_MAX];
    const char *name[OP_TIMER_MAX];
    const char *kname[OP_TIMER_MAX]; /* the launch's kernel (hip.kernel.*), or NULL */
    int layer_first[UOCR_DECODER_LAYERS], layer_last[UOCR_DECODER_LAYERS];
    int n;
};

/* Persistent runs need every CU of the device: runs of different engines in
 * one process are serialised. */
static std::mutex g_run_mutex;

#define HIPCHK(expr, what)                                                                        \
    do {                                                                                          \
        const hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess) return bfail(err, err_size, "%s: %s", (what), hipGetErrorString(e_)); \
    } while (0)

/* Counted allocations: the hot-path guard compares the counts. */
static hipError_t counted_malloc(uocr_hip_ctx *c, void **p, size_t bytes) {
    const hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) {
        ++c->alloc_count;
        c->alloc_bytes += bytes;
    }
    return e;
}

static hipError_t counted_host_malloc(uocr_hip_ctx *c, void **p, size_t bytes) {
    const hipError_t e = hipHostMalloc(p, bytes, hipHostMallocDefault);
    if (e == hipSuccess) {
        ++c->alloc_count;
        c->alloc_bytes += bytes;
    }
    return e;
}

/* Hot-path allocation guard: generation fails when prefill or the decode
 * loop allocated device or pinned memory, or the arenas changed size. */
struct alloc_guard {
    uint64_t count, bytes, warena, rarena;
};

static alloc_guard guard_begin(const uocr_hip_ctx *c) {
    return alloc_guard{c->alloc_count, c->alloc_bytes, c->warena_bytes, c->rarena_bytes};
}

static int guard_end(const uocr_hip_ctx *c, const alloc_guard &g, const char *label, char *err, size_t err_size) {
    if (c->alloc_count != g.count || c->warena_bytes != g.warena || c->rarena_bytes != g.rarena) {
        return bfail(err, err_size, "%s allocated device memory (%llu allocation(s), %llu bytes)", label,
                     (unsigned long long)(c->alloc_count - g.count), (unsigned long long)(c->alloc_bytes - g.bytes));
    }
    return 1;
}

/* UOCR_HIP_FAULT_ALLOC test hook: one counted 256-byte allocation inside the
 * guarded region (freed at once), so tests can see the guard fail a request. */
static void fault_alloc(uocr_hip_ctx *c, int where) {
    if (c->fault_alloc != where) return;
    void *p = nullptr;
    if (counted_malloc(c, &p, 256u) == hipSuccess) (void)hipFree(p);
}

extern "C" int uocr_hip_is_available(char *why, size_t why_size) {
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) {
        if (why != nullptr && why_size > 0u) {
            snprintf(why, why_size, "no HIP device is available (%s)", e != hipSuccess ? hipGetErrorString(e) : "0 devices");
        }
        return 0;
    }
    return 1;
}

extern "C" uocr_hip_ctx *uocr_hip_context_create(char *err, size_t err_size) {
    if (!uocr_hip_is_available(err, err_size)) return nullptr;
    uocr_hip_ctx *ctx = (uocr_hip_ctx *)calloc(1, sizeof(uocr_hip_ctx));
    if (ctx == nullptr) {
        bfail(err, err_size, "failed to allocate HIP context");
        return nullptr;
    }
    const char *dev = getenv("UOCR_HIP_DEVICE");
    ctx->device = dev != nullptr ? atoi(dev) : 0;
    if (hipSetDevice(ctx->device) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        bfail(err, err_size, "failed to initialise HIP device %d", ctx->device);
        free(ctx);
        return nullptr;
    }
    /* inv_freq[d] = 2^(d * (-2 log2(theta) / head_dim)), golden.py:410-414 */
    ctx->trace_step = -1;
    ctx->last_path = -1;
    const char *re = getenv("UOCR_HIP_RUN_EVENTS");
    ctx->run_events = re != nullptr && atoi(re) != 0;
    const char *pd = getenv("UOCR_HIP_DECODER_PROFILE_DETAIL");
    ctx->profile_detail = pd != nullptr ? atoi(pd) : 0;
    const char *fa = getenv("UOCR_HIP_FAULT_ALLOC");
    ctx->fault_alloc = fa == nullptr ? 0 : (strcmp(fa, "prefill") == 0 ? 1 : (strcmp(fa, "decode") == 0 ? 2 : 0));
    const float freq_scale = -2.0f * log2f((float)UOCR_ROPE_THETA) / (float)UOCR_HEAD_DIM;
    for (int d = 0; d < UOCR_K_HEAD_DIM / 2; ++d) ctx->invf[d] = exp2f((float)d * freq_scale);
    return ctx;
}

static void release_graphs(uocr_hip_ctx *ctx) {
    if (ctx->g_mfma != nullptr) {
        (void)hipGraphExecDestroy(ctx->g_mfma);
        ctx->g_mfma = nullptr;
    }
    ctx->g_mfma_P = ctx->last_mfma_P = 0u;
    if (ctx->graphs_ready) {
        (void)hipGraphExecDestroy(ctx->g_decode);
        (void)hipGraphExecDestroy(ctx->g_decode_chunk);
        (void)hipGraphExecDestroy(ctx->g_prefill);
        ctx->graphs_ready = 0;
    }
}

static void release_runtime(uocr_hip_ctx *ctx) {
    release_graphs(ctx);
    if (ctx->rarena != nullptr) {
        (void)hipFree(ctx->rarena);
        if (ctx->mem != nullptr) {
            uocr_memory_release(ctx->mem, UOCR_MEMORY_KV_CACHE, ctx->kv_bytes);
            uocr_memory_release(ctx->mem, UOCR_MEMORY_DECODER_SCRATCH, ctx->scratch_bytes);
            uocr_memory_release(ctx->mem, UOCR_MEMORY_MOE_SCRATCH, ctx->moe_bytes);
            uocr_memory_release(ctx->mem, UOCR_MEMORY_LOGITS_READBACK, ctx->logits_bytes);
            uocr_memory_release(ctx->mem, UOCR_MEMORY_PROMPT_EMBEDDINGS, ctx->prompt_bytes);
        }
    }
    if (ctx->h_tokens != nullptr) (void)hipHostFree(ctx->h_tokens);
    if (ctx->h_scores != nullptr) (void)hipHostFree(ctx->h_scores);
    if (ctx->h_prompt != nullptr) (void)hipHostFree(ctx->h_prompt);
    ctx->rarena = nullptr;
    ctx->h_tokens = nullptr;
    ctx->h_scores = nullptr;
    ctx->h_prompt = nullptr;
    ctx->runtime_ready = 0;
}

extern "C" void uocr_hip_context_destroy(uocr_hip_ctx *ctx) {
    if (ctx == nullptr) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    release_runtime(ctx);
    if (ctx->warena != nullptr) (void)hipFree(ctx->warena);
    if (ctx->d_trace != nullptr) (void)hipFree(ctx->d_trace);
    if (ctx->d_force != nullptr) (void)hipFree(ctx->d_force);
    (void)hipStreamDestroy(ctx->stream);
    free(ctx);
}

extern "C" void uocr_hip_context_set_profile(uocr_hip_ctx *ctx, uocr_profile_state *profile) {
    if (ctx != nullptr) ctx->profile = profile;
}

extern "C" void uocr_hip_context_set_memory_tracker(uocr_hip_ctx *ctx, uocr_memory_tracker *tracker) {
    if (ctx != nullptr) ctx->mem = tracker;
}

extern "C" uint64_t uocr_hip_context_weight_bytes(const uocr_hip_ctx *ctx) {
    return ctx != nullptr ? ctx->warena_bytes : 0u;
}

/* ---- weight residency ---------------------------------------------------- */

namespace {

struct placer {
    uint64_t off = 0;
    uint64_t take(uint64_t bytes) {
        const uint64_t at = off;
        off = align256(off + bytes);
        return at;
    }
};

uint64_t tensor_bytes(const uocr_bound_tensor &t) {
    return align256(t.w_bytes) + align256(t.s_bytes);
}

}  // namespace

static int upload(uocr_hip_ctx *ctx, placer &p, const uocr_bound_tensor &t, uocr_qmat *out, char *err, size_t err_size) {
    const uint64_t wo = p.take(t.w_bytes);
    HIPCHK(hipMemcpy(ctx->warena + wo, t.w, t.w_bytes, hipMemcpyHostToDevice), "weight upload");
    out->w = ctx->warena + wo;
    out->qtype = t.qtype;
    out->s = nullptr;
    if (t.s != nullptr) {
        const uint64_t so = p.take(t.s_bytes);
        HIPCHK(hipMemcpy(ctx->warena + so, t.s, t.s_bytes, hipMemcpyHostToDevice), "scale upload");
        out->s = (const uint16_t *)(ctx->warena + so);
    }
    return 1;
}

/* The router folded into the post-attention norm weight, transposed:
 * fold[i][e] = R[e][i] * nw[i] (exact in fp32: a product of two fp16
 * values).  The O-projection kernel accumulates z[e] = sum_i fold[i][e] *
 * a[i] in int64 fixed point (2^32 units), so the fold is used only when no
 * sum can leave that range: max_e sum_i |fold[i][e]| * 65504 (the largest
 * fp16 magnitude of a[i]) < 2^31.  Otherwise *out stays NULL and the layer
 * keeps the separate router kernel. */
static int upload_router_fold(uocr_hip_ctx *ctx, placer &p, const uocr_bound_tensor &R, const uocr_bound_tensor &nw,
                              const float **out, const float **all, char *err, size_t err_size) {
    constexpr uint32_t E = UOCR_ROUTED_EXPERTS;
    *out = nullptr;
    *all = nullptr;
    const uint64_t bytes = (uint64_t)H_SIZE * E * 4u;
    const uint64_t off = p.take(bytes);
    if (R.qtype != UOCR_QT_F16 || R.w_bytes < (uint64_t)E * H_SIZE * 2u || nw.w_bytes < (uint64_t)H_SIZE * 2u) {
        return 1;
    }
    const _Float16 *r = (const _Float16 *)R.w, *w = (const _Float16 *)nw.w;
    std::vector<float> fold((size_t)H_SIZE * E);
    double worst = 0.0;
    for (uint32_t e = 0; e < E; ++e) {
        double tot = 0.0;
        for (uint32_t i = 0; i < H_SIZE; ++i) {
            const float f = (float)r[(size_t)e * H_SIZE + i] * (float)w[i];
            fold[(size_t)i * E + e] = f;
            tot += fabs((double)f);
        }
        worst = tot > worst ? tot : worst;
    }
    HIPCHK(hipMemcpy(ctx->warena + off, fold.data(), bytes, hipMemcpyHostToDevice), "router fold upload");
    *all = (const float *)(ctx->warena + off);
    if (worst * 65504.0 < 2147483648.0) *out = *all;
    return 1;
}

/* Uploads one projection of all 64 experts into an evenly strided slab. */
static int upload_slab(uocr_hip_ctx *ctx, placer &p, const uocr_bound_tensor *ex, uocr_qmat *out, uint64_t *w_stride,
                       uint64_t *s_stride, char *err, size_t err_size) {
    const uint64_t ws = align256(ex[0].w_bytes);
    const uint64_t ss = align256(ex[0].s_bytes);
    const uint64_t wo = p.take(ws * UOCR_ROUTED_EXPERTS);
    const uint64_t so = ex[0].s != nullptr ? p.take(ss * UOCR_ROUTED_EXPERTS) : 0u;
    for (uint32_t e = 0; e < UOCR_ROUTED_EXPERTS; ++e) {
        HIPCHK(hipMemcpy(ctx->warena + wo + e * ws, ex[e].w, ex[e].w_bytes, hipMemcpyHostToDevice), "expert upload");
        if (ex[e].s != nullptr) {
            HIPCHK(hipMemcpy(ctx->warena + so + e * ss, ex[e].s, ex[e].s_bytes, hipMemcpyHostToDevice), "expert scale upload");
        }
    }
    out->w = ctx->warena + wo;
    out->s = ex[0].s != nullptr ? (const uint16_t *)(ctx->warena + so) : nullptr;
    out->qtype = ex[0].qtype;
    *w_stride = ws;
    *s_stride = ss / 2u;
    return 1;
}

/* The persistent decode run's view of the model (device pointers of every
 * layer) and whether this model, device and environment can use it:
 * it is the default decode wherever it is supported (config 5: Q4 3,873
 * against about 3,500 tok/s for the per-step graphs, Q8 3,178 against
 * 3,102); UOCR_HIP_RUN=1 / 0 forces either.  The run needs Q8 attention with
 * Q4 or Q8 everywhere else (fp16 weights keep the graphs), fp16 routers (for
 * the fold) and 256 CUs. */
static int setup_run(uocr_hip_ctx *ctx, char *err, size_t err_size) {
    uocr_run_model &m = ctx->run_model;
    memset(&m, 0, sizeof(m));
    bool ok = true;
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const dev_layer &D = ctx->L[l];
        uocr_run_layer &R = m.L[l];
        R.q = D.q.w;
        R.k = D.k.w;
        R.v = D.v.w;
        R.o = D.o.w;
        R.qs = D.q.s;
        R.ks = D.k.s;
        R.vs = D.v.s;
        R.os = D.o.s;
        R.in_norm = D.in_norm;
        R.post_norm = D.post_norm;
        ok = ok && D.q.qtype == D.k.qtype && D.q.qtype == D.v.qtype && D.q.qtype == D.o.qtype;
        if (l == 0u) {
            R.gate = D.gate.w;
            R.up = D.up.w;
            R.down = D.down.w;
            R.gs = D.gate.s;
            R.us = D.up.s;
            R.ds = D.down.s;
            ok = ok && D.gate.qtype == D.up.qtype && D.gate.qtype == D.down.qtype;
            m.qf = D.gate.qtype;
        } else {
            R.fold = D.rfold_all;
            R.fold_o = D.rfold_o;
            R.router = D.router;
            if (R.fold != nullptr && R.fold_o != nullptr) {
                HIPCHK(uocr_run_fold_o(nullptr, D.o.qtype, D.o.w, D.o.s, R.fold, (float *)R.fold_o), "router fold_o");
            }
            R.sg = D.sgate.w;
            R.su = D.sup.w;
            R.sd = D.sdown.w;
            R.sgs = D.sgate.s;
            R.sus = D.sup.s;
            R.sds = D.sdown.s;
            R.eg = D.slab.gate.w;
            R.eu = D.slab.up.w;
            R.ed = D.slab.down.w;
            R.egs = D.slab.gate.s;
            R.eus = D.slab.up.s;
            R.eds = D.slab.down.s;
            R.gu_w_stride = D.slab.gu_w_stride;
            R.gu_s_stride = D.slab.gu_s_stride;
            R.dn_w_stride = D.slab.dn_w_stride;
            R.dn_s_stride = D.slab.dn_s_stride;
            ok = ok && R.fold != nullptr && R.fold_o != nullptr && R.router != nullptr;
            for (const uocr_qmat *q : {&D.sgate, &D.sup, &D.sdown, &D.slab.gate, &D.slab.up, &D.slab.down}) {
                ok = ok && q->qtype == ctx->L[0].gate.qtype;
            }
        }
        ok = ok && D.q.qtype == ctx->L[0].q.qtype;
    }
    m.qa = ctx->L[0].q.qtype;
    m.lm = ctx->lm_head.w;
    m.lms = ctx->lm_head.s;
    m.emb = ctx->embed.w;
    m.embs = ctx->embed.s;
    m.final_norm = ctx->final_norm;
    m.ql = ctx->lm_head.qtype;
    m.qe = ctx->embed.qtype;
    memcpy(m.invf, ctx->invf, sizeof(m.invf));
    /* UOCR_HIP_RUN_LIMIT_US: the longest a run workgroup waits for a packet
     * before the run gives up (default 50 ms; the request is then served
     * again on the per-step kernels) */
    const char *lu = getenv("UOCR_HIP_RUN_LIMIT_US");
    m.limit_ticks = (lu != nullptr ? strtoull(lu, nullptr, 10) : 50000ull) * 100ull;
    HIPCHK(hipMemcpy(ctx->d_run_model, &m, sizeof(m), hipMemcpyHostToDevice), "run model upload");
    int cus = 0;
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device);
    const char *ru = getenv("UOCR_HIP_RUN");
    const bool want = ru != nullptr ? atoi(ru) != 0 : true;
    const bool can = ok && uocr_run_supported(&m) && cus == (int)UOCR_RUN_BLOCKS;
    /* UOCR_HIP_RUN=1 forces the run: a model or device without it fails the
     * mapping instead of decoding on the per-step kernels */
    if (ru != nullptr && want && !can) {
        return bfail(err, err_size,
                     "UOCR_HIP_RUN=1 but the persistent decode run is unavailable (%s)",
                     !uocr_run_supported(&m) ? "qtype mix has no run kernel"
                                             : "device CU count is not 256");
    }
    ctx->run_ok = can && want;
    return 1;
}

extern "C" int uocr_hip_context_map_model(uocr_hip_ctx *ctx, const uocr_decoder_bindings *b, char *err, size_t err_size) {
    if (ctx == nullptr || b == nullptr) return bfail(err, err_size, "invalid map_model request");
    HIPCHK(hipSetDevice(ctx->device), "hipSetDevice");
    if (ctx->warena != nullptr) {
        (void)hipFree(ctx->warena);
        ctx->warena = nullptr;
        ctx->mapped = 0;
        release_graphs(ctx);
    }
    /* UOCR_HIP_NO_ROUTER_FOLD=1 keeps the separate router kernel in every layer */
    const char *nf = getenv("UOCR_HIP_NO_ROUTER_FOLD");
    const bool no_fold = nf != nullptr && atoi(nf) != 0;
    /* UOCR_HIP_NO_SELECT_FOLD=1 chooses each token in a finalize launch after the LM head */
    const char *ns = getenv("UOCR_HIP_NO_SELECT_FOLD");
    ctx->fold_select = !(ns != nullptr && atoi(ns) != 0);
    /* UOCR_HIP_NO_PREFILL_KSPLIT=1 runs every prefill GEMM unsplit */
    const char *nk = getenv("UOCR_HIP_NO_PREFILL_KSPLIT");
    ctx->prefill_ksplit = !(nk != nullptr && atoi(nk) != 0);
    /* size pass */
    uint64_t total = tensor_bytes(b->embed) + tensor_bytes(b->lm_head) + tensor_bytes(b->final_norm);
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const uocr_bound_layer &L = b->layers[l];
        total += tensor_bytes(L.in_norm) + tensor_bytes(L.post_norm) + tensor_bytes(L.q) + tensor_bytes(L.k) +
                 tensor_bytes(L.v) + tensor_bytes(L.o);
        if (l == 0u) {
            total += tensor_bytes(L.gate) + tensor_bytes(L.up) + tensor_bytes(L.down);
        } else {
            total += tensor_bytes(L.router) + tensor_bytes(L.sgate) + tensor_bytes(L.sup) + tensor_bytes(L.sdown);
            total += UOCR_ROUTED_EXPERTS * (tensor_bytes(L.egate[0]) + tensor_bytes(L.eup[0]) + tensor_bytes(L.edown[0]));
            total += 2u * align256((uint64_t)H_SIZE * UOCR_ROUTED_EXPERTS * 4u); /* fold, fold_o */
        }
    }
    /* GEMM-packed copies of the Q4/Q8 layer payloads (MFMA prefill) */
    auto packed_bytes = [](const uocr_bound_tensor &t, uint64_t count) -> uint64_t {
        return t.qtype == UOCR_QT_F16 ? 0u : count * align256(t.w_bytes);
    };
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const uocr_bound_layer &L = b->layers[l];
        total += packed_bytes(L.q, 1) + packed_bytes(L.k, 1) + packed_bytes(L.v, 1) + packed_bytes(L.o, 1);
        if (l == 0u) {
            total += packed_bytes(L.gate, 1) + packed_bytes(L.up, 1) + packed_bytes(L.down, 1);
        } else {
            total += packed_bytes(L.sgate, 1) + packed_bytes(L.sup, 1) + packed_bytes(L.sdown, 1);
            total += packed_bytes(L.egate[0], UOCR_ROUTED_EXPERTS) + packed_bytes(L.eup[0], UOCR_ROUTED_EXPERTS) +
                     packed_bytes(L.edown[0], UOCR_ROUTED_EXPERTS);
        }
    }
    const uint64_t run_model_off = total;
    total += align256(sizeof(uocr_run_model));
    HIPCHK(counted_malloc(ctx, (void **)&ctx->warena, total), "weight arena allocation");
    ctx->warena_bytes = total;
    placer p;
    uocr_qmat fn;
    if (!upload(ctx, p, b->embed, &ctx->embed, err, err_size) || !upload(ctx, p, b->lm_head, &ctx->lm_head, err, err_size) ||
        !upload(ctx, p, b->final_norm, &fn, err, err_size)) {
        return 0;
    }
    ctx->final_norm = (const uint16_t *)fn.w;
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const uocr_bound_layer &S = b->layers[l];
        dev_layer &D = ctx->L[l];
        memset(&D, 0, sizeof(D));
        uocr_qmat n1, n2;
        if (!upload(ctx, p, S.in_norm, &n1, err, err_size) || !upload(ctx, p, S.post_norm, &n2, err, err_size) ||
            !upload(ctx, p, S.q, &D.q, err, err_size) || !upload(ctx, p, S.k, &D.k, err, err_size) ||
            !upload(ctx, p, S.v, &D.v, err, err_size) || !upload(ctx, p, S.o, &D.o, err, err_size)) {
            return 0;
        }
        D.in_norm = (const uint16_t *)n1.w;
        D.post_norm = (const uint16_t *)n2.w;
        if (l == 0u) {
            if (!upload(ctx, p, S.gate, &D.gate, err, err_size) || !upload(ctx, p, S.up, &D.up, err, err_size) ||
                !upload(ctx, p, S.down, &D.down, err, err_size)) {
                return 0;
            }
            continue;
        }
        uocr_qmat r;
        if (!upload(ctx, p, S.router, &r, err, err_size) || !upload(ctx, p, S.sgate, &D.sgate, err, err_size) ||
            !upload(ctx, p, S.sup, &D.sup, err, err_size) || !upload(ctx, p, S.sdown, &D.sdown, err, err_size)) {
            return 0;
        }
        D.router = (const uint16_t *)r.w;
        if (!upload_router_fold(ctx, p, S.router, S.post_norm, &D.rfold, &D.rfold_all, err, err_size)) return 0;
        if (no_fold) D.rfold = nullptr;
        uocr_expert_slab &sl = D.slab;
        uint64_t ws2, ss2;
        if (!upload_slab(ctx, p, S.egate, &sl.gate, &sl.gu_w_stride, &sl.gu_s_stride, err, err_size) ||
            !upload_slab(ctx, p, S.eup, &sl.up, &ws2, &ss2, err, err_size) ||
            !upload_slab(ctx, p, S.edown, &sl.down, &sl.dn_w_stride, &sl.dn_s_stride, err, err_size)) {
            return 0;
        }
        if (ws2 != sl.gu_w_stride || ss2 != sl.gu_s_stride) return bfail(err, err_size, "expert gate/up slabs differ in stride");
    }
    for (uint32_t l = 1; l < UOCR_DECODER_LAYERS; ++l) {
        ctx->L[l].rfold_o = (const float *)(ctx->warena + p.take((uint64_t)H_SIZE * UOCR_ROUTED_EXPERTS * 4u));
    }
    /* GEMM-packed copies: rows x K per matrix, experts at the slab stride.
     * Each copy's range is checked against the arena before its kernel
     * writes it; a failed check or launch fails the mapping (pack_bad). */
    const char *pack_bad = nullptr;
    auto pack = [&](const uocr_qmat &m, uint32_t rows, uint32_t K, uint32_t count, uint64_t stride,
                    uint64_t bytes) -> const void * {
        if (m.qtype == UOCR_QT_F16 || pack_bad != nullptr) return nullptr;
        const uint64_t need = count == 1u ? align256(bytes) : count * stride;
        if (p.off + need > run_model_off) {
            pack_bad = "weight arena overflow (GEMM-packed copies)";
            return nullptr;
        }
        uint8_t *dst = ctx->warena + p.take(need);
        if (uocr_launch_pack_gemm_rows(nullptr, m.qtype, m.w, dst, rows, K, count, count == 1u ? 0u : stride) !=
            hipSuccess) {
            pack_bad = "GEMM weight packing launch failed";
            return nullptr;
        }
        return dst;
    };
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        dev_layer &D = ctx->L[l];
        const uocr_bound_layer &S = b->layers[l];
        const uint32_t H = H_SIZE, I0 = UOCR_DENSE_LAYER0_INTERMEDIATE, SI = UOCR_MOE_SHARED_INTERMEDIATE,
                       EI = UOCR_MOE_EXPERT_INTERMEDIATE;
        D.pq = pack(D.q, H, H, 1, 0, S.q.w_bytes);
        D.pk = pack(D.k, H, H, 1, 0, S.k.w_bytes);
        D.pv = pack(D.v, H, H, 1, 0, S.v.w_bytes);
        D.po = pack(D.o, H, H, 1, 0, S.o.w_bytes);
        if (l == 0u) {
            D.pgate = pack(D.gate, I0, H, 1, 0, S.gate.w_bytes);
            D.pup = pack(D.up, I0, H, 1, 0, S.up.w_bytes);
            D.pdown = pack(D.down, H, I0, 1, 0, S.down.w_bytes);
            continue;
        }
        D.psg = pack(D.sgate, SI, H, 1, 0, S.sgate.w_bytes);
        D.psu = pack(D.sup, SI, H, 1, 0, S.sup.w_bytes);
        D.psd = pack(D.sdown, H, SI, 1, 0, S.sdown.w_bytes);
        D.peg = pack(D.slab.gate, EI, H, UOCR_ROUTED_EXPERTS, D.slab.gu_w_stride, 0);
        D.peu = pack(D.slab.up, EI, H, UOCR_ROUTED_EXPERTS, D.slab.gu_w_stride, 0);
        D.ped = pack(D.slab.down, H, EI, UOCR_ROUTED_EXPERTS, D.slab.dn_w_stride, 0);
    }
    if (pack_bad != nullptr) return bfail(err, err_size, "%s", pack_bad);
    HIPCHK(hipGetLastError(), "GEMM weight packing");
    if (p.off > run_model_off) return bfail(err, err_size, "weight arena overflow");
    ctx->d_run_model = (uocr_run_model *)(ctx->warena + run_model_off);
    if (!setup_run(ctx, err, err_size)) return 0;
    /* the uploads ran on the null stream; the engine's stream is non-blocking,
     * so wait for them before any kernel can read the weights */
    HIPCHK(hipDeviceSynchronize(), "weight upload sync");
    ctx->mapped = 1;
    return 1;
}

/* ---- runtime arenas ------------------------------------------------------- */

extern "C" int uocr_hip_context_allocate_runtime(uocr_hip_ctx *ctx, uint32_t prompt_capacity, uint32_t max_gen,
                                                 char *err, size_t err_size) {
    if (ctx == nullptr || prompt_capacity == 0u || max_gen == 0u) return bfail(err, err_size, "invalid runtime arena request");
    if (ctx->runtime_ready && prompt_capacity <= ctx->prompt_cap && max_gen <= ctx->max_gen) return 1;
    HIPCHK(hipSetDevice(ctx->device), "hipSetDevice");
    HIPCHK(hipStreamSynchronize(ctx->stream), "stream sync");
    release_runtime(ctx);
    const uint32_t cap = prompt_capacity + UOCR_GENERATED_RING_WINDOW;
    const uint64_t kv_one = (uint64_t)UOCR_DECODER_LAYERS * UOCR_ATTENTION_HEADS * cap * UOCR_HEAD_DIM * 2u;
    placer p;
    const uint64_t o_kc = p.take(kv_one), o_vc = p.take(kv_one);
    const uint64_t o_h = p.take(H_SIZE * 2u), o_a = p.take(H_SIZE * 2u), o_q = p.take(H_SIZE * 2u), o_c = p.take(H_SIZE * 2u);
    const uint64_t o_state = p.take(sizeof(uocr_step_state));
    const uint64_t o_apart = p.take(UOCR_ATTN_PARTIAL_FLOATS * 4u), o_logits = p.take(64u * 4u);
    const uint64_t o_lgpart = p.take(4u * 64u * 4u);
    const uint64_t o_rids = p.take(64u), o_rwts = p.take(64u), o_racc = p.take(UOCR_ROUTER_ACC_WORDS * 8u);
    const uint64_t scratch_end = p.off;
    const uint64_t o_mid = p.take(UOCR_DENSE_LAYER0_INTERMEDIATE * 2u), o_smid = p.take(UOCR_MOE_SHARED_INTERMEDIATE * 2u);
    const uint64_t moe_end = p.off;
    const uint64_t o_lpart = p.take(UOCR_LM_PARTIAL_WORDS * 4u);
    const uint64_t o_tok = p.take((uint64_t)max_gen * 4u), o_sc = p.take((uint64_t)max_gen * 4u);
    const uint64_t logits_end = p.off;
    const uint64_t o_prompt = p.take((uint64_t)prompt_capacity * H_SIZE * 2u);
    const uint64_t o_dids = p.take((uint64_t)prompt_capacity * 4u), o_dmask = p.take(prompt_capacity);
    const uint64_t prompt_end = p.off;
    const uint64_t Pc = prompt_capacity, PK = Pc * UOCR_MOE_TOP_K;
    const uint32_t max_tiles = (uint32_t)((PK + 63u) / 64u + UOCR_ROUTED_EXPERTS);
    const uint64_t o_pxn = p.take(Pc * H_SIZE * 2u), o_prope = p.take(Pc * 64u * 8u);
    const uint64_t o_pq = p.take(Pc * H_SIZE * 2u), o_pctx = p.take(Pc * H_SIZE * 2u), o_pa = p.take(Pc * H_SIZE * 2u);
    const uint64_t o_pmid = p.take(Pc * UOCR_DENSE_LAYER0_INTERMEDIATE * 2u);
    const uint64_t o_psmid = p.take(Pc * UOCR_MOE_SHARED_INTERMEDIATE * 2u), o_psout = p.take(Pc * H_SIZE * 2u);
    const uint64_t o_prmid = p.take(PK * UOCR_MOE_EXPERT_INTERMEDIATE * 2u);
    const uint64_t o_plog = p.take(Pc * UOCR_ROUTED_EXPERTS * 4u), o_pwts = p.take(PK * 4u);
    const uint64_t o_py = p.take(PK * H_SIZE * 2u), o_pids = p.take(PK * 4u);
    const uint64_t o_poff = p.take(64u * 4u);
    const uint64_t o_pte = p.take(max_tiles * 4u), o_pts0 = p.take(max_tiles * 4u), o_pts1 = p.take(max_tiles * 4u);
    const uint64_t o_pnt = p.take(4u), o_plt = p.take(PK * 4u), o_plp = p.take(PK * 4u);
    const uint64_t o_pfa = p.take(uocr_flash_attn_ws_bytes());
    /* split-K partials of the O projection and the dense down (UOCR_PREFILL_KSPLIT_MAX splits x
     * P x 1280, fp32) */
    const uint64_t o_pkp = p.take(Pc * H_SIZE * UOCR_PREFILL_KSPLIT_MAX * 4u);
    const uint64_t o_run = p.take(uocr_run_arena_bytes());
    const uint64_t total = p.off;
    HIPCHK(counted_malloc(ctx, (void **)&ctx->rarena, total), "runtime arena allocation");
    /* cleared on the engine's stream (non-blocking, so not ordered against a
     * null-stream hipMemset) and waited for */
    HIPCHK(hipMemsetAsync(ctx->rarena, 0, total, ctx->stream), "runtime arena clear");
    HIPCHK(hipStreamSynchronize(ctx->stream), "runtime arena clear sync");
    uint8_t *b = ctx->rarena;
    ctx->kc = (uint16_t *)(b + o_kc);
    ctx->vc = (uint16_t *)(b + o_vc);
    ctx->h = (uint16_t *)(b + o_h);
    ctx->a = (uint16_t *)(b + o_a);
    ctx->q = (uint16_t *)(b + o_q);
    ctx->ctxv = (uint16_t *)(b + o_c);
    ctx->state = (uocr_step_state *)(b + o_state);
    ctx->attn_part = (float *)(b + o_apart);
    ctx->logits = (float *)(b + o_logits);
    ctx->lg_part = (float *)(b + o_lgpart);
    ctx->route_ids = (uint32_t *)(b + o_rids);
    ctx->route_w = (float *)(b + o_rwts);
    ctx->racc = (int64_t *)(b + o_racc);
    ctx->mid = (uint16_t *)(b + o_mid);
    ctx->smid = (uint16_t *)(b + o_smid);
    ctx->lm_part = (uint32_t *)(b + o_lpart);
    ctx->tokens = (int32_t *)(b + o_tok);
    ctx->scores = (float *)(b + o_sc);
    ctx->prompt = (uint16_t *)(b + o_prompt);
    ctx->d_ids = (int32_t *)(b + o_dids);
    ctx->d_mask = (uint8_t *)(b + o_dmask);
    ctx->p_xn = (uint16_t *)(b + o_pxn);
    ctx->p_q = (uint16_t *)(b + o_pq);
    ctx->p_ctx = (uint16_t *)(b + o_pctx);
    ctx->p_a = (uint16_t *)(b + o_pa);
    ctx->p_mid = (uint16_t *)(b + o_pmid);
    ctx->p_smid = (uint16_t *)(b + o_psmid);
    ctx->p_sout = (uint16_t *)(b + o_psout);
    ctx->p_rmid = (uint16_t *)(b + o_prmid);
    ctx->p_logits = (float *)(b + o_plog);
    ctx->p_wts = (float *)(b + o_pwts);
    ctx->p_y = (uint16_t *)(b + o_py);
    ctx->p_ids = (int32_t *)(b + o_pids);
    ctx->p_offsets = (int32_t *)(b + o_poff);
    ctx->p_tile_e = (int32_t *)(b + o_pte);
    ctx->p_tile_s0 = (int32_t *)(b + o_pts0);
    ctx->p_tile_s1 = (int32_t *)(b + o_pts1);
    ctx->p_ntiles = (int32_t *)(b + o_pnt);
    ctx->p_list_tok = (int32_t *)(b + o_plt);
    ctx->p_list_pair = (int32_t *)(b + o_plp);
    ctx->p_fa_ws = (float *)(b + o_pfa);
    ctx->p_rope = (float *)(b + o_prope);
    ctx->p_kpart = (float *)(b + o_pkp);
    ctx->run_arena = b + o_run;
    ctx->run_tag = 1u; /* the arena is zero: tag 0 never matches */
    ctx->p_max_tiles = max_tiles;
    ctx->rarena_bytes = total;
    ctx->kv_bytes = 2u * kv_one;
    ctx->scratch_bytes = scratch_end - o_h;
    ctx->moe_bytes = moe_end - scratch_end;
    ctx->logits_bytes = logits_end - moe_end;
    ctx->prompt_bytes = prompt_end - logits_end;
    ctx->prefill_bytes = total - prompt_end;
    HIPCHK(counted_host_malloc(ctx, (void **)&ctx->h_tokens, (size_t)max_gen * 4u), "pinned token buffer");
    HIPCHK(counted_host_malloc(ctx, (void **)&ctx->h_scores, (size_t)max_gen * 4u), "pinned score buffer");
    HIPCHK(counted_host_malloc(ctx, (void **)&ctx->h_prompt, (size_t)prompt_capacity * H_SIZE * 2u),
           "pinned prompt staging");
    if (ctx->mem != nullptr) {
        uocr_memory_reserve(ctx->mem, UOCR_MEMORY_KV_CACHE, ctx->kv_bytes);
        uocr_memory_reserve(ctx->mem, UOCR_MEMORY_DECODER_SCRATCH, ctx->scratch_bytes + ctx->prefill_bytes);
        uocr_memory_reserve(ctx->mem, UOCR_MEMORY_MOE_SCRATCH, ctx->moe_bytes);
        uocr_memory_reserve(ctx->mem, UOCR_MEMORY_LOGITS_READBACK, ctx->logits_bytes);
        uocr_memory_reserve(ctx->mem, UOCR_MEMORY_PROMPT_EMBEDDINGS, ctx->prompt_bytes);
    }
    ctx->prompt_cap = prompt_capacity;
    ctx->cache_cap = cap;
    ctx->max_gen = max_gen;
    ctx->runtime_ready = 1;
    return 1;
}

/* ---- step enqueue ----------------------------------------------------------- */

/* sel: layer 0's QKV launch chooses the token from the LM-head keys and
 * stages its embedding row (a decode step); else h already holds the
 * layer input (a prompt position). */
/* Per-op decode timing: an event pair around one launch, named with the
 * reference's decode roles (uocr_metal.m:14338-14496) under hip.decode.*;
 * a fused launch carries the role of its first op:
 *   attention_projections  QKV (+ attention norm, RoPE, KV write) and O
 *                          (+ attention merge, router fold)
 *   attention              split-K attention
 *   dense_mlp              layer 0's SwiGLU and down
 *   moe_router             router logits (layers without the fold)
 *   moe_routed_experts     top-6 + routed and shared gate/up; routed and
 *                          shared down + combine
 *   lm_head                final norm + LM head + argmax (+ selection) */
static void tm_begin(uocr_hip_ctx *c, const char *name, const char *kname) {
    op_timer *t = c->tm;
    if (t == nullptr || t->n >= OP_TIMER_MAX) return;
    t->name[t->n] = name;
    t->kname[t->n] = c->profile_detail >= 4 ? kname : nullptr;
    (void)hipEventRecord(t->ev[2 * t->n], c->stream);
}

static void tm_end(uocr_hip_ctx *c) {
    op_timer *t = c->tm;
    if (t == nullptr || t->n >= OP_TIMER_MAX) return;
    (void)hipEventRecord(t->ev[2 * t->n + 1], c->stream);
    ++t->n;
}

/* After the step's work is complete: every timed launch into the profile,
 * and per layer the span from its first launch's start to its last's end. */
static void tm_flush(uocr_hip_ctx *c) {
    op_timer *t = c->tm;
    if (t == nullptr || c->profile == nullptr) return;
    for (int i = 0; i < t->n; ++i) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, t->ev[2 * i], t->ev[2 * i + 1]) != hipSuccess) continue;
        uocr_profile_add_ms(c->profile, t->name[i], ms);
        if (t->kname[i] != nullptr) uocr_profile_add_ms(c->profile, t->kname[i], ms);
    }
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const int a = t->layer_first[l], b = t->layer_last[l];
        float ms = 0.0f;
        if (a >= 0 && b >= a && hipEventElapsedTime(&ms, t->ev[2 * a], t->ev[2 * b + 1]) == hipSuccess) {
            uocr_profile_add_ms(c->profile, "hip.decode.layer", ms);
        }
        t->layer_first[l] = t->layer_last[l] = -1;
    }
    t->n = 0;
}

static hipError_t enqueue_layers(uocr_hip_ctx *c, bool sel) {
    hipStream_t s = c->stream;
    const uint64_t kv_layer = (uint64_t)UOCR_ATTENTION_HEADS * c->cache_cap * UOCR_HEAD_DIM;
    hipError_t e = hipSuccess;
    const char *role = nullptr;
#define ENQK(k, x)                    \
    do {                              \
        if (role != nullptr) tm_begin(c, role, "hip.kernel." k); \
        e = (x);                      \
        if (e != hipSuccess) return e; \
        if (role != nullptr) tm_end(c); \
    } while (0)
#define ROLE(r) role = c->tm != nullptr ? (r) : nullptr
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const dev_layer &L = c->L[l];
        uint16_t *kc = c->kc + l * kv_layer, *vc = c->vc + l * kv_layer;
        if (c->tm != nullptr) c->tm->layer_first[l] = c->tm->n;
        ROLE("hip.decode.attention_projections");
        if (sel && l == 0u) {
            ENQK("k_qkv_rope", uocr_launch_qkv_rope_select(s, L.q, L.k, L.v, L.in_norm, c->state, c->q, kc, vc, c->cache_cap,
                                            (const uint64_t *)c->lm_part, c->embed, UOCR_VOCAB_SIZE, c->tokens,
                                            c->scores, c->h));
        } else {
            ENQK("k_qkv_rope", uocr_launch_qkv_rope(s, L.q, L.k, L.v, c->h, L.in_norm, c->state, c->q, kc, vc, c->cache_cap));
        }
        ROLE("hip.decode.attention");
        ENQK("k_attention", uocr_launch_attention(s, c->q, kc, vc, c->cache_cap, c->state, c->attn_part, c->racc,
                                  sel && l == 0u ? (uint64_t *)c->lm_part : nullptr));
        ROLE("hip.decode.attention_projections");
        ENQK("k_attn_out", uocr_launch_attn_out(s, L.o, c->attn_part, c->h, c->a, nullptr, L.rfold, c->racc));
        if (l == 0u) {
            ROLE("hip.decode.dense_mlp");
            ENQK("k_swiglu", uocr_launch_swiglu(s, L.gate, L.up, UOCR_DENSE_LAYER0_INTERMEDIATE, H_SIZE, c->a, L.post_norm, c->mid));
            ENQK("k_gemv", uocr_launch_gemv(s, L.down, H_SIZE, UOCR_DENSE_LAYER0_INTERMEDIATE, c->mid, nullptr, c->a, c->h));
        } else {
            /* with the fold, attn_out has produced the un-normalised logits */
            ROLE("hip.decode.moe_router");
            if (L.rfold == nullptr) ENQK("k_router_logits", uocr_launch_router_logits(s, L.router, c->a, L.post_norm, c->logits));
            ROLE("hip.decode.moe_routed_experts");
            ENQK("k_moe_gate_up", uocr_launch_moe_gate_up(s, &L.slab, L.sgate, L.sup, L.rfold == nullptr ? c->logits : nullptr,
                                        L.rfold == nullptr ? nullptr : c->racc, 0, c->a, L.post_norm, c->mid, c->smid,
                                        c->route_ids, c->route_w, L.router, L.rfold == nullptr ? nullptr : c->lg_part));
            /* with the fold, the routing weights come from the exact logits'
             * quarters of the gate/up launch, taken by the down launch */
            ENQK("k_moe_down", uocr_launch_moe_down(s, &L.slab, c->route_ids, c->route_w, c->mid, L.sdown, c->smid, c->a, c->h,
                                                    L.rfold == nullptr ? nullptr : c->lg_part, c->route_w));
            if (c->trace_step >= 0 && (uint32_t)c->trace_step < c->trace_steps) {
                role = nullptr; /* not a decode launch */
                ENQK("trace", hipMemcpyAsync(c->d_trace + ((size_t)c->trace_step * 11u + (l - 1u)) * UOCR_MOE_TOP_K, c->route_ids,
                                   UOCR_MOE_TOP_K * 4u, hipMemcpyDeviceToDevice, s));
                ENQK("trace", hipMemcpyAsync(c->d_trace + ((size_t)(c->trace_steps + c->trace_step) * 11u + (l - 1u)) * UOCR_MOE_TOP_K,
                                   c->route_w, UOCR_MOE_TOP_K * 4u, hipMemcpyDeviceToDevice, s));
                uint16_t *ta = (uint16_t *)(c->d_trace + 2u * (size_t)c->trace_steps * 11u * UOCR_MOE_TOP_K);
                ENQK("trace", hipMemcpyAsync(ta + ((size_t)c->trace_step * 11u + (l - 1u)) * H_SIZE, c->a, H_SIZE * 2u,
                                   hipMemcpyDeviceToDevice, s));
            }
        }
        if (c->tm != nullptr) c->tm->layer_last[l] = c->tm->n - 1;
    }
    return e;
#undef ROLE
#undef ENQK
}

/* The LM head of a decode step: argmax keys and the step-state advance
 * (k_lm_keys).  With fold_select the token is chosen by layer 0's QKV launch
 * (enqueue_layers with sel); otherwise, or with last (the final step, no
 * layers follow), a finalize launch chooses it and, unless last, gathers its
 * embedding row into h. */
static hipError_t enqueue_select(uocr_hip_ctx *c, bool last) {
    tm_begin(c, "hip.decode.lm_head", "hip.kernel.k_lm_keys");
    hipError_t e = uocr_launch_lm_keys(c->stream, c->lm_head, UOCR_VOCAB_SIZE, c->h, c->final_norm,
                                       (uint64_t *)c->lm_part, c->state, 1, c->invf);
    if (e == hipSuccess) tm_end(c);
    if (e != hipSuccess || (c->fold_select && !last)) return e;
    uocr_qmat none = {nullptr, nullptr, UOCR_QT_Q4};
    tm_begin(c, "hip.decode.lm_head", "hip.kernel.k_lm_finalize");
    e = uocr_launch_lm_finalize(c->stream, (uint64_t *)c->lm_part, c->state, 1, c->tokens, c->scores,
                                last ? none : c->embed, UOCR_VOCAB_SIZE, c->h);
    if (e == hipSuccess) tm_end(c);
    return e;
}

static hipError_t enqueue_decode_step(uocr_hip_ctx *c) {
    hipError_t e = enqueue_select(c, false);
    if (e == hipSuccess) e = enqueue_layers(c, c->fold_select != 0);
    return e;
}

static hipError_t enqueue_prefill_step(uocr_hip_ctx *c) {
    hipError_t e = uocr_launch_prefill_next(c->stream, c->state, c->prompt, c->h, c->invf);
    if (e == hipSuccess) e = enqueue_layers(c, false);
    return e;
}

/* Plain prefill GEMM with split K where its grid is small (the partials
 * buffer holds UOCR_PREFILL_KSPLIT_MAX x P x 1280 floats; the split count is
 * clamped to what it holds at this N).  Used for the O projection and layer
 * 0's dense down (K = 6848): measured at P = 932, O 26.3 -> 16 + 5 us
 * (reduce), while the router logits (11.4 -> 6.6 + 4.9) and the shared down
 * (23.6 -> 19 + 5.2) gain nothing, an extra eager launch costing about 5 us. */
static void with_ksplit(uocr_gemm_desc &d, float *part) {
    const uint32_t s = std::min<uint32_t>(uocr_gemm_ksplit(d.M, d.N, d.K), UOCR_PREFILL_KSPLIT_MAX * H_SIZE / d.N);
    if (s > 1u) {
        d.ksplit = s;
        d.part = part;
    }
}

static uocr_gemm_desc gdesc(const uint16_t *A, uint32_t lda, uint32_t M, uint32_t N, uint32_t K, void *out,
                           uint32_t ldo) {
    uocr_gemm_desc d;
    memset(&d, 0, sizeof(d));
    d.A = A;
    d.lda = lda;
    d.M = M;
    d.N = N;
    d.K = K;
    d.out = out;
    d.ldo = ldo;
    return d;
}

/* All P prompt rows (c->prompt, updated in place as the residual stream)
 * through the 12 layers on MFMA GEMMs; K/V of positions 0..P-1 land in the
 * cache slots 0..P-1 and the last row's hidden state in c->h. */
/* m with its payload replaced by the GEMM-packed copy (when there is one). */
static uocr_qmat packed_of(const uocr_qmat &m, const void *pw) {
    uocr_qmat r = m;
    if (pw != nullptr) r.w = pw;
    return r;
}

static hipError_t enqueue_prefill_mfma(uocr_hip_ctx *c, uint32_t P) {
    hipStream_t s = c->stream;
    const uint64_t kv_layer = (uint64_t)UOCR_ATTENTION_HEADS * c->cache_cap * UOCR_HEAD_DIM;
    uint16_t *H = c->prompt;
    hipError_t e = hipSuccess;
#define ENQ(x)                        \
    do {                              \
        e = (x);                      \
        if (e != hipSuccess) return e; \
    } while (0)
    /* each layer's input norm comes out of the previous layer's last kernel
     * (the combine, or layer 0's down reduce); only layer 0 launches it */
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const dev_layer &L = c->L[l];
        const uint16_t *next_norm = l + 1u < UOCR_DECODER_LAYERS ? c->L[l + 1u].in_norm : nullptr;
        uint16_t *kc = c->kc + l * kv_layer, *vc = c->vc + l * kv_layer;
        if (l == 0u) {
            ENQ(uocr_launch_rows_rmsnorm(s, H, L.in_norm, P, c->p_xn));
            ENQ(uocr_launch_rope_table(s, c->invf, P, c->p_rope));
        }
        uocr_gemm_desc d = gdesc(c->p_xn, H_SIZE, P, 3u * H_SIZE, H_SIZE, c->p_q, 3u * H_SIZE);
        d.W[0] = packed_of(L.q, L.pq);
        d.W[1] = packed_of(L.k, L.pk);
        d.W[2] = packed_of(L.v, L.pv);
        d.packed = L.pq != nullptr && L.pk != nullptr && L.pv != nullptr;
        if (!d.packed) {
            d.W[0] = L.q;
            d.W[1] = L.k;
            d.W[2] = L.v;
        }
        d.nseg = H_SIZE;
        ENQ(uocr_launch_gemm_qkv_rope(s, &d, c->p_rope, c->p_q, kc, vc, c->cache_cap));
        ENQ(uocr_launch_flash_attn(s, c->p_q, kc, vc, c->cache_cap, P, c->p_ctx, c->p_fa_ws));
        d = gdesc(c->p_ctx, H_SIZE, P, H_SIZE, H_SIZE, c->p_a, H_SIZE);
        d.W[0] = packed_of(L.o, L.po);
        d.packed = L.po != nullptr;
        d.res = H;
        d.ldr = H_SIZE;
        if (c->prefill_ksplit) with_ksplit(d, c->p_kpart);
        d.norm_w = L.post_norm;
        d.norm_out = c->p_xn;
        ENQ(uocr_launch_gemm(s, UOCR_GEMM_F16, &d));
        if (l == 0u) {
            const uint32_t I0 = UOCR_DENSE_LAYER0_INTERMEDIATE;
            d = gdesc(c->p_xn, H_SIZE, P, I0, H_SIZE, c->p_mid, I0);
            d.packed = L.pgate != nullptr && L.pup != nullptr;
            d.W[0] = d.packed ? packed_of(L.gate, L.pgate) : L.gate;
            d.W[1] = d.packed ? packed_of(L.up, L.pup) : L.up;
            ENQ(uocr_launch_gemm(s, UOCR_GEMM_SWIGLU, &d));
            d = gdesc(c->p_mid, I0, P, H_SIZE, I0, H, H_SIZE);
            d.W[0] = packed_of(L.down, L.pdown);
            d.packed = L.pdown != nullptr;
            d.res = c->p_a;
            d.ldr = H_SIZE;
            if (c->prefill_ksplit) with_ksplit(d, c->p_kpart);
            d.norm_w = next_norm;
            d.norm_out = next_norm != nullptr ? c->p_xn : nullptr;
            ENQ(uocr_launch_gemm(s, UOCR_GEMM_F16, &d));
            continue;
        }
        const uint32_t SI = UOCR_MOE_SHARED_INTERMEDIATE, EI = UOCR_MOE_EXPERT_INTERMEDIATE;
        /* the router logits share a launch with the shared gate/up (both read
         * xn), the shared down with the routed down */
        uocr_gemm_desc dr = gdesc(c->p_xn, H_SIZE, P, UOCR_ROUTED_EXPERTS, H_SIZE, c->p_logits, UOCR_ROUTED_EXPERTS);
        dr.W[0].w = L.router;
        dr.W[0].s = nullptr;
        dr.W[0].qtype = UOCR_QT_F16;
        uocr_gemm_desc dsg = gdesc(c->p_xn, H_SIZE, P, SI, H_SIZE, c->p_smid, SI);
        dsg.packed = L.psg != nullptr && L.psu != nullptr;
        dsg.W[0] = dsg.packed ? packed_of(L.sgate, L.psg) : L.sgate;
        dsg.W[1] = dsg.packed ? packed_of(L.sup, L.psu) : L.sup;
        ENQ(uocr_launch_gemm_pair(s, UOCR_GEMM_SWIGLU, &dsg, UOCR_GEMM_F32, &dr));
        ENQ(uocr_launch_route_rows(s, c->p_logits, P, 0, c->p_ids, c->p_wts, c->p_offsets, c->p_tile_e, c->p_tile_s0, c->p_tile_s1, c->p_ntiles, c->p_list_tok,
                                   c->p_list_pair));
        uocr_gemm_desc dsd = gdesc(c->p_smid, SI, P, H_SIZE, SI, c->p_sout, H_SIZE);
        dsd.W[0] = packed_of(L.sdown, L.psd);
        dsd.packed = L.psd != nullptr;
        d = gdesc(c->p_xn, H_SIZE, 0, EI, H_SIZE, c->p_rmid, EI);
        d.packed = L.peg != nullptr && L.peu != nullptr;
        d.W[0] = d.packed ? packed_of(L.slab.gate, L.peg) : L.slab.gate;
        d.W[1] = d.packed ? packed_of(L.slab.up, L.peu) : L.slab.up;
        d.w_stride = L.slab.gu_w_stride;
        d.s_stride = L.slab.gu_s_stride;
        d.a_idx = c->p_list_tok;
        d.o_idx = c->p_list_pair;
        d.tile_e = c->p_tile_e;
        d.tile_s0 = c->p_tile_s0;
        d.tile_s1 = c->p_tile_s1;
        d.ntiles = c->p_ntiles;
        d.max_tiles = c->p_max_tiles;
        /* the shared down shares the routed down's launch (2.77 against 2.83 ms
         * beside the routed gate/up; UOCR_HIP_SHARED_DOWN_WITH=gu for that) */
        static const int sd_down = [] {
            const char *e = getenv("UOCR_HIP_SHARED_DOWN_WITH");
            return e != nullptr && strcmp(e, "gu") == 0 ? 0 : 1;
        }();
        if (sd_down) {
            ENQ(uocr_launch_gemm(s, UOCR_GEMM_SWIGLU, &d));
        } else {
            ENQ(uocr_launch_gemm_pair(s, UOCR_GEMM_F16, &dsd, UOCR_GEMM_SWIGLU, &d));
        }
        uocr_gemm_desc dd = d;
        dd.A = c->p_rmid;
        dd.lda = EI;
        dd.N = H_SIZE;
        dd.K = EI;
        dd.W[0] = packed_of(L.slab.down, L.ped);
        dd.packed = L.ped != nullptr;
        dd.W[1] = uocr_qmat{nullptr, nullptr, 0};
        dd.w_stride = L.slab.dn_w_stride;
        dd.s_stride = L.slab.dn_s_stride;
        dd.a_idx = c->p_list_pair;
        /* per-pair expert outputs in fp16, as the reference keeps them */
        uint16_t *y16 = c->p_y;
        dd.out = y16;
        dd.ldo = H_SIZE;
        if (sd_down) {
            ENQ(uocr_launch_gemm_pair(s, UOCR_GEMM_F16, &dsd, UOCR_GEMM_F16, &dd));
        } else {
            ENQ(uocr_launch_gemm(s, UOCR_GEMM_F16, &dd));
        }
        if (next_norm != nullptr) {
            ENQ(uocr_launch_moe_combine_norm_h(s, y16, c->p_wts, c->p_sout, c->p_a, P, H, next_norm, c->p_xn));
        } else {
            ENQ(uocr_launch_moe_combine_h(s, y16, c->p_wts, c->p_sout, c->p_a, P, H));
        }
    }
    return hipMemcpyAsync(c->h, H + (size_t)(P - 1u) * H_SIZE, H_SIZE * 2u, hipMemcpyDeviceToDevice, s);
#undef ENQ
}

/* DECODE_CHUNK decode steps in one graph: the device-side step state
 * advances from one step to the next, so the steps replay unchanged, and a
 * chunk pays one graph launch instead of DECODE_CHUNK (a launch boundary
 * between graphs costs about 6 us, between kernels of a graph about 1.4 us). */
static hipError_t enqueue_decode_chunk(uocr_hip_ctx *c) {
    hipError_t e = hipSuccess;
    for (uint32_t i = 0; i < DECODE_CHUNK && e == hipSuccess; ++i) e = enqueue_decode_step(c);
    return e;
}

static int capture(uocr_hip_ctx *c, hipError_t (*fn)(uocr_hip_ctx *), hipGraphExec_t *out, char *err, size_t err_size) {
    hipGraph_t g = nullptr;
    HIPCHK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "graph capture begin");
    const hipError_t e = fn(c);
    const hipError_t e2 = hipStreamEndCapture(c->stream, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
        if (g != nullptr) (void)hipGraphDestroy(g);
        return bfail(err, err_size, "graph capture failed: %s", hipGetErrorString(e != hipSuccess ? e : e2));
    }
    const hipError_t e3 = hipGraphInstantiate(out, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    HIPCHK(e3, "graph instantiate");
    return 1;
}

static hipError_t enqueue_prefill_mfma_cap(uocr_hip_ctx *c) {
    return enqueue_prefill_mfma(c, c->cap_P);
}

/* The MFMA prefill of P rows: replayed from its graph when this length was
 * captured; captured when the same length comes twice in a row (a first
 * length runs eagerly, so prompts of changing lengths pay no capture); eager
 * otherwise.  Inside a graph the prefill's ~190 launches cost about 1.5 us
 * each instead of about 5. */
static int run_prefill_mfma(uocr_hip_ctx *c, uint32_t P, int use_graph, char *err, size_t err_size) {
    if (use_graph && c->g_mfma != nullptr && c->g_mfma_P == P) {
        HIPCHK(hipGraphLaunch(c->g_mfma, c->stream), "prefill graph launch");
        return 1;
    }
    if (use_graph && c->last_mfma_P == P) {
        if (c->g_mfma != nullptr) {
            (void)hipGraphExecDestroy(c->g_mfma);
            c->g_mfma = nullptr;
            c->g_mfma_P = 0u;
        }
        c->cap_P = P;
        if (!capture(c, enqueue_prefill_mfma_cap, &c->g_mfma, err, err_size)) {
            c->g_mfma = nullptr;
            return 0;
        }
        c->g_mfma_P = P;
        HIPCHK(hipGraphLaunch(c->g_mfma, c->stream), "prefill graph launch");
        return 1;
    }
    c->last_mfma_P = P;
    HIPCHK(enqueue_prefill_mfma(c, P), "MFMA prefill");
    return 1;
}

/* ---- generation -------------------------------------------------------------- */

__global__ void k_fill_u32(uint32_t *p, size_t n, uint32_t v) {
    const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (i < n) p[i] = v;
}

extern "C" int uocr_hip_context_decode_path(const uocr_hip_ctx *c) {
    return c != nullptr ? c->last_path : -1;
}

static int scan_chunk(uocr_hip_ctx *c, uint32_t from, uint32_t to, int ignore_eos, uint32_t *count, int *eos) {
    for (uint32_t i = from; i < to; ++i) {
        const int32_t id = c->h_tokens[i];
        if (id < 0 || (uint32_t)id >= UOCR_VOCAB_SIZE) return 0;
        *count = i + 1u;
        if (!ignore_eos && id == UOCR_TOKEN_EOS) {
            *eos = 1;
            return 1;
        }
    }
    return 1;
}

/* The decode loop on the persistent run: launches of DECODE_CHUNK steps,
 * the first starting from the prefill's hidden state (published with a tag
 * of its own), token ids read back one chunk behind the GPU. */
static int decode_run(uocr_hip_ctx *c, uint32_t P, uint32_t N, int ignore_eos, uint64_t t0, uint64_t t1,
                      const alloc_guard &dg, uocr_hip_decoder_result *res, char *err, size_t err_size) {
    hipStream_t s = c->stream;
    std::lock_guard<std::mutex> lock(g_run_mutex);
    const uint32_t seed_tag = c->run_tag, tag0 = seed_tag + 1u;
    c->run_tag = tag0 + N;
    HIPCHK(uocr_run_reset(s, c->run_arena), "run reset");
    HIPCHK(uocr_run_seed(s, c->run_arena, c->h, seed_tag), "run seed");
    uint32_t count = 0, scanned = 0, issued = 0, chunk = 0;
    int eos = 0, ok = 1;
    hipEvent_t ev[2];
    HIPCHK(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming), "event create");
    HIPCHK(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming), "event create");
    /* per-launch timing (UOCR_HIP_RUN_EVENTS=1 with profiling): an event pair
     * around each launch on the engine stream, reported as
     * hip.kernel.k_decode_run once the loop has finished */
    const bool kev = c->run_events != 0 && c->profile != nullptr && c->profile->report.enabled != 0u;
    std::vector<hipEvent_t> kt;
    if (kev) {
        kt.resize(2u * ((N + DECODE_CHUNK - 1u) / DECODE_CHUNK));
        for (hipEvent_t &x : kt) HIPCHK(hipEventCreate(&x), "event create");
    }
    while (issued < N && !eos && ok) {
        const uint32_t end = issued + DECODE_CHUNK < N ? issued + DECODE_CHUNK : N;
        if (kev) (void)hipEventRecord(kt[2u * chunk], s);
        const hipError_t e = uocr_run_launch(s, c->d_run_model, &c->run_model, c->run_arena, c->kc, c->vc, c->cache_cap,
                                             (int32_t)P, (int32_t)issued, (int32_t)(end - issued), end == N ? 1 : 0,
                                             tag0 + issued, c->tokens, c->scores, c->h, c->d_trace, c->trace_steps,
                                             c->d_force, c->force_n);
        if (e != hipSuccess) {
            ok = bfail(err, err_size, "decode run of steps %u-%u: %s", issued, end - 1u, hipGetErrorString(e));
            break;
        }
        if (kev) (void)hipEventRecord(kt[2u * chunk + 1u], s);
        if (hipMemcpyAsync(c->h_tokens + issued, c->tokens + issued, (size_t)(end - issued) * 4u, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipEventRecord(ev[chunk & 1u], s) != hipSuccess) {
            ok = bfail(err, err_size, "token readback failed");
            break;
        }
        if (chunk > 0u) {
            if (hipEventSynchronize(ev[(chunk - 1u) & 1u]) != hipSuccess) {
                ok = bfail(err, err_size, "decode chunk wait failed");
                break;
            }
            if (!scan_chunk(c, scanned, issued, ignore_eos, &count, &eos)) ok = bfail(err, err_size, "decode selected an invalid token id");
            scanned = issued;
        }
        issued = end;
        ++chunk;
    }
    const hipError_t se = hipStreamSynchronize(s);
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
    for (uint32_t i = 0; kev && i < chunk; ++i) {
        float ms = 0.0f;
        if (se == hipSuccess && hipEventElapsedTime(&ms, kt[2u * i], kt[2u * i + 1u]) == hipSuccess) {
            uocr_profile_add_ms(c->profile, "hip.kernel.k_decode_run", ms);
        }
    }
    for (hipEvent_t x : kt) (void)hipEventDestroy(x);
    if (se != hipSuccess) return bfail(err, err_size, "decode sync: %s", hipGetErrorString(se));
    uint32_t ctl[4] = {0u, 0u, 0u, 0u};
    HIPCHK(hipMemcpy(ctl, c->run_arena, sizeof(ctl), hipMemcpyDeviceToHost), "run status readback");
    if (ctl[UOCR_RUN_CTL_ABORT] != 0u) {
        c->run_aborted = 1;
        return bfail(err, err_size, "decode run timed out waiting at stage %u of step %u (workgroup %u)",
                     ctl[UOCR_RUN_CTL_WHERE], ctl[UOCR_RUN_CTL_STEP], ctl[UOCR_RUN_CTL_BLOCK]);
    }
    if (!ok) return 0;
    if (!eos && !scan_chunk(c, scanned, issued, ignore_eos, &count, &eos)) {
        return bfail(err, err_size, "decode selected an invalid token id");
    }
    fault_alloc(c, 2);
    if (!guard_end(c, dg, "HIP decode loop", err, err_size)) return 0;
    const uint64_t t2 = uocr_now_ns();
    memcpy(res->generated_ids, c->h_tokens, (size_t)count * 4u);
    if (res->generated_scores != nullptr) {
        HIPCHK(hipMemcpy(res->generated_scores, c->scores, (size_t)count * 4u, hipMemcpyDeviceToHost), "score readback");
    }
    res->generated_count = count;
    res->stopped_on_eos = (uint32_t)eos;
    res->prefill_ms = (double)(t1 - t0) / 1.0e6;
    res->decode_ms = (double)(t2 - t1) / 1.0e6;
    if (c->profile != nullptr) {
        uocr_profile_add_ms(c->profile, "hip.prefill", res->prefill_ms);
        uocr_profile_add_ms(c->profile, "hip.decode_loop", res->decode_ms);
        c->profile->report.metal_command_buffer_count += chunk;
        c->profile->report.metal_command_buffer_wait_count += chunk + 1u;
    }
    return 1;
}

/* The eager decode loop, one synchronised step at a time; the host scans
 * every step for EOS.  With timed, an event pair brackets each launch and the
 * step's times go to the profile report (hip.decode.*); with a decode trace
 * on, the router's selections are copied out after each gate/up launch. */
static int decode_timed(uocr_hip_ctx *c, uint32_t P, uint32_t N, int ignore_eos, uint64_t t0, uint64_t t1,
                        const alloc_guard &dg, bool timed, uocr_hip_decoder_result *res, char *err, size_t err_size) {
    hipStream_t s = c->stream;
    op_timer *t = (op_timer *)calloc(1, sizeof(op_timer));
    if (t == nullptr) return bfail(err, err_size, "profile timer allocation failed");
    int made = 0, ok = 1;
    for (; made < 2 * OP_TIMER_MAX && hipEventCreate(&t->ev[made]) == hipSuccess; ++made) {
    }
    if (made < 2 * OP_TIMER_MAX) ok = bfail(err, err_size, "profile event creation failed");
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) t->layer_first[l] = t->layer_last[l] = -1;
    uint32_t count = 0;
    int eos = 0;
    if (ok && uocr_launch_decode_state(s, c->state, (int32_t)P, 0, c->invf) != hipSuccess) {
        ok = bfail(err, err_size, "decode state init failed");
    }
    c->tm = timed ? t : nullptr;
    /* teacher forcing: the finalize launch selects and embeds the step's own
     * token, then the forced token's row replaces it */
    const int fold_select = c->fold_select;
    if (c->force_n != 0u) c->fold_select = 0;
    for (uint32_t step = 0; ok && step < N && !eos; ++step) {
        c->trace_step = (int32_t)step;
        hipError_t e;
        if (step + 1u == N) {
            e = enqueue_select(c, true);
        } else if (step < c->force_n) {
            e = enqueue_select(c, false);
            if (e == hipSuccess) e = uocr_launch_embed(s, c->embed, UOCR_VOCAB_SIZE, c->d_force + step, nullptr, c->h);
            if (e == hipSuccess) e = enqueue_layers(c, false);
        } else {
            e = enqueue_decode_step(c);
        }
        if (e != hipSuccess || hipMemcpyAsync(c->h_tokens + step, c->tokens + step, 4u, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess) {
            ok = bfail(err, err_size, "timed decode step %u failed", step);
            break;
        }
        tm_flush(c);
        if (!scan_chunk(c, step, step + 1u, ignore_eos, &count, &eos)) ok = bfail(err, err_size, "decode selected an invalid token id");
    }
    c->tm = nullptr;
    c->trace_step = -1;
    c->fold_select = fold_select;
    for (int i = 0; i < made; ++i) (void)hipEventDestroy(t->ev[i]);
    free(t);
    if (!ok) return 0;
    fault_alloc(c, 2);
    if (!guard_end(c, dg, "HIP decode loop", err, err_size)) return 0;
    const uint64_t t2 = uocr_now_ns();
    memcpy(res->generated_ids, c->h_tokens, (size_t)count * 4u);
    if (res->generated_scores != nullptr) {
        HIPCHK(hipMemcpy(res->generated_scores, c->scores, (size_t)count * 4u, hipMemcpyDeviceToHost), "score readback");
    }
    res->generated_count = count;
    res->stopped_on_eos = (uint32_t)eos;
    res->prefill_ms = (double)(t1 - t0) / 1.0e6;
    res->decode_ms = (double)(t2 - t1) / 1.0e6;
    if (c->profile != nullptr) {
        uocr_profile_add_ms(c->profile, "hip.prefill", res->prefill_ms);
        uocr_profile_add_ms(c->profile, "hip.decode_loop", res->decode_ms);
    }
    return 1;
}

extern "C" int uocr_hip_context_generate(uocr_hip_ctx *c, const uocr_hip_decoder_request *req,
                                         uocr_hip_decoder_result *res, char *err, size_t err_size) {
    if (c == nullptr || req == nullptr || res == nullptr || req->input_ids == nullptr) {
        return bfail(err, err_size, "invalid HIP generation request");
    }
    if (!c->mapped) return bfail(err, err_size, "HIP context has no mapped model");
    const uint32_t P = req->n_tokens, N = req->max_new_tokens;
    if (P == 0u || N == 0u) return bfail(err, err_size, "generation needs a prompt and max_new_tokens > 0");
    if (res->generated_ids == nullptr || res->generated_capacity < N) return bfail(err, err_size, "result capacity too small");
    if (!uocr_hip_context_allocate_runtime(c, P > c->prompt_cap ? P : (c->prompt_cap ? c->prompt_cap : P),
                                           N > c->max_gen ? N : (c->max_gen ? c->max_gen : N), err, err_size)) {
        return 0;
    }
    HIPCHK(hipSetDevice(c->device), "hipSetDevice");
    const int use_graph = (req->flags & UOCR_GEN_NO_GRAPH) == 0u;
    if (use_graph && !c->graphs_ready) {
        if (!capture(c, enqueue_decode_step, &c->g_decode, err, err_size)) return 0;
        if (!capture(c, enqueue_decode_chunk, &c->g_decode_chunk, err, err_size)) {
            (void)hipGraphExecDestroy(c->g_decode);
            return 0;
        }
        if (!capture(c, enqueue_prefill_step, &c->g_prefill, err, err_size)) {
            (void)hipGraphExecDestroy(c->g_decode);
            (void)hipGraphExecDestroy(c->g_decode_chunk);
            return 0;
        }
        c->graphs_ready = 1;
    }
    hipStream_t s = c->stream;
    const uint64_t t0 = uocr_now_ns();
    const alloc_guard pg = guard_begin(c);

    /* prompt assembly: image rows from the caller, text rows gathered on device */
    uint32_t n_img = 0;
    for (uint32_t i = 0; i < P; ++i) {
        if (req->image_mask != nullptr && req->image_mask[i] != 0u) {
            if (req->image_rows == nullptr || n_img >= req->n_image_rows) {
                return bfail(err, err_size, "prompt has more image positions than image rows");
            }
            memcpy(c->h_prompt + (size_t)i * H_SIZE, req->image_rows + (size_t)n_img * H_SIZE, H_SIZE * 2u);
            ++n_img;
        }
    }
    if (n_img != 0u) {
        HIPCHK(hipMemcpyAsync(c->prompt, c->h_prompt, (size_t)P * H_SIZE * 2u, hipMemcpyHostToDevice, s), "prompt upload");
    }
    HIPCHK(hipMemcpyAsync(c->d_ids, req->input_ids, (size_t)P * 4u, hipMemcpyHostToDevice, s), "ids upload");
    const uint8_t *dmask = nullptr;
    if (req->image_mask != nullptr) {
        HIPCHK(hipMemcpyAsync(c->d_mask, req->image_mask, P, hipMemcpyHostToDevice, s), "mask upload");
        dmask = c->d_mask;
    }
    HIPCHK(uocr_launch_embed_rows(s, c->embed, UOCR_VOCAB_SIZE, c->d_ids, dmask, P, c->prompt), "prompt embedding");

    /* prefill */
    HIPCHK(uocr_launch_decode_state(s, c->state, (int32_t)P, 0, c->invf), "state init");
    if ((req->flags & UOCR_GEN_TOKEN_PREFILL) == 0u) {
        if (!run_prefill_mfma(c, P, use_graph, err, err_size)) return 0;
    } else {
        for (uint32_t i = 0; i < P; ++i) {
            if (use_graph) {
                HIPCHK(hipGraphLaunch(c->g_prefill, s), "prefill graph launch");
            } else {
                HIPCHK(enqueue_prefill_step(c), "prefill step");
            }
        }
    }
    fault_alloc(c, 1);
    HIPCHK(hipStreamSynchronize(s), "prefill sync");
    if (!guard_end(c, pg, "HIP prompt prefill", err, err_size)) return 0;
    const alloc_guard dg = guard_begin(c);
    const uint64_t t1 = uocr_now_ns();

    /* decode: chunks of DECODE_CHUNK steps; the host scans chunk k-1 while
     * chunk k runs.  A chunk is one persistent run launch, or (UOCR_GEN_NO_RUN,
     * unsupported models) one replay of the captured 8-step graph. */
    const int ignore_eos = (req->flags & UOCR_GEN_IGNORE_EOS) != 0u;
    const bool timed = c->profile_detail >= 3 && c->profile != nullptr && c->profile->report.enabled != 0u;
    const bool use_run = c->run_ok && use_graph && !timed && (req->flags & UOCR_GEN_NO_RUN) == 0u;
    if (c->trace_steps != 0u) {
        /* steps this generation does not reach read as 0xffffffff */
        const size_t n = 2u * (size_t)c->trace_steps * 11u * UOCR_MOE_TOP_K + (size_t)c->trace_steps * 11u * H_SIZE / 2u;
        hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((n + 255u) / 256u)), dim3(256), 0, s, c->d_trace, n, 0xffffffffu);
        HIPCHK(hipGetLastError(), "trace clear");
    }
    if (use_run) {
        c->last_path = 1;
        c->run_aborted = 0;
        if (decode_run(c, P, N, ignore_eos, t0, t1, dg, res, err, err_size)) return 1;
        if (!c->run_aborted) return 0;
        /* a run that gave up waiting (a workgroup not scheduled for 50 ms,
         * e.g. CUs taken by another process) leaves the device usable: the
         * request is served again, prefill included, on the per-step kernels */
        uocr_hip_decoder_request again = *req;
        again.flags |= UOCR_GEN_NO_RUN;
        if (!uocr_hip_context_generate(c, &again, res, err, err_size)) return 0;
        c->last_path = 2;
        return 1;
    }
    c->last_path = 0;
    if (timed || c->trace_steps != 0u || c->force_n != 0u) return decode_timed(c, P, N, ignore_eos, t0, t1, dg, timed, res, err, err_size);
    HIPCHK(uocr_launch_decode_state(s, c->state, (int32_t)P, 0, c->invf), "decode state init");
    uint32_t count = 0, scanned = 0;
    int eos = 0;
    hipEvent_t ev[2];
    HIPCHK(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming), "event create");
    HIPCHK(hipEventCreateWithFlags(&ev[1], hipEventDisableTiming), "event create");
    uint32_t issued = 0, chunk = 0;
    int ok = 1;
    while (issued < N && !eos && ok) {
        const uint32_t end = issued + DECODE_CHUNK < N ? issued + DECODE_CHUNK : N;
        if (use_graph && end - issued == DECODE_CHUNK && end < N) {
            /* a whole chunk of full decode steps: one graph launch */
            const hipError_t e = hipGraphLaunch(c->g_decode_chunk, s);
            if (e != hipSuccess) ok = bfail(err, err_size, "decode steps %u-%u: %s", issued, end - 1u, hipGetErrorString(e));
        }
        for (uint32_t t = issued; t < end && ok && !(use_graph && end - issued == DECODE_CHUNK && end < N); ++t) {
            hipError_t e;
            if (t + 1u < N) {
                e = use_graph ? hipGraphLaunch(c->g_decode, s) : enqueue_decode_step(c);
            } else {
                e = enqueue_select(c, true);
            }
            if (e != hipSuccess) ok = bfail(err, err_size, "decode step %u: %s", t, hipGetErrorString(e));
        }
        if (!ok) break;
        if (hipMemcpyAsync(c->h_tokens + issued, c->tokens + issued, (size_t)(end - issued) * 4u, hipMemcpyDeviceToHost, s) != hipSuccess ||
            hipEventRecord(ev[chunk & 1u], s) != hipSuccess) {
            ok = bfail(err, err_size, "token readback failed");
            break;
        }
        if (chunk > 0u) {
            if (hipEventSynchronize(ev[(chunk - 1u) & 1u]) != hipSuccess) {
                ok = bfail(err, err_size, "decode chunk wait failed");
                break;
            }
            if (!scan_chunk(c, scanned, issued, ignore_eos, &count, &eos)) ok = bfail(err, err_size, "decode selected an invalid token id");
            scanned = issued;
        }
        issued = end;
        ++chunk;
    }
    const hipError_t se = hipStreamSynchronize(s);
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
    if (se != hipSuccess) return bfail(err, err_size, "decode sync: %s", hipGetErrorString(se));
    if (!ok) return 0;
    if (!eos && !scan_chunk(c, scanned, issued, ignore_eos, &count, &eos)) {
        return bfail(err, err_size, "decode selected an invalid token id");
    }
    fault_alloc(c, 2);
    if (!guard_end(c, dg, "HIP decode loop", err, err_size)) return 0;
    const uint64_t t2 = uocr_now_ns();
    memcpy(res->generated_ids, c->h_tokens, (size_t)count * 4u);
    if (res->generated_scores != nullptr) {
        HIPCHK(hipMemcpy(res->generated_scores, c->scores, (size_t)count * 4u, hipMemcpyDeviceToHost), "score readback");
    }
    res->generated_count = count;
    res->stopped_on_eos = (uint32_t)eos;
    res->prefill_ms = (double)(t1 - t0) / 1.0e6;
    res->decode_ms = (double)(t2 - t1) / 1.0e6;
    if (c->profile != nullptr) {
        uocr_profile_add_ms(c->profile, "hip.prefill", res->prefill_ms);
        uocr_profile_add_ms(c->profile, "hip.decode_loop", res->decode_ms);
        c->profile->report.metal_command_buffer_count += use_graph ? (uint64_t)P + issued : 0u;
        c->profile->report.metal_command_buffer_wait_count += chunk + 1u;
    }
    return 1;
}

/* ---- decode trace ----------------------------------------------------------- */

extern "C" int uocr_hip_context_trace_enable(uocr_hip_ctx *c, uint32_t steps, char *err, size_t err_size) {
    if (c == nullptr) return bfail(err, err_size, "invalid HIP context");
    HIPCHK(hipSetDevice(c->device), "hipSetDevice");
    if (c->d_trace != nullptr) {
        HIPCHK(hipStreamSynchronize(c->stream), "stream sync");
        (void)hipFree(c->d_trace);
        c->d_trace = nullptr;
    }
    c->trace_steps = 0u;
    if (steps == 0u) return 1;
    const size_t bytes = 2u * (size_t)steps * 11u * UOCR_MOE_TOP_K * 4u + (size_t)steps * 11u * H_SIZE * 2u;
    HIPCHK(counted_malloc(c, (void **)&c->d_trace, bytes), "trace buffer allocation");
    c->trace_steps = steps;
    return 1;
}

extern "C" int uocr_hip_context_trace_force(uocr_hip_ctx *c, const int32_t *ids, uint32_t n, char *err,
                                            size_t err_size) {
    if (c == nullptr || (n != 0u && ids == nullptr)) return bfail(err, err_size, "invalid trace_force request");
    HIPCHK(hipSetDevice(c->device), "hipSetDevice");
    HIPCHK(hipStreamSynchronize(c->stream), "stream sync");
    if (c->d_force != nullptr) {
        (void)hipFree(c->d_force);
        c->d_force = nullptr;
    }
    c->force_n = 0u;
    if (n == 0u) return 1;
    for (uint32_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= (int32_t)UOCR_VOCAB_SIZE) return bfail(err, err_size, "forced id %u out of vocabulary", i);
    }
    HIPCHK(counted_malloc(c, (void **)&c->d_force, (size_t)n * 4u), "forced id allocation");
    HIPCHK(hipMemcpy(c->d_force, ids, (size_t)n * 4u, hipMemcpyHostToDevice), "forced id upload");
    c->force_n = n;
    return 1;
}

extern "C" int uocr_hip_context_trace_read(uocr_hip_ctx *c, uint32_t *expert_ids, uint16_t *hidden, char *err,
                                           size_t err_size) {
    return uocr_hip_context_trace_read2(c, expert_ids, nullptr, hidden, err, err_size);
}

extern "C" int uocr_hip_context_trace_read_inputs(uocr_hip_ctx *c, uint16_t *inputs, char *err, size_t err_size) {
    if (c == nullptr || !c->runtime_ready || inputs == nullptr) return bfail(err, err_size, "invalid trace readback");
    HIPCHK(hipSetDevice(c->device), "hipSetDevice");
    HIPCHK(hipStreamSynchronize(c->stream), "stream sync");
    if (c->trace_steps != 0u) {
        const size_t n = (size_t)c->trace_steps * 11u * UOCR_MOE_TOP_K;
        HIPCHK(hipMemcpy(inputs, c->d_trace + 2u * n, (size_t)c->trace_steps * 11u * H_SIZE * 2u, hipMemcpyDeviceToHost),
               "trace input readback");
    }
    return 1;
}

extern "C" int uocr_hip_context_trace_read2(uocr_hip_ctx *c, uint32_t *expert_ids, float *weights, uint16_t *hidden,
                                            char *err, size_t err_size) {
    if (c == nullptr || !c->runtime_ready) return bfail(err, err_size, "HIP context has no runtime");
    HIPCHK(hipSetDevice(c->device), "hipSetDevice");
    HIPCHK(hipStreamSynchronize(c->stream), "stream sync");
    const size_t n = (size_t)c->trace_steps * 11u * UOCR_MOE_TOP_K;
    if (expert_ids != nullptr && c->trace_steps != 0u) {
        HIPCHK(hipMemcpy(expert_ids, c->d_trace, n * 4u, hipMemcpyDeviceToHost), "trace readback");
    }
    if (weights != nullptr && c->trace_steps != 0u) {
        HIPCHK(hipMemcpy(weights, c->d_trace + n, n * 4u, hipMemcpyDeviceToHost), "trace weight readback");
    }
    if (hidden != nullptr) HIPCHK(hipMemcpy(hidden, c->h, H_SIZE * 2u, hipMemcpyDeviceToHost), "hidden readback");
    return 1;
}
