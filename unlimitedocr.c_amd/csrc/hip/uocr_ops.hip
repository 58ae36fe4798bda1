/*
 * uocr_ops.hip - operator-level C ABI (include/uocr_hip.h, group 2 and 3).
 *
 * Each operator validates its arguments on the host, then enqueues the same
 * kernels the engine's decode graph uses on one library stream (device 0).
 */
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "uocr_hip.h"
#include "uocr_kernels.h"

namespace {

pthread_once_t g_once = PTHREAD_ONCE_INIT;
hipStream_t g_stream = nullptr;
hipEvent_t g_ev0 = nullptr, g_ev1 = nullptr;
hipGraph_t g_graph = nullptr;
hipGraphExec_t g_graph_exec = nullptr;
hipError_t g_init_error = hipSuccess;
void *g_scratch_dev = nullptr; /* device address of `scratch` on device 0 */
hipError_t g_scratch_err = hipSuccess;
thread_local char g_err[512] = "OK";

void take_scratch_address();

void init_stream() {
    g_init_error = hipSetDevice(0);
    if (g_init_error == hipSuccess) g_init_error = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking);
    if (g_init_error == hipSuccess) g_init_error = hipEventCreate(&g_ev0);
    if (g_init_error == hipSuccess) g_init_error = hipEventCreate(&g_ev1);
    if (g_init_error == hipSuccess) take_scratch_address();
}

int op_fail(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

hipStream_t stream_or_fail(int *status) {
    pthread_once(&g_once, init_stream);
    if (g_init_error != hipSuccess) {
        *status = op_fail(UOCR_ERROR_UNSUPPORTED, "HIP unavailable: %s", hipGetErrorString(g_init_error));
        return nullptr;
    }
    *status = UOCR_OK;
    return g_stream;
}

int hip_status(hipError_t e, const char *what) {
    if (e == hipSuccess) return UOCR_OK;
    if (e == hipErrorInvalidValue) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "%s: invalid argument or shape", what);
    return op_fail(UOCR_ERROR_INTERNAL, "%s: %s", what, hipGetErrorString(e));
}

bool qt_ok(uint32_t q) {
    return q == UOCR_QT_F16 || q == UOCR_QT_Q8 || q == UOCR_QT_Q4;
}

uocr_qmat qm(uint32_t qt, const void *w, const void *s) {
    uocr_qmat m;
    m.w = w;
    m.s = (const uint16_t *)s;
    m.qtype = qt;
    return m;
}

/* workspace layout */
constexpr size_t A256(size_t v) {
    return (v + 255u) & ~(size_t)255u;
}
constexpr size_t WS_STATE = 0;
constexpr size_t WS_APART = WS_STATE + A256(sizeof(uocr_step_state));
constexpr size_t WS_LOGITS = WS_APART + A256(UOCR_ATTN_PARTIAL_FLOATS_WIDE * 4u);
static_assert(UOCR_ATTN_PARTIAL_FLOATS_WIDE >= UOCR_ATTN_PARTIAL_FLOATS, "wide partials layout");
constexpr size_t WS_LPART = WS_LOGITS + 256u;
constexpr size_t WS_IDS = WS_LPART + A256(UOCR_LM_PARTIAL_WORDS * 4u);
constexpr size_t WS_WTS = WS_IDS + 256u;
constexpr size_t WS_MID = WS_WTS + 256u;
constexpr size_t WS_SMID = WS_MID + A256(6848u * 2u);
constexpr size_t WS_Q = WS_SMID + A256(1792u * 2u);
constexpr size_t WS_CTX = WS_Q + A256(1280u * 2u);
constexpr size_t WS_TOTAL = WS_CTX + A256(1280u * 2u);

template <typename T>
T *ws(void *base, size_t off) {
    return (T *)((uint8_t *)base + off);
}

}  // namespace

#define STREAM_OR_RETURN(s)             \
    int st_ = UOCR_OK;                  \
    hipStream_t s = stream_or_fail(&st_); \
    if (s == nullptr) return st_

extern "C" size_t uocr_op_workspace_bytes(void) {
    return WS_TOTAL;
}

extern "C" int uocr_op_gemv(uint32_t qtype, const void *w, const void *s, uint32_t rows, uint32_t k, const void *x,
                            const void *residual, void *y) {
    if (!qt_ok(qtype)) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "unsupported qtype %u", qtype);
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_gemv(st, qm(qtype, w, s), rows, k, (const uint16_t *)x, nullptr,
                                       (const uint16_t *)residual, (uint16_t *)y),
                      "gemv");
}

extern "C" int uocr_op_swiglu(uint32_t qtype, const void *gw, const void *gs, const void *uw, const void *us,
                              uint32_t rows, uint32_t k, const void *x, const void *norm_w, void *mid) {
    if (!qt_ok(qtype)) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "unsupported qtype %u", qtype);
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_swiglu(st, qm(qtype, gw, gs), qm(qtype, uw, us), rows, k, (const uint16_t *)x,
                                         (const uint16_t *)norm_w, (uint16_t *)mid),
                      "swiglu");
}

extern "C" int uocr_op_rmsnorm(const void *x, const void *w, uint32_t n, void *y) {
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_rmsnorm(st, (const uint16_t *)x, (const uint16_t *)w, n, (uint16_t *)y), "rmsnorm");
}

extern "C" int uocr_op_lm_head_argmax(uint32_t qtype, const void *w, const void *s, uint32_t vocab, const void *x,
                                      const void *norm_w, void *workspace, int32_t *token, float *score) {
    if (!qt_ok(qtype) || workspace == nullptr || token == nullptr || vocab == 0u) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid lm_head_argmax arguments");
    }
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_lm_head(st, qm(qtype, w, s), vocab, (const uint16_t *)x, (const uint16_t *)norm_w,
                                          ws<uint32_t>(workspace, WS_LPART), nullptr, 0, token, score,
                                          qm(qtype, nullptr, nullptr), nullptr, nullptr),
                      "lm_head_argmax");
}

extern "C" int uocr_op_lm_head_keys(uint32_t qtype, const void *w, const void *s, uint32_t vocab, const void *x,
                                    const void *norm_w, uint64_t *keys) {
    if (!qt_ok(qtype) || keys == nullptr || vocab == 0u) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid lm_head_keys arguments");
    }
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_lm_keys(st, qm(qtype, w, s), vocab, (const uint16_t *)x, (const uint16_t *)norm_w,
                                          keys, nullptr, 0, nullptr),
                      "lm_head_keys");
}

extern "C" int uocr_op_router(const void *router_w, const void *x, const void *norm_w, int norm_topk, void *workspace,
                              uint32_t *ids, float *weights) {
    if (workspace == nullptr) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "router needs a workspace");
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_router(st, (const uint16_t *)router_w, (const uint16_t *)x, (const uint16_t *)norm_w,
                                         norm_topk, ws<float>(workspace, WS_LOGITS), ids, weights),
                      "router");
}

extern "C" int uocr_op_moe_ffn(const uocr_op_moe_weights *m, const void *x, const void *norm_w, const void *residual,
                               int norm_topk, void *workspace, void *out, uint32_t *ids, float *weights) {
    if (m == nullptr || x == nullptr || residual == nullptr || workspace == nullptr || out == nullptr ||
        !qt_ok(m->expert_qtype) || !qt_ok(m->shared_qtype)) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid moe_ffn arguments");
    }
    STREAM_OR_RETURN(st);
    uocr_expert_slab sl;
    sl.gate = qm(m->expert_qtype, m->gate_w, m->gate_s);
    sl.up = qm(m->expert_qtype, m->up_w, m->up_s);
    sl.down = qm(m->expert_qtype, m->down_w, m->down_s);
    sl.gu_w_stride = m->gu_w_stride;
    sl.gu_s_stride = m->gu_s_stride;
    sl.dn_w_stride = m->dn_w_stride;
    sl.dn_s_stride = m->dn_s_stride;
    uint32_t *wids = ids != nullptr ? ids : ws<uint32_t>(workspace, WS_IDS);
    float *wwts = weights != nullptr ? weights : ws<float>(workspace, WS_WTS);
    float *logits = ws<float>(workspace, WS_LOGITS);
    uint16_t *mid = ws<uint16_t>(workspace, WS_MID), *smid = ws<uint16_t>(workspace, WS_SMID);
    const uint16_t *xx = (const uint16_t *)x, *nw = (const uint16_t *)norm_w;
    int r = hip_status(uocr_launch_router_logits(st, (const uint16_t *)m->router, xx, nw, logits), "moe router");
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_moe_gate_up(st, &sl, qm(m->shared_qtype, m->sgate_w, m->sgate_s),
                                               qm(m->shared_qtype, m->sup_w, m->sup_s), logits, nullptr, norm_topk, xx, nw, mid,
                                               smid, wids, wwts, nullptr, nullptr),
                       "moe gate/up");
    }
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_moe_down(st, &sl, wids, wwts, mid, qm(m->shared_qtype, m->sdown_w, m->sdown_s),
                                            smid, (const uint16_t *)residual, (uint16_t *)out, nullptr, nullptr),
                       "moe down/combine");
    }
    return r;
}

extern "C" int uocr_op_moe_gate_up(const uocr_op_moe_weights *m, const float *logits, const void *x, const void *norm_w,
                                   int norm_topk, void *mid, void *smid, uint32_t *ids, float *weights) {
    if (m == nullptr || logits == nullptr || x == nullptr || mid == nullptr || smid == nullptr || ids == nullptr ||
        weights == nullptr || !qt_ok(m->expert_qtype) || !qt_ok(m->shared_qtype)) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid moe_gate_up arguments");
    }
    STREAM_OR_RETURN(st);
    uocr_expert_slab sl;
    sl.gate = qm(m->expert_qtype, m->gate_w, m->gate_s);
    sl.up = qm(m->expert_qtype, m->up_w, m->up_s);
    sl.down = qm(m->expert_qtype, m->down_w, m->down_s);
    sl.gu_w_stride = m->gu_w_stride;
    sl.gu_s_stride = m->gu_s_stride;
    sl.dn_w_stride = m->dn_w_stride;
    sl.dn_s_stride = m->dn_s_stride;
    return hip_status(uocr_launch_moe_gate_up(st, &sl, qm(m->shared_qtype, m->sgate_w, m->sgate_s),
                                              qm(m->shared_qtype, m->sup_w, m->sup_s), logits, nullptr, norm_topk,
                                              (const uint16_t *)x, (const uint16_t *)norm_w, (uint16_t *)mid,
                                              (uint16_t *)smid, ids, weights, nullptr, nullptr),
                      "moe gate/up");
}

static void rope_inv_freq(float *invf) {
    const float freq_scale = -2.0f * log2f(10000.0f) / (float)UOCR_K_HEAD_DIM;
    for (int d = 0; d < UOCR_K_HEAD_DIM / 2; ++d) invf[d] = exp2f((float)d * freq_scale);
}

static int plan_ok(uint32_t cap, uint32_t P, uint32_t g) {
    if (P == 0u || (uint64_t)P + (g < UOCR_K_RING ? g : UOCR_K_RING) > cap) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "attention plan (prompt %u, generated %u) exceeds cache capacity %u", P,
                       g, cap);
    }
    return UOCR_OK;
}

static int set_plan(hipStream_t st, void *workspace, uint32_t cap, uint32_t P, uint32_t g) {
    const int r = plan_ok(cap, P, g);
    if (r != UOCR_OK) return r;
    float invf[UOCR_K_HEAD_DIM / 2];
    rope_inv_freq(invf);
    uocr_step_state *state = ws<uocr_step_state>(workspace, WS_STATE);
    if (g == 0u) return hip_status(uocr_launch_prefill_state(st, state, (int32_t)P - 1, invf), "attention plan");
    return hip_status(uocr_launch_decode_state(st, state, (int32_t)P, (int32_t)g - 1, invf), "attention plan");
}

/* Blocks per head of the operators' decode attention (wide partials
 * layout): enough splits that each block's K/V range is small, at most one
 * block per CU (10 heads x 25 splits = 250 blocks for 256 CUs); short
 * caches keep 16.  UOCR_OP_ATT_SPLITS (1-32) overrides it, for measurement. */
static uint32_t op_att_splits(uint32_t cap) {
    static const int forced = [] {
        const char *e = getenv("UOCR_OP_ATT_SPLITS");
        const int v = e != nullptr ? atoi(e) : 0;
        return v >= 1 && v <= UOCR_K_ATTN_SPLITS_WIDE ? v : 0;
    }();
    if (forced != 0) return (uint32_t)forced;
    return cap >= 2048u ? 25u : 16u;
}

extern "C" int uocr_op_attention_decode(const void *q, const void *k_cache, const void *v_cache,
                                        uint32_t cache_capacity, uint32_t prompt_length, uint32_t generated_count,
                                        void *workspace, void *out) {
    if (q == nullptr || k_cache == nullptr || v_cache == nullptr || workspace == nullptr || out == nullptr) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid attention_decode arguments");
    }
    STREAM_OR_RETURN(st);
    const int r = set_plan(st, workspace, cache_capacity, prompt_length, generated_count);
    if (r != UOCR_OK) return r;
    int r2 = hip_status(uocr_launch_attention_wide(st, (const uint16_t *)q, (const uint16_t *)k_cache,
                                                   (const uint16_t *)v_cache, cache_capacity,
                                                   ws<uocr_step_state>(workspace, WS_STATE),
                                                   ws<float>(workspace, WS_APART), op_att_splits(cache_capacity)),
                        "attention_decode");
    if (r2 != UOCR_OK) return r2;
    return hip_status(uocr_launch_attn_merge_wide(st, ws<float>(workspace, WS_APART), (uint16_t *)out),
                      "attention merge");
}

extern "C" int uocr_op_attention_block(uint32_t qtype, const void *wq, const void *sq, const void *wk, const void *sk,
                                       const void *wv, const void *sv, const void *wo, const void *so,
                                       const void *hidden, const void *norm_w, void *k_cache, void *v_cache,
                                       uint32_t cache_capacity, uint32_t prompt_length, uint32_t generated_count,
                                       void *workspace, void *out) {
    if (!qt_ok(qtype) || hidden == nullptr || norm_w == nullptr || workspace == nullptr || out == nullptr ||
        generated_count == 0u) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid attention_block arguments");
    }
    STREAM_OR_RETURN(st);
    uocr_step_state *state = ws<uocr_step_state>(workspace, WS_STATE);
    uint16_t *qb = ws<uint16_t>(workspace, WS_Q), *cb = ws<uint16_t>(workspace, WS_CTX);
    /* the step plan (slot, RoPE, attention length) is computed by the QKV
     * launch itself: one launch fewer than a separate plan kernel */
    int r = plan_ok(cache_capacity, prompt_length, generated_count);
    if (r == UOCR_OK) {
        float invf[UOCR_K_HEAD_DIM / 2];
        rope_inv_freq(invf);
        r = hip_status(uocr_launch_qkv_rope_plan(st, qm(qtype, wq, sq), qm(qtype, wk, sk), qm(qtype, wv, sv),
                                                 (const uint16_t *)hidden, (const uint16_t *)norm_w, state, qb,
                                                 (uint16_t *)k_cache, (uint16_t *)v_cache, cache_capacity,
                                                 (int32_t)prompt_length, (int32_t)generated_count - 1, invf),
                       "qkv_rope");
    }
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_attention_wide(st, qb, (const uint16_t *)k_cache, (const uint16_t *)v_cache,
                                                  cache_capacity, state, ws<float>(workspace, WS_APART),
                                                  op_att_splits(cache_capacity)),
                       "attention");
    }
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_attn_out_wide(st, qm(qtype, wo, so), ws<float>(workspace, WS_APART),
                                                 (const uint16_t *)hidden, (uint16_t *)out, cb),
                       "o_proj");
    }
    return r;
}

extern "C" int uocr_op_embed(uint32_t qtype, const void *w, const void *s, uint32_t vocab, const int32_t *token,
                             void *out) {
    if (!qt_ok(qtype) || token == nullptr) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid embed arguments");
    STREAM_OR_RETURN(st);
    return hip_status(uocr_launch_embed(st, qm(qtype, w, s), vocab, token, nullptr, (uint16_t *)out), "embed");
}

/* ---- prefill operators ------------------------------------------------------ */

extern "C" int uocr_op_gemm(uint32_t qtype, const void *w, const void *s, uint32_t m, uint32_t n, uint32_t k,
                            const void *x, const void *residual, void *y) {
    if (!qt_ok(qtype) || w == nullptr || x == nullptr || y == nullptr || m == 0u || n == 0u || k == 0u ||
        k % 64u != 0u || (qtype != UOCR_QT_F16 && s == nullptr)) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid gemm arguments (k must be a multiple of 64)");
    }
    STREAM_OR_RETURN(st);
    uocr_gemm_desc d;
    memset(&d, 0, sizeof(d));
    d.A = (const uint16_t *)x;
    d.lda = k;
    d.M = m;
    d.N = n;
    d.K = k;
    d.W[0] = qm(qtype, w, s);
    d.out = y;
    d.ldo = n;
    d.res = (const uint16_t *)residual;
    d.ldr = n;
    return hip_status(uocr_launch_gemm(st, UOCR_GEMM_F16, &d), "gemm");
}

/* Split-K partials of the vision linear: grown on demand, kept until the
 * process ends (outgrown buffers too, since captured graphs may reference
 * them; one current buffer per process, so concurrent calls are not
 * supported).  Only long-K GEMMs on grids under half a block per CU split K
 * (at least 4 K steps per split, at most 8 splits): the partials round trip
 * and the reduce launch cost more than the unsplit kernel elsewhere (257 x
 * 4096 -> 1024: 56 -> 20 us split; 640 x 1024 -> 3072: 28 us split against
 * 14-20 us unsplit). */
static float *g_vision_part = nullptr;
static size_t g_vision_part_bytes = 0;
/* Guards the lazily allocated operator buffers (g_vision_part, the prefill
 * attention partials): held from the size check through the launch, so two
 * threads never allocate twice or launch into a buffer being replaced; the
 * launches then serialise on the operator stream. */
static pthread_mutex_t g_lazy_mu = PTHREAD_MUTEX_INITIALIZER;
struct lazy_lock {
    lazy_lock() { pthread_mutex_lock(&g_lazy_mu); }
    ~lazy_lock() { pthread_mutex_unlock(&g_lazy_mu); }
};

static uint32_t vision_ksplit(uint32_t m, uint32_t n, uint32_t k) {
    const uint32_t blocks = ((m + 63u) / 64u) * ((n + 127u) / 128u), steps = k / 64u;
    if (blocks >= 128u || steps < 32u) return 1u;
    uint32_t s = 1u;
    while (s < 8u && blocks * s < 512u && steps / (2u * s) >= 4u) s *= 2u;
    return s;
}

extern "C" int uocr_op_vision_linear(uint32_t qtype, const void *w, const void *s, const void *bias, uint32_t m,
                                     uint32_t k, uint32_t n, uint32_t act, uint32_t split, const void *x, void *dst0,
                                     void *dst1, void *dst2) {
    if (!qt_ok(qtype) || w == nullptr || bias == nullptr || x == nullptr || dst0 == nullptr || m == 0u || n == 0u ||
        k == 0u || k % 64u != 0u || (qtype != UOCR_QT_F16 && s == nullptr) || act > UOCR_VISION_ACT_GELU_ERF ||
        (split != 0u && (n != 3u * split || dst1 == nullptr || dst2 == nullptr))) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT,
                       "invalid vision linear arguments (k % 64 == 0, bias required, split: n == 3 * split)");
    }
    STREAM_OR_RETURN(st);
    uocr_gemm_desc d;
    memset(&d, 0, sizeof(d));
    d.A = (const uint16_t *)x;
    d.lda = k;
    d.M = m;
    d.N = n;
    d.K = k;
    d.W[0] = qm(qtype, w, s);
    d.out = dst0;
    d.ldo = n;
    d.bias = (const uint16_t *)bias;
    d.act = act;
    d.split = split;
    d.out1 = dst1;
    d.out2 = dst2;
    d.ksplit = vision_ksplit(m, n, k);
    lazy_lock lk;
    if (d.ksplit > 1u) {
        const size_t need = (size_t)d.ksplit * m * n * sizeof(float);
        if (need > g_vision_part_bytes) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
                void *p = nullptr;
                /* a smaller buffer is kept, not freed: a graph captured
                 * earlier may still replay into it */
                if (hipMalloc(&p, need) == hipSuccess) {
                    g_vision_part = (float *)p;
                    g_vision_part_bytes = need;
                }
            }
        }
        /* no room (or a capture in progress): the unsplit kernel, same result
         * up to fp32 summation order */
        if (need > g_vision_part_bytes) d.ksplit = 1u;
        d.part = g_vision_part;
    }
    return hip_status(uocr_launch_gemm(st, UOCR_GEMM_VISION, &d), "vision linear");
}

extern "C" int uocr_op_prefill_attention(const void *q, const void *k_cache, const void *v_cache,
                                         uint32_t cache_capacity, uint32_t prompt_length, void *ctx) {
    if (q == nullptr || k_cache == nullptr || v_cache == nullptr || ctx == nullptr || prompt_length == 0u ||
        prompt_length > cache_capacity) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid prefill_attention arguments");
    }
    STREAM_OR_RETURN(st);
    /* key-split partials: allocated on first need outside graph capture and
     * kept (calls must not overlap); without them the unsplit kernel runs */
    static float *fa_ws = nullptr;
    lazy_lock lk;
    if (fa_ws == nullptr) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
            void *p = nullptr;
            if (hipMalloc(&p, uocr_flash_attn_ws_bytes()) == hipSuccess) fa_ws = (float *)p;
        }
    }
    return hip_status(uocr_launch_flash_attn(st, (const uint16_t *)q, (const uint16_t *)k_cache,
                                             (const uint16_t *)v_cache, cache_capacity, prompt_length, (uint16_t *)ctx,
                                             fa_ws),
                      "prefill_attention");
}

namespace {
/* workspace layout of uocr_op_moe_ffn_rows for P rows */
struct MoeRowsWs {
    size_t xn = 0, logits = 0, ids = 0, wts = 0, offsets = 0, te = 0, ts0 = 0, ts1 = 0, nt = 0, ltok = 0, lpair = 0,
           smid = 0, sout = 0, rmid = 0, y = 0, total = 0;
    uint32_t max_tiles = 0;
    explicit constexpr MoeRowsWs(size_t P) {
        const size_t PK = P * 6u;
        max_tiles = (uint32_t)((PK + 63u) / 64u + 64u);
        size_t o = 0;
        auto take = [&](size_t bytes) {
            const size_t r = o;
            o += A256(bytes);
            return r;
        };
        xn = take(P * 1280u * 2u);
        logits = take(P * 64u * 4u);
        ids = take(PK * 4u);
        wts = take(PK * 4u);
        offsets = take(256u);
        te = take(max_tiles * 4u);
        ts0 = take(max_tiles * 4u);
        ts1 = take(max_tiles * 4u);
        nt = take(4u);
        ltok = take(PK * 4u);
        lpair = take(PK * 4u);
        smid = take(P * 1792u * 2u);
        sout = take(P * 1280u * 2u);
        rmid = take(PK * 896u * 2u);
        y = take(PK * 1280u * 4u);
        total = o;
    }
};
}  // namespace

extern "C" size_t uocr_op_moe_rows_workspace_bytes(uint32_t rows) {
    return MoeRowsWs(rows).total;
}

/* The static scratch of uocr_op_moe_ffn_rows_static: the workspace of
 * UOCR_OP_STATIC_MAX_ROWS rows in a file-scope device array (each device
 * holds its own copy until the process ends).  Host code never passes the
 * array's name to a kernel: it is a host-side stand-in, not a device address.
 * The device address comes from hipGetSymbolAddress, taken once per device
 * with that device current (the operator stream runs on device 0: taken in
 * init_stream). */
constexpr size_t STATIC_SCRATCH_BYTES = 3235840u;
static_assert(MoeRowsWs(UOCR_OP_STATIC_MAX_ROWS).total <= STATIC_SCRATCH_BYTES, "static scratch holds the maximum rows");
static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {
void take_scratch_address() {
    void *p = nullptr;
    g_scratch_err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_dev = g_scratch_err == hipSuccess ? p : nullptr;
}
}  // namespace

static int moe_rows(hipStream_t st, const uocr_op_moe_weights *m, const void *x, const void *norm_w,
                    const void *residual, uint32_t rows, int norm_topk, void *workspace, void *out) {
    const MoeRowsWs L(rows);
    uint8_t *b = (uint8_t *)workspace;
    const uint32_t P = rows;
    uint16_t *xn = (uint16_t *)(b + L.xn);
    int r = UOCR_OK;
    if (norm_w != nullptr) {
        r = hip_status(uocr_launch_rows_rmsnorm(st, (const uint16_t *)x, (const uint16_t *)norm_w, P, xn), "rmsnorm");
    } else {
        r = hip_status(hipMemcpyAsync(xn, x, (size_t)P * 1280u * 2u, hipMemcpyDeviceToDevice, st), "copy");
    }
    uocr_gemm_desc d;
    memset(&d, 0, sizeof(d));
    d.A = xn;
    d.lda = 1280u;
    d.M = P;
    d.N = 64u;
    d.K = 1280u;
    d.W[0] = qm(UOCR_QT_F16, m->router, nullptr);
    d.out = b + L.logits;
    d.ldo = 64u;
    if (r == UOCR_OK) r = hip_status(uocr_launch_gemm(st, UOCR_GEMM_F32, &d), "router gemm");
    int32_t *ids = (int32_t *)(b + L.ids);
    float *wts = (float *)(b + L.wts);
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_route_rows(st, (const float *)(b + L.logits), P, norm_topk, ids, wts,
                                              (int32_t *)(b + L.offsets), (int32_t *)(b + L.te), (int32_t *)(b + L.ts0),
                                              (int32_t *)(b + L.ts1), (int32_t *)(b + L.nt), (int32_t *)(b + L.ltok),
                                              (int32_t *)(b + L.lpair)),
                       "routing");
    }
    d.N = 1792u;
    d.W[0] = qm(m->shared_qtype, m->sgate_w, m->sgate_s);
    d.W[1] = qm(m->shared_qtype, m->sup_w, m->sup_s);
    d.out = b + L.smid;
    d.ldo = 1792u;
    if (r == UOCR_OK) r = hip_status(uocr_launch_gemm(st, UOCR_GEMM_SWIGLU, &d), "shared gate/up gemm");
    uocr_gemm_desc sd;
    memset(&sd, 0, sizeof(sd));
    sd.A = (const uint16_t *)(b + L.smid);
    sd.lda = 1792u;
    sd.M = P;
    sd.N = 1280u;
    sd.K = 1792u;
    sd.W[0] = qm(m->shared_qtype, m->sdown_w, m->sdown_s);
    sd.out = b + L.sout;
    sd.ldo = 1280u;
    if (r == UOCR_OK) r = hip_status(uocr_launch_gemm(st, UOCR_GEMM_F16, &sd), "shared down gemm");
    uocr_gemm_desc gd;
    memset(&gd, 0, sizeof(gd));
    gd.A = xn;
    gd.lda = 1280u;
    gd.N = 896u;
    gd.K = 1280u;
    gd.W[0] = qm(m->expert_qtype, m->gate_w, m->gate_s);
    gd.W[1] = qm(m->expert_qtype, m->up_w, m->up_s);
    gd.w_stride = m->gu_w_stride;
    gd.s_stride = m->gu_s_stride;
    gd.a_idx = (const int32_t *)(b + L.ltok);
    gd.o_idx = (const int32_t *)(b + L.lpair);
    gd.tile_e = (const int32_t *)(b + L.te);
    gd.tile_s0 = (const int32_t *)(b + L.ts0);
    gd.tile_s1 = (const int32_t *)(b + L.ts1);
    gd.ntiles = (const int32_t *)(b + L.nt);
    gd.max_tiles = L.max_tiles;
    gd.out = b + L.rmid;
    gd.ldo = 896u;
    if (r == UOCR_OK) r = hip_status(uocr_launch_gemm(st, UOCR_GEMM_SWIGLU, &gd), "routed gate/up gemm");
    uocr_gemm_desc dd = gd;
    dd.A = (const uint16_t *)(b + L.rmid);
    dd.lda = 896u;
    dd.N = 1280u;
    dd.K = 896u;
    dd.W[0] = qm(m->expert_qtype, m->down_w, m->down_s);
    dd.W[1] = qm(0u, nullptr, nullptr);
    dd.w_stride = m->dn_w_stride;
    dd.s_stride = m->dn_s_stride;
    dd.a_idx = (const int32_t *)(b + L.lpair);
    dd.out = b + L.y;
    dd.ldo = 1280u;
    if (r == UOCR_OK) r = hip_status(uocr_launch_gemm(st, UOCR_GEMM_F32, &dd), "routed down gemm");
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_moe_combine(st, (const float *)(b + L.y), wts, (const uint16_t *)(b + L.sout),
                                               (const uint16_t *)residual, P, (uint16_t *)out),
                       "combine");
    }
    return r;
}

extern "C" int uocr_op_moe_ffn_rows(const uocr_op_moe_weights *m, const void *x, const void *norm_w,
                                    const void *residual, uint32_t rows, int norm_topk, void *workspace, void *out) {
    if (m == nullptr || x == nullptr || residual == nullptr || workspace == nullptr || out == nullptr || rows == 0u ||
        !qt_ok(m->expert_qtype) || !qt_ok(m->shared_qtype) || m->router == nullptr) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid moe_ffn_rows arguments");
    }
    STREAM_OR_RETURN(st);
    return moe_rows(st, m, x, norm_w, residual, rows, norm_topk, workspace, out);
}

extern "C" int uocr_op_moe_ffn_rows_static(const uocr_op_moe_weights *m, const void *x, const void *norm_w,
                                           const void *residual, uint32_t rows, int norm_topk, void *out) {
    if (m == nullptr || x == nullptr || residual == nullptr || out == nullptr || rows == 0u ||
        !qt_ok(m->expert_qtype) || !qt_ok(m->shared_qtype) || m->router == nullptr) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "invalid moe_ffn_rows_static arguments");
    }
    if (rows > UOCR_OP_STATIC_MAX_ROWS) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT,
                       "moe_ffn_rows_static: %u rows exceed the static scratch's maximum of %u rows (use "
                       "uocr_op_moe_ffn_rows with a workspace)",
                       rows, UOCR_OP_STATIC_MAX_ROWS);
    }
    STREAM_OR_RETURN(st);
    if (g_scratch_dev == nullptr) {
        return op_fail(UOCR_ERROR_INTERNAL, "static scratch address unavailable: %s", hipGetErrorString(g_scratch_err));
    }
    return moe_rows(st, m, x, norm_w, residual, rows, norm_topk, g_scratch_dev, out);
}

/* ---- plumbing -------------------------------------------------------------- */

extern "C" int uocr_hip_device_count(void) {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
}

extern "C" void *uocr_hip_alloc(size_t bytes) {
    int st = UOCR_OK;
    if (stream_or_fail(&st) == nullptr) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        op_fail(UOCR_ERROR_OUT_OF_MEMORY, "hipMalloc(%zu) failed", bytes);
        return nullptr;
    }
    /* zeroed on the library stream and waited for (a plain hipMemset runs on
     * the null stream, which the non-blocking library stream does not order
     * against): operator workspaces rely on it, the LM-head selection's keys
     * and ticket counter start at zero */
    if (hipMemsetAsync(p, 0, bytes, g_stream) != hipSuccess || hipStreamSynchronize(g_stream) != hipSuccess) {
        (void)hipFree(p);
        op_fail(UOCR_ERROR_INTERNAL, "hipMemset(%zu) failed", bytes);
        return nullptr;
    }
    return p;
}

extern "C" int uocr_hip_free(void *p) {
    if (p == nullptr) return UOCR_OK;
    return hip_status(hipFree(p), "hipFree");
}

extern "C" int uocr_hip_upload(void *dst, const void *src, size_t bytes) {
    STREAM_OR_RETURN(st);
    int r = hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st), "upload");
    return r == UOCR_OK ? hip_status(hipStreamSynchronize(st), "upload sync") : r;
}

extern "C" int uocr_hip_download(void *dst, const void *src, size_t bytes) {
    STREAM_OR_RETURN(st);
    int r = hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st), "download");
    return r == UOCR_OK ? hip_status(hipStreamSynchronize(st), "download sync") : r;
}

extern "C" int uocr_hip_memset(void *dst, int value, size_t bytes) {
    STREAM_OR_RETURN(st);
    /* a memset recorded into a captured graph has given wrong results on
     * replays after the first: refuse while the operator stream captures */
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t ce = hipStreamIsCapturing(st, &cs);
    if (ce != hipSuccess) return hip_status(ce, "memset capture query");
    if (cs != hipStreamCaptureStatusNone) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "memset refused: the operator stream is capturing a graph");
    }
    return hip_status(hipMemsetAsync(dst, value, bytes, st), "memset");
}

extern "C" int uocr_hip_copy(void *dst, const void *src, size_t bytes) {
    STREAM_OR_RETURN(st);
    return hip_status(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st), "copy");
}

extern "C" int uocr_hip_sync(void) {
    STREAM_OR_RETURN(st);
    return hip_status(hipStreamSynchronize(st), "sync");
}

extern "C" const char *uocr_hip_op_error(void) {
    return g_err;
}

extern "C" int uocr_hip_timer_begin(void) {
    STREAM_OR_RETURN(st);
    return hip_status(hipEventRecord(g_ev0, st), "timer begin");
}

extern "C" float uocr_hip_timer_end_ms(void) {
    int status = UOCR_OK;
    hipStream_t st = stream_or_fail(&status);
    if (st == nullptr) return -1.0f;
    float ms = -1.0f;
    if (hipEventRecord(g_ev1, st) != hipSuccess || hipEventSynchronize(g_ev1) != hipSuccess ||
        hipEventElapsedTime(&ms, g_ev0, g_ev1) != hipSuccess) {
        return -1.0f;
    }
    return ms;
}

extern "C" int uocr_hip_capture_begin(void) {
    STREAM_OR_RETURN(st);
    if (g_graph != nullptr || g_graph_exec != nullptr) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "a graph is held");
    return hip_status(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture begin");
}

extern "C" int uocr_hip_capture_end(void) {
    STREAM_OR_RETURN(st);
    int r = hip_status(hipStreamEndCapture(st, &g_graph), "capture end");
    if (r == UOCR_OK) r = hip_status(hipGraphInstantiate(&g_graph_exec, g_graph, nullptr, nullptr, 0), "instantiate");
    if (r != UOCR_OK) uocr_hip_graph_release();
    return r;
}

extern "C" int uocr_hip_graph_replay(uint32_t times) {
    STREAM_OR_RETURN(st);
    if (g_graph_exec == nullptr) return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "no captured graph");
    for (uint32_t i = 0; i < times; ++i) {
        int r = hip_status(hipGraphLaunch(g_graph_exec, st), "graph launch");
        if (r != UOCR_OK) return r;
    }
    return UOCR_OK;
}

extern "C" int uocr_hip_graph_release(void) {
    if (g_graph_exec != nullptr) (void)hipGraphExecDestroy(g_graph_exec);
    if (g_graph != nullptr) (void)hipGraphDestroy(g_graph);
    g_graph_exec = nullptr;
    g_graph = nullptr;
    return UOCR_OK;
}
