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
hipError_t g_init_error = hipSuccess;
thread_local char g_err[512] = "OK";

void init_stream() {
    g_init_error = hipSetDevice(0);
    if (g_init_error == hipSuccess) g_init_error = hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking);
    if (g_init_error == hipSuccess) g_init_error = hipEventCreate(&g_ev0);
    if (g_init_error == hipSuccess) g_init_error = hipEventCreate(&g_ev1);
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
constexpr size_t WS_APART = WS_STATE + 256u;
constexpr size_t WS_LOGITS = WS_APART + A256(UOCR_ATTN_PARTIAL_FLOATS * 4u);
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
                                          qm(qtype, nullptr, nullptr), nullptr),
                      "lm_head_argmax");
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
                                               qm(m->shared_qtype, m->sup_w, m->sup_s), logits, norm_topk, xx, nw, mid,
                                               smid, wids, wwts),
                       "moe gate/up");
    }
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_moe_down(st, &sl, wids, wwts, mid, qm(m->shared_qtype, m->sdown_w, m->sdown_s),
                                            smid, (const uint16_t *)residual, (uint16_t *)out),
                       "moe down/combine");
    }
    return r;
}

static int set_plan(hipStream_t st, void *workspace, uint32_t cap, uint32_t P, uint32_t g) {
    if (P == 0u || (uint64_t)P + (g < UOCR_K_RING ? g : UOCR_K_RING) > cap) {
        return op_fail(UOCR_ERROR_INVALID_ARGUMENT, "attention plan (prompt %u, generated %u) exceeds cache capacity %u", P,
                       g, cap);
    }
    uocr_step_state *state = ws<uocr_step_state>(workspace, WS_STATE);
    if (g == 0u) return hip_status(uocr_launch_prefill_state(st, state, (int32_t)P - 1), "attention plan");
    return hip_status(uocr_launch_decode_state(st, state, (int32_t)P, (int32_t)g - 1), "attention plan");
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
    int r2 = hip_status(uocr_launch_attention(st, (const uint16_t *)q, (const uint16_t *)k_cache,
                                              (const uint16_t *)v_cache, cache_capacity,
                                              ws<uocr_step_state>(workspace, WS_STATE), ws<float>(workspace, WS_APART)),
                        "attention_decode");
    if (r2 != UOCR_OK) return r2;
    return hip_status(uocr_launch_attn_merge(st, ws<float>(workspace, WS_APART), (uint16_t *)out), "attention merge");
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
    float invf[UOCR_K_HEAD_DIM / 2];
    const float freq_scale = -2.0f * log2f(10000.0f) / (float)UOCR_K_HEAD_DIM;
    for (int d = 0; d < UOCR_K_HEAD_DIM / 2; ++d) invf[d] = exp2f((float)d * freq_scale);
    uocr_step_state *state = ws<uocr_step_state>(workspace, WS_STATE);
    uint16_t *qb = ws<uint16_t>(workspace, WS_Q), *cb = ws<uint16_t>(workspace, WS_CTX);
    int r = set_plan(st, workspace, cache_capacity, prompt_length, generated_count);
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_qkv_rope(st, qm(qtype, wq, sq), qm(qtype, wk, sk), qm(qtype, wv, sv),
                                            (const uint16_t *)hidden, (const uint16_t *)norm_w, invf, state, qb,
                                            (uint16_t *)k_cache, (uint16_t *)v_cache, cache_capacity),
                       "qkv_rope");
    }
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_attention(st, qb, (const uint16_t *)k_cache, (const uint16_t *)v_cache,
                                             cache_capacity, state, ws<float>(workspace, WS_APART)),
                       "attention");
    }
    if (r == UOCR_OK) {
        r = hip_status(uocr_launch_attn_out(st, qm(qtype, wo, so), ws<float>(workspace, WS_APART),
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
    return hip_status(hipMemsetAsync(dst, value, bytes, st), "memset");
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
