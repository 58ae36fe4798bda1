/*
 * uocr_kernels.hip - hand-written gfx950 (CDNA4, wave64) kernels for the
 * batch-1 decode token loop of the UnlimitedOCR language model.
 *
 * Design (MI355X-first, not a translation of the Metal kernels):
 *  - Batch-1 decode is HBM-bound.  Weights stream once per token with 128-bit
 *    global loads; each lane owns one 16-byte chunk of a row per iteration and
 *    dequantises it in registers (Q4_0 group-half-split nibbles, Q8_0, f16).
 *  - The activation vector is staged once per workgroup in LDS as fp16; when
 *    the consumer of an RMSNorm output is a GEMV, the norm is recomputed in
 *    the GEMV prologue instead of a separate launch (same fp16 values).
 *  - Row dots reduce across the 64-lane wavefront with DPP row permutes
 *    (quad_perm / row_half_mirror / row_mirror) plus 4 readlanes, no LDS.
 *  - RoPE and the KV-cache write are fused into the QKV GEMV epilogue (a
 *    wave owns rows d and d+64 of one head, the split-half rotation pair).
 *  - Decode attention is split-K over the context (32 blocks per head, 16
 *    lanes x 8 dims per cached token) with an online-softmax partial per
 *    block and a last-block log-sum-exp merge, so no second launch is needed.
 *  - The MoE router is one 1024-thread workgroup; the softmax and greedy
 *    top-6 run in a single wavefront (one expert per lane, 64-bit keys of
 *    (probability bits, inverted id) so ties go to the lower id).
 *  - Routed experts are gathered by id from a per-layer expert slab; the down
 *    projection fuses the weighted combine, the shared-expert down GEMV and
 *    the residual add (single fp16 rounding).
 *  - The LM head fuses the final RMSNorm and a two-pass argmax whose second
 *    pass runs in the last block to finish (NaN rows skipped, ties to the
 *    lowest id); it also advances the device-side step state so a captured
 *    decode graph can be replayed per token.
 * Cross-block hand-offs use __threadfence() + a device-scope counter that
 * the last block resets, so every launch leaves its counters at zero and no
 * block ever waits on another.
 */
#include "uocr_kernels.h"

#include <math.h>

typedef _Float16 h16;

#define BLOCK 256
#define NONE_ID 0xffffffffu

/* ------------------------------------------------------------------------ */
/* wavefront / block reductions                                              */
/* ------------------------------------------------------------------------ */

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}

/* Every lane receives the sum over its 16-lane DPP row. */
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);   /* quad_perm [1,0,3,2] */
    v += dpp_f<0x4E>(v);   /* quad_perm [2,3,0,1] */
    v += dpp_f<0x141>(v);  /* row_half_mirror */
    v += dpp_f<0x140>(v);  /* row_mirror */
    return v;
}

__device__ __forceinline__ float lane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

/* Wave-uniform sum of all 64 lanes (all lanes must be active). */
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned lo = __shfl_xor((unsigned)(v & 0xffffffffull), o);
        const unsigned hi = __shfl_xor((unsigned)(v >> 32), o);
        const unsigned long long u = ((unsigned long long)hi << 32) | lo;
        v = u > v ? u : v;
    }
    return v;
}

/* Sum over the block; every thread receives the result. red: >= 16 floats. */
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float silu_f(float g) {
    return g / (1.0f + expf(-g));
}

/* Stage K fp16 activations into LDS; with nw, apply RMSNorm (eps 1e-6):
 * xs[i] = f16(x[i] * inv_rms * nw[i]) (norm.metal:12-40 arithmetic). */
__device__ __forceinline__ void stage_x(h16 *xs, const h16 *x, const h16 *nw, int K, float *red) {
    if (nw != nullptr) {
        float ss = 0.0f;
        for (int i = threadIdx.x; i < K; i += blockDim.x) {
            const float v = (float)x[i];
            ss = fmaf(v, v, ss);
        }
        ss = block_sum(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)K + 1.0e-6f);
        for (int i = threadIdx.x; i < K; i += blockDim.x) xs[i] = (h16)(((float)x[i] * inv) * (float)nw[i]);
    } else {
        const uint4 *src = (const uint4 *)x;
        uint4 *dst = (uint4 *)xs;
        for (int i = threadIdx.x; i < K / 8; i += blockDim.x) dst[i] = src[i];
    }
    __syncthreads();
}

/* ------------------------------------------------------------------------ */
/* 16-byte chunk dequant-dots                                                */
/* ------------------------------------------------------------------------ */

template <int QT>
__device__ __forceinline__ uint32_t row_bytes(uint32_t K) {
    return QT == 4 ? K / 2u : (QT == 3 ? K : 2u * K);
}

template <int QT>
__device__ __forceinline__ uint32_t chunk_group(uint32_t c) {
    return QT == 4 ? (c >> 1) : (c >> 2);
}

union h16x8 {
    uint4 u;
    h16 h[8];
};

template <int QT>
__device__ __forceinline__ float chunk_dot(const uint4 w, const h16 *xs, uint32_t c);

/* Q4_0: chunk c is bytes 16*(c&1)..+15 of 64-column group c>>1; its low
 * nibbles are columns g*64+16*(c&1)+i and its high nibbles the same +32. */
template <>
__device__ __forceinline__ float chunk_dot<4>(const uint4 w, const h16 *xs, uint32_t c) {
    const h16 *xl = xs + (c >> 1) * 64u + (c & 1u) * 16u;
    h16x8 l0, l1, g0, g1;
    l0.u = ((const uint4 *)xl)[0];
    l1.u = ((const uint4 *)xl)[1];
    g0.u = ((const uint4 *)(xl + 32))[0];
    g1.u = ((const uint4 *)(xl + 32))[1];
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    float s = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t byte = (wv[b] >> (8 * i)) & 0xffu;
            const int k = 4 * b + i;
            const float xlo = (float)(k < 8 ? l0.h[k] : l1.h[k - 8]);
            const float xhi = (float)(k < 8 ? g0.h[k] : g1.h[k - 8]);
            s = fmaf((float)((int)(byte & 15u) - 8), xlo, s);
            s = fmaf((float)((int)(byte >> 4) - 8), xhi, s);
        }
    }
    return s;
}

/* Q8_0: chunk c is columns 16c..16c+15 (group c>>2). */
template <>
__device__ __forceinline__ float chunk_dot<3>(const uint4 w, const h16 *xs, uint32_t c) {
    const h16 *xp = xs + 16u * c;
    h16x8 a, b;
    a.u = ((const uint4 *)xp)[0];
    b.u = ((const uint4 *)xp)[1];
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = (int)(int8_t)((wv[j] >> (8 * i)) & 0xffu);
            const int k = 4 * j + i;
            s = fmaf((float)q, (float)(k < 8 ? a.h[k] : b.h[k - 8]), s);
        }
    }
    return s;
}

/* f16: chunk c is columns 8c..8c+7. */
template <>
__device__ __forceinline__ float chunk_dot<1>(const uint4 w, const h16 *xs, uint32_t c) {
    h16x8 a, b;
    a.u = ((const uint4 *)(xs + 8u * c))[0];
    b.u = w;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = fmaf((float)b.h[i], (float)a.h[i], s);
    return s;
}

/* NR independent row dots by one wavefront; loads of all NR rows are issued
 * before any arithmetic.  Returns wave-uniform results. */
template <int QT, int NR>
__device__ __forceinline__ void rows_dot(const uint8_t *const *W, const h16 *const *S, const h16 *const *X,
                                         uint32_t C, uint32_t lane, float *out) {
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;
    for (uint32_t c = lane; c < C; c += 64u) {
        uint4 w[NR];
        float sc[NR];
#pragma unroll
        for (int r = 0; r < NR; ++r) w[r] = *(const uint4 *)(W[r] + 16u * c);
        if (QT != 1) {
#pragma unroll
            for (int r = 0; r < NR; ++r) sc[r] = (float)S[r][chunk_group<QT>(c)];
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const float d = chunk_dot<QT>(w[r], X[r], c);
            acc[r] = QT == 1 ? acc[r] + d : fmaf(d, sc[r], acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) out[r] = wave_sum(acc[r]);
}

/* ------------------------------------------------------------------------ */
/* GEMV family                                                               */
/* ------------------------------------------------------------------------ */

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

template <int QT, int EPI>
__global__ __launch_bounds__(BLOCK) void k_gemv(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                const uint8_t *__restrict__ W2, const h16 *__restrict__ S2,
                                                uint32_t rows, uint32_t K, const h16 *__restrict__ x,
                                                const h16 *__restrict__ nw, const h16 *__restrict__ res,
                                                h16 *__restrict__ y, uint32_t rpb) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_MAX_K];
    __shared__ float red[16];
    stage_x(xs, x, nw, (int)K, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const uint32_t r0 = blockIdx.x * rpb;
    const uint32_t r1 = min(rows, r0 + rpb);
    if (EPI == EPI_SWIGLU) {
        for (uint32_t r = r0 + wave; r < r1; r += 4u) {
            const uint8_t *Wp[2] = {W + (size_t)r * rb, W2 + (size_t)r * rb};
            const h16 *Sp[2] = {S + (size_t)r * G, S2 + (size_t)r * G};
            const h16 *Xp[2] = {xs, xs};
            float d[2];
            rows_dot<QT, 2>(Wp, Sp, Xp, C, lane, d);
            if (lane == 0u) y[r] = (h16)(silu_f(d[0]) * d[1]);
        }
    } else {
        for (uint32_t r = r0 + wave; r < r1; r += 8u) {
            const uint32_t rr = (r + 4u < r1) ? r + 4u : r;
            const uint8_t *Wp[2] = {W + (size_t)r * rb, W + (size_t)rr * rb};
            const h16 *Sp[2] = {S + (size_t)r * G, S + (size_t)rr * G};
            const h16 *Xp[2] = {xs, xs};
            float d[2];
            rows_dot<QT, 2>(Wp, Sp, Xp, C, lane, d);
            if (lane == 0u) {
                if (EPI == EPI_RESID) {
                    y[r] = (h16)(d[0] + (float)res[r]);
                    if (rr != r) y[rr] = (h16)(d[1] + (float)res[rr]);
                } else {
                    y[r] = (h16)d[0];
                    if (rr != r) y[rr] = (h16)d[1];
                }
            }
        }
    }
}

__global__ __launch_bounds__(BLOCK) void k_rmsnorm(const h16 *x, const h16 *nw, uint32_t n, h16 *y) {
    __shared__ float red[16];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = (float)x[i];
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + 1.0e-6f);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) y[i] = (h16)(((float)x[i] * inv) * (float)nw[i]);
}

/* ------------------------------------------------------------------------ */
/* QKV + RoPE + KV write                                                     */
/* ------------------------------------------------------------------------ */

struct RopeTab {
    float f[UOCR_K_HEAD_DIM / 2];
};

/* Work item i (0..1919): matrix m = i/640 (q,k,v), head h, pair d; the wave
 * computes rows h*128+d and h*128+d+64 of matrix m. */
template <int QT>
__global__ __launch_bounds__(BLOCK) void k_qkv_rope(uocr_qmat Q, uocr_qmat Km, uocr_qmat V, const h16 *__restrict__ hin,
                                                    const h16 *__restrict__ nw, RopeTab rope,
                                                    const uocr_step_state *__restrict__ st, h16 *__restrict__ qout,
                                                    h16 *__restrict__ kc, h16 *__restrict__ vc, uint32_t cap,
                                                    uint32_t ipb) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    stage_x(xs, hin, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t K = UOCR_K_HIDDEN, rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const int32_t pos = st->pos;
    const uint32_t ct = (uint32_t)st->cache_token;
    const uint32_t i0 = blockIdx.x * ipb, i1 = min(1920u, i0 + ipb);
    for (uint32_t it = i0 + wave; it < i1; it += 4u) {
        const uint32_t m = it / 640u, rem = it % 640u, h = rem / 64u, d = rem % 64u;
        const uocr_qmat M = m == 0u ? Q : (m == 1u ? Km : V);
        const uint32_t ra = h * 128u + d, rbw = ra + 64u;
        const uint8_t *Wp[2] = {(const uint8_t *)M.w + (size_t)ra * rb, (const uint8_t *)M.w + (size_t)rbw * rb};
        const h16 *Sp[2] = {(const h16 *)M.s + (size_t)ra * G, (const h16 *)M.s + (size_t)rbw * G};
        const h16 *Xp[2] = {xs, xs};
        float dd[2];
        rows_dot<QT, 2>(Wp, Sp, Xp, C, lane, dd);
        if (lane == 0u) {
            const h16 a = (h16)dd[0], b = (h16)dd[1];
            const size_t cix = ((size_t)h * cap + ct) * 128u + d;
            if (m == 2u) {
                vc[cix] = a;
                vc[cix + 64u] = b;
            } else {
                const float ang = (float)pos * rope.f[d];
                const float cs = cosf(ang), sn = sinf(ang);
                const float fa = (float)a, fb = (float)b;
                const h16 na = (h16)(fa * cs - fb * sn), nb = (h16)(fa * sn + fb * cs);
                if (m == 0u) {
                    qout[h * 128u + d] = na;
                    qout[h * 128u + d + 64u] = nb;
                } else {
                    kc[cix] = na;
                    kc[cix + 64u] = nb;
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* split-K decode attention                                                  */
/* ------------------------------------------------------------------------ */

__global__ __launch_bounds__(BLOCK) void k_attention(const h16 *__restrict__ q, const h16 *__restrict__ kc,
                                                     const h16 *__restrict__ vc, uint32_t cap,
                                                     const uocr_step_state *__restrict__ st, float *part,
                                                     uint32_t *cnt, h16 *__restrict__ ctx) {
    __shared__ float sm[16], sl[16];
    __shared__ float sacc[16][UOCR_K_HEAD_DIM];
    __shared__ int is_last;
    const int h = blockIdx.y, s = blockIdx.x, S = gridDim.x;
    const int P = st->attn_prompt, L = st->attn_len, fg = st->first_gen;
    const int chunk = (L + S - 1) / S;
    const int i0 = s * chunk, i1 = min(L, i0 + chunk);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, p = lane & 15;
    const float scale = 0.08838834764831845f; /* 1/sqrt(128) */

    float qv[8];
    {
        h16x8 t;
        t.u = *(const uint4 *)(q + h * 128 + 8 * p);
#pragma unroll
        for (int j = 0; j < 8; ++j) qv[j] = (float)t.h[j];
    }
    float m = -INFINITY, l = 0.0f, acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    const h16 *kh = kc + (size_t)h * cap * 128u;
    const h16 *vh = vc + (size_t)h * cap * 128u;
    for (int i = i0 + wave * 4 + g; i < i1; i += 16) {
        const int t = i < P ? i : P + (fg + i - P) % UOCR_K_RING;
        h16x8 kk, vv;
        kk.u = *(const uint4 *)(kh + (size_t)t * 128u + 8 * p);
        vv.u = *(const uint4 *)(vh + (size_t)t * 128u + 8 * p);
        float d = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) d = fmaf(qv[j], (float)kk.h[j], d);
        const float sc = row16_sum(d) * scale;
        const float mn = fmaxf(m, sc);
        const float corr = expf(m - mn), e = expf(sc - mn);
        l = l * corr + e;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(e, (float)vv.h[j], acc[j] * corr);
        m = mn;
    }
    const int gid = wave * 4 + g;
    if (p == 0) {
        sm[gid] = m;
        sl[gid] = l;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) sacc[gid][8 * p + j] = acc[j];
    __syncthreads();
    if (threadIdx.x < UOCR_K_HEAD_DIM) {
        const int d = threadIdx.x;
        float M = -INFINITY;
        for (int k = 0; k < 16; ++k) M = fmaxf(M, sm[k]);
        float Ls = 0.0f, A = 0.0f;
        if (M != -INFINITY) {
            for (int k = 0; k < 16; ++k) {
                const float f = expf(sm[k] - M);
                Ls = fmaf(sl[k], f, Ls);
                A = fmaf(sacc[k][d], f, A);
            }
        }
        float *pp = part + (size_t)(h * S + s) * (UOCR_K_HEAD_DIM + 2);
        pp[2 + d] = A;
        if (d == 0) {
            pp[0] = M;
            pp[1] = Ls;
        }
        __threadfence();
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(&cnt[h], 1u);
        is_last = (prev == (uint32_t)(S - 1));
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    if (threadIdx.x < UOCR_K_HEAD_DIM) {
        const int d = threadIdx.x;
        const float *ph = part + (size_t)h * S * (UOCR_K_HEAD_DIM + 2);
        float M = -INFINITY;
        for (int k = 0; k < S; ++k) M = fmaxf(M, __builtin_nontemporal_load(ph + (size_t)k * (UOCR_K_HEAD_DIM + 2)));
        float Ls = 0.0f, A = 0.0f;
        for (int k = 0; k < S; ++k) {
            const float *pk = ph + (size_t)k * (UOCR_K_HEAD_DIM + 2);
            const float mk = __builtin_nontemporal_load(pk);
            if (mk == -INFINITY) continue;
            const float f = expf(mk - M);
            Ls = fmaf(__builtin_nontemporal_load(pk + 1), f, Ls);
            A = fmaf(__builtin_nontemporal_load(pk + 2 + d), f, A);
        }
        ctx[h * 128 + d] = (h16)(A / Ls);
    }
    if (threadIdx.x == 0) cnt[h] = 0u;
}

/* ------------------------------------------------------------------------ */
/* MoE router: one 1024-thread workgroup                                     */
/* ------------------------------------------------------------------------ */

__global__ __launch_bounds__(1024) void k_router(const h16 *__restrict__ R, const h16 *__restrict__ x,
                                                 const h16 *__restrict__ nw, int norm_topk, uint32_t *ids,
                                                 float *wts) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    __shared__ float logits[UOCR_K_EXPERTS];
    stage_x(xs, x, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rb = UOCR_K_HIDDEN * 2u, C = rb / 16u;
    {
        const uint32_t e0 = wave * 4u;
        const uint8_t *Wp[4];
        const h16 *Sp[4] = {nullptr, nullptr, nullptr, nullptr};
        const h16 *Xp[4] = {xs, xs, xs, xs};
        for (int j = 0; j < 4; ++j) Wp[j] = (const uint8_t *)R + (size_t)(e0 + j) * rb;
        float d[4];
        rows_dot<1, 4>(Wp, Sp, Xp, C, lane, d);
        if (lane == 0u) {
            for (int j = 0; j < 4; ++j) logits[e0 + j] = d[j];
        }
    }
    __syncthreads();
    if (wave != 0u) return;
    const float lg = logits[lane];
    const float mx = wave_max(lg);
    const float pe = expf(lg - mx);
    const float den = wave_sum(pe);
    const float prob = pe / den;
    unsigned long long key = ((unsigned long long)__float_as_uint(prob) << 32) | (0xffffffffu - lane);
    float sel_w[UOCR_K_TOPK];
    uint32_t sel_id[UOCR_K_TOPK];
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        const unsigned long long best = wave_max_u64(key);
        const uint32_t e = 0xffffffffu - (uint32_t)(best & 0xffffffffull);
        sel_id[r] = e;
        sel_w[r] = __uint_as_float((uint32_t)(best >> 32));
        tot += sel_w[r];
        if (lane == e) key = 0ull;
    }
    if (lane == 0u) {
        for (int r = 0; r < UOCR_K_TOPK; ++r) {
            ids[r] = sel_id[r];
            wts[r] = norm_topk ? sel_w[r] / tot : sel_w[r];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* routed experts                                                            */
/* ------------------------------------------------------------------------ */

template <int QT>
__global__ __launch_bounds__(BLOCK) void k_moe_gate_up(uocr_expert_slab sl, const uint32_t *__restrict__ ids,
                                                       const h16 *__restrict__ x, const h16 *__restrict__ nw,
                                                       h16 *__restrict__ mid, uint32_t rpb) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    stage_x(xs, x, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t I = 896u, K = UOCR_K_HIDDEN, rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const uint32_t rows = UOCR_K_TOPK * I;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min(rows, r0 + rpb);
    for (uint32_t r = r0 + wave; r < r1; r += 4u) {
        const uint32_t rank = r / I, col = r % I;
        const uint32_t e = ids[rank];
        if (e >= UOCR_K_EXPERTS) {
            if (lane == 0u) mid[r] = (h16)0.0f;
            continue;
        }
        const uint8_t *Wp[2] = {(const uint8_t *)sl.gate.w + e * sl.gu_w_stride + (size_t)col * rb,
                                (const uint8_t *)sl.up.w + e * sl.gu_w_stride + (size_t)col * rb};
        const h16 *Sp[2] = {(const h16 *)sl.gate.s + e * sl.gu_s_stride + (size_t)col * G,
                            (const h16 *)sl.up.s + e * sl.gu_s_stride + (size_t)col * G};
        const h16 *Xp[2] = {xs, xs};
        float d[2];
        rows_dot<QT, 2>(Wp, Sp, Xp, C, lane, d);
        if (lane == 0u) mid[r] = (h16)(silu_f(d[0]) * d[1]);
    }
}

template <int QT, int QS>
__global__ __launch_bounds__(BLOCK) void k_moe_down(uocr_expert_slab sl, const uint32_t *__restrict__ ids,
                                                    const float *__restrict__ wts, const h16 *__restrict__ mid,
                                                    uocr_qmat SD, const h16 *__restrict__ smid,
                                                    const h16 *__restrict__ res, h16 *__restrict__ out,
                                                    uint32_t rpb) {
    constexpr uint32_t I = 896u, SI = 1792u;
    __shared__ __attribute__((aligned(16))) h16 ms[UOCR_K_TOPK * I + SI];
    {
        const uint4 *a = (const uint4 *)mid;
        const uint4 *b = (const uint4 *)smid;
        uint4 *d = (uint4 *)ms;
        for (uint32_t i = threadIdx.x; i < UOCR_K_TOPK * I / 8u; i += blockDim.x) d[i] = a[i];
        for (uint32_t i = threadIdx.x; i < SI / 8u; i += blockDim.x) d[UOCR_K_TOPK * I / 8u + i] = b[i];
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t e[UOCR_K_TOPK];
    float w[UOCR_K_TOPK];
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        const uint32_t id = ids[r];
        e[r] = id < UOCR_K_EXPERTS ? id : 0u;
        w[r] = id < UOCR_K_EXPERTS ? wts[r] : 0.0f;
    }
    const uint32_t rbD = row_bytes<QT>(I), CD = rbD / 16u, GD = I / 64u;
    const uint32_t rbS = row_bytes<QS>(SI), CS = rbS / 16u, GS = SI / 64u;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min((uint32_t)UOCR_K_HIDDEN, r0 + rpb);
    for (uint32_t c = r0 + wave; c < r1; c += 4u) {
        const uint8_t *Wp[UOCR_K_TOPK];
        const h16 *Sp[UOCR_K_TOPK];
        const h16 *Xp[UOCR_K_TOPK];
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) {
            Wp[r] = (const uint8_t *)sl.down.w + e[r] * sl.dn_w_stride + (size_t)c * rbD;
            Sp[r] = (const h16 *)sl.down.s + e[r] * sl.dn_s_stride + (size_t)c * GD;
            Xp[r] = ms + r * I;
        }
        float d[UOCR_K_TOPK];
        rows_dot<QT, UOCR_K_TOPK>(Wp, Sp, Xp, CD, lane, d);
        const uint8_t *Ws[1] = {(const uint8_t *)SD.w + (size_t)c * rbS};
        const h16 *Ss[1] = {(const h16 *)SD.s + (size_t)c * GS};
        const h16 *Xs[1] = {ms + UOCR_K_TOPK * I};
        float sd[1];
        rows_dot<QS, 1>(Ws, Ss, Xs, CS, lane, sd);
        if (lane == 0u) {
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < UOCR_K_TOPK; ++r) acc = fmaf(w[r], d[r], acc);
            out[c] = (h16)(acc + (float)(h16)sd[0] + (float)res[c]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* LM head + argmax                                                          */
/* ------------------------------------------------------------------------ */

__device__ __forceinline__ bool better(float s, uint32_t id, float bs, uint32_t bid) {
    return id != NONE_ID && (bid == NONE_ID || s > bs || (s == bs && id < bid));
}

template <int QT>
__global__ __launch_bounds__(BLOCK) void k_lm_head(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                   uint32_t vocab, const h16 *__restrict__ x,
                                                   const h16 *__restrict__ nw, uint32_t *part, uint32_t *cnt,
                                                   uocr_step_state *st, int advance, int32_t *tokens,
                                                   float *scores, uint32_t rpb) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    __shared__ float bsc[BLOCK];
    __shared__ uint32_t bidv[BLOCK];
    __shared__ int is_last;
    stage_x(xs, x, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t K = UOCR_K_HIDDEN, rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min(vocab, r0 + rpb);
    float bs = -INFINITY;
    uint32_t bid = NONE_ID;
    for (uint32_t r = r0 + wave; r < r1; r += 8u) {
        const uint32_t rr = (r + 4u < r1) ? r + 4u : r;
        const uint8_t *Wp[2] = {W + (size_t)r * rb, W + (size_t)rr * rb};
        const h16 *Sp[2] = {S + (size_t)r * G, S + (size_t)rr * G};
        const h16 *Xp[2] = {xs, xs};
        float d[2];
        rows_dot<QT, 2>(Wp, Sp, Xp, C, lane, d);
        if (!isnan(d[0]) && better(d[0], r, bs, bid)) {
            bs = d[0];
            bid = r;
        }
        if (rr != r && !isnan(d[1]) && better(d[1], rr, bs, bid)) {
            bs = d[1];
            bid = rr;
        }
    }
    if (lane == 0u) {
        bsc[wave] = bs;
        bidv[wave] = bid;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = -INFINITY;
        uint32_t bi = NONE_ID;
        for (int i = 0; i < BLOCK / 64; ++i) {
            if (better(bsc[i], bidv[i], b, bi)) {
                b = bsc[i];
                bi = bidv[i];
            }
        }
        part[2u * blockIdx.x] = __float_as_uint(b);
        part[2u * blockIdx.x + 1u] = bi;
        __threadfence();
        const uint32_t prev = atomicAdd(cnt, 1u);
        is_last = (prev == gridDim.x - 1u);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    float b = -INFINITY;
    uint32_t bi = NONE_ID;
    for (uint32_t i = threadIdx.x; i < gridDim.x; i += blockDim.x) {
        const float s = __uint_as_float(__builtin_nontemporal_load(part + 2u * i));
        const uint32_t id = __builtin_nontemporal_load(part + 2u * i + 1u);
        if (better(s, id, b, bi)) {
            b = s;
            bi = id;
        }
    }
    bsc[threadIdx.x] = b;
    bidv[threadIdx.x] = bi;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < BLOCK; ++i) {
            if (better(bsc[i], bidv[i], b, bi)) {
                b = bsc[i];
                bi = bidv[i];
            }
        }
        const int32_t id = bi == NONE_ID ? 0 : (int32_t)bi;
        const int32_t t = st != nullptr ? st->t : 0;
        tokens[t] = id;
        if (scores != nullptr) scores[t] = bi == NONE_ID ? -INFINITY : b;
        if (st != nullptr && advance) {
            const int32_t P = st->prompt_len;
            const int32_t gcount = t + 1;
            const int32_t live = gcount < UOCR_K_RING ? gcount : UOCR_K_RING;
            st->cur_token = id;
            st->pos = P + t;
            st->cache_token = P + (t % UOCR_K_RING);
            st->attn_prompt = P;
            st->attn_len = P + live;
            st->first_gen = gcount - live;
            st->t = t + 1;
        }
        *cnt = 0u;
    }
}

/* ------------------------------------------------------------------------ */
/* embedding gather, state                                                   */
/* ------------------------------------------------------------------------ */

template <int QT>
__device__ __forceinline__ void k_embed_row_body(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                 uint32_t vocab, int32_t tok, h16 *__restrict__ out) {
    const uint32_t K = UOCR_K_HIDDEN;
    for (uint32_t c = threadIdx.x; c < K; c += blockDim.x) {
        float v = 0.0f;
        if (tok >= 0 && (uint32_t)tok < vocab) {
            const size_t r = (size_t)tok;
            if (QT == 1) {
                v = (float)((const h16 *)W)[r * K + c];
            } else {
                const float sc = (float)S[r * (K / 64u) + c / 64u];
                if (QT == 3) {
                    v = (float)((const int8_t *)W)[r * K + c] * sc;
                } else {
                    const uint32_t j = c % 64u;
                    const uint8_t b = W[r * (K / 2u) + (c / 64u) * 32u + (j & 31u)];
                    v = (float)((int)(j < 32u ? (b & 15u) : (b >> 4)) - 8) * sc;
                }
            }
        }
        out[c] = (h16)v;
    }
}

template <int QT>
__global__ __launch_bounds__(BLOCK) void k_embed(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                 uint32_t vocab, const int32_t *token,
                                                 const uocr_step_state *st, h16 *__restrict__ out) {
    k_embed_row_body<QT>(W, S, vocab, token != nullptr ? token[0] : st->cur_token, out);
}

/* Text rows of the prompt embedding: row b = dequant(E[ids[b]]) unless
 * mask[b] (image rows are placed by the host). */
template <int QT>
__global__ __launch_bounds__(BLOCK) void k_embed_rows(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                      uint32_t vocab, const int32_t *__restrict__ ids,
                                                      const uint8_t *__restrict__ mask, h16 *__restrict__ out) {
    const uint32_t b = blockIdx.x;
    if (mask != nullptr && mask[b] != 0u) return;
    k_embed_row_body<QT>(W, S, vocab, ids[b], out + (size_t)b * UOCR_K_HIDDEN);
}

/* One replayable prefill step: position i = st->t; copy prompt row i into h
 * and set the causal-prefix attention plan; then st->t = i + 1. */
__global__ __launch_bounds__(BLOCK) void k_prefill_next(uocr_step_state *st, const h16 *__restrict__ prompt,
                                                        h16 *__restrict__ h) {
    const int32_t i = st->t;
    const uint4 *src = (const uint4 *)(prompt + (size_t)i * UOCR_K_HIDDEN);
    uint4 *dst = (uint4 *)h;
    for (uint32_t c = threadIdx.x; c < UOCR_K_HIDDEN / 8u; c += blockDim.x) dst[c] = src[c];
    __syncthreads();
    if (threadIdx.x == 0) {
        st->pos = i;
        st->cache_token = i;
        st->attn_prompt = i + 1;
        st->attn_len = i + 1;
        st->first_gen = 0;
        st->t = i + 1;
    }
}

__global__ void k_prefill_state(uocr_step_state *st, int32_t i) {
    st->pos = i;
    st->cache_token = i;
    st->attn_prompt = i + 1;
    st->attn_len = i + 1;
    st->first_gen = 0;
}

__global__ void k_decode_state(uocr_step_state *st, int32_t P, int32_t t) {
    const int32_t gcount = t + 1;
    const int32_t live = gcount < UOCR_K_RING ? gcount : UOCR_K_RING;
    st->t = t;
    st->prompt_len = P;
    st->pos = P + t;
    st->cache_token = P + (t % UOCR_K_RING);
    st->attn_prompt = P;
    st->attn_len = P + live;
    st->first_gen = gcount - live;
}

/* ------------------------------------------------------------------------ */
/* launchers                                                                 */
/* ------------------------------------------------------------------------ */

static bool qt_ok(uint32_t q) {
    return q == UOCR_QT_F16 || q == UOCR_QT_Q8 || q == UOCR_QT_Q4;
}

static bool mat_ok(uocr_qmat m) {
    return m.w != nullptr && qt_ok(m.qtype) && (m.qtype == UOCR_QT_F16 || m.s != nullptr);
}

static uint32_t rows_per_block(uint32_t rows, uint32_t target_blocks) {
    uint32_t rpb = (rows + target_blocks - 1u) / target_blocks;
    rpb = (rpb + 3u) & ~3u;
    return rpb < 4u ? 4u : rpb;
}

#define DISPATCH_QT(qt, F, ...)                                      \
    do {                                                             \
        switch (qt) {                                                \
            case UOCR_QT_F16: F<1>(__VA_ARGS__); break;              \
            case UOCR_QT_Q8: F<3>(__VA_ARGS__); break;               \
            default: F<4>(__VA_ARGS__); break;                       \
        }                                                            \
    } while (0)

template <int QT>
static void launch_gemv_qt(hipStream_t st, int epi, uocr_qmat W, uocr_qmat W2, uint32_t rows, uint32_t K,
                           const uint16_t *x, const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    const uint32_t rpb = rows_per_block(rows, 512u);
    const dim3 grid((rows + rpb - 1u) / rpb);
    const uint8_t *w = (const uint8_t *)W.w, *w2 = (const uint8_t *)W2.w;
    const h16 *s = (const h16 *)W.s, *s2 = (const h16 *)W2.s;
    if (epi == EPI_SWIGLU) {
        hipLaunchKernelGGL((k_gemv<QT, EPI_SWIGLU>), grid, dim3(BLOCK), 0, st, w, s, w2, s2, rows, K, (const h16 *)x,
                           (const h16 *)nw, (const h16 *)res, (h16 *)y, rpb);
    } else if (epi == EPI_RESID) {
        hipLaunchKernelGGL((k_gemv<QT, EPI_RESID>), grid, dim3(BLOCK), 0, st, w, s, w2, s2, rows, K, (const h16 *)x,
                           (const h16 *)nw, (const h16 *)res, (h16 *)y, rpb);
    } else {
        hipLaunchKernelGGL((k_gemv<QT, EPI_STORE>), grid, dim3(BLOCK), 0, st, w, s, w2, s2, rows, K, (const h16 *)x,
                           (const h16 *)nw, (const h16 *)res, (h16 *)y, rpb);
    }
}

extern "C" hipError_t uocr_launch_gemv(hipStream_t st, uocr_qmat W, uint32_t rows, uint32_t K, const uint16_t *x,
                                       const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    if (!mat_ok(W) || x == nullptr || y == nullptr || rows == 0u || K == 0u || K % 64u != 0u || K > UOCR_K_MAX_K) {
        return hipErrorInvalidValue;
    }
    const int epi = res != nullptr ? EPI_RESID : EPI_STORE;
    DISPATCH_QT(W.qtype, launch_gemv_qt, st, epi, W, W, rows, K, x, nw, res, y);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_swiglu(hipStream_t st, uocr_qmat G, uocr_qmat U, uint32_t rows, uint32_t K,
                                         const uint16_t *x, const uint16_t *nw, uint16_t *mid) {
    if (!mat_ok(G) || !mat_ok(U) || G.qtype != U.qtype || x == nullptr || mid == nullptr || rows == 0u ||
        K == 0u || K % 64u != 0u || K > UOCR_K_MAX_K) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(G.qtype, launch_gemv_qt, st, EPI_SWIGLU, G, U, rows, K, x, nw, nullptr, mid);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_rmsnorm(hipStream_t st, const uint16_t *x, const uint16_t *nw, uint32_t n,
                                          uint16_t *y) {
    if (x == nullptr || nw == nullptr || y == nullptr || n == 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(BLOCK), 0, st, (const h16 *)x, (const h16 *)nw, n, (h16 *)y);
    return hipGetLastError();
}

template <int QT>
static void launch_qkv_qt(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                          const uint16_t *nw, const RopeTab &tab, const uocr_step_state *state, uint16_t *qout,
                          uint16_t *kc, uint16_t *vc, uint32_t cap) {
    const uint32_t ipb = 8u;
    hipLaunchKernelGGL((k_qkv_rope<QT>), dim3(1920u / ipb), dim3(BLOCK), 0, st, Q, K, V, (const h16 *)h,
                       (const h16 *)nw, tab, state, (h16 *)qout, (h16 *)kc, (h16 *)vc, cap, ipb);
}

extern "C" hipError_t uocr_launch_qkv_rope(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                                           const uint16_t *nw, const float *inv_freq, const uocr_step_state *state,
                                           uint16_t *qout, uint16_t *kcache, uint16_t *vcache,
                                           uint32_t cache_capacity) {
    if (!mat_ok(Q) || !mat_ok(K) || !mat_ok(V) || Q.qtype != K.qtype || Q.qtype != V.qtype || h == nullptr ||
        nw == nullptr || inv_freq == nullptr || state == nullptr || qout == nullptr || kcache == nullptr ||
        vcache == nullptr || cache_capacity == 0u) {
        return hipErrorInvalidValue;
    }
    RopeTab tab;
    for (int i = 0; i < UOCR_K_HEAD_DIM / 2; ++i) tab.f[i] = inv_freq[i];
    DISPATCH_QT(Q.qtype, launch_qkv_qt, st, Q, K, V, h, nw, tab, state, qout, kcache, vcache, cache_capacity);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_attention(hipStream_t st, const uint16_t *q, const uint16_t *kcache,
                                            const uint16_t *vcache, uint32_t cache_capacity,
                                            const uocr_step_state *state, float *partials, uint32_t *counters,
                                            uint16_t *ctx) {
    if (q == nullptr || kcache == nullptr || vcache == nullptr || cache_capacity == 0u || state == nullptr ||
        partials == nullptr || counters == nullptr || ctx == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k_attention, dim3(UOCR_K_ATTN_SPLITS, UOCR_K_HEADS), dim3(BLOCK), 0, st, (const h16 *)q,
                       (const h16 *)kcache, (const h16 *)vcache, cache_capacity, state, partials, counters,
                       (h16 *)ctx);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_router(hipStream_t st, const uint16_t *R, const uint16_t *x, const uint16_t *nw,
                                         int norm_topk, uint32_t *ids, float *weights) {
    if (R == nullptr || x == nullptr || ids == nullptr || weights == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_router, dim3(1), dim3(1024), 0, st, (const h16 *)R, (const h16 *)x, (const h16 *)nw,
                       norm_topk, ids, weights);
    return hipGetLastError();
}

template <int QT>
static void launch_moe_gu_qt(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids, const uint16_t *x,
                             const uint16_t *nw, uint16_t *mid) {
    const uint32_t rows = UOCR_K_TOPK * 896u;
    const uint32_t rpb = rows_per_block(rows, 512u);
    hipLaunchKernelGGL((k_moe_gate_up<QT>), dim3((rows + rpb - 1u) / rpb), dim3(BLOCK), 0, st, *slab, ids,
                       (const h16 *)x, (const h16 *)nw, (h16 *)mid, rpb);
}

extern "C" hipError_t uocr_launch_moe_gate_up(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids,
                                              const uint16_t *x, const uint16_t *nw, uint16_t *mid) {
    if (slab == nullptr || !mat_ok(slab->gate) || !mat_ok(slab->up) || slab->gate.qtype != slab->up.qtype ||
        ids == nullptr || x == nullptr || mid == nullptr) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(slab->gate.qtype, launch_moe_gu_qt, st, slab, ids, x, nw, mid);
    return hipGetLastError();
}

template <int QT, int QS>
static void launch_moe_down_qs(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids, const float *w,
                               const uint16_t *mid, uocr_qmat SD, const uint16_t *smid, const uint16_t *res,
                               uint16_t *out) {
    const uint32_t rpb = 4u;
    hipLaunchKernelGGL((k_moe_down<QT, QS>), dim3(UOCR_K_HIDDEN / rpb), dim3(BLOCK), 0, st, *slab, ids, w,
                       (const h16 *)mid, SD, (const h16 *)smid, (const h16 *)res, (h16 *)out, rpb);
}

template <int QT>
static void launch_moe_down_qt(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids, const float *w,
                               const uint16_t *mid, uocr_qmat SD, const uint16_t *smid, const uint16_t *res,
                               uint16_t *out) {
    switch (SD.qtype) {
        case UOCR_QT_F16: launch_moe_down_qs<QT, 1>(st, slab, ids, w, mid, SD, smid, res, out); break;
        case UOCR_QT_Q8: launch_moe_down_qs<QT, 3>(st, slab, ids, w, mid, SD, smid, res, out); break;
        default: launch_moe_down_qs<QT, 4>(st, slab, ids, w, mid, SD, smid, res, out); break;
    }
}

extern "C" hipError_t uocr_launch_moe_down(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids,
                                           const float *weights, const uint16_t *mid, uocr_qmat SD,
                                           const uint16_t *smid, const uint16_t *res, uint16_t *out) {
    if (slab == nullptr || !mat_ok(slab->down) || !mat_ok(SD) || ids == nullptr || weights == nullptr ||
        mid == nullptr || smid == nullptr || res == nullptr || out == nullptr) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(slab->down.qtype, launch_moe_down_qt, st, slab, ids, weights, mid, SD, smid, res, out);
    return hipGetLastError();
}

template <int QT>
static void launch_lm_qt(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x, const uint16_t *nw,
                         uint32_t *part, uint32_t *cnt, uocr_step_state *state, int advance, int32_t *tokens,
                         float *scores) {
    uint32_t rpb = (vocab + UOCR_K_LM_BLOCKS - 1u) / UOCR_K_LM_BLOCKS;
    rpb = (rpb + 7u) & ~7u;
    if (rpb < 8u) rpb = 8u;
    hipLaunchKernelGGL((k_lm_head<QT>), dim3((vocab + rpb - 1u) / rpb), dim3(BLOCK), 0, st, (const uint8_t *)W.w,
                       (const h16 *)W.s, vocab, (const h16 *)x, (const h16 *)nw, part, cnt, state, advance, tokens,
                       scores, rpb);
}

extern "C" hipError_t uocr_launch_lm_head(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x,
                                          const uint16_t *nw, uint32_t *partials, uint32_t *counter,
                                          uocr_step_state *state, int advance, int32_t *tokens, float *scores) {
    if (!mat_ok(W) || vocab == 0u || x == nullptr || partials == nullptr || counter == nullptr ||
        tokens == nullptr || (advance && state == nullptr)) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(W.qtype, launch_lm_qt, st, W, vocab, x, nw, partials, counter, state, advance, tokens, scores);
    return hipGetLastError();
}

template <int QT>
static void launch_embed_qt(hipStream_t st, uocr_qmat E, uint32_t vocab, const int32_t *token,
                            const uocr_step_state *state, uint16_t *out) {
    hipLaunchKernelGGL((k_embed<QT>), dim3(1), dim3(BLOCK), 0, st, (const uint8_t *)E.w, (const h16 *)E.s, vocab,
                       token, state, (h16 *)out);
}

extern "C" hipError_t uocr_launch_embed(hipStream_t st, uocr_qmat E, uint32_t vocab, const int32_t *token,
                                        const uocr_step_state *state, uint16_t *out) {
    if (!mat_ok(E) || out == nullptr || (token == nullptr && state == nullptr)) return hipErrorInvalidValue;
    DISPATCH_QT(E.qtype, launch_embed_qt, st, E, vocab, token, state, out);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_prefill_state(hipStream_t st, uocr_step_state *state, int32_t i) {
    if (state == nullptr || i < 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_prefill_state, dim3(1), dim3(1), 0, st, state, i);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_decode_state(hipStream_t st, uocr_step_state *state, int32_t prompt_len, int32_t t) {
    if (state == nullptr || prompt_len <= 0 || t < 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_decode_state, dim3(1), dim3(1), 0, st, state, prompt_len, t);
    return hipGetLastError();
}

template <int QT>
static void launch_embed_rows_qt(hipStream_t st, uocr_qmat E, uint32_t vocab, const int32_t *ids,
                                 const uint8_t *mask, uint32_t n, uint16_t *out) {
    hipLaunchKernelGGL((k_embed_rows<QT>), dim3(n), dim3(BLOCK), 0, st, (const uint8_t *)E.w, (const h16 *)E.s, vocab,
                       ids, mask, (h16 *)out);
}

extern "C" hipError_t uocr_launch_embed_rows(hipStream_t st, uocr_qmat E, uint32_t vocab, const int32_t *ids,
                                             const uint8_t *mask, uint32_t n, uint16_t *out) {
    if (!mat_ok(E) || ids == nullptr || out == nullptr || n == 0u) return hipErrorInvalidValue;
    DISPATCH_QT(E.qtype, launch_embed_rows_qt, st, E, vocab, ids, mask, n, out);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_prefill_next(hipStream_t st, uocr_step_state *state, const uint16_t *prompt,
                                               uint16_t *h) {
    if (state == nullptr || prompt == nullptr || h == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_prefill_next, dim3(1), dim3(BLOCK), 0, st, state, (const h16 *)prompt, (h16 *)h);
    return hipGetLastError();
}
