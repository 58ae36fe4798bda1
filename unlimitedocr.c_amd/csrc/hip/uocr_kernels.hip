/*
 * uocr_kernels.hip - hand-written gfx950 (CDNA4, wave64) kernels for the
 * batch-1 decode token loop of the UnlimitedOCR language model.
 *
 * Design (MI355X-first, not a translation of the Metal kernels):
 *  - Batch-1 decode is HBM/latency-bound.  Every GEMV assigns a group of LPR
 *    lanes to a row; each lane owns 16-byte chunks sub, sub+LPR, ... of the
 *    row and issues all of its (up to 8) 128-bit loads and scale loads
 *    before any arithmetic, so a wavefront keeps 64 x 8 x 16 B of weights in
 *    flight.  LPR is chosen per (qtype, K) so a row takes at most 8 loads per
 *    lane (e.g. Q4 K=1280: 8 lanes x 5 loads, 8 rows per wavefront).
 *  - Dequantisation happens in registers (Q4_0 group-half-split nibbles,
 *    Q8_0, f16); the activation vector is staged once per workgroup in LDS as
 *    fp16, with the producing RMSNorm recomputed in the prologue instead of a
 *    separate launch.  Group sums use DPP row permutes (quad_perm,
 *    row_half_mirror, row_mirror) and lane swizzles beyond 16 lanes.
 *  - RoPE and the KV-cache write are fused into the QKV GEMV epilogue (one
 *    lane group owns rows d and d+64 of one head, the rotation pair).
 *  - Decode attention is split-K over the context (32 blocks per head, 16
 *    lanes x 8 dims per cached token) with an online softmax; a 10-block
 *    merge kernel combines the log-sum-exp partials.
 *  - The MoE router logits are computed by spare blocks of the shared-expert
 *    gate/up launch; the routed gate/up and down-combine kernels recompute
 *    the greedy top-6 from the 64 logits in one wavefront (64-bit keys of
 *    probability bits and inverted id, so ties go to the lower id).
 *  - The down-combine kernel fuses the 6 routed down projections, their
 *    weighted sum, the shared-expert down GEMV and the residual add.
 *  - The LM head is a fused final-RMSNorm GEMV writing per-block argmax
 *    partials; a one-block finalize picks the token (NaN rows skipped, ties to
 *    the lowest id), advances the device-side step state and gathers the next
 *    token's embedding row, so a captured decode graph can be replayed.
 * No kernel waits on another block and none uses a device-scope fence
 * (on gfx950 one costs an L2 writeback and invalidate per wavefront); every
 * cross-block hand-off is a kernel boundary.
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

/* Sum over aligned groups of LPR lanes; every lane receives its group's sum.
 * DPP quad/half-row/row permutes inside 16-lane rows, then lane swizzles. */
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    if (LPR >= 2) v += dpp_f<0xB1>(v);
    if (LPR >= 4) v += dpp_f<0x4E>(v);
    if (LPR >= 8) v += dpp_f<0x141>(v);
    if (LPR >= 16) v += dpp_f<0x140>(v);
    if (LPR >= 32) v += __shfl_xor(v, 16);
    if (LPR >= 64) v += __shfl_xor(v, 32);
    return v;
}

/* Row dots by a group of LPR lanes: lane `sub` of the group owns the 16-byte
 * chunks sub, sub+LPR, ... of its row.  The first J chunks of every one of the
 * NM rows are loaded (with their scales) before any arithmetic, so a wave
 * keeps 64*J*NM loads in flight; chunks past J*LPR fall to a tail loop.  W, S,
 * X are per-lane pointers (row payload, row scales, activation in LDS).
 * Every lane receives the NM dot products of its group. */
template <int QT, int LPR, int J, int NM>
__device__ __forceinline__ void group_dot(const uint8_t *const *W, const h16 *const *S, const h16 *const *X,
                                          uint32_t C, uint32_t sub, float *out) {
    uint4 w[NM][J];
    float sc[NM][J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t c = sub + LPR * j;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            w[m][j] = c < C ? *(const uint4 *)(W[m] + 16u * c) : make_uint4(0u, 0u, 0u, 0u);
            if (QT != 1) sc[m][j] = c < C ? (float)S[m][chunk_group<QT>(c)] : 0.0f;
        }
    }
    float acc[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m] = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t c = sub + LPR * j;
        if (c < C) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float d = chunk_dot<QT>(w[m][j], X[m], c);
                acc[m] = QT == 1 ? acc[m] + d : fmaf(d, sc[m][j], acc[m]);
            }
        }
    }
    for (uint32_t c = sub + LPR * J; c < C; c += LPR) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const float d = chunk_dot<QT>(*(const uint4 *)(W[m] + 16u * c), X[m], c);
            acc[m] = QT == 1 ? acc[m] + d : fmaf(d, (float)S[m][chunk_group<QT>(c)], acc[m]);
        }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m) out[m] = group_sum<LPR>(acc[m]);
}

/* Greedy top-6 over 64 router logits by one wavefront (one expert per lane):
 * max-subtracted softmax, then 6 rounds of a 64-bit max over
 * (probability bits, inverted id) so ties go to the lower id
 * (uocr_cpu_ref.c:443-463, moe.metal:12-18).  Raw probabilities unless
 * norm_topk.  Results land in ids/w (LDS). */
__device__ __forceinline__ void topk6_wave(const float *logits, int norm_topk, uint32_t *ids, float *w) {
    const uint32_t lane = threadIdx.x & 63u;
    const float lg = logits[lane];
    const float mx = wave_max(lg);
    const float pe = expf(lg - mx);
    const float prob = pe / wave_sum(pe);
    unsigned long long key = ((unsigned long long)__float_as_uint(prob) << 32) | (0xffffffffu - lane);
    float sel[UOCR_K_TOPK];
    uint32_t sid[UOCR_K_TOPK];
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        const unsigned long long best = wave_max_u64(key);
        sid[r] = 0xffffffffu - (uint32_t)(best & 0xffffffffull);
        sel[r] = __uint_as_float((uint32_t)(best >> 32));
        tot += sel[r];
        if (lane == sid[r]) key = 0ull;
    }
    if (lane == 0u) {
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) {
            ids[r] = sid[r];
            w[r] = norm_topk ? sel[r] / tot : sel[r];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GEMV family                                                               */
/* ------------------------------------------------------------------------ */

#define GBLOCK 128 /* GEMV-family workgroup: 2 wavefronts */

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

template <int QT, int LPR, int EPI>
__global__ __launch_bounds__(GBLOCK) void k_gemv(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                 const uint8_t *__restrict__ W2, const h16 *__restrict__ S2,
                                                 uint32_t rows, uint32_t K, const h16 *__restrict__ x,
                                                 const h16 *__restrict__ nw, const h16 *__restrict__ res,
                                                 h16 *__restrict__ y, uint32_t rpb) {
    constexpr uint32_t R = 64u / LPR;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_MAX_K];
    __shared__ float red[16];
    stage_x(xs, x, nw, (int)K, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const uint32_t sub = lane % LPR, grp = lane / LPR;
    const uint32_t rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min(rows, r0 + rpb);
    for (uint32_t base = r0 + wave * R; base < r1; base += nwave * R) {
        const uint32_t r = base + grp;
        const uint32_t rr = r < r1 ? r : r1 - 1u;
        if (EPI == EPI_SWIGLU) {
            const uint8_t *Wp[2] = {W + (size_t)rr * rb, W2 + (size_t)rr * rb};
            const h16 *Sp[2] = {S + (size_t)rr * G, S2 + (size_t)rr * G};
            const h16 *Xp[2] = {xs, xs};
            float d[2];
            group_dot<QT, LPR, 8, 2>(Wp, Sp, Xp, C, sub, d);
            if (r < r1 && sub == 0u) y[r] = (h16)(silu_f(d[0]) * d[1]);
        } else {
            const uint8_t *Wp[1] = {W + (size_t)rr * rb};
            const h16 *Sp[1] = {S + (size_t)rr * G};
            const h16 *Xp[1] = {xs};
            float d[1];
            group_dot<QT, LPR, 8, 1>(Wp, Sp, Xp, C, sub, d);
            if (r < r1 && sub == 0u) y[r] = (h16)(EPI == EPI_RESID ? d[0] + (float)res[r] : d[0]);
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

/* Work item i (0..1919): matrix m = i/640 (q,k,v), head h, pair d; a lane
 * group computes rows h*128+d and h*128+d+64 of matrix m, rounds them to
 * fp16, rotates q/k by the split-half RoPE at st->pos and stores q, or k/v
 * into the cache slot st->cache_token. */
template <int QT, int LPR>
__global__ __launch_bounds__(GBLOCK) void k_qkv_rope(uocr_qmat Q, uocr_qmat Km, uocr_qmat V, const h16 *__restrict__ hin,
                                                     const h16 *__restrict__ nw, RopeTab rope,
                                                     const uocr_step_state *__restrict__ st, h16 *__restrict__ qout,
                                                     h16 *__restrict__ kc, h16 *__restrict__ vc, uint32_t cap,
                                                     uint32_t ipb) {
    constexpr uint32_t R = 64u / LPR;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    stage_x(xs, hin, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const uint32_t sub = lane % LPR, grp = lane / LPR;
    const uint32_t K = UOCR_K_HIDDEN, rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const int32_t pos = st->pos;
    const uint32_t ct = (uint32_t)st->cache_token;
    const uint32_t i0 = blockIdx.x * ipb, i1 = min(1920u, i0 + ipb);
    for (uint32_t base = i0 + wave * R; base < i1; base += nwave * R) {
        const uint32_t it = min(base + grp, i1 - 1u);
        const uint32_t m = it / 640u, rem = it % 640u, h = rem / 64u, d = rem % 64u;
        const uocr_qmat M = m == 0u ? Q : (m == 1u ? Km : V);
        const uint32_t ra = h * 128u + d, rbw = ra + 64u;
        const uint8_t *Wp[2] = {(const uint8_t *)M.w + (size_t)ra * rb, (const uint8_t *)M.w + (size_t)rbw * rb};
        const h16 *Sp[2] = {(const h16 *)M.s + (size_t)ra * G, (const h16 *)M.s + (size_t)rbw * G};
        const h16 *Xp[2] = {xs, xs};
        float dd[2];
        group_dot<QT, LPR, 8, 2>(Wp, Sp, Xp, C, sub, dd);
        if (sub == 0u && base + grp < i1) {
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
/* split-K decode attention + merge                                          */
/* ------------------------------------------------------------------------ */

/* Block (s, h) covers attention indices [s*chunk, (s+1)*chunk) of head h:
 * 16 lanes x 8 dims per cached token, 16 tokens per block in flight, an
 * online softmax per 16-lane group, then a block merge into one (max, sum,
 * acc[128]) partial.  Indices >= attn_prompt map into the 128-token ring
 * (attention_decode.metal:25-33). */
__global__ __launch_bounds__(BLOCK) void k_attention(const h16 *__restrict__ q, const h16 *__restrict__ kc,
                                                     const h16 *__restrict__ vc, uint32_t cap,
                                                     const uocr_step_state *__restrict__ st, float *__restrict__ part) {
    __shared__ float sm[16], sl[16];
    __shared__ float sacc[16][UOCR_K_HEAD_DIM];
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
    }
}

/* Log-sum-exp merge of the S partials of one head -> fp16 context. */
__global__ __launch_bounds__(UOCR_K_HEAD_DIM) void k_attention_merge(const float *__restrict__ part, uint32_t S,
                                                                     h16 *__restrict__ ctx) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float *ph = part + (size_t)h * S * (UOCR_K_HEAD_DIM + 2);
    float M = -INFINITY;
    for (uint32_t k = 0; k < S; ++k) M = fmaxf(M, ph[(size_t)k * (UOCR_K_HEAD_DIM + 2)]);
    float Ls = 0.0f, A = 0.0f;
    for (uint32_t k = 0; k < S; ++k) {
        const float *pk = ph + (size_t)k * (UOCR_K_HEAD_DIM + 2);
        if (pk[0] == -INFINITY) continue;
        const float f = expf(pk[0] - M);
        Ls = fmaf(pk[1], f, Ls);
        A = fmaf(pk[2 + d], f, A);
    }
    ctx[h * 128 + d] = (h16)(A / Ls);
}

/* ------------------------------------------------------------------------ */
/* MoE: shared experts + router logits, routed gate/up, down-combine         */
/* ------------------------------------------------------------------------ */

/* Blocks [0, nb_shared) compute the shared-expert SwiGLU rows (1792) and the
 * remaining blocks the 64 router logits (fp16 rows, fp32 dot); both read the
 * same RMSNorm'd input, so one launch serves both. */
template <int QS, int LPRS>
__global__ __launch_bounds__(GBLOCK) void k_moe_shared_router(uocr_qmat SG, uocr_qmat SU, const h16 *__restrict__ R,
                                                              const h16 *__restrict__ x, const h16 *__restrict__ nw,
                                                              h16 *__restrict__ smid, float *__restrict__ logits,
                                                              uint32_t nb_shared, uint32_t rpb_shared,
                                                              uint32_t rpb_router) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    stage_x(xs, x, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    if (blockIdx.x < nb_shared) {
        constexpr uint32_t RS = 64u / LPRS;
        const uint32_t sub = lane % LPRS, grp = lane / LPRS;
        const uint32_t rb = row_bytes<QS>(UOCR_K_HIDDEN), C = rb / 16u, G = UOCR_K_HIDDEN / 64u;
        const uint32_t r0 = blockIdx.x * rpb_shared, r1 = min(1792u, r0 + rpb_shared);
        for (uint32_t base = r0 + wave * RS; base < r1; base += nwave * RS) {
            const uint32_t r = base + grp, rr = r < r1 ? r : r1 - 1u;
            const uint8_t *Wp[2] = {(const uint8_t *)SG.w + (size_t)rr * rb, (const uint8_t *)SU.w + (size_t)rr * rb};
            const h16 *Sp[2] = {(const h16 *)SG.s + (size_t)rr * G, (const h16 *)SU.s + (size_t)rr * G};
            const h16 *Xp[2] = {xs, xs};
            float d[2];
            group_dot<QS, LPRS, 8, 2>(Wp, Sp, Xp, C, sub, d);
            if (r < r1 && sub == 0u) smid[r] = (h16)(silu_f(d[0]) * d[1]);
        }
    } else {
        constexpr uint32_t LPR = 32u, RR = 2u;
        const uint32_t sub = lane % LPR, grp = lane / LPR;
        const uint32_t rb = UOCR_K_HIDDEN * 2u, C = rb / 16u;
        const uint32_t r0 = (blockIdx.x - nb_shared) * rpb_router, r1 = min(64u, r0 + rpb_router);
        for (uint32_t base = r0 + wave * RR; base < r1; base += nwave * RR) {
            const uint32_t r = base + grp, rr = r < r1 ? r : r1 - 1u;
            const uint8_t *Wp[1] = {(const uint8_t *)R + (size_t)rr * rb};
            const h16 *Sp[1] = {nullptr};
            const h16 *Xp[1] = {xs};
            float d[1];
            group_dot<1, LPR, 8, 1>(Wp, Sp, Xp, C, sub, d);
            if (r < r1 && sub == 0u) logits[r] = d[0];
        }
    }
}

/* Router top-6 from logits (one wavefront). */
__global__ __launch_bounds__(64) void k_router_topk(const float *__restrict__ logits, int norm_topk, uint32_t *ids,
                                                    float *w) {
    __shared__ uint32_t sid[UOCR_K_TOPK];
    __shared__ float sw[UOCR_K_TOPK];
    topk6_wave(logits, norm_topk, sid, sw);
    __syncthreads();
    if (threadIdx.x < UOCR_K_TOPK) {
        ids[threadIdx.x] = sid[threadIdx.x];
        w[threadIdx.x] = sw[threadIdx.x];
    }
}

/* Routed gate/up: the block recomputes the top-6 from the logits, then
 * mid[r*896 + c] = f16(silu(G_e[c].xin) * (U_e[c].xin)), e = ids[r]. */
template <int QT, int LPR>
__global__ __launch_bounds__(GBLOCK) void k_moe_gate_up(uocr_expert_slab sl, const float *__restrict__ logits,
                                                        int norm_topk, const h16 *__restrict__ x,
                                                        const h16 *__restrict__ nw, h16 *__restrict__ mid,
                                                        uint32_t *ids_out, float *w_out, uint32_t rpb) {
    constexpr uint32_t R = 64u / LPR;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    __shared__ uint32_t sid[UOCR_K_TOPK];
    __shared__ float sw[UOCR_K_TOPK];
    if (threadIdx.x < 64u) topk6_wave(logits, norm_topk, sid, sw);
    stage_x(xs, x, nw, UOCR_K_HIDDEN, red);
    if (blockIdx.x == 0u && ids_out != nullptr && threadIdx.x < UOCR_K_TOPK) {
        ids_out[threadIdx.x] = sid[threadIdx.x];
        w_out[threadIdx.x] = sw[threadIdx.x];
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const uint32_t sub = lane % LPR, grp = lane / LPR;
    const uint32_t I = 896u, K = UOCR_K_HIDDEN, rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const uint32_t rows = UOCR_K_TOPK * I;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min(rows, r0 + rpb);
    for (uint32_t base = r0 + wave * R; base < r1; base += nwave * R) {
        const uint32_t r = base + grp, rr = r < r1 ? r : r1 - 1u;
        const uint32_t rank = rr / I, col = rr % I;
        const uint32_t e = sid[rank] < UOCR_K_EXPERTS ? sid[rank] : 0u;
        const uint8_t *Wp[2] = {(const uint8_t *)sl.gate.w + e * sl.gu_w_stride + (size_t)col * rb,
                                (const uint8_t *)sl.up.w + e * sl.gu_w_stride + (size_t)col * rb};
        const h16 *Sp[2] = {(const h16 *)sl.gate.s + e * sl.gu_s_stride + (size_t)col * G,
                            (const h16 *)sl.up.s + e * sl.gu_s_stride + (size_t)col * G};
        const h16 *Xp[2] = {xs, xs};
        float d[2];
        group_dot<QT, LPR, 8, 2>(Wp, Sp, Xp, C, sub, d);
        if (r < r1 && sub == 0u) mid[r] = (h16)(silu_f(d[0]) * d[1]);
    }
}

/* Down projection of the 6 routed experts + weighted combine + shared-expert
 * down + residual, one fp16 rounding:
 * out[c] = f16(sum_r w_r * D_e[c].mid_r + f16(SD[c].smid) + res[c]). */
template <int QT, int QS, int LPR>
__global__ __launch_bounds__(GBLOCK) void k_moe_down(uocr_expert_slab sl, const float *__restrict__ logits,
                                                     int norm_topk, const h16 *__restrict__ mid, uocr_qmat SD,
                                                     const h16 *__restrict__ smid, const h16 *__restrict__ res,
                                                     h16 *__restrict__ out, uint32_t rpb) {
    constexpr uint32_t I = 896u, SI = 1792u, R = 64u / LPR;
    __shared__ __attribute__((aligned(16))) h16 ms[UOCR_K_TOPK * I + SI];
    __shared__ uint32_t sid[UOCR_K_TOPK];
    __shared__ float sw[UOCR_K_TOPK];
    if (threadIdx.x < 64u) topk6_wave(logits, norm_topk, sid, sw);
    {
        const uint4 *a = (const uint4 *)mid;
        const uint4 *b = (const uint4 *)smid;
        uint4 *d = (uint4 *)ms;
        for (uint32_t i = threadIdx.x; i < UOCR_K_TOPK * I / 8u; i += blockDim.x) d[i] = a[i];
        for (uint32_t i = threadIdx.x; i < SI / 8u; i += blockDim.x) d[UOCR_K_TOPK * I / 8u + i] = b[i];
    }
    __syncthreads();
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const uint32_t sub = lane % LPR, grp = lane / LPR;
    uint32_t e[UOCR_K_TOPK];
    float w[UOCR_K_TOPK];
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        e[r] = sid[r] < UOCR_K_EXPERTS ? sid[r] : 0u;
        w[r] = sid[r] < UOCR_K_EXPERTS ? sw[r] : 0.0f;
    }
    const uint32_t rbD = row_bytes<QT>(I), CD = rbD / 16u, GD = I / 64u;
    const uint32_t rbS = row_bytes<QS>(SI), CS = rbS / 16u, GS = SI / 64u;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min((uint32_t)UOCR_K_HIDDEN, r0 + rpb);
    for (uint32_t base = r0 + wave * R; base < r1; base += nwave * R) {
        const uint32_t c = base + grp, cc = c < r1 ? c : r1 - 1u;
        const uint8_t *Wp[UOCR_K_TOPK];
        const h16 *Sp[UOCR_K_TOPK];
        const h16 *Xp[UOCR_K_TOPK];
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) {
            Wp[r] = (const uint8_t *)sl.down.w + e[r] * sl.dn_w_stride + (size_t)cc * rbD;
            Sp[r] = (const h16 *)sl.down.s + e[r] * sl.dn_s_stride + (size_t)cc * GD;
            Xp[r] = ms + r * I;
        }
        float d[UOCR_K_TOPK];
        group_dot<QT, LPR, 2, UOCR_K_TOPK>(Wp, Sp, Xp, CD, sub, d);
        const uint8_t *Ws[1] = {(const uint8_t *)SD.w + (size_t)cc * rbS};
        const h16 *Ss[1] = {(const h16 *)SD.s + (size_t)cc * GS};
        const h16 *Xs[1] = {ms + UOCR_K_TOPK * I};
        float sd[1];
        group_dot<QS, LPR, 4, 1>(Ws, Ss, Xs, CS, sub, sd);
        if (c < r1 && sub == 0u) {
            float acc = 0.0f;
#pragma unroll
            for (int r = 0; r < UOCR_K_TOPK; ++r) acc = fmaf(w[r], d[r], acc);
            out[c] = (h16)(acc + (float)(h16)sd[0] + (float)res[c]);
        }
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
/* LM head + argmax                                                          */
/* ------------------------------------------------------------------------ */

__device__ __forceinline__ bool better(float s, uint32_t id, float bs, uint32_t bid) {
    return id != NONE_ID && (bid == NONE_ID || s > bs || (s == bs && id < bid));
}

/* Pass 1: fused final RMSNorm + GEMV over vocab rows; each block writes its
 * best (score, id) with NaN rows skipped and ties to the lowest id. */
template <int QT, int LPR>
__global__ __launch_bounds__(GBLOCK) void k_lm_head(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                    uint32_t vocab, const h16 *__restrict__ x,
                                                    const h16 *__restrict__ nw, uint32_t *__restrict__ part,
                                                    uint32_t rpb) {
    constexpr uint32_t R = 64u / LPR;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    __shared__ float bsc[GBLOCK];
    __shared__ uint32_t bidv[GBLOCK];
    stage_x(xs, x, nw, UOCR_K_HIDDEN, red);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, nwave = blockDim.x >> 6;
    const uint32_t sub = lane % LPR, grp = lane / LPR;
    const uint32_t K = UOCR_K_HIDDEN, rb = row_bytes<QT>(K), C = rb / 16u, G = K / 64u;
    const uint32_t r0 = blockIdx.x * rpb, r1 = min(vocab, r0 + rpb);
    float bs = -INFINITY;
    uint32_t bid = NONE_ID;
    for (uint32_t base = r0 + wave * R; base < r1; base += nwave * R) {
        const uint32_t r = base + grp, rr = r < r1 ? r : r1 - 1u;
        const uint8_t *Wp[1] = {W + (size_t)rr * rb};
        const h16 *Sp[1] = {S + (size_t)rr * G};
        const h16 *Xp[1] = {xs};
        float d[1];
        group_dot<QT, LPR, 8, 1>(Wp, Sp, Xp, C, sub, d);
        if (r < r1 && !isnan(d[0]) && better(d[0], r, bs, bid)) {
            bs = d[0];
            bid = r;
        }
    }
    bsc[threadIdx.x] = bs;
    bidv[threadIdx.x] = bid;
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = -INFINITY;
        uint32_t bi = NONE_ID;
        for (uint32_t i = 0; i < blockDim.x; i += LPR) {
            if (better(bsc[i], bidv[i], b, bi)) {
                b = bsc[i];
                bi = bidv[i];
            }
        }
        part[2u * blockIdx.x] = __float_as_uint(b);
        part[2u * blockIdx.x + 1u] = bi;
    }
}

/* Pass 2 (one block): reduce the partials to the token id (none valid -> 0,
 * score -inf), store it at tokens[state->t] (or [0] without state); with
 * advance, write the next decode position into *state (uocr_metal.m:14239
 * and the ring plan of attention_decode.metal:25-33) and gather the selected
 * token's embedding row into h (embedding_q4.metal:21-56). */
template <int QE>
__global__ __launch_bounds__(BLOCK) void k_lm_finalize(const uint32_t *__restrict__ part, uint32_t nparts,
                                                       uocr_step_state *st, int advance, int32_t *tokens,
                                                       float *scores, const uint8_t *__restrict__ EW,
                                                       const h16 *__restrict__ ES, uint32_t vocab,
                                                       h16 *__restrict__ hout) {
    __shared__ float bsc[BLOCK];
    __shared__ uint32_t bidv[BLOCK];
    __shared__ int32_t chosen;
    float b = -INFINITY;
    uint32_t bi = NONE_ID;
    for (uint32_t i = threadIdx.x; i < nparts; i += blockDim.x) {
        const float s = __uint_as_float(part[2u * i]);
        const uint32_t id = part[2u * i + 1u];
        if (better(s, id, b, bi)) {
            b = s;
            bi = id;
        }
    }
    bsc[threadIdx.x] = b;
    bidv[threadIdx.x] = bi;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t i = 1; i < blockDim.x; ++i) {
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
        chosen = id;
    }
    __syncthreads();
    if (advance && EW != nullptr) k_embed_row_body<QE>(EW, ES, vocab, chosen, hout);
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

static uint32_t chunks_of(uint32_t qt, uint32_t K) {
    return (qt == UOCR_QT_Q4 ? K / 2u : (qt == UOCR_QT_Q8 ? K : 2u * K)) / 16u;
}

/* lanes per row: the smallest group that covers a row in at most 8 loads */
static uint32_t pick_lpr(uint32_t C) {
    for (uint32_t l = 4u; l < 64u; l *= 2u) {
        if (C <= 8u * l) return l;
    }
    return 64u;
}

/* K = 1280 rows: Q4 -> 8 lanes, Q8 -> 16, f16 -> 32 (5 loads per lane) */
#define LPR_1280(QT) ((QT) == 4 ? 8 : ((QT) == 3 ? 16 : 32))
/* K = 896 with 2 loads per lane: Q4 -> 16, Q8 -> 32, f16 -> 64 */
#define LPR_896(QT) ((QT) == 4 ? 16 : ((QT) == 3 ? 32 : 64))

#define DISPATCH_QT(qt, F, ...)                                      \
    do {                                                             \
        switch (qt) {                                                \
            case UOCR_QT_F16: F<1>(__VA_ARGS__); break;              \
            case UOCR_QT_Q8: F<3>(__VA_ARGS__); break;               \
            default: F<4>(__VA_ARGS__); break;                       \
        }                                                            \
    } while (0)

template <int QT, int LPR>
static void launch_gemv_l(hipStream_t st, int epi, uocr_qmat W, uocr_qmat W2, uint32_t rows, uint32_t K,
                          const uint16_t *x, const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    const uint32_t pass = 2u * (64u / LPR);
    const uint32_t passes = (rows + pass * 1024u - 1u) / (pass * 1024u);
    const uint32_t rpb = pass * passes;
    const dim3 grid((rows + rpb - 1u) / rpb);
    const uint8_t *w = (const uint8_t *)W.w, *w2 = (const uint8_t *)W2.w;
    const h16 *s = (const h16 *)W.s, *s2 = (const h16 *)W2.s;
    if (epi == EPI_SWIGLU) {
        hipLaunchKernelGGL((k_gemv<QT, LPR, EPI_SWIGLU>), grid, dim3(GBLOCK), 0, st, w, s, w2, s2, rows, K,
                           (const h16 *)x, (const h16 *)nw, (const h16 *)res, (h16 *)y, rpb);
    } else if (epi == EPI_RESID) {
        hipLaunchKernelGGL((k_gemv<QT, LPR, EPI_RESID>), grid, dim3(GBLOCK), 0, st, w, s, w2, s2, rows, K,
                           (const h16 *)x, (const h16 *)nw, (const h16 *)res, (h16 *)y, rpb);
    } else {
        hipLaunchKernelGGL((k_gemv<QT, LPR, EPI_STORE>), grid, dim3(GBLOCK), 0, st, w, s, w2, s2, rows, K,
                           (const h16 *)x, (const h16 *)nw, (const h16 *)res, (h16 *)y, rpb);
    }
}

template <int QT>
static void launch_gemv_qt(hipStream_t st, int epi, uocr_qmat W, uocr_qmat W2, uint32_t rows, uint32_t K,
                           const uint16_t *x, const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    switch (pick_lpr(chunks_of(QT, K))) {
        case 4: launch_gemv_l<QT, 4>(st, epi, W, W2, rows, K, x, nw, res, y); break;
        case 8: launch_gemv_l<QT, 8>(st, epi, W, W2, rows, K, x, nw, res, y); break;
        case 16: launch_gemv_l<QT, 16>(st, epi, W, W2, rows, K, x, nw, res, y); break;
        case 32: launch_gemv_l<QT, 32>(st, epi, W, W2, rows, K, x, nw, res, y); break;
        default: launch_gemv_l<QT, 64>(st, epi, W, W2, rows, K, x, nw, res, y); break;
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
    constexpr int LPR = LPR_1280(QT);
    const uint32_t ipb = 2u * (64u / LPR);
    hipLaunchKernelGGL((k_qkv_rope<QT, LPR>), dim3((1920u + ipb - 1u) / ipb), dim3(GBLOCK), 0, st, Q, K, V,
                       (const h16 *)h, (const h16 *)nw, tab, state, (h16 *)qout, (h16 *)kc, (h16 *)vc, cap, ipb);
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
                                            const uocr_step_state *state, float *partials, uint16_t *ctx) {
    if (q == nullptr || kcache == nullptr || vcache == nullptr || cache_capacity == 0u || state == nullptr ||
        partials == nullptr || ctx == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k_attention, dim3(UOCR_K_ATTN_SPLITS, UOCR_K_HEADS), dim3(BLOCK), 0, st, (const h16 *)q,
                       (const h16 *)kcache, (const h16 *)vcache, cache_capacity, state, partials);
    hipLaunchKernelGGL(k_attention_merge, dim3(UOCR_K_HEADS), dim3(UOCR_K_HEAD_DIM), 0, st, (const float *)partials,
                       (uint32_t)UOCR_K_ATTN_SPLITS, (h16 *)ctx);
    return hipGetLastError();
}

template <int QS>
static void launch_shared_router_qs(hipStream_t st, uocr_qmat SG, uocr_qmat SU, const uint16_t *R, const uint16_t *x,
                                    const uint16_t *nw, uint16_t *smid, float *logits, bool with_shared) {
    constexpr int LPRS = LPR_1280(QS);
    const uint32_t rpb_s = 2u * (64u / LPRS);
    const uint32_t nb_s = with_shared ? (1792u + rpb_s - 1u) / rpb_s : 0u;
    const uint32_t rpb_r = 4u, nb_r = 64u / rpb_r;
    hipLaunchKernelGGL((k_moe_shared_router<QS, LPRS>), dim3(nb_s + nb_r), dim3(GBLOCK), 0, st, SG, SU,
                       (const h16 *)R, (const h16 *)x, (const h16 *)nw, (h16 *)smid, logits, nb_s, rpb_s, rpb_r);
}

extern "C" hipError_t uocr_launch_moe_shared_router(hipStream_t st, uocr_qmat SG, uocr_qmat SU, const uint16_t *R,
                                                    const uint16_t *x, const uint16_t *nw, uint16_t *smid,
                                                    float *logits) {
    if (!mat_ok(SG) || !mat_ok(SU) || SG.qtype != SU.qtype || R == nullptr || x == nullptr || smid == nullptr ||
        logits == nullptr) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(SG.qtype, launch_shared_router_qs, st, SG, SU, R, x, nw, smid, logits, true);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_router(hipStream_t st, const uint16_t *R, const uint16_t *x, const uint16_t *nw,
                                         int norm_topk, float *logits, uint32_t *ids, float *weights) {
    if (R == nullptr || x == nullptr || logits == nullptr || ids == nullptr || weights == nullptr) {
        return hipErrorInvalidValue;
    }
    uocr_qmat none = {R, nullptr, UOCR_QT_F16};
    launch_shared_router_qs<1>(st, none, none, R, x, nw, nullptr, logits, false);
    hipLaunchKernelGGL(k_router_topk, dim3(1), dim3(64), 0, st, (const float *)logits, norm_topk, ids, weights);
    return hipGetLastError();
}

template <int QT>
static void launch_moe_gu_qt(hipStream_t st, const uocr_expert_slab *slab, const float *logits, int norm_topk,
                             const uint16_t *x, const uint16_t *nw, uint16_t *mid, uint32_t *ids_out, float *w_out) {
    constexpr int LPR = LPR_1280(QT);
    const uint32_t rows = UOCR_K_TOPK * 896u;
    const uint32_t rpb = 2u * (64u / LPR);
    hipLaunchKernelGGL((k_moe_gate_up<QT, LPR>), dim3((rows + rpb - 1u) / rpb), dim3(GBLOCK), 0, st, *slab, logits,
                       norm_topk, (const h16 *)x, (const h16 *)nw, (h16 *)mid, ids_out, w_out, rpb);
}

extern "C" hipError_t uocr_launch_moe_gate_up(hipStream_t st, const uocr_expert_slab *slab, const float *logits,
                                              int norm_topk, const uint16_t *x, const uint16_t *nw, uint16_t *mid,
                                              uint32_t *ids_out, float *weights_out) {
    if (slab == nullptr || !mat_ok(slab->gate) || !mat_ok(slab->up) || slab->gate.qtype != slab->up.qtype ||
        logits == nullptr || x == nullptr || mid == nullptr || ((ids_out == nullptr) != (weights_out == nullptr))) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(slab->gate.qtype, launch_moe_gu_qt, st, slab, logits, norm_topk, x, nw, mid, ids_out, weights_out);
    return hipGetLastError();
}

template <int QT, int QS>
static void launch_moe_down_qs(hipStream_t st, const uocr_expert_slab *slab, const float *logits, int norm_topk,
                               const uint16_t *mid, uocr_qmat SD, const uint16_t *smid, const uint16_t *res,
                               uint16_t *out) {
    constexpr int LPR = LPR_896(QT);
    const uint32_t rpb = 2u * (64u / LPR);
    hipLaunchKernelGGL((k_moe_down<QT, QS, LPR>), dim3((UOCR_K_HIDDEN + rpb - 1u) / rpb), dim3(GBLOCK), 0, st, *slab,
                       logits, norm_topk, (const h16 *)mid, SD, (const h16 *)smid, (const h16 *)res, (h16 *)out,
                       rpb);
}

template <int QT>
static void launch_moe_down_qt(hipStream_t st, const uocr_expert_slab *slab, const float *logits, int norm_topk,
                               const uint16_t *mid, uocr_qmat SD, const uint16_t *smid, const uint16_t *res,
                               uint16_t *out) {
    switch (SD.qtype) {
        case UOCR_QT_F16: launch_moe_down_qs<QT, 1>(st, slab, logits, norm_topk, mid, SD, smid, res, out); break;
        case UOCR_QT_Q8: launch_moe_down_qs<QT, 3>(st, slab, logits, norm_topk, mid, SD, smid, res, out); break;
        default: launch_moe_down_qs<QT, 4>(st, slab, logits, norm_topk, mid, SD, smid, res, out); break;
    }
}

extern "C" hipError_t uocr_launch_moe_down(hipStream_t st, const uocr_expert_slab *slab, const float *logits,
                                           int norm_topk, const uint16_t *mid, uocr_qmat SD, const uint16_t *smid,
                                           const uint16_t *res, uint16_t *out) {
    if (slab == nullptr || !mat_ok(slab->down) || !mat_ok(SD) || logits == nullptr || mid == nullptr ||
        smid == nullptr || res == nullptr || out == nullptr) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(slab->down.qtype, launch_moe_down_qt, st, slab, logits, norm_topk, mid, SD, smid, res, out);
    return hipGetLastError();
}

template <int QT>
static uint32_t launch_lm_qt(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x, const uint16_t *nw,
                             uint32_t *part) {
    constexpr int LPR = LPR_1280(QT);
    const uint32_t pass = 2u * (64u / LPR);
    uint32_t rpb = (vocab + UOCR_K_LM_BLOCKS - 1u) / UOCR_K_LM_BLOCKS;
    rpb = (rpb + pass - 1u) / pass * pass;
    const uint32_t nb = (vocab + rpb - 1u) / rpb;
    hipLaunchKernelGGL((k_lm_head<QT, LPR>), dim3(nb), dim3(GBLOCK), 0, st, (const uint8_t *)W.w, (const h16 *)W.s,
                       vocab, (const h16 *)x, (const h16 *)nw, part, rpb);
    return nb;
}

template <int QE>
static void launch_lm_fin(hipStream_t st, const uint32_t *part, uint32_t nb, uocr_step_state *state, int advance,
                          int32_t *tokens, float *scores, uocr_qmat E, uint32_t vocab, uint16_t *hout) {
    hipLaunchKernelGGL((k_lm_finalize<QE>), dim3(1), dim3(BLOCK), 0, st, part, nb, state, advance, tokens, scores,
                       (const uint8_t *)E.w, (const h16 *)E.s, vocab, (h16 *)hout);
}

extern "C" hipError_t uocr_launch_lm_head(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x,
                                          const uint16_t *nw, uint32_t *partials, uocr_step_state *state, int advance,
                                          int32_t *tokens, float *scores, uocr_qmat E, uint16_t *hout) {
    if (!mat_ok(W) || vocab == 0u || x == nullptr || partials == nullptr || tokens == nullptr ||
        (advance && state == nullptr) || (E.w != nullptr && (!mat_ok(E) || hout == nullptr))) {
        return hipErrorInvalidValue;
    }
    uint32_t nb = 0;
    switch (W.qtype) {
        case UOCR_QT_F16: nb = launch_lm_qt<1>(st, W, vocab, x, nw, partials); break;
        case UOCR_QT_Q8: nb = launch_lm_qt<3>(st, W, vocab, x, nw, partials); break;
        default: nb = launch_lm_qt<4>(st, W, vocab, x, nw, partials); break;
    }
    DISPATCH_QT(E.w != nullptr ? E.qtype : UOCR_QT_Q4, launch_lm_fin, st, partials, nb, state, advance, tokens, scores,
                E, vocab, hout);
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
