/*
 * uocr_kernels.hip - hand-written gfx950 (CDNA4, wave64) kernels for the
 * batch-1 decode token loop of the UnlimitedOCR language model.
 *
 * Design (MI355X-first, not a translation of the Metal kernels):
 *  - Batch-1 decode is bound by HBM bandwidth and, at this model size, by
 *    the latency of each launch's dependent memory round trips.  Every kernel
 *    therefore issues its weight loads first (they depend on nothing), then
 *    stages the activation vector (with the producing RMSNorm recomputed in
 *    the prologue), so a kernel costs one memory round trip plus its
 *    streaming time.  GEMVs that take several row passes per wavefront
 *    double-buffer the next pass's loads behind the current pass's math.
 *  - A GEMV row belongs to a group of LPR lanes; lane `sub` owns 16-byte
 *    chunks sub, sub+LPR, ... (J of them, all loads in flight together).
 *    LPR is the smallest power of two that covers a row in at most 7 chunks
 *    per lane (K = 1280: Q4 8 lanes, Q8 16, f16 32).
 *  - Dequantisation is exact and packed: a nibble n (or a biased int8 byte)
 *    is placed under an fp16 exponent of 1024 with one byte permute, giving
 *    the half 1024 + n; one packed fp16 subtract yields the integer weight
 *    exactly, and v_dot2_f32_f16 accumulates weight x activation pairs in
 *    fp32.  Each 16-byte chunk's sum is scaled by its group's fp16 scale.
 *  - Group sums use DPP row permutes (quad_perm, row_half_mirror,
 *    row_mirror) and lane swizzles beyond 16 lanes.
 *  - RoPE and the KV-cache write are fused into the QKV GEMV epilogue (one
 *    lane group owns rows d and d+64 of one head, the rotation pair).
 *  - Decode attention is split-K over the live KV slots (16 blocks per head,
 *    slots partitioned by the cache capacity so the first K/V loads do not
 *    wait for the step state; a 16-lane group per slot, 5 slots in flight per
 *    group).  The log-sum-exp merge of the partials runs in the prologue of
 *    the O projection, overlapped with that kernel's weight loads.
 *  - The MoE router (64 fp16 rows) is one block of the shared-expert gate/up
 *    launch; it runs the greedy top-6 in one wavefront (64-bit keys of
 *    probability bits and inverted id, so ties go to the lower id) and
 *    publishes ids and weights for the routed kernels.
 *  - The down-combine kernel fuses the 6 routed down projections, their
 *    weighted sum, the shared-expert down GEMV and the residual add.
 *  - The LM head is a streaming final-RMSNorm GEMV writing one argmax
 *    partial per block; a one-block finalize picks the token (NaN rows
 *    skipped, ties to the lowest id), advances the device-side step state and
 *    gathers the next token's embedding row, so a captured decode graph can
 *    be replayed.
 *
 * Every cross-block hand-off is a kernel boundary: no kernel waits for
 * another block and none uses a device-scope fence (on gfx950 such a fence
 * writes back and invalidates the whole L2 of the XCD).
 */
#include "uocr_kernels.h"
#include "uocr_dev.h"

#include <math.h>
#include <string.h>


#define BLOCK 256
#define NWAVE (BLOCK / 64)
#define SMALL_BLOCK 128 /* one-pass GEMVs with few rows: 2 wavefronts, more CUs */


/* The attention projections' weights (q/k/v in k_qkv_rope, O in
 * k_attn_out) are read non-temporally, so the Infinity Cache keeps the
 * weights that stay resident across steps with less pressure (measured:
 * Q8 decode 3,059 -> 3,103 tok/s, fp16 2,479 -> 2,560). */
/* The shared experts stay resident across steps when quantised (Q4 40 MB,
 * Q8 75 MB); in fp16 (138 MB) they do not fit beside the other resident
 * weights and are read non-temporally (measured: fp16 decode 2,515 -> 2,561
 * tok/s; Q8 with them non-temporal 3,105 -> 3,089). */
template <int QS>
__host__ __device__ constexpr bool shared_nt() {
    return QS == 1;
}
#ifndef UOCR_ATT_W_NT
#define UOCR_ATT_W_NT true
#endif

/* ------------------------------------------------------------------------ */
/* opt-in per-block timeline (builds with -DUOCR_TIMELINE only)              */
/* ------------------------------------------------------------------------ */
#ifdef UOCR_TIMELINE
struct TlRec {
    uint32_t kid, block, xcc, pad;
    uint64_t t0, t1;
};
__device__ TlRec *g_tl_buf;
__device__ unsigned g_tl_cap;
__device__ unsigned g_tl_n[256]; /* records per region (block id % 256): few same-line atomics per launch */
/* thread 0 of every block records (kernel, block, XCD, start, end) in
 * s_memrealtime ticks (100 MHz) when the block leaves the kernel */
struct TlScope {
    uint64_t t0;
    uint32_t kid;
    __device__ explicit TlScope(uint32_t k) : kid(k) { t0 = __builtin_amdgcn_s_memrealtime(); }
    __device__ ~TlScope() {
        if (threadIdx.x == 0 && g_tl_buf != nullptr) {
            const unsigned b = (blockIdx.x + blockIdx.y * gridDim.x) & 255u, per = g_tl_cap / 256u;
            const unsigned j = atomicAdd(&g_tl_n[b], 1u), i = b * per + j;
            if (j < per) {
                TlRec r;
                r.kid = kid;
                r.block = blockIdx.x + blockIdx.y * gridDim.x;
                r.xcc = (uint32_t)__builtin_amdgcn_s_getreg(20 | (3 << 11)) & 0xfu; /* HW_REG_XCC_ID */
                r.pad = 0;
                r.t0 = t0;
                r.t1 = __builtin_amdgcn_s_memrealtime();
                g_tl_buf[i] = r;
            }
        }
    }
};
#define TL(k) TlScope tl_scope_(k)
extern "C" __attribute__((visibility("default"))) int uocr_hip_timeline(void *buf, unsigned cap) {
    static const unsigned zero[256] = {0};
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_tl_buf), &buf, sizeof(buf)) != hipSuccess) return -1;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_tl_cap), &cap, sizeof(cap)) != hipSuccess) return -1;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_tl_n), zero, sizeof(zero)) != hipSuccess) return -1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}
#else
#define TL(k)
#endif


/* ------------------------------------------------------------------------ */
/* streaming GEMV family                                                      */
/* ------------------------------------------------------------------------ */

enum { EPI_LINEAR = 0, EPI_SWIGLU = 1, EPI_ARGMAX = 2 };


/* Row groups of R = 64/LPR rows are dealt to wavefronts round-robin over the
 * grid; a wavefront loads its next group while it reduces the current one.
 *  EPI_LINEAR: y[r] = f16(W_r.xin (+ res[r]))
 *  EPI_SWIGLU: y[r] = f16(silu(W_r.xin) * (W2_r.xin))
 *  EPI_ARGMAX: the block's best (score, row) in thread 0's best/best_id
 *              (NaN skipped, ties to the lower row). */
template <int QT, int LPR, int J, int EPI>
__device__ __forceinline__ void stream_rows(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                            const uint8_t *__restrict__ W2, const h16 *__restrict__ S2, u32 rows,
                                            u32 K, const h16 *__restrict__ x, const h16 *__restrict__ nw,
                                            const h16 *__restrict__ res, h16 *__restrict__ y, float &best,
                                            u32 &best_id) {
    constexpr u32 R = 64u / LPR;
    constexpr int NM = EPI == EPI_SWIGLU ? 2 : 1;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_MAX_K];
    __shared__ float red[16];
    __shared__ float bsc[NWAVE];
    __shared__ u32 bidv[NWAVE];
    const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const u32 sub = lane % LPR, grp = lane / LPR;
    const u32 C = chunks_per_row<QT>(K), rb = 16u * C, G = K / 64u;
    const u32 ngroups = (rows + R - 1u) / R;
    const u32 stride = gridDim.x * NWAVE;
    u32 g = blockIdx.x * NWAVE + wave;

    RowFrag<J> fa[NM], fb[NM];
    auto load = [&](RowFrag<J>(&f)[NM], u32 gg) {
        const u32 r = min(gg * R + grp, rows - 1u);
        frag_load<QT, LPR, J, EPI == EPI_ARGMAX && UOCR_NT_STREAM>(f[0], W + (size_t)r * rb, S + (size_t)r * G, C, sub);
        if (NM == 2) frag_load<QT, LPR, J>(f[NM - 1], W2 + (size_t)r * rb, S2 + (size_t)r * G, C, sub);
    };
    float bs = -INFINITY;
    u32 bid = NONE_ID;
    /* LM head (Q4/Q8): offset-free chunk dots (chunk_dot_u), the bias back
     * from the chunk sums of the staged activation */
    constexpr bool XU = EPI == EPI_ARGMAX && QT != 1;
    float nx[J];
    auto finish = [&](const RowFrag<J>(&f)[NM], u32 gg) {
        const u32 r = gg * R + grp;
        const float d0 = XU ? group_sum<LPR>(frag_dot_u<XU ? QT : 4, LPR, J>(f[0], xs, nx, C, sub))
                            : group_sum<LPR>(frag_dot<QT, LPR, J>(f[0], xs, C, sub));
        if (EPI == EPI_SWIGLU) {
            const float d1 = group_sum<LPR>(frag_dot<QT, LPR, J>(f[NM - 1], xs, C, sub));
            if (r < rows && sub == 0u) y[r] = (h16)(silu_f(d0) * d1);
        } else if (EPI == EPI_LINEAR) {
            if (r < rows && sub == 0u) y[r] = (h16)(res != nullptr ? d0 + (float)res[r] : d0);
        } else {
            if (r < rows && !isnan(d0) && better(d0, r, bs, bid)) {
                bs = d0;
                bid = r;
            }
        }
    };

    XStage<UOCR_K_MAX_K, BLOCK> sx;
    stage_load(sx, x, nw, (int)K);
    load(fa, min(g, ngroups - 1u));
    stage_store(sx, xs, nw, (int)K, red);
    if constexpr (XU) {
        /* chunk sums: a Q4 chunk is two runs of 16 columns (one per thread
         * of a pair), a Q8 chunk one run */
        __shared__ float xsum[UOCR_K_HIDDEN / 16u];
        const u32 t = threadIdx.x, np = QT == 4 ? 2u * C : C;
        float ps = 0.0f;
        if (t < np && t < 2u * (UOCR_K_HIDDEN / 32u)) {
            const u32 q = QT == 4 ? t >> 1 : t;
            const u32 c0 = QT == 4 ? (q >> 1) * 64u + (q & 1u) * 16u + (t & 1u) * 32u : 16u * q;
            const uint4 u0 = *(const uint4 *)(xs + c0), u1 = *(const uint4 *)(xs + c0 + 8u);
            const u32 wv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const h16x2 v = __builtin_bit_cast(h16x2, wv[k]);
                ps += (float)v.x + (float)v.y;
            }
        }
        if (QT == 4) ps += __shfl_xor(ps, 1);
        if (t < np && (QT != 4 || (t & 1u) == 0u)) xsum[QT == 4 ? t >> 1 : t] = ps;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < J; ++j) nx[j] = -chunk_bias<XU ? QT : 4>() * xsum[min(sub + LPR * (u32)j, C - 1u)];
    }
    while (g < ngroups) {
        const u32 g1 = g + stride;
        if (g1 < ngroups) load(fb, g1);
        finish(fa, g);
        if (g1 >= ngroups) break;
        const u32 g2 = g1 + stride;
        if (g2 < ngroups) load(fa, g2);
        finish(fb, g1);
        g = g2;
    }

    if (EPI == EPI_ARGMAX) {
        /* wave argmax over the group leaders, then over the block's waves */
#pragma unroll
        for (int o = LPR; o < 64; o <<= 1) {
            const float os = __shfl_xor(bs, o);
            const u32 oid = (u32)__shfl_xor((int)bid, o);
            if (better(os, oid, bs, bid)) {
                bs = os;
                bid = oid;
            }
        }
        if (lane == 0u) {
            bsc[wave] = bs;
            bidv[wave] = bid;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            float b = bsc[0];
            u32 bi = bidv[0];
            for (int i = 1; i < NWAVE; ++i) {
                if (better(bsc[i], bidv[i], b, bi)) {
                    b = bsc[i];
                    bi = bidv[i];
                }
            }
            best = b;
            best_id = bi;
        }
    }
}

/* GEMV launch of stream_rows (EPI_LINEAR, EPI_SWIGLU; the LM head's
 * EPI_ARGMAX runs inside k_lm_keys). */
template <int QT, int LPR, int J, int EPI>
__global__ __launch_bounds__(BLOCK) void k_stream(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                  const uint8_t *__restrict__ W2, const h16 *__restrict__ S2,
                                                  u32 rows, u32 K, const h16 *__restrict__ x,
                                                  const h16 *__restrict__ nw, const h16 *__restrict__ res,
                                                  h16 *__restrict__ y) {
    TL(7);
    static_assert(EPI != EPI_ARGMAX, "the argmax epilogue runs in k_lm_keys");
    float b = -INFINITY;
    u32 bi = NONE_ID;
    stream_rows<QT, LPR, J, EPI>(W, S, W2, S2, rows, K, x, nw, res, y, b, bi);
}

__global__ __launch_bounds__(BLOCK) void k_rmsnorm(const h16 *x, const h16 *nw, u32 n, h16 *y) {
    __shared__ float red[16];
    float ss = 0.0f;
    for (u32 i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = (float)x[i];
        ss = fmaf(v, v, ss);
    }
    ss = block_sum(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + 1.0e-6f);
    for (u32 i = threadIdx.x; i < n; i += blockDim.x) y[i] = (h16)(((float)x[i] * inv) * (float)nw[i]);
}

/* ------------------------------------------------------------------------ */
/* QKV + RoPE + KV write                                                     */
/* ------------------------------------------------------------------------ */

struct RopeTab {
    float f[UOCR_K_HEAD_DIM / 2];
};

/* cos/sin(pos * inv_freq[d]) of a step's position into the step state
 * (threads d < 64), so the 12 QKV launches of the step read them instead of
 * evaluating trig on their critical path (rope.metal:16-70 angle form). */
__device__ __forceinline__ void set_rope(uocr_step_state *st, int32_t pos, const RopeTab &tab) {
    const u32 d = threadIdx.x;
    if (d < UOCR_K_HEAD_DIM / 2) {
        const float ang = (float)pos * tab.f[d];
        st->rope_cos[d] = cosf(ang);
        st->rope_sin[d] = sinf(ang);
    }
}

/* Token selection folded into layer 0's QKV launch of a decode step
 * (QE = the embedding's qtype; 0: plain QKV).  Every wavefront reads the 16
 * argmax keys the LM-head launch left, takes the largest (the token; 0 when
 * no row was valid) and stages the token's embedding row, dequantised as
 * embed_row_body does, as its activation; block 0 also stores that row as
 * the hidden state h (the residual of layer 0), the token and its score at
 * tokens[st->t - 1] and st->cur_token.  The keys and weights are requested
 * before the embedding row, so the row's dependent load overlaps the weight
 * loads. */
struct SelArgs {
    const unsigned long long *keys;
    const uint8_t *EW;
    const h16 *ES;
    u32 vocab;
    int32_t *tokens;
    float *scores;
    uocr_step_state *stw;
    h16 *hout;
};

/* 8 embedding values (columns 8i..8i+7) of row tok as fp16(q * scale). */
template <int QE>
__device__ __forceinline__ uint4 embed_piece(const SelArgs &sa, int32_t tok, u32 i) {
    constexpr u32 K = UOCR_K_HIDDEN;
    union h8 {
        uint4 u;
        h16 h[8];
    } o;
    o.u = make_uint4(0u, 0u, 0u, 0u);
    if (tok < 0 || (u32)tok >= sa.vocab) return o.u;
    const size_t r = (size_t)tok;
    if (QE == 1) return ((const uint4 *)((const h16 *)sa.EW + r * K))[i];
    const float sc = (float)sa.ES[r * (K / 64u) + i / 8u];
    if (QE == 3) {
        const uint2 v = *(const uint2 *)(sa.EW + r * K + 8u * i);
        const u32 w[2] = {v.x, v.y};
#pragma unroll
        for (int j = 0; j < 8; ++j) o.h[j] = (h16)((float)(int8_t)((w[j / 4] >> (8 * (j % 4))) & 0xffu) * sc);
    } else {
        const u32 j0 = (i % 8u) * 8u;
        const uint2 v = *(const uint2 *)(sa.EW + r * (K / 2u) + (i / 8u) * 32u + (j0 & 31u));
        const u32 w[2] = {v.x, v.y}, sh = j0 < 32u ? 0u : 4u;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int q = (int)((w[j / 4] >> (8 * (j % 4) + sh)) & 15u) - 8;
            o.h[j] = (h16)((float)q * sc);
        }
    }
    return o.u;
}

/* Work item i (0..1919): matrix m = i/640 (q,k,v), head h, pair d; a lane
 * group computes rows h*128+d and h*128+d+64 of matrix m, rounds them to
 * fp16, rotates q/k by the split-half RoPE at st->pos and stores q, or k/v
 * into the cache slot st->cache_token.  One item per lane group. */
/* The step plan a standalone attention-block call computes in its QKV
 * launch instead of a separate plan launch: decode step t after a P-token
 * prompt (k_decode_state's arithmetic). */
struct QkvPlan {
    int32_t P, t;
    uocr_step_state *st;
    RopeTab tab;
};

/* The plan as a kernel argument only where it is used. */
template <bool PLAN>
struct PlanArg {
    char none;
};
template <>
struct PlanArg<true> {
    QkvPlan p;
};

/* Slot, cos and sin of pair d for the QKV stores: from the step state, or
 * (PLAN) computed from the plan, whose step state block 0 also writes. */
template <bool PLAN>
__device__ __forceinline__ void qkv_slot(const uocr_step_state *__restrict__ st, const QkvPlan &pl, u32 d, u32 &ct,
                                         float &cs, float &sn) {
    if (PLAN) {
        const int32_t pos = pl.P + pl.t;
        ct = (u32)(pl.P + (pl.t % UOCR_K_RING));
        const float ang = (float)pos * pl.tab.f[d];
        cs = cosf(ang);
        sn = sinf(ang);
        if (blockIdx.x == 0u) {
            uocr_step_state *sw = pl.st;
            if (threadIdx.x < UOCR_K_HEAD_DIM / 2) {
                const float a2 = (float)pos * pl.tab.f[threadIdx.x];
                sw->rope_cos[threadIdx.x] = cosf(a2);
                sw->rope_sin[threadIdx.x] = sinf(a2);
            }
            if (threadIdx.x == 0) {
                const int32_t gcount = pl.t + 1;
                const int32_t live = gcount < UOCR_K_RING ? gcount : UOCR_K_RING;
                sw->t = pl.t;
                sw->prompt_len = pl.P;
                sw->pos = pos;
                sw->cache_token = (int32_t)ct;
                sw->attn_prompt = pl.P;
                sw->attn_len = pl.P + live;
                sw->first_gen = gcount - live;
            }
        }
    } else {
        ct = (u32)st->cache_token;
        cs = st->rope_cos[d];
        sn = st->rope_sin[d];
    }
}

template <int QT, int QE, bool PLAN = false>
__global__ __launch_bounds__(SMALL_BLOCK) void k_qkv_rope(uocr_qmat Q, uocr_qmat Km, uocr_qmat V, const h16 *__restrict__ hin,
                                                    const h16 *__restrict__ nw,
                                                    const uocr_step_state *__restrict__ st, h16 *__restrict__ qout,
                                                    h16 *__restrict__ kc, h16 *__restrict__ vc, u32 cap, SelArgs sa,
                                                    PlanArg<PLAN> pa) {
    TL(1);
    constexpr u32 K = UOCR_K_HIDDEN, C = chunks_per_row<QT>(K), LPR = lpr_lat(C), J = j_lat(C), R = 64u / LPR;
    constexpr u32 rb = 16u * C, G = K / 64u;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const u32 sub = lane % LPR, grp = lane / LPR;
    const u32 item = (blockIdx.x * (SMALL_BLOCK / 64) + wave) * R + grp;
    const u32 it = min(item, 1919u);
    const u32 m = it / 640u, rem = it % 640u, h = rem / 64u, d = rem % 64u;
    const uocr_qmat M = m == 0u ? Q : (m == 1u ? Km : V);
    const u32 ra = h * 128u + d, rbw = ra + 64u;
    XStage<UOCR_K_HIDDEN, SMALL_BLOCK> sx;
    constexpr int PER = XStage<UOCR_K_HIDDEN, SMALL_BLOCK>::PER;
    unsigned long long key = 0ull;
    if (QE == 0) {
        stage_load(sx, hin, nw, UOCR_K_HIDDEN);
    } else {
        if (lane < UOCR_LM_KEYS) key = sa.keys[lane];
#pragma unroll
        for (int p = 0; p < PER; ++p) sx.w[p] = ((const uint4 *)nw)[min((int)threadIdx.x + p * SMALL_BLOCK, (int)K / 8 - 1)];
    }
    RowFrag<J> fa, fb;
    frag_load<QT, LPR, J, UOCR_ATT_W_NT>(fa, (const uint8_t *)M.w + (size_t)ra * rb, (const h16 *)M.s + (size_t)ra * G, C, sub);
    frag_load<QT, LPR, J, UOCR_ATT_W_NT>(fb, (const uint8_t *)M.w + (size_t)rbw * rb, (const h16 *)M.s + (size_t)rbw * G, C, sub);
    u32 ct;
    float cs, sn;
    {
        if constexpr (PLAN) {
            qkv_slot<true>(st, pa.p, d, ct, cs, sn);
        } else {
            QkvPlan none{};
            qkv_slot<false>(st, none, d, ct, cs, sn);
        }
    }
    if (QE != 0) {
        asm volatile("" : "+v"(key)::"memory");
        float b;
        u32 bi;
        key_winner(wave_max_u64(key), b, bi);
        const int32_t tok = bi == NONE_ID ? 0 : (int32_t)bi;
#pragma unroll
        for (int p = 0; p < PER; ++p) sx.x[p] = embed_piece<QE>(sa, tok, (u32)min((int)threadIdx.x + p * SMALL_BLOCK, (int)K / 8 - 1));
        if (blockIdx.x == 0) {
#pragma unroll
            for (int p = 0; p < PER; ++p) {
                const int i = (int)threadIdx.x + p * SMALL_BLOCK;
                if (i < (int)K / 8) ((uint4 *)sa.hout)[i] = sx.x[p];
            }
            if (threadIdx.x == 0) {
                const int32_t t = st->t - 1;
                sa.tokens[t] = tok;
                if (sa.scores != nullptr) sa.scores[t] = b;
                sa.stw->cur_token = tok;
            }
        }
    }
    stage_store(sx, xs, nw, UOCR_K_HIDDEN, red);
    const float da = group_sum<LPR>(frag_dot<QT, LPR, J>(fa, xs, C, sub));
    const float db = group_sum<LPR>(frag_dot<QT, LPR, J>(fb, xs, C, sub));
    if (sub == 0u && item < 1920u) {
        const h16 a = (h16)da, b = (h16)db;
        const size_t cix = ((size_t)h * cap + ct) * 128u + d;
        if (m == 2u) {
            vc[cix] = a;
            vc[cix + 64u] = b;
        } else {
            const float fa2 = (float)a, fb2 = (float)b;
            const h16 na = (h16)(fa2 * cs - fb2 * sn), nb = (h16)(fa2 * sn + fb2 * cs);
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

/* ------------------------------------------------------------------------ */
/* split-K decode attention; merge in the O-projection prologue              */
/* ------------------------------------------------------------------------ */

/* Threads of an attention block: 32 slot groups of 16 lanes (8 dims per
 * lane).  A group holds U slots in flight (the launch picks U so that one
 * round of loads covers the block's range up to 4,608 slots of cache). */
constexpr int ATT_THREADS = 512;
constexpr int ATT_GROUPS = ATT_THREADS / 16;

/* Live KV slots of a step are always [0, attn_len): the prompt slots
 * [0, P) plus the ring slots [P, P + live) (before the ring wraps these hold
 * generated tokens 0..live-1 in order; after it wraps all 128 slots are
 * live).  Softmax over a set does not depend on the visiting order, so the
 * kernel addresses slot i for attention index i and needs no ring
 * arithmetic (attention_decode.metal:25-33 maps logical indices instead; the
 * results differ only in fp32 summation order).
 *
 * Block (s, h) owns slots [s*chunk, (s+1)*chunk) with chunk fixed by the
 * cache capacity.  Blocks whose range lies below the last UOCR_K_RING slots
 * (live in every decode step whose prompt fills the cache) issue their first
 * K/V loads before the step state (attention length) arrives; the others
 * read it first, so ring slots not generated yet are not fetched.  Slots >=
 * attn_len are masked.  A 16-lane group handles one slot (8 dims per lane),
 * U slots in flight per group, with an online softmax; the block writes one
 * partial (max, sum, acc[128] / sum) per head:
 *   fp16 acc/sum at ((h16 *)part)[(h*S + s)*128 + d],
 *   fp32 (max, sum) at part[H*S*128 + (h*S + s)*2]. */
template <int ATT_UNROLL, int SL = UOCR_K_ATTN_SPLITS>
__global__ __launch_bounds__(ATT_THREADS) void k_attention(const h16 *__restrict__ q, const h16 *__restrict__ kc,
                                                     const h16 *__restrict__ vc, u32 cap,
                                                     const uocr_step_state *__restrict__ st, float *__restrict__ part,
                                                     long long *__restrict__ racc,
                                                     unsigned long long *__restrict__ clear_keys) {
    TL(2);
    /* SL: splits of the partials' layout; the grid runs gridDim.x <= SL of
     * them, and block (s, h) with s < SL - gridDim.x also marks the unused
     * split gridDim.x + s of head h empty (max -inf, sum 0) */
    constexpr int S = SL;
    const int SE = (int)gridDim.x;
    if (racc != nullptr && blockIdx.x == 0 && blockIdx.y == 0) {
        for (int i = threadIdx.x; i < UOCR_ROUTER_ACC_WORDS; i += ATT_THREADS) racc[i] = 0;
    }
    /* the LM-head keys, read by layer 0's QKV launch, are re-armed for the
     * next step (kernel order: every reader has finished) */
    if (clear_keys != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < UOCR_LM_KEYS) {
        clear_keys[threadIdx.x] = 0ull;
    }
    constexpr int NW = ATT_THREADS / 64;
    __shared__ float sm[NW], sl[NW];
    __shared__ float sacc[NW][UOCR_K_HEAD_DIM];
    const int h = blockIdx.y, s = blockIdx.x;
    const int chunk = ((int)cap + SE - 1) / SE;
    const int i0 = s * chunk, iend = min((int)cap, i0 + chunk);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int gq = lane >> 4, p = lane & 15;
    const int gid = wave * 4 + gq;
    const float scale = 0.08838834764831845f; /* 1/sqrt(128) */
    const h16 *kh = kc + (size_t)h * cap * 128u + 8 * p;
    const h16 *vh = vc + (size_t)h * cap * 128u + 8 * p;

    union h8 {
        uint4 u;
        h16 h[8];
    };
    h8 kk[ATT_UNROLL], vv[ATT_UNROLL];
    /* slots past the block's range (or, once the step state is in, past
     * attn_len) re-read the range's last slot: the re-reads hit the caches
     * instead of fetching the neighbouring split's slots */
    int lim = max(iend - 1, 0);
    auto load = [&](int ib) {
#pragma unroll
        for (int u = 0; u < ATT_UNROLL; ++u) {
            const int t = min(ib + ATT_GROUPS * u, lim);
            kk[u].u = *(const uint4 *)(kh + (size_t)t * 128u);
            vv[u].u = *(const uint4 *)(vh + (size_t)t * 128u);
        }
    };
    h8 qq;
    qq.u = *(const uint4 *)(q + h * 128 + 8 * p);
    const bool late = iend > (int)cap - min((int)cap, (int)UOCR_K_RING);
    int i1 = iend;
    if (late) {
        i1 = min(st->attn_len, iend);
        lim = max(i1 - 1, 0);
    }
    load(i0 + gid);
    hold(qq.u);
    i1 = min(st->attn_len, iend);
    lim = max(min(i1, iend) - 1, 0);
    float qv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) qv[j] = (float)qq.h[j];
    float m = -INFINITY, l = 0.0f, acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int ib = i0 + gid;;) {
        /* all slot scores first (independent), then one softmax update */
        float sc[ATT_UNROLL];
        float mn = m;
#pragma unroll
        for (int u = 0; u < ATT_UNROLL; ++u) {
            float d = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) d = fmaf(qv[j], (float)kk[u].h[j], d);
            sc[u] = ib + ATT_GROUPS * u < i1 ? row16_sum(d) * scale : -INFINITY;
            mn = fmaxf(mn, sc[u]);
        }
        if (mn != -INFINITY) {
            const float corr = expf(m - mn);
            l *= corr;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] *= corr;
#pragma unroll
            for (int u = 0; u < ATT_UNROLL; ++u) {
                const float e = expf(sc[u] - mn);
                l += e;
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = fmaf(e, (float)vv[u].h[j], acc[j]);
            }
            m = mn;
        }
        ib += ATT_GROUPS * ATT_UNROLL;
        if (ib >= i1) break;
        load(ib);
    }
    {
        /* the wave's four slot groups (lanes p, p+16, p+32, p+48 hold the
         * same dims) merged in registers */
        float Mw = fmaxf(m, __shfl_xor(m, 16));
        Mw = fmaxf(Mw, __shfl_xor(Mw, 32));
        const float f = m == -INFINITY ? 0.0f : expf(m - Mw);
        l *= f;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[j] *= f;
            acc[j] += __shfl_xor(acc[j], 16);
            acc[j] += __shfl_xor(acc[j], 32);
        }
        if (gq == 0) {
            if (p == 0) {
                sm[wave] = Mw;
                sl[wave] = l;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) sacc[wave][8 * p + j] = acc[j];
        }
    }
    __syncthreads();
    if (threadIdx.x < UOCR_K_HEAD_DIM) {
        const int d = threadIdx.x;
        float M = -INFINITY;
#pragma unroll
        for (int k = 0; k < NW; ++k) M = fmaxf(M, sm[k]);
        float Ls = 0.0f, A = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (int k = 0; k < NW; ++k) {
                const float f = expf(sm[k] - M);
                Ls = fmaf(sl[k], f, Ls);
                A = fmaf(sacc[k][d], f, A);
            }
        }
        /* normalised accumulator in fp16; (max, sum) in fp32 */
        ((h16 *)part)[(size_t)(h * S + s) * UOCR_K_HEAD_DIM + d] = (h16)(Ls > 0.0f ? A / Ls : 0.0f);
        if (d == 0) {
            float *ml = part + (size_t)UOCR_K_HEADS * S * UOCR_K_HEAD_DIM + (size_t)(h * S + s) * 2u;
            ml[0] = M;
            ml[1] = Ls;
        }
        if (S > 1 && s < S - SE) {
            const int se = SE + s;
            ((h16 *)part)[(size_t)(h * S + se) * UOCR_K_HEAD_DIM + d] = (h16)0.0f;
            if (d == 0) {
                float *ml = part + (size_t)UOCR_K_HEADS * S * UOCR_K_HEAD_DIM + (size_t)(h * S + se) * 2u;
                ml[0] = -INFINITY;
                ml[1] = 0.0f;
            }
        }
    }
}

/* Log-sum-exp merge of the S attention partials into fp16 ctx[1280] in LDS
 * (all threads of a BLOCK-thread block).  Split k of head h left its
 * normalised accumulator accn_k = acc_k / L_k in fp16 (a weighted mean of V
 * rows, so within the V range) and (M_k, L_k) in fp32; then
 *   ctx_h = sum_k w_k accn_k,  w_k = L_k exp(M_k - M_h) / sum_k' L_k' exp(M_k' - M_h).
 * Threads t < H*S compute the weights into LDS; thread t < 160 owns dims
 * 8t..8t+7 and sums their S split values (loads issued by merge_load,
 * before the caller's weight loads). */
template <int S>
struct MergeLoads {
    static constexpr int NML = (UOCR_K_HEADS * S + BLOCK - 1) / BLOCK; /* (max, sum) pairs per thread */
    uint4 a[S];
    float2 ml[NML];
};

template <int S>
__device__ __forceinline__ void merge_load(MergeLoads<S> &m, const float *__restrict__ part) {
    constexpr int HD = UOCR_K_HEAD_DIM, NO = UOCR_K_HIDDEN / 8;
    const int t = threadIdx.x;
    const int o = min(t, NO - 1), hh = o / (HD / 8), d8 = o % (HD / 8);
    const h16 *accn = (const h16 *)part;
#pragma unroll
    for (int k = 0; k < S; ++k) m.a[k] = *(const uint4 *)(accn + (size_t)(hh * S + k) * HD + 8 * d8);
#pragma unroll
    for (int i = 0; i < MergeLoads<S>::NML; ++i) {
        m.ml[i] = *(const float2 *)(part + (size_t)UOCR_K_HEADS * S * HD + 2u * min(t + i * BLOCK, UOCR_K_HEADS * S - 1));
    }
}

template <int S>
__device__ __forceinline__ void merge_finish(MergeLoads<S> &m, h16 *ctx, float *wk) {
    constexpr int HD = UOCR_K_HEAD_DIM, NO = UOCR_K_HIDDEN / 8;
    static_assert(S == 4 || S == 8 || S == 16 || S == 32, "split weights use aligned S-lane groups");
    static_assert(BLOCK % S == 0, "a thread's (max, sum) pairs belong to whole S-lane groups");
#pragma unroll
    for (int i = 0; i < MergeLoads<S>::NML; ++i) hold(m.ml[i]);
#pragma unroll
    for (int k = 0; k < S; ++k) hold(m.a[k]);
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < MergeLoads<S>::NML; ++i) {
        /* lanes S*h..S*h+S-1 of this pass hold the splits of head h */
        const int j = t + i * BLOCK;
        float M = m.ml[i].x;
#pragma unroll
        for (int o = 1; o < S; o <<= 1) M = fmaxf(M, __shfl_xor(M, o));
        const float lf = m.ml[i].x == -INFINITY ? 0.0f : m.ml[i].y * expf(m.ml[i].x - M);
        const float w = lf / group_sum<S>(lf);
        if (j < UOCR_K_HEADS * S) wk[j] = w;
    }
    __syncthreads();
    if (t < NO) {
        const int hh = t / (HD / 8);
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll
        for (int k = 0; k < S; ++k) {
            const float w = wk[hh * S + k];
            const u32 u[4] = {m.a[k].x, m.a[k].y, m.a[k].z, m.a[k].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const h16x2 v = __builtin_bit_cast(h16x2, u[j]);
                acc[2 * j] = fmaf((float)v.x, w, acc[2 * j]);
                acc[2 * j + 1] = fmaf((float)v.y, w, acc[2 * j + 1]);
            }
        }
        h16x2 r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = h16x2{(h16)acc[2 * j], (h16)acc[2 * j + 1]};
        ((uint4 *)ctx)[t] = __builtin_bit_cast(uint4, r);
    }
    __syncthreads();
}

/* O projection with the attention merge in its prologue:
 * out[r] = f16(O_r . ctx + res[r]), ctx = merge of the partials (fp16, the
 * reference's attention-output rounding point).  Block 0 also stores ctx
 * when ctx_out is set.  One row per lane group.
 * FOLD: the block also adds z[e] += sum over its rows i of fold[i][e] *
 * out[i] to racc[e] as round(z * 2^32) (integer adds: the total does not
 * depend on the order in which blocks arrive).  With fold = R * post_norm,
 * z * inv_rms(out) are the router logits R . rmsnorm(out) of the MoE
 * (moe.metal:53-189), less the fp16 rounding of the normalised vector. */
template <int QT, bool FOLD, int S = UOCR_K_ATTN_SPLITS>
__global__ __launch_bounds__(BLOCK) void k_attn_out(uocr_qmat O, const float *__restrict__ part,
                                                    const h16 *__restrict__ res, h16 *__restrict__ out,
                                                    h16 *__restrict__ ctx_out, const float *__restrict__ fold,
                                                    long long *__restrict__ racc) {
    TL(3);
    constexpr u32 K = UOCR_K_HIDDEN, C = chunks_per_row<QT>(K), LPR = lpr_for(C), J = j_for(C), R = 64u / LPR;
    constexpr u32 rb = 16u * C, G = K / 64u;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float wk[UOCR_K_HEADS * S];
    const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const u32 sub = lane % LPR, grp = lane / LPR;
    const u32 r = (blockIdx.x * NWAVE + wave) * R + grp, rr = min(r, K - 1u);
    MergeLoads<S> ml;
    merge_load(ml, part);
    RowFrag<J> f;
    frag_load<QT, LPR, J, UOCR_ATT_W_NT>(f, (const uint8_t *)O.w + (size_t)rr * rb, (const h16 *)O.s + (size_t)rr * G, C, sub);
    const float rv = (float)res[rr];
    const u32 row0 = (blockIdx.x * NWAVE + wave) * R;
    float fw[FOLD ? R : 1];
    if (FOLD) {
#pragma unroll
        for (u32 g = 0; g < R; ++g) fw[g] = fold[(size_t)min(row0 + g, K - 1u) * UOCR_K_EXPERTS + lane];
    }
    merge_finish(ml, xs, wk);
    if (ctx_out != nullptr && blockIdx.x == 0) {
        for (u32 i = threadIdx.x; i < K / 8u; i += blockDim.x) ((uint4 *)ctx_out)[i] = ((const uint4 *)xs)[i];
    }
    const float d = group_sum<LPR>(frag_dot<QT, LPR, J>(f, xs, C, sub));
    const h16 o = (h16)(d + rv);
    if (r < K && sub == 0u) out[r] = o;
    if (FOLD) {
        __shared__ float zp[NWAVE][UOCR_K_EXPERTS];
        float z = 0.0f;
#pragma unroll
        for (u32 g = 0; g < R; ++g) {
            const float av = lane_f((float)o, (int)(g * LPR));
            z = row0 + g < K ? fmaf(fw[g], av, z) : z;
        }
        zp[wave][lane] = z;
        __syncthreads();
        if (wave == 0u) {
            float t = zp[0][lane];
#pragma unroll
            for (u32 w = 1; w < NWAVE; ++w) t += zp[w][lane];
            const long long q = __float2ll_rn(t * (float)(1ull << UOCR_K_ROUTER_FIX_SHIFT));
            /* blocks spread over the accumulator copies: fewer same-line
             * atomics queue at the memory side */
            atomicAdd((unsigned long long *)racc + (blockIdx.x % UOCR_K_ROUTER_ACC_COPIES) * UOCR_K_EXPERTS + lane,
                      (unsigned long long)q);
        }
    }
}

/* Merge alone (operator API): ctx = merge of the partials. */
template <int S>
__global__ __launch_bounds__(BLOCK) void k_attn_merge(const float *__restrict__ part, h16 *__restrict__ ctx) {
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float wk[UOCR_K_HEADS * S];
    MergeLoads<S> ml;
    merge_load(ml, part);
    merge_finish(ml, xs, wk);
    for (u32 i = threadIdx.x; i < UOCR_K_HIDDEN / 8u; i += blockDim.x) ((uint4 *)ctx)[i] = ((const uint4 *)xs)[i];
}

/* ------------------------------------------------------------------------ */
/* MoE: shared experts + router, routed gate/up, down-combine                */
/* ------------------------------------------------------------------------ */

/* Router logits: block b stages rmsnorm(x) once in LDS and its 8
 * wavefronts compute logits 8b..8b+7 = R_r . rmsnorm(x) (fp16 rows, fp32
 * dots): the input row and the norm weight are read by 8 blocks rather than
 * by one block per logit. */
#define ROUTER_ROWS 8u
__global__ __launch_bounds__(64 * ROUTER_ROWS) void k_router_logits(const h16 *__restrict__ Rw,
                                                                    const h16 *__restrict__ x,
                                                                    const h16 *__restrict__ nw,
                                                                    float *__restrict__ logits) {
    TL(8);
    constexpr u32 C = chunks_per_row<1>(UOCR_K_HIDDEN), LPR = 64u, J = (C + LPR - 1u) / LPR, rb = 16u * C;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    const u32 r = blockIdx.x * ROUTER_ROWS + (threadIdx.x >> 6), sub = threadIdx.x & 63u;
    XStage<UOCR_K_HIDDEN, 64 * ROUTER_ROWS> sx;
    stage_load(sx, x, nw, UOCR_K_HIDDEN);
    RowFrag<J> f;
    frag_load<1, LPR, J>(f, (const uint8_t *)Rw + (size_t)r * rb, nullptr, C, sub);
    stage_store(sx, xs, nw, UOCR_K_HIDDEN, red);
    const float d = group_sum<LPR>(frag_dot<1, LPR, J>(f, xs, C, sub));
    if (sub == 0u) logits[r] = d;
}

/* Top-6 alone (operator API): one wavefront. */
__global__ __launch_bounds__(64) void k_router_topk(const float *__restrict__ logits, int norm_topk, u32 *ids,
                                                    float *weights) {
    u32 sid[UOCR_K_TOPK];
    float sw[UOCR_K_TOPK];
    topk6(logits[threadIdx.x], norm_topk, sid, sw);
    if (threadIdx.x < UOCR_K_TOPK) {
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) {
            if (threadIdx.x == (u32)r) {
                ids[r] = sid[r];
                weights[r] = sw[r];
            }
        }
    }
}

/* Gate/up of the routed and the shared experts in one launch.
 * Blocks [0, nb_routed): every wavefront recomputes the top-6 from the 64
 * router logits (cheaper than another launch), then one row pair per lane
 * group: mid[r*896 + c] = f16(silu(G_e[c].xin) * (U_e[c].xin)), e = the
 * rank-r expert; block 0 publishes ids/weights for the down kernel.
 * Blocks [nb_routed, ...): smid[c] = f16(silu(SG[c].xin) * (SU[c].xin)),
 * c < 1792.  xin = x or rmsnorm(x, nw).
 * FOLD: racc holds the un-normalised logits z of k_attn_out (fixed point,
 * summed over the accumulator copies);
 * the top-6 is taken on z (same order), and block 0 turns z * inv_rms(x)
 * into the probabilities once x is staged. */
template <int QT, int QS, bool FOLD>
__global__ __launch_bounds__(SMALL_BLOCK) void k_moe_gate_up(uocr_expert_slab sl, uocr_qmat SG, uocr_qmat SU,
                                                             const float *__restrict__ logits,
                                                             const long long *__restrict__ racc, int norm_topk,
                                                             const h16 *__restrict__ x, const h16 *__restrict__ nw,
                                                             h16 *__restrict__ mid, h16 *__restrict__ smid,
                                                             u32 *__restrict__ ids_out, float *__restrict__ w_out,
                                                             u32 nb_routed, const h16 *__restrict__ router,
                                                             float *__restrict__ lg_part) {
    TL(4);
    constexpr u32 K = UOCR_K_HIDDEN, G = K / 64u, I = 896u, ROWS = UOCR_K_TOPK * I, SI = 1792u;
    constexpr u32 NWV = SMALL_BLOCK / 64u;
    __shared__ __attribute__((aligned(16))) h16 xs[UOCR_K_HIDDEN];
    __shared__ float red[16];
    const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (blockIdx.x >= nb_routed) {
        constexpr u32 C = chunks_per_row<QS>(K), LPR = lpr_lat(C), J = j_lat(C), R = 64u / LPR, rb = 16u * C;
        const u32 sub = lane % LPR, grp = lane / LPR;
        const u32 r = ((blockIdx.x - nb_routed) * NWV + wave) * R + grp, rr = min(r, SI - 1u);
        XStage<UOCR_K_HIDDEN, SMALL_BLOCK> sx;
        stage_load(sx, x, nw, UOCR_K_HIDDEN);
        RowFrag<J> fg, fu;
        frag_load<QS, LPR, J, shared_nt<QS>()>(fg, (const uint8_t *)SG.w + (size_t)rr * rb, (const h16 *)SG.s + (size_t)rr * G, C, sub);
        frag_load<QS, LPR, J, shared_nt<QS>()>(fu, (const uint8_t *)SU.w + (size_t)rr * rb, (const h16 *)SU.s + (size_t)rr * G, C, sub);
        stage_store(sx, xs, nw, UOCR_K_HIDDEN, red);
        const float dg = group_sum<LPR>(frag_dot<QS, LPR, J>(fg, xs, C, sub));
        const float du = group_sum<LPR>(frag_dot<QS, LPR, J>(fu, xs, C, sub));
        if (r < SI && sub == 0u) smid[r] = (h16)(silu_f(dg) * du);
        return;
    }
    constexpr u32 C = chunks_per_row<QT>(K), LPR = lpr_lat(C), J = j_lat(C), R = 64u / LPR, rb = 16u * C;
    const u32 sub = lane % LPR, grp = lane / LPR;
    float lg;
    if (FOLD) {
        long long zq[UOCR_K_ROUTER_ACC_COPIES];
#pragma unroll
        for (int k = 0; k < UOCR_K_ROUTER_ACC_COPIES; ++k) zq[k] = racc[k * UOCR_K_EXPERTS + lane];
        long long zt = 0;
#pragma unroll
        for (int k = 0; k < UOCR_K_ROUTER_ACC_COPIES; ++k) zt += zq[k];
        lg = (float)zt * (1.0f / (float)(1ull << UOCR_K_ROUTER_FIX_SHIFT));
    } else {
        lg = logits[lane];
    }
    XStage<UOCR_K_HIDDEN, SMALL_BLOCK> sx;
    stage_load(sx, x, nw, UOCR_K_HIDDEN);
    u32 sid[UOCR_K_TOPK];
    float sw[UOCR_K_TOPK];
    if (FOLD) {
        topk6_ids(lg, sid);
    } else {
        topk6(lg, norm_topk, sid, sw);
    }
    if (!FOLD && blockIdx.x == 0u && wave == 0u && lane < UOCR_K_TOPK) {
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) {
            if (lane == (u32)r) {
                ids_out[r] = sid[r];
                w_out[r] = sw[r];
            }
        }
    }
    const u32 r = (blockIdx.x * NWV + wave) * R + grp, rr = min(r, ROWS - 1u);
    const u32 rank = rr / I, col = rr % I;
    u32 e = sid[0];
#pragma unroll
    for (int k = 1; k < UOCR_K_TOPK; ++k) e = rank == (u32)k ? sid[k] : e;
    e = e < UOCR_K_EXPERTS ? e : 0u;
    RowFrag<J> fg, fu;
    frag_load<QT, LPR, J, UOCR_NT_STREAM>(fg, (const uint8_t *)sl.gate.w + e * sl.gu_w_stride + (size_t)col * rb,
                          (const h16 *)sl.gate.s + e * sl.gu_s_stride + (size_t)col * G, C, sub);
    frag_load<QT, LPR, J, UOCR_NT_STREAM>(fu, (const uint8_t *)sl.up.w + e * sl.gu_w_stride + (size_t)col * rb,
                          (const h16 *)sl.up.s + e * sl.gu_s_stride + (size_t)col * G, C, sub);
    /* FOLD: the experts come from z; the routing weights from the exact
     * logits, summed over the normalised row as the reference rounds it (xs):
     * block b < 256 writes quarter b % 4 of logit b / 4 (columns [320 q,
     * + 320) in order), and k_moe_down takes the softmax */
    constexpr u32 LQ = 4u, LC = K / LQ, LPL = LC / 64u;
    const bool lgb = FOLD && lg_part != nullptr && blockIdx.x < UOCR_K_EXPERTS * LQ && wave == 0u;
    h16 rv[LPL];
    if (lgb) {
        const h16 *rr = router + (size_t)(blockIdx.x / LQ) * K + (blockIdx.x % LQ) * LC + lane * LPL;
#pragma unroll
        for (u32 k = 0; k < LPL; ++k) rv[k] = rr[k];
    }
    const float inv = stage_store(sx, xs, nw, UOCR_K_HIDDEN, red);
    (void)inv;
    if (lgb) {
        const h16 *xr = xs + (blockIdx.x % LQ) * LC + lane * LPL;
        float part = 0.0f;
#pragma unroll
        for (u32 k = 0; k < LPL; ++k) part = fmaf((float)xr[k], (float)rv[k], part);
        part = wave_sum(part);
        if (lane == 0u) lg_part[blockIdx.x] = part;
    }
    if (FOLD && blockIdx.x == 0u && wave == 0u && lane < UOCR_K_TOPK) {
#pragma unroll
        for (int k = 0; k < UOCR_K_TOPK; ++k) {
            if (lane == (u32)k) ids_out[k] = sid[k];
        }
    }
    const float dg = group_sum<LPR>(frag_dot<QT, LPR, J>(fg, xs, C, sub));
    const float du = group_sum<LPR>(frag_dot<QT, LPR, J>(fu, xs, C, sub));
    if (r < ROWS && sub == 0u) mid[r] = (h16)(silu_f(dg) * du);
}

/* Lanes per output row of the down-combine: Q4 32, Q8 and f16 64 (one or
 * two chunk slots per routed row of K = 896), so 1280 rows spread over
 * 160-320 workgroups. */
__host__ __device__ constexpr u32 lpr_down(int QT) {
    return QT == 4 ? 32u : 64u;
}

/* Down projection of the 6 routed experts + weighted combine + shared-expert
 * down + residual, one fp16 rounding:
 * out[c] = f16(sum_r w_r * D_e[c].mid_r + f16(SD[c].smid) + res[c]). */
template <int QT, int QS>
__global__ __launch_bounds__(BLOCK) void k_moe_down(uocr_expert_slab sl, const u32 *__restrict__ ids,
                                                    const float *__restrict__ wts, const h16 *__restrict__ mid,
                                                    uocr_qmat SD, const h16 *__restrict__ smid,
                                                    const h16 *__restrict__ res, h16 *__restrict__ out,
                                                    const float *__restrict__ lg_part, float *__restrict__ w_out) {
    TL(5);
    constexpr u32 I = 896u, SI = 1792u, LPR = lpr_down(QT), R = 64u / LPR;
    constexpr u32 CD = chunks_per_row<QT>(I), JD = (CD + LPR - 1u) / LPR, GD = I / 64u;
    constexpr u32 CS = chunks_per_row<QS>(SI), JS = (CS + LPR - 1u) / LPR, GS = SI / 64u;
    __shared__ __attribute__((aligned(16))) h16 ms[UOCR_K_TOPK * I + SI];
    const u32 lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const u32 sub = lane % LPR, grp = lane / LPR;
    const u32 c = (blockIdx.x * NWAVE + wave) * R + grp, cc = min(c, (u32)UOCR_K_HIDDEN - 1u);
    /* mids first (consumed first), then the shared-down row, then the routed
     * rows once the expert ids are in */
    constexpr u32 NMID = (UOCR_K_TOPK * I + SI) / 8u, PER = (NMID + BLOCK - 1u) / BLOCK;
    uint4 mv[PER];
#pragma unroll
    for (u32 p = 0; p < PER; ++p) {
        const u32 i = min(threadIdx.x + p * BLOCK, NMID - 1u);
        const uint4 *src = i < UOCR_K_TOPK * I / 8u ? (const uint4 *)mid + i : (const uint4 *)smid + (i - UOCR_K_TOPK * I / 8u);
        mv[p] = *src;
    }
    RowFrag<JS> fs;
    frag_load<QS, LPR, JS, shared_nt<QS>()>(fs, (const uint8_t *)SD.w + (size_t)cc * 16u * CS, (const h16 *)SD.s + (size_t)cc * GS, CS,
                           sub);
    u32 e[UOCR_K_TOPK];
    float w[UOCR_K_TOPK];
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        e[r] = ids[r]; /* all 12 loads unconditional: one scalar round trip */
        w[r] = wts[r];
    }
    if (lg_part != nullptr) {
        /* routing weights from the gate/up kernel's logit quarters (lane e:
         * the four quarters of logit e in order): raw softmax probabilities,
         * max-subtracted (moe.metal:53-193); every wavefront takes them */
        const float4 q = ((const float4 *)lg_part)[lane];
        const float p = router_prob(((q.x + q.y) + q.z) + q.w);
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) w[r] = __shfl(p, (int)(e[r] < UOCR_K_EXPERTS ? e[r] : 0u));
        if (w_out != nullptr && blockIdx.x == 0u && wave == 0u && lane < UOCR_K_TOPK) {
            float mine = w[0];
#pragma unroll
            for (int r = 1; r < UOCR_K_TOPK; ++r) mine = lane == (u32)r ? w[r] : mine;
            w_out[lane] = mine;
        }
    }
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        w[r] = e[r] < UOCR_K_EXPERTS ? w[r] : 0.0f;
        e[r] = e[r] < UOCR_K_EXPERTS ? e[r] : 0u;
    }
    RowFrag<JD> fd[UOCR_K_TOPK];
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        frag_load<QT, LPR, JD, UOCR_NT_STREAM>(fd[r], (const uint8_t *)sl.down.w + e[r] * sl.dn_w_stride + (size_t)cc * 16u * CD,
                               (const h16 *)sl.down.s + e[r] * sl.dn_s_stride + (size_t)cc * GD, CD, sub);
    }
#pragma unroll
    for (u32 p = 0; p < PER; ++p) hold(mv[p]);
#pragma unroll
    for (u32 p = 0; p < PER; ++p) {
        const u32 i = threadIdx.x + p * BLOCK;
        if (i < NMID) ((uint4 *)ms)[i] = mv[p];
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        acc = fmaf(w[r], group_sum<LPR>(frag_dot<QT, LPR, JD>(fd[r], ms + r * I, CD, sub)), acc);
    }
    const float sd = group_sum<LPR>(frag_dot<QS, LPR, JS>(fs, ms + UOCR_K_TOPK * I, CS, sub));
    if (c < UOCR_K_HIDDEN && sub == 0u) out[c] = (h16)(acc + (float)(h16)sd + (float)res[c]);
}

/* ------------------------------------------------------------------------ */
/* embedding gather, state                                                   */
/* ------------------------------------------------------------------------ */

template <int QT>
__device__ __forceinline__ void embed_row_body(const uint8_t *__restrict__ W, const h16 *__restrict__ S, u32 vocab,
                                               int32_t tok, h16 *__restrict__ out) {
    const u32 K = UOCR_K_HIDDEN;
    for (u32 c = threadIdx.x; c < K; c += blockDim.x) {
        float v = 0.0f;
        if (tok >= 0 && (u32)tok < vocab) {
            const size_t r = (size_t)tok;
            if (QT == 1) {
                v = (float)((const h16 *)W)[r * K + c];
            } else {
                const float sc = (float)S[r * (K / 64u) + c / 64u];
                if (QT == 3) {
                    v = (float)((const int8_t *)W)[r * K + c] * sc;
                } else {
                    const u32 j = c % 64u;
                    const uint8_t b = W[r * (K / 2u) + (c / 64u) * 32u + (j & 31u)];
                    v = (float)((int)(j < 32u ? (b & 15u) : (b >> 4)) - 8) * sc;
                }
            }
        }
        out[c] = (h16)v;
    }
}

template <int QT>
__global__ __launch_bounds__(BLOCK) void k_embed(const uint8_t *__restrict__ W, const h16 *__restrict__ S, u32 vocab,
                                                 const int32_t *token, const uocr_step_state *st,
                                                 h16 *__restrict__ out) {
    embed_row_body<QT>(W, S, vocab, token != nullptr ? token[0] : st->cur_token, out);
}

/* Text rows of the prompt embedding: row b = dequant(E[ids[b]]) unless
 * mask[b] (image rows are placed by the host). */
template <int QT>
__global__ __launch_bounds__(BLOCK) void k_embed_rows(const uint8_t *__restrict__ W, const h16 *__restrict__ S,
                                                      u32 vocab, const int32_t *__restrict__ ids,
                                                      const uint8_t *__restrict__ mask, h16 *__restrict__ out) {
    const u32 b = blockIdx.x;
    if (mask != nullptr && mask[b] != 0u) return;
    embed_row_body<QT>(W, S, vocab, ids[b], out + (size_t)b * UOCR_K_HIDDEN);
}

/* One replayable prefill step: position i = st->t; copy prompt row i into h
 * and set the causal-prefix attention plan; then st->t = i + 1. */
__global__ __launch_bounds__(BLOCK) void k_prefill_next(uocr_step_state *st, const h16 *__restrict__ prompt,
                                                        h16 *__restrict__ h, RopeTab tab) {
    const int32_t i = st->t;
    const uint4 *src = (const uint4 *)(prompt + (size_t)i * UOCR_K_HIDDEN);
    uint4 *dst = (uint4 *)h;
    for (u32 c = threadIdx.x; c < UOCR_K_HIDDEN / 8u; c += blockDim.x) dst[c] = src[c];
    set_rope(st, i, tab);
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

__global__ void k_prefill_state(uocr_step_state *st, int32_t i, RopeTab tab) {
    set_rope(st, i, tab);
    if (threadIdx.x == 0) {
        st->pos = i;
        st->cache_token = i;
        st->attn_prompt = i + 1;
        st->attn_len = i + 1;
        st->first_gen = 0;
    }
}

__global__ void k_decode_state(uocr_step_state *st, int32_t P, int32_t t, RopeTab tab) {
    set_rope(st, P + t, tab);
    if (threadIdx.x == 0) {
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
}

/* ------------------------------------------------------------------------ */
/* LM head finalize                                                          */
/* ------------------------------------------------------------------------ */

/* Step-state advance for decode step t = st->t (thread 0 of one block, then
 * the RoPE table by threads < 64): position P + t, its KV slot on the
 * ring plan, attention length, t + 1.  It does not depend on the token, so
 * the LM-head launch performs it; the token is chosen by the next kernel. */
__device__ __forceinline__ void advance_state(uocr_step_state *st, const RopeTab &tab, int with_rope) {
    __shared__ int32_t next_pos;
    if (threadIdx.x == 0) {
        const int32_t t = st->t, P = st->prompt_len;
        const int32_t gcount = t + 1;
        const int32_t live = gcount < UOCR_K_RING ? gcount : UOCR_K_RING;
        st->pos = P + t;
        st->cache_token = P + (t % UOCR_K_RING);
        st->attn_prompt = P;
        st->attn_len = P + live;
        st->first_gen = gcount - live;
        st->t = t + 1;
        next_pos = P + t;
    }
    __syncthreads();
    if (with_rope) set_rope(st, next_pos, tab);
}

/* Final norm + LM-head GEMV + argmax: every block reduces its rows to a best
 * (score, row) and adds its key with an atomic max into keys[block % 16]
 * (non-returning: nothing in this launch waits for it).  With advance,
 * block 0 also advances the step state after its rows.  The token itself is
 * chosen from the 16 keys by the next launch (k_qkv_rope's SEL form in a
 * decode step, or k_lm_finalize), after the kernel boundary. */
template <int QT, int LPR, int J>
__global__ __launch_bounds__(BLOCK) void k_lm_keys(const uint8_t *__restrict__ W, const h16 *__restrict__ S, u32 rows,
                                                   const h16 *__restrict__ x, const h16 *__restrict__ nw,
                                                   unsigned long long *keys, uocr_step_state *st, int advance,
                                                   RopeTab tab, int with_rope) {
    TL(6);
    float b = -INFINITY;
    u32 bi = NONE_ID;
    stream_rows<QT, LPR, J, EPI_ARGMAX>(W, S, nullptr, nullptr, rows, UOCR_K_HIDDEN, x, nw, nullptr, nullptr, b, bi);
    if (threadIdx.x == 0) {
        __hip_atomic_fetch_max(keys + blockIdx.x % UOCR_LM_KEYS, argmax_key(b, bi), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    if (advance && st != nullptr && blockIdx.x == 0) advance_state(st, tab, with_rope);
}

/* One wavefront: reads and clears the 16 keys, stores the token (and score)
 * at tokens[st->t - 1] (advance; the LM-head launch already advanced t) or
 * tokens[0], sets st->cur_token, and with EW gathers the token's embedding
 * row into hout (all of the wavefront). */
template <int QE>
__global__ __launch_bounds__(64) void k_lm_finalize(unsigned long long *keys, uocr_step_state *st, int advance,
                                                    int32_t *tokens, float *scores, const uint8_t *__restrict__ EW,
                                                    const h16 *__restrict__ ES, u32 vocab, h16 *__restrict__ hout) {
    const u32 lane = threadIdx.x;
    unsigned long long k = 0ull;
    if (lane < UOCR_LM_KEYS) k = __hip_atomic_exchange(keys + lane, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long best = wave_max_u64(k);
    float b;
    u32 bi;
    key_winner(best, b, bi);
    const int32_t id = bi == NONE_ID ? 0 : (int32_t)bi;
    if (lane == 0) {
        const int32_t t = advance && st != nullptr ? st->t - 1 : 0;
        tokens[t] = id;
        if (scores != nullptr) scores[t] = b;
        if (advance && st != nullptr) st->cur_token = id;
    }
    if (EW != nullptr) embed_row_body<QE>(EW, ES, vocab, id, hout);
}


/* ------------------------------------------------------------------------ */
/* launchers                                                                 */
/* ------------------------------------------------------------------------ */

static bool qt_ok(u32 q) {
    return q == UOCR_QT_F16 || q == UOCR_QT_Q8 || q == UOCR_QT_Q4;
}

static bool mat_ok(uocr_qmat m) {
    return m.w != nullptr && qt_ok(m.qtype) && (m.qtype == UOCR_QT_F16 || m.s != nullptr);
}

static u32 chunks_of(u32 qt, u32 K) {
    return qt == UOCR_QT_Q4 ? K / 32u : (qt == UOCR_QT_Q8 ? K / 16u : K / 8u);
}

#define DISPATCH_QT(qt, F, ...)                                      \
    do {                                                             \
        switch (qt) {                                                \
            case UOCR_QT_F16: F<1>(__VA_ARGS__); break;              \
            case UOCR_QT_Q8: F<3>(__VA_ARGS__); break;               \
            default: F<4>(__VA_ARGS__); break;                       \
        }                                                            \
    } while (0)

/* Workgroups that fit on the device at once for a streaming kernel: waves
 * per SIMD from its register use, 4 SIMDs per CU. */
template <typename KFn>
static u32 resident_blocks(KFn fn) {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
            cus = 256;
        }
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, BLOCK, 0) != hipSuccess || per_cu <= 0) per_cu = 1;
    return (u32)(cus * per_cu);
}

template <int QT, int LPR, int J, int EPI>
static void launch_stream_lj(hipStream_t st, uocr_qmat W, uocr_qmat W2, u32 rows, u32 K, const uint16_t *x,
                             const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    constexpr u32 R = 64u / LPR;
    auto fn = k_stream<QT, LPR, J, EPI>;
    const u32 groups = (rows + R - 1u) / R;
    u32 nb = (groups + NWAVE - 1u) / NWAVE;
    const u32 cap = resident_blocks(fn);
    if (nb > cap) nb = cap;
    hipLaunchKernelGGL(fn, dim3(nb), dim3(BLOCK), 0, st, (const uint8_t *)W.w, (const h16 *)W.s,
                       (const uint8_t *)W2.w, (const h16 *)W2.s, rows, K, (const h16 *)x, (const h16 *)nw,
                       (const h16 *)res, (h16 *)y);
}

template <int QT, int EPI>
static void launch_stream(hipStream_t st, uocr_qmat W, uocr_qmat W2, u32 rows, u32 K, const uint16_t *x,
                          const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    const u32 C = chunks_of(QT, K);
    const u32 lpr = lpr_for(C), j = (C + lpr - 1u) / lpr;
#define LS(L, JJ) launch_stream_lj<QT, L, JJ, EPI>(st, W, W2, rows, K, x, nw, res, y)
    switch (lpr) {
        case 4: if (j <= 5) LS(4, 5); else LS(4, 7); break;
        case 8: if (j <= 5) LS(8, 5); else LS(8, 7); break;
        case 16: if (j <= 5) LS(16, 5); else LS(16, 7); break;
        case 32: if (j <= 5) LS(32, 5); else LS(32, 7); break;
        default: if (j <= 7) LS(64, 7); else LS(64, 16); break;
    }
#undef LS
}

extern "C" hipError_t uocr_launch_gemv(hipStream_t st, uocr_qmat W, uint32_t rows, uint32_t K, const uint16_t *x,
                                       const uint16_t *nw, const uint16_t *res, uint16_t *y) {
    if (!mat_ok(W) || x == nullptr || y == nullptr || rows == 0u || K == 0u || K % 64u != 0u || K > UOCR_K_MAX_K) {
        return hipErrorInvalidValue;
    }
    switch (W.qtype) {
        case UOCR_QT_F16: launch_stream<1, EPI_LINEAR>(st, W, W, rows, K, x, nw, res, y); break;
        case UOCR_QT_Q8: launch_stream<3, EPI_LINEAR>(st, W, W, rows, K, x, nw, res, y); break;
        default: launch_stream<4, EPI_LINEAR>(st, W, W, rows, K, x, nw, res, y); break;
    }
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_swiglu(hipStream_t st, uocr_qmat G, uocr_qmat U, uint32_t rows, uint32_t K,
                                         const uint16_t *x, const uint16_t *nw, uint16_t *mid) {
    if (!mat_ok(G) || !mat_ok(U) || G.qtype != U.qtype || x == nullptr || mid == nullptr || rows == 0u ||
        K == 0u || K % 64u != 0u || K > UOCR_K_MAX_K) {
        return hipErrorInvalidValue;
    }
    switch (G.qtype) {
        case UOCR_QT_F16: launch_stream<1, EPI_SWIGLU>(st, G, U, rows, K, x, nw, nullptr, mid); break;
        case UOCR_QT_Q8: launch_stream<3, EPI_SWIGLU>(st, G, U, rows, K, x, nw, nullptr, mid); break;
        default: launch_stream<4, EPI_SWIGLU>(st, G, U, rows, K, x, nw, nullptr, mid); break;
    }
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_rmsnorm(hipStream_t st, const uint16_t *x, const uint16_t *nw, uint32_t n,
                                          uint16_t *y) {
    if (x == nullptr || nw == nullptr || y == nullptr || n == 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(BLOCK), 0, st, (const h16 *)x, (const h16 *)nw, n, (h16 *)y);
    return hipGetLastError();
}

template <int QT, int QE>
static void launch_qkv_qe(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                          const uint16_t *nw, const uocr_step_state *state, uint16_t *qout, uint16_t *kc,
                          uint16_t *vc, u32 cap, const SelArgs &sa) {
    constexpr u32 R = 64u / lpr_lat(chunks_per_row<QT>(UOCR_K_HIDDEN));
    constexpr u32 ipb = (SMALL_BLOCK / 64) * R;
    hipLaunchKernelGGL((k_qkv_rope<QT, QE>), dim3((1920u + ipb - 1u) / ipb), dim3(SMALL_BLOCK), 0, st, Q, K, V,
                       (const h16 *)h, (const h16 *)nw, state, (h16 *)qout, (h16 *)kc, (h16 *)vc, cap, sa,
                       PlanArg<false>{});
}

template <int QT>
static void launch_qkv_plan_qt(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                               const uint16_t *nw, uocr_step_state *state, uint16_t *qout, uint16_t *kc,
                               uint16_t *vc, u32 cap, const QkvPlan &pl) {
    constexpr u32 R = 64u / lpr_lat(chunks_per_row<QT>(UOCR_K_HIDDEN));
    constexpr u32 ipb = (SMALL_BLOCK / 64) * R;
    SelArgs sa;
    memset(&sa, 0, sizeof(sa));
    PlanArg<true> pa;
    pa.p = pl;
    hipLaunchKernelGGL((k_qkv_rope<QT, 0, true>), dim3((1920u + ipb - 1u) / ipb), dim3(SMALL_BLOCK), 0, st, Q, K, V,
                       (const h16 *)h, (const h16 *)nw, (const uocr_step_state *)state, (h16 *)qout, (h16 *)kc,
                       (h16 *)vc, cap, sa, pa);
}

template <int QT>
static void launch_qkv_qt(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                          const uint16_t *nw, const uocr_step_state *state, uint16_t *qout, uint16_t *kc,
                          uint16_t *vc, u32 cap, const SelArgs &sa, u32 qe) {
    switch (qe) {
        case 0u: launch_qkv_qe<QT, 0>(st, Q, K, V, h, nw, state, qout, kc, vc, cap, sa); break;
        case UOCR_QT_F16: launch_qkv_qe<QT, 1>(st, Q, K, V, h, nw, state, qout, kc, vc, cap, sa); break;
        case UOCR_QT_Q8: launch_qkv_qe<QT, 3>(st, Q, K, V, h, nw, state, qout, kc, vc, cap, sa); break;
        default: launch_qkv_qe<QT, 4>(st, Q, K, V, h, nw, state, qout, kc, vc, cap, sa); break;
    }
}

extern "C" hipError_t uocr_launch_qkv_rope(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V, const uint16_t *h,
                                           const uint16_t *nw, const uocr_step_state *state, uint16_t *qout,
                                           uint16_t *kcache, uint16_t *vcache, uint32_t cache_capacity) {
    if (!mat_ok(Q) || !mat_ok(K) || !mat_ok(V) || Q.qtype != K.qtype || Q.qtype != V.qtype || h == nullptr ||
        nw == nullptr || state == nullptr || qout == nullptr || kcache == nullptr || vcache == nullptr ||
        cache_capacity == 0u) {
        return hipErrorInvalidValue;
    }
    SelArgs sa;
    memset(&sa, 0, sizeof(sa));
    DISPATCH_QT(Q.qtype, launch_qkv_qt, st, Q, K, V, h, nw, state, qout, kcache, vcache, cache_capacity, sa, 0u);
    return hipGetLastError();
}

static RopeTab rope_tab(const float *inv_freq);

extern "C" hipError_t uocr_launch_qkv_rope_plan(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V,
                                                const uint16_t *h, const uint16_t *nw, uocr_step_state *state,
                                                uint16_t *qout, uint16_t *kcache, uint16_t *vcache,
                                                uint32_t cache_capacity, int32_t prompt_len, int32_t t,
                                                const float *inv_freq) {
    if (!mat_ok(Q) || !mat_ok(K) || !mat_ok(V) || Q.qtype != K.qtype || Q.qtype != V.qtype || h == nullptr ||
        nw == nullptr || state == nullptr || qout == nullptr || kcache == nullptr || vcache == nullptr ||
        cache_capacity == 0u || inv_freq == nullptr || prompt_len <= 0 || t < 0) {
        return hipErrorInvalidValue;
    }
    QkvPlan pl;
    pl.P = prompt_len;
    pl.t = t;
    pl.st = state;
    pl.tab = rope_tab(inv_freq);
    DISPATCH_QT(Q.qtype, launch_qkv_plan_qt, st, Q, K, V, h, nw, state, qout, kcache, vcache, cache_capacity, pl);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_qkv_rope_select(hipStream_t st, uocr_qmat Q, uocr_qmat K, uocr_qmat V,
                                                  const uint16_t *nw, uocr_step_state *state, uint16_t *qout,
                                                  uint16_t *kcache, uint16_t *vcache, uint32_t cache_capacity,
                                                  const uint64_t *keys, uocr_qmat E, uint32_t vocab, int32_t *tokens,
                                                  float *scores, uint16_t *hout) {
    if (!mat_ok(Q) || !mat_ok(K) || !mat_ok(V) || Q.qtype != K.qtype || Q.qtype != V.qtype || nw == nullptr ||
        state == nullptr || qout == nullptr || kcache == nullptr || vcache == nullptr || cache_capacity == 0u ||
        keys == nullptr || !mat_ok(E) || vocab == 0u || tokens == nullptr || hout == nullptr) {
        return hipErrorInvalidValue;
    }
    SelArgs sa;
    sa.keys = (const unsigned long long *)keys;
    sa.EW = (const uint8_t *)E.w;
    sa.ES = (const h16 *)E.s;
    sa.vocab = vocab;
    sa.tokens = tokens;
    sa.scores = scores;
    sa.stw = state;
    sa.hout = (h16 *)hout;
    DISPATCH_QT(Q.qtype, launch_qkv_qt, st, Q, K, V, nullptr, nw, state, qout, kcache, vcache, cache_capacity, sa,
                E.qtype);
    return hipGetLastError();
}

/* splits blocks per head over a partials layout of SL splits; one round of
 * loads per block where the range allows it */
template <int SL>
static void launch_attention_sl(hipStream_t st, const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache,
                                uint32_t cache_capacity, const uocr_step_state *state, float *partials,
                                int64_t *router_acc, uint64_t *clear_keys, uint32_t splits) {
    const u32 chunk = (cache_capacity + splits - 1u) / splits;
    auto *kern = chunk <= 2u * ATT_GROUPS   ? k_attention<2, SL>
                 : chunk <= 3u * ATT_GROUPS ? k_attention<3, SL>
                 : chunk <= 5u * ATT_GROUPS ? k_attention<5, SL>
                 : chunk <= 6u * ATT_GROUPS ? k_attention<6, SL>
                                            : k_attention<9, SL>;
    hipLaunchKernelGGL(kern, dim3(splits, UOCR_K_HEADS), dim3(ATT_THREADS), 0, st, (const h16 *)q,
                       (const h16 *)kcache, (const h16 *)vcache, cache_capacity, state, partials,
                       (long long *)router_acc, (unsigned long long *)clear_keys);
}

extern "C" hipError_t uocr_launch_attention(hipStream_t st, const uint16_t *q, const uint16_t *kcache,
                                            const uint16_t *vcache, uint32_t cache_capacity,
                                            const uocr_step_state *state, float *partials, int64_t *router_acc,
                                            uint64_t *clear_keys) {
    if (q == nullptr || kcache == nullptr || vcache == nullptr || cache_capacity == 0u || state == nullptr ||
        partials == nullptr) {
        return hipErrorInvalidValue;
    }
    launch_attention_sl<UOCR_K_ATTN_SPLITS>(st, q, kcache, vcache, cache_capacity, state, partials, router_acc,
                                            clear_keys, UOCR_K_ATTN_SPLITS);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_attention_wide(hipStream_t st, const uint16_t *q, const uint16_t *kcache,
                                                 const uint16_t *vcache, uint32_t cache_capacity,
                                                 const uocr_step_state *state, float *partials, uint32_t splits) {
    if (q == nullptr || kcache == nullptr || vcache == nullptr || cache_capacity == 0u || state == nullptr ||
        partials == nullptr || splits == 0u || splits > UOCR_K_ATTN_SPLITS_WIDE) {
        return hipErrorInvalidValue;
    }
    launch_attention_sl<UOCR_K_ATTN_SPLITS_WIDE>(st, q, kcache, vcache, cache_capacity, state, partials, nullptr,
                                                 nullptr, splits);
    return hipGetLastError();
}

template <int QT>
static void launch_attn_out_qt(hipStream_t st, uocr_qmat O, const float *partials, const uint16_t *res, uint16_t *out,
                               uint16_t *ctx_out, const float *fold, int64_t *racc) {
    constexpr u32 rpb = NWAVE * (64u / lpr_for(chunks_per_row<QT>(UOCR_K_HIDDEN)));
    const dim3 grid((UOCR_K_HIDDEN + rpb - 1u) / rpb);
    if (fold != nullptr) {
        hipLaunchKernelGGL((k_attn_out<QT, true>), grid, dim3(BLOCK), 0, st, O, partials, (const h16 *)res,
                           (h16 *)out, (h16 *)ctx_out, fold, (long long *)racc);
    } else {
        hipLaunchKernelGGL((k_attn_out<QT, false>), grid, dim3(BLOCK), 0, st, O, partials, (const h16 *)res,
                           (h16 *)out, (h16 *)ctx_out, nullptr, nullptr);
    }
}

extern "C" hipError_t uocr_launch_attn_out(hipStream_t st, uocr_qmat O, const float *partials, const uint16_t *res,
                                           uint16_t *out, uint16_t *ctx_out, const float *router_fold,
                                           int64_t *router_acc) {
    if (!mat_ok(O) || partials == nullptr || res == nullptr || out == nullptr ||
        (router_fold != nullptr && router_acc == nullptr)) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(O.qtype, launch_attn_out_qt, st, O, partials, res, out, ctx_out, router_fold, router_acc);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_attn_merge(hipStream_t st, const float *partials, uint16_t *ctx) {
    if (partials == nullptr || ctx == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_attn_merge<UOCR_K_ATTN_SPLITS>, dim3(1), dim3(BLOCK), 0, st, partials, (h16 *)ctx);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_attn_merge_wide(hipStream_t st, const float *partials, uint16_t *ctx) {
    if (partials == nullptr || ctx == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_attn_merge<UOCR_K_ATTN_SPLITS_WIDE>, dim3(1), dim3(BLOCK), 0, st, partials, (h16 *)ctx);
    return hipGetLastError();
}

template <int QT>
static void launch_attn_out_wide_qt(hipStream_t st, uocr_qmat O, const float *partials, const uint16_t *res,
                                    uint16_t *out, uint16_t *ctx_out) {
    constexpr u32 rpb = NWAVE * (64u / lpr_for(chunks_per_row<QT>(UOCR_K_HIDDEN)));
    hipLaunchKernelGGL((k_attn_out<QT, false, UOCR_K_ATTN_SPLITS_WIDE>), dim3((UOCR_K_HIDDEN + rpb - 1u) / rpb),
                       dim3(BLOCK), 0, st, O, partials, (const h16 *)res, (h16 *)out, (h16 *)ctx_out, nullptr, nullptr);
}

extern "C" hipError_t uocr_launch_attn_out_wide(hipStream_t st, uocr_qmat O, const float *partials,
                                                const uint16_t *res, uint16_t *out, uint16_t *ctx_out) {
    if (!mat_ok(O) || partials == nullptr || res == nullptr || out == nullptr) return hipErrorInvalidValue;
    DISPATCH_QT(O.qtype, launch_attn_out_wide_qt, st, O, partials, res, out, ctx_out);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_router_logits(hipStream_t st, const uint16_t *R, const uint16_t *x,
                                                const uint16_t *nw, float *logits) {
    if (R == nullptr || x == nullptr || logits == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_router_logits, dim3(UOCR_K_EXPERTS / ROUTER_ROWS), dim3(64 * ROUTER_ROWS), 0, st,
                       (const h16 *)R, (const h16 *)x, (const h16 *)nw, logits);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_router(hipStream_t st, const uint16_t *R, const uint16_t *x, const uint16_t *nw,
                                         int norm_topk, float *logits, uint32_t *ids, float *weights) {
    if (ids == nullptr || weights == nullptr) return hipErrorInvalidValue;
    const hipError_t e = uocr_launch_router_logits(st, R, x, nw, logits);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_router_topk, dim3(1), dim3(64), 0, st, (const float *)logits, norm_topk, ids, weights);
    return hipGetLastError();
}

template <int QT, int QS>
static void launch_moe_gu_qs(hipStream_t st, const uocr_expert_slab *slab, uocr_qmat SG, uocr_qmat SU,
                             const float *logits, const int64_t *racc, int norm_topk, const uint16_t *x,
                             const uint16_t *nw, uint16_t *mid, uint16_t *smid, u32 *ids, float *wts,
                             const uint16_t *router, float *lg_part) {
    constexpr u32 NWV = SMALL_BLOCK / 64u;
    constexpr u32 rpb = NWV * (64u / lpr_lat(chunks_per_row<QT>(UOCR_K_HIDDEN)));
    constexpr u32 rpb_s = NWV * (64u / lpr_lat(chunks_per_row<QS>(UOCR_K_HIDDEN)));
    constexpr u32 nbr = (UOCR_K_TOPK * 896u + rpb - 1u) / rpb, nbs = (1792u + rpb_s - 1u) / rpb_s;
    if (racc != nullptr) {
        hipLaunchKernelGGL((k_moe_gate_up<QT, QS, true>), dim3(nbr + nbs), dim3(SMALL_BLOCK), 0, st, *slab, SG, SU,
                           nullptr, (const long long *)racc, norm_topk, (const h16 *)x, (const h16 *)nw, (h16 *)mid,
                           (h16 *)smid, ids, wts, nbr, (const h16 *)router, lg_part);
    } else {
        hipLaunchKernelGGL((k_moe_gate_up<QT, QS, false>), dim3(nbr + nbs), dim3(SMALL_BLOCK), 0, st, *slab, SG, SU,
                           logits, nullptr, norm_topk, (const h16 *)x, (const h16 *)nw, (h16 *)mid, (h16 *)smid, ids,
                           wts, nbr, nullptr, nullptr);
    }
}

template <int QT>
static void launch_moe_gu_qt(hipStream_t st, const uocr_expert_slab *slab, uocr_qmat SG, uocr_qmat SU,
                             const float *logits, const int64_t *racc, int norm_topk, const uint16_t *x,
                             const uint16_t *nw, uint16_t *mid, uint16_t *smid, u32 *ids, float *wts,
                             const uint16_t *router, float *lg_part) {
#define GU(QS) launch_moe_gu_qs<QT, QS>(st, slab, SG, SU, logits, racc, norm_topk, x, nw, mid, smid, ids, wts, router, lg_part)
    switch (SG.qtype) {
        case UOCR_QT_F16: GU(1); break;
        case UOCR_QT_Q8: GU(3); break;
        default: GU(4); break;
    }
#undef GU
}

extern "C" hipError_t uocr_launch_moe_gate_up(hipStream_t st, const uocr_expert_slab *slab, uocr_qmat SG,
                                              uocr_qmat SU, const float *logits, const int64_t *router_acc,
                                              int norm_topk, const uint16_t *x, const uint16_t *nw, uint16_t *mid,
                                              uint16_t *smid, uint32_t *ids, float *weights, const uint16_t *router,
                                              float *lg_part) {
    if (slab == nullptr || !mat_ok(slab->gate) || !mat_ok(slab->up) || slab->gate.qtype != slab->up.qtype ||
        !mat_ok(SG) || !mat_ok(SU) || SG.qtype != SU.qtype || (logits == nullptr) == (router_acc == nullptr) ||
        x == nullptr || mid == nullptr || smid == nullptr || ids == nullptr || weights == nullptr ||
        (lg_part != nullptr && (router == nullptr || router_acc == nullptr || nw == nullptr))) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(slab->gate.qtype, launch_moe_gu_qt, st, slab, SG, SU, logits, router_acc, norm_topk, x, nw, mid, smid,
                ids, weights, router, lg_part);
    return hipGetLastError();
}

template <int QT, int QS>
static void launch_moe_down_qs(hipStream_t st, const uocr_expert_slab *slab, const u32 *ids, const float *wts,
                               const uint16_t *mid, uocr_qmat SD, const uint16_t *smid, const uint16_t *res,
                               uint16_t *out, const float *lg_part, float *w_out) {
    constexpr u32 rpb = NWAVE * (64u / lpr_down(QT));
    hipLaunchKernelGGL((k_moe_down<QT, QS>), dim3((UOCR_K_HIDDEN + rpb - 1u) / rpb), dim3(BLOCK), 0, st, *slab, ids,
                       wts, (const h16 *)mid, SD, (const h16 *)smid, (const h16 *)res, (h16 *)out, lg_part, w_out);
}

template <int QT>
static void launch_moe_down_qt(hipStream_t st, const uocr_expert_slab *slab, const u32 *ids, const float *wts,
                               const uint16_t *mid, uocr_qmat SD, const uint16_t *smid, const uint16_t *res,
                               uint16_t *out, const float *lg_part, float *w_out) {
    switch (SD.qtype) {
        case UOCR_QT_F16: launch_moe_down_qs<QT, 1>(st, slab, ids, wts, mid, SD, smid, res, out, lg_part, w_out); break;
        case UOCR_QT_Q8: launch_moe_down_qs<QT, 3>(st, slab, ids, wts, mid, SD, smid, res, out, lg_part, w_out); break;
        default: launch_moe_down_qs<QT, 4>(st, slab, ids, wts, mid, SD, smid, res, out, lg_part, w_out); break;
    }
}

extern "C" hipError_t uocr_launch_moe_down(hipStream_t st, const uocr_expert_slab *slab, const uint32_t *ids,
                                           const float *weights, const uint16_t *mid, uocr_qmat SD,
                                           const uint16_t *smid, const uint16_t *res, uint16_t *out,
                                           const float *lg_part, float *w_out) {
    if (slab == nullptr || !mat_ok(slab->down) || !mat_ok(SD) || ids == nullptr ||
        (weights == nullptr && lg_part == nullptr) || mid == nullptr || smid == nullptr || res == nullptr ||
        out == nullptr) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(slab->down.qtype, launch_moe_down_qt, st, slab, ids, weights, mid, SD, smid, res, out, lg_part, w_out);
    return hipGetLastError();
}

static RopeTab rope_tab(const float *inv_freq) {
    RopeTab tab;
    for (int i = 0; i < UOCR_K_HEAD_DIM / 2; ++i) tab.f[i] = inv_freq != nullptr ? inv_freq[i] : 0.0f;
    return tab;
}

template <int QT>
static void launch_lm_keys_qt(hipStream_t st, uocr_qmat W, u32 vocab, const uint16_t *x, const uint16_t *nw,
                              uint64_t *keys, uocr_step_state *state, int advance, const float *inv_freq) {
    constexpr u32 C = chunks_per_row<QT>(UOCR_K_HIDDEN), LPR = lpr_for(C), J = j_for(C), R = 64u / LPR;
    auto fn = k_lm_keys<QT, LPR, J>;
    const u32 groups = (vocab + R - 1u) / R;
    u32 nb = (groups + NWAVE - 1u) / NWAVE;
    nb = min(nb, min(resident_blocks(fn), (u32)UOCR_K_LM_BLOCKS));
    hipLaunchKernelGGL(fn, dim3(nb), dim3(BLOCK), 0, st, (const uint8_t *)W.w, (const h16 *)W.s, vocab,
                       (const h16 *)x, (const h16 *)nw, (unsigned long long *)keys, state, advance,
                       rope_tab(inv_freq), inv_freq != nullptr ? 1 : 0);
}

extern "C" hipError_t uocr_launch_lm_keys(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x,
                                          const uint16_t *nw, uint64_t *keys, uocr_step_state *state, int advance,
                                          const float *inv_freq) {
    if (!mat_ok(W) || vocab == 0u || x == nullptr || keys == nullptr || (advance && state == nullptr)) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(W.qtype, launch_lm_keys_qt, st, W, vocab, x, nw, keys, state, advance, inv_freq);
    return hipGetLastError();
}

template <int QE>
static void launch_lm_finalize_qe(hipStream_t st, uint64_t *keys, uocr_step_state *state, int advance,
                                  int32_t *tokens, float *scores, uocr_qmat E, u32 vocab, uint16_t *hout) {
    hipLaunchKernelGGL((k_lm_finalize<QE>), dim3(1), dim3(64), 0, st, (unsigned long long *)keys, state, advance,
                       tokens, scores, (const uint8_t *)E.w, (const h16 *)E.s, vocab, (h16 *)hout);
}

extern "C" hipError_t uocr_launch_lm_finalize(hipStream_t st, uint64_t *keys, uocr_step_state *state, int advance,
                                              int32_t *tokens, float *scores, uocr_qmat E, uint32_t vocab,
                                              uint16_t *hout) {
    if (keys == nullptr || tokens == nullptr || (advance && state == nullptr) ||
        (E.w != nullptr && (!mat_ok(E) || hout == nullptr))) {
        return hipErrorInvalidValue;
    }
    DISPATCH_QT(E.w != nullptr ? E.qtype : UOCR_QT_Q4, launch_lm_finalize_qe, st, keys, state, advance, tokens,
                scores, E, vocab, hout);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_lm_head(hipStream_t st, uocr_qmat W, uint32_t vocab, const uint16_t *x,
                                          const uint16_t *nw, uint32_t *partials, uocr_step_state *state, int advance,
                                          int32_t *tokens, float *scores, uocr_qmat E, uint16_t *hout,
                                          const float *inv_freq) {
    if (!mat_ok(W) || vocab == 0u || x == nullptr || partials == nullptr || tokens == nullptr ||
        (advance && state == nullptr) || (E.w != nullptr && (!mat_ok(E) || hout == nullptr))) {
        return hipErrorInvalidValue;
    }
    const hipError_t e = uocr_launch_lm_keys(st, W, vocab, x, nw, (uint64_t *)partials, state, advance, inv_freq);
    if (e != hipSuccess) return e;
    return uocr_launch_lm_finalize(st, (uint64_t *)partials, state, advance, tokens, scores, E, vocab, hout);
}

template <int QT>
static void launch_embed_qt(hipStream_t st, uocr_qmat E, u32 vocab, const int32_t *token,
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
static void launch_embed_rows_qt(hipStream_t st, uocr_qmat E, u32 vocab, const int32_t *ids, const uint8_t *mask,
                                 u32 n, uint16_t *out) {
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
                                               uint16_t *h, const float *inv_freq) {
    if (state == nullptr || prompt == nullptr || h == nullptr || inv_freq == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_prefill_next, dim3(1), dim3(BLOCK), 0, st, state, (const h16 *)prompt, (h16 *)h,
                       rope_tab(inv_freq));
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_prefill_state(hipStream_t st, uocr_step_state *state, int32_t i,
                                                const float *inv_freq) {
    if (state == nullptr || i < 0 || inv_freq == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_prefill_state, dim3(1), dim3(64), 0, st, state, i, rope_tab(inv_freq));
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_decode_state(hipStream_t st, uocr_step_state *state, int32_t prompt_len, int32_t t,
                                               const float *inv_freq) {
    if (state == nullptr || prompt_len <= 0 || t < 0 || inv_freq == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_decode_state, dim3(1), dim3(64), 0, st, state, prompt_len, t, rope_tab(inv_freq));
    return hipGetLastError();
}
