/*
 * uocr_dev.h - device helpers shared by the decode kernels of
 * libunlimitedocr.so (uocr_kernels.hip, uocr_decode_run.hip): wavefront and
 * block reductions, activation staging, the exact packed Q8_0 / Q4_0 / f16
 * 16-byte chunk dequant-dots, lane-group row fragments, the router's greedy
 * top-6 and the 64-bit argmax keys of the LM head.
 */
#ifndef UOCR_DEV_H
#define UOCR_DEV_H

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "uocr_kernels.h"

typedef _Float16 h16;
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32;

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

/* 64-bit argmax key of a (score, row) pair: the largest key is the highest
 * score with the lowest row among equals; -0 ranks as +0; 0 means no valid
 * row (lm_head_q4.metal:48-97, sampling.metal:173-200: NaN rows skipped,
 * ties to the lowest id, none valid -> token 0). */
__device__ __forceinline__ unsigned long long argmax_key(float b, u32 bi) {
    if (bi == NONE_ID) return 0ull;
    const u32 u = __float_as_uint(b == 0.0f ? 0.0f : b);
    const u32 o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xffffffffu - bi);
}

__device__ __forceinline__ void key_winner(unsigned long long best, float &b, u32 &bi) {
    if (best == 0ull) {
        b = -INFINITY;
        bi = NONE_ID;
    } else {
        const u32 o = (u32)(best >> 32);
        b = __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
        bi = 0xffffffffu - (u32)best;
    }
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

/* Compiler-only fence on loaded values: every memory access before it stays
 * before it, and v is consumed only after it.  Placed after a kernel's
 * weight loads, it makes the compiler wait for an earlier-issued activation
 * load with an in-order count that leaves the weight loads in flight
 * (vector loads retire in issue order). */
__device__ __forceinline__ void hold(uint4 &v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)::"memory");
}
__device__ __forceinline__ void hold(float4 &v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w)::"memory");
}
__device__ __forceinline__ void hold(float2 &v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y)::"memory");
}

/* ------------------------------------------------------------------------ */
/* activation staging                                                        */
/* ------------------------------------------------------------------------ */

/* Activation staging in two halves so the activation loads are issued
 * before a kernel's weight loads (vector loads retire in order: a load issued
 * after the weights could only be consumed once every weight load is back).
 * stage_load puts this thread's 16-byte pieces of x (and of the RMSNorm
 * weight nw) in registers; stage_store, called after the weight loads are
 * issued, applies RMSNorm (eps 1e-6) when nw is set,
 *   xs[i] = f16(x[i] * inv_rms * nw[i])   (norm.metal:12-40 arithmetic:
 *   fp32 sum of squares, one rounding per element),
 * writes xs to LDS and synchronises the block, and returns inv_rms (1 without
 * nw).  KMAX and NT (threads) are
 * compile-time; the runtime K (multiple of 8, <= KMAX) masks the pieces. */
template <int KMAX, int NT>
struct XStage {
    static constexpr int PER = (KMAX / 8 + NT - 1) / NT;
    uint4 x[PER], w[PER];
};

template <int KMAX, int NT>
__device__ __forceinline__ void stage_load(XStage<KMAX, NT> &sx, const h16 *x, const h16 *nw, int K) {
    /* branch-free (clamped index, nw aliased to x when absent) so the
     * compiler keeps every load ahead of the first wait */
    const uint4 *xp = (const uint4 *)x, *wp = (const uint4 *)(nw != nullptr ? nw : x);
    const int last = K / 8 - 1;
#pragma unroll
    for (int p = 0; p < XStage<KMAX, NT>::PER; ++p) {
        const int i = min((int)threadIdx.x + p * NT, last);
        sx.x[p] = xp[i];
        sx.w[p] = wp[i];
    }
}

template <int KMAX, int NT>
__device__ __forceinline__ float stage_store(XStage<KMAX, NT> &sx, h16 *xs, const h16 *nw, int K, float *red) {
#pragma unroll
    for (int p = 0; p < XStage<KMAX, NT>::PER; ++p) {
        hold(sx.x[p]);
        hold(sx.w[p]);
    }
    union h8 {
        uint4 u;
        h16 h[8];
    };
    float inv = 1.0f;
    if (nw != nullptr) {
        float ss = 0.0f;
#pragma unroll
        for (int p = 0; p < XStage<KMAX, NT>::PER; ++p) {
            if ((int)threadIdx.x + p * NT < K / 8) {
                h8 v;
                v.u = sx.x[p];
#pragma unroll
                for (int j = 0; j < 8; ++j) ss = fmaf((float)v.h[j], (float)v.h[j], ss);
            }
        }
        ss = block_sum(ss, red);
        inv = 1.0f / sqrtf(ss / (float)K + 1.0e-6f);
#pragma unroll
        for (int p = 0; p < XStage<KMAX, NT>::PER; ++p) {
            const int i = threadIdx.x + p * NT;
            if (i < K / 8) {
                h8 v, w;
                v.u = sx.x[p];
                w.u = sx.w[p];
#pragma unroll
                for (int j = 0; j < 8; ++j) v.h[j] = (h16)(((float)v.h[j] * inv) * (float)w.h[j]);
                ((uint4 *)xs)[i] = v.u;
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < XStage<KMAX, NT>::PER; ++p) {
            const int i = threadIdx.x + p * NT;
            if (i < K / 8) ((uint4 *)xs)[i] = sx.x[p];
        }
    }
    __syncthreads();
    return inv;
}

/* ------------------------------------------------------------------------ */
/* 16-byte chunk dequant-dots                                                */
/* ------------------------------------------------------------------------ */

/* Chunks per row and chunks per 64-column scale group. */
template <int QT>
__host__ __device__ constexpr u32 chunks_per_row(u32 K) {
    return QT == 4 ? K / 32u : (QT == 3 ? K / 16u : K / 8u);
}
template <int QT>
__host__ __device__ constexpr u32 chunks_per_group() {
    return QT == 4 ? 2u : 4u;
}

__device__ __forceinline__ h16x2 as_h2(u32 v) {
    return __builtin_bit_cast(h16x2, v);
}

/* fp16 pair (1024 + b0, 1024 + b1) from bytes b0, b1 of v selected by SEL. */
template <u32 SEL>
__device__ __forceinline__ h16x2 magic_pair(u32 v) {
    return as_h2(__builtin_amdgcn_perm(0x64646464u, v, SEL));
}
#define SEL01 0x04010400u /* bytes 0,1 */
#define SEL23 0x04030402u /* bytes 2,3 */

__device__ __forceinline__ float dot2(h16x2 a, u32 x, float acc) {
    return __builtin_amdgcn_fdot2(a, as_h2(x), acc, false);
}

template <int QT>
__device__ __forceinline__ float chunk_dot(const uint4 w, const h16 *xs, u32 c);

/* Q4_0: chunk c is bytes 16*(c&1)..+15 of 64-column group c>>1; byte i holds
 * column g*64 + 16*(c&1) + i in its low nibble and the same + 32 in its high
 * nibble, each stored as q + 8. */
template <>
__device__ __forceinline__ float chunk_dot<4>(const uint4 w, const h16 *xs, u32 c) {
    const uint4 *xp = (const uint4 *)(xs + (c >> 1) * 64u + (c & 1u) * 16u);
    const uint4 l0 = xp[0], l1 = xp[1], g0 = xp[4], g1 = xp[5];
    const u32 xl[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    const u32 xh[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const u32 wv[4] = {w.x, w.y, w.z, w.w};
    /* low nibbles: 1024 + q + 8 - 1032 = q; high nibbles stay in place
     * (bytes 16 (q + 8)): 1024 + 16 (q + 8) - 1152 = 16 q, exact, summed in
     * a second chain and scaled back by 1/16 (exact) */
    const h16x2 bl = {(h16)1032.0f, (h16)1032.0f}, bh = {(h16)1152.0f, (h16)1152.0f};
    float dl = 0.0f, dh = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32 lo = wv[b] & 0x0F0F0F0Fu, hi = wv[b] & 0xF0F0F0F0u;
        dl = dot2(magic_pair<SEL01>(lo) - bl, xl[2 * b], dl);
        dh = dot2(magic_pair<SEL01>(hi) - bh, xh[2 * b], dh);
        dl = dot2(magic_pair<SEL23>(lo) - bl, xl[2 * b + 1], dl);
        dh = dot2(magic_pair<SEL23>(hi) - bh, xh[2 * b + 1], dh);
    }
    return fmaf(dh, 0.0625f, dl);
}

/* Q8_0: chunk c is columns 16c..16c+15; byte ^ 0x80 = q + 128. */
template <>
__device__ __forceinline__ float chunk_dot<3>(const uint4 w, const h16 *xs, u32 c) {
    const uint4 *xp = (const uint4 *)(xs + 16u * c);
    const uint4 a = xp[0], b4 = xp[1];
    const u32 xv[8] = {a.x, a.y, a.z, a.w, b4.x, b4.y, b4.z, b4.w};
    const u32 wv[4] = {w.x, w.y, w.z, w.w};
    const h16x2 bias = {(h16)1152.0f, (h16)1152.0f};
    float d = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32 u = wv[b] ^ 0x80808080u;
        d = dot2(magic_pair<SEL01>(u) - bias, xv[2 * b], d);
        d = dot2(magic_pair<SEL23>(u) - bias, xv[2 * b + 1], d);
    }
    return d;
}

/* f16: chunk c is columns 8c..8c+7. */
template <>
__device__ __forceinline__ float chunk_dot<1>(const uint4 w, const h16 *xs, u32 c) {
    const uint4 a = *(const uint4 *)(xs + 8u * c);
    float d = 0.0f;
    d = dot2(as_h2(w.x), a.x, d);
    d = dot2(as_h2(w.y), a.y, d);
    d = dot2(as_h2(w.z), a.z, d);
    d = dot2(as_h2(w.w), a.w, d);
    return d;
}

/* Offset-free chunk dots.  Each weight byte is taken as the unsigned
 * integer u it stores (Q4: q + 8 per nibble, Q8: q + 128 after flipping the
 * sign bit) and placed in an fp16 subnormal, u * 2^-24 (exact), so a weight
 * pair costs one v_perm and no bias subtraction; the returned raw dot is
 * sum(u * x) * 2^-24.  chunk_value() restores q = u - bias with the sum of
 * the chunk's activations:  scale * (2^24 raw - bias * xsum).  fp16
 * subnormals are preserved by the dot instructions (the kernels run with
 * fp16 denormals enabled, the compiler's default). */
template <int QT>
__device__ __forceinline__ float chunk_dot_u(const uint4 w, const h16 *xs, u32 c);

template <>
__device__ __forceinline__ float chunk_dot_u<4>(const uint4 w, const h16 *xs, u32 c) {
    const uint4 *xp = (const uint4 *)(xs + (c >> 1) * 64u + (c & 1u) * 16u);
    const uint4 l0 = xp[0], l1 = xp[1], g0 = xp[4], g1 = xp[5];
    const u32 xl[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
    const u32 xh[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const u32 wv[4] = {w.x, w.y, w.z, w.w};
    /* high nibbles stay in place (bytes 16 u): their chain is scaled by 1/16 */
    float dl = 0.0f, dh = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32 lo = wv[b] & 0x0F0F0F0Fu, hi = wv[b] & 0xF0F0F0F0u;
        dl = dot2(as_h2(__builtin_amdgcn_perm(0u, lo, SEL01)), xl[2 * b], dl);
        dh = dot2(as_h2(__builtin_amdgcn_perm(0u, hi, SEL01)), xh[2 * b], dh);
        dl = dot2(as_h2(__builtin_amdgcn_perm(0u, lo, SEL23)), xl[2 * b + 1], dl);
        dh = dot2(as_h2(__builtin_amdgcn_perm(0u, hi, SEL23)), xh[2 * b + 1], dh);
    }
    return fmaf(dh, 0.0625f, dl);
}

template <>
__device__ __forceinline__ float chunk_dot_u<3>(const uint4 w, const h16 *xs, u32 c) {
    const uint4 *xp = (const uint4 *)(xs + 16u * c);
    const uint4 a = xp[0], b4 = xp[1];
    const u32 xv[8] = {a.x, a.y, a.z, a.w, b4.x, b4.y, b4.z, b4.w};
    const u32 wv[4] = {w.x, w.y, w.z, w.w};
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const u32 u = wv[b] ^ 0x80808080u;
        d0 = dot2(as_h2(__builtin_amdgcn_perm(0u, u, SEL01)), xv[2 * b], d0);
        d1 = dot2(as_h2(__builtin_amdgcn_perm(0u, u, SEL23)), xv[2 * b + 1], d1);
    }
    return d0 + d1;
}

template <int QT>
__host__ __device__ constexpr float chunk_bias() {
    return QT == 4 ? 8.0f : 128.0f;
}
/* scale * (q . x) of a chunk from its raw dot and nx = -bias * xsum */
__device__ __forceinline__ float chunk_value(float raw, float scale, float nx) {
    return scale * fmaf(raw, 16777216.0f, nx);
}

/* Chunk sums of an activation row held as 8-element pieces, thread t of a
 * wavefront-aligned range holding the fp32 sum p of piece t (0 past the
 * row): Q4 chunk 2g + h is pieces 8g + 2h, +1, +4, +5 (columns 64g + 16h
 * and + 32), a Q8 chunk pieces 2c, 2c + 1.  Every lane of the wavefront
 * calls it. */
__device__ __forceinline__ void piece_sums(float p, u32 t, u32 npieces, float *x4, float *x8) {
    const float s1 = p + __shfl_xor(p, 1);
    const float s2 = s1 + __shfl_xor(s1, 4);
    if (t < npieces) {
        if (x8 != nullptr && (t & 1u) == 0u) x8[t >> 1] = s1;
        if (x4 != nullptr && (t & 7u) == 0u) x4[t >> 2] = s2;
        if (x4 != nullptr && (t & 7u) == 2u) x4[(t >> 2) + 1u] = s2;
    }
}

/* Sum over aligned groups of LPR lanes; every lane receives its group's sum. */
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

/* In-flight loads of one row for one lane: chunks sub + LPR*j, j < J. */
template <int J>
struct RowFrag {
    uint4 w[J];
    h16 s[J];
};

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

/* NT: non-temporal loads, for weights read once per token (the LM head, the
 * routed experts), so they do not displace reused weights from the caches. */
template <int QT, int LPR, int J, bool NT = false>
__device__ __forceinline__ void frag_load(RowFrag<J> &f, const uint8_t *W, const h16 *S, u32 C, u32 sub) {
    /* branch-free: chunks past the row re-read its last chunk and are
     * dropped in frag_dot, so no wait lands between the loads */
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const u32 c = min(sub + LPR * j, C - 1u);
        if (NT) {
            f.w[j] = __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4v *)(W + 16u * c)));
            if (QT != 1) f.s[j] = __builtin_nontemporal_load(S + c / chunks_per_group<QT>());
        } else {
            f.w[j] = *(const uint4 *)(W + 16u * c);
            if (QT != 1) f.s[j] = S[c / chunks_per_group<QT>()];
        }
    }
}
#ifndef UOCR_NT_STREAM
#define UOCR_NT_STREAM true
#endif

/* Lane-partial dot of a loaded row with the LDS activation xs. */
template <int QT, int LPR, int J>
__device__ __forceinline__ float frag_dot(const RowFrag<J> &f, const h16 *xs, u32 C, u32 sub) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const u32 c = sub + LPR * j;
        if (LPR * (j + 1) <= C || c < C) {
            const float d = chunk_dot<QT>(f.w[j], xs, min(c, C - 1u));
            const float v = QT == 1 ? d : d * (float)f.s[j];
            acc += c < C ? v : 0.0f;
        }
    }
    return acc;
}

/* frag_dot() over offset-free chunk dots; nx[j] = -bias * (activation sum
 * of the lane's chunk slot j). */
template <int QT, int LPR, int J>
__device__ __forceinline__ float frag_dot_u(const RowFrag<J> &f, const h16 *xs, const float (&nx)[J], u32 C, u32 sub) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const u32 c = sub + LPR * j;
        if (LPR * (j + 1) <= (int)C || c < C) {
            const float v = chunk_value(chunk_dot_u<QT>(f.w[j], xs, min(c, C - 1u)), (float)f.s[j], nx[j]);
            acc += c < C ? v : 0.0f;
        }
    }
    return acc;
}

/* Lanes per row and chunk slots per lane for a row of C chunks: the smallest
 * power of two >= 4 with C <= 7 * LPR (else 64 lanes, up to 16 slots). */
__host__ __device__ constexpr u32 lpr_for(u32 C) {
    return C <= 28u ? 4u : (C <= 56u ? 8u : (C <= 112u ? 16u : (C <= 224u ? 32u : 64u)));
}
__host__ __device__ constexpr u32 j_for(u32 C) {
    return (C + lpr_for(C) - 1u) / lpr_for(C);
}

/* One-pass GEMVs are latency-bound (about one wavefront per SIMD), so they
 * spread a row over more lanes: at most 3 chunk slots per lane below 64
 * lanes, which shortens each wavefront's dequant-dot stream. */
__host__ __device__ constexpr u32 lpr_lat(u32 C) {
    return C <= 12u ? 4u : (C <= 24u ? 8u : (C <= 48u ? 16u : (C <= 96u ? 32u : 64u)));
}
__host__ __device__ constexpr u32 j_lat(u32 C) {
    return (C + lpr_lat(C) - 1u) / lpr_lat(C);
}

/* Wave-uniform max of all 64 lanes with DPP row steps and readlanes. */
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

/* Wave-uniform max of a 32-bit unsigned value over all 64 lanes (DPP row
 * steps, then readlanes of the four row results). */
__device__ __forceinline__ u32 wave_max_u32(u32 v) {
    v = max(v, (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, true));
    v = max(v, (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, true));
    v = max(v, (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, true));
    v = max(v, (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, true));
    const u32 a = (u32)__builtin_amdgcn_readlane((int)v, 0), b = (u32)__builtin_amdgcn_readlane((int)v, 16);
    const u32 c = (u32)__builtin_amdgcn_readlane((int)v, 32), d = (u32)__builtin_amdgcn_readlane((int)v, 48);
    return max(max(a, b), max(c, d));
}

/* Six rounds of "largest key, lowest lane among equals" over one wavefront
 * (a DPP wave max of the key and a ballot of the lanes holding it); sid gets
 * the lanes, best the keys.  Wave-uniform results. */
__device__ __forceinline__ void top6_keys(u32 key, u32 (&sid)[UOCR_K_TOPK], u32 (&best)[UOCR_K_TOPK]) {
    const u32 lane = threadIdx.x & 63u;
    bool live = true;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        best[r] = wave_max_u32(live ? key : 0u);
        const unsigned long long m = __ballot(live && key == best[r]);
        const u32 l = (u32)__builtin_ctzll(m);
        sid[r] = l;
        live = live && lane != l;
    }
}

/* Max-subtracted softmax of the 64 router logits (one per lane). */
__device__ __forceinline__ float router_prob(float lg) {
    const float mx = wave_max_dpp(lg);
    const float pe = expf(lg - mx);
    return pe / wave_sum(pe);
}

/* Greedy top-6 over 64 router logits by one wavefront (one expert per lane):
 * max-subtracted softmax, then 6 rounds of "largest probability, lowest id
 * among equals" (uocr_cpu_ref.c:443-463, moe.metal:12-18); probabilities
 * are non-negative, so their bits order as unsigned integers.  Raw
 * probabilities unless norm_topk.  The results are wave-uniform. */
__device__ __forceinline__ void topk6(float lg, int norm_topk, u32 (&sid)[UOCR_K_TOPK], float (&sw)[UOCR_K_TOPK]) {
    u32 best[UOCR_K_TOPK];
    top6_keys(__float_as_uint(router_prob(lg)), sid, best);
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        sw[r] = __uint_as_float(best[r]);
        tot += sw[r];
    }
    if (norm_topk) {
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) sw[r] /= tot;
    }
}

/* Top-6 ids from un-normalised logits z = logits / inv_rms: softmax is
 * monotone and inv_rms > 0, so z orders the experts as the probabilities
 * do.  The key maps floats to unsigned integers in the same order. */
__device__ __forceinline__ void topk6_ids(float z, u32 (&sid)[UOCR_K_TOPK]) {
    const u32 b = __float_as_uint(z);
    u32 best[UOCR_K_TOPK];
    top6_keys((b & 0x80000000u) ? ~b : (b | 0x80000000u), sid, best);
}

/* Probabilities of the selected experts sid from the logits (one per lane),
 * with topk6's arithmetic. */
__device__ __forceinline__ void topk6_weights(float lg, int norm_topk, const u32 (&sid)[UOCR_K_TOPK],
                                              float (&sw)[UOCR_K_TOPK]) {
    const float prob = router_prob(lg);
    float tot = 0.0f;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        sw[r] = lane_f(prob, (int)sid[r]);
        tot += sw[r];
    }
    if (norm_topk) {
#pragma unroll
        for (int r = 0; r < UOCR_K_TOPK; ++r) sw[r] /= tot;
    }
}

__device__ __forceinline__ bool better(float s, u32 id, float bs, u32 bid) {
    return id != NONE_ID && (bid == NONE_ID || s > bs || (s == bs && id < bid));
}

#endif /* UOCR_DEV_H */
