/*
 * uocr_prefill.hip - MFMA prompt prefill for the UnlimitedOCR decoder on
 * gfx950 (replaces the reference's prefill path, uocr_metal.m:14550-14908,
 * with its tiled GEMMs gemm_q4.metal / gemm_q8.metal).
 *
 * All P prompt rows go through each layer together, so the projections are
 * real GEMMs [P x K] x [K x N]:
 *  - k_gemm: 64 x 128 output tiles, K in 64-column steps (one quantisation
 *    group).  Activation tiles are staged in LDS as fp16 (double-buffered);
 *    each wavefront dequantises its own 32 weight rows straight into MFMA
 *    operand registers as fp16(q * scale), the reference's prefill staging
 *    (gemm_q4.metal:48-55: half(float(q) * scale)), and
 *    v_mfma_f32_32x32x16_f16 accumulates in fp32.  Epilogues: fp16 store with
 *    optional residual, fp32 store, and SwiGLU over two weight matrices.  In
 *    grouped mode a tile table maps each block to an expert's bucket of
 *    (token, rank) pairs: rows are gathered through an index list and the
 *    expert's weights are addressed by slab stride.
 *  - k_flash_attn: causal attention over the prompt slots, one block per
 *    (64-query tile, head): S = Q K^T and O += P V on MFMA, fp32 online
 *    softmax in LDS.
 *  - routing (top-6 per token, expert buckets), RoPE + KV scatter, MoE
 *    combine and row RMSNorm kernels.
 * fp16 rounding happens where the decode path rounds (norm, q/k/v, RoPE,
 * attention output, O + residual, SwiGLU mids, shared output, layer output).
 */
#include "uocr_kernels.h"

#include <math.h>

#include <type_traits>

typedef _Float16 h16;
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32;

#define PB 256 /* threads per prefill block */
#define TM 64  /* GEMM tile rows */
#define GTM TM /* tile rows of the grouped (expert-bucket) GEMMs */
#define TN 128 /* GEMM tile columns */
#define TK 64  /* one quantisation group */
#define LDA (TK + 8) /* padded LDS row of the activation tile (halves) */
#ifndef GDEPTH
#define GDEPTH 2 /* K steps in flight per GEMM block (2, 3 and 5 measured: 2 best on the SAM shapes, equal on the prefill) */
#endif
/* The SwiGLU GEMMs (two weight matrices) keep one K step in flight: 16
 * fewer registers take them from 2 to 3 wavefronts per SIMD (routed gate/up
 * 66.8 -> 62.4 us, dense gate/up 62.9 -> 60.8 us); the one-matrix GEMMs run
 * 4 per SIMD either way and lose with one step (dense down 44.4 -> 48.7 us). */
#ifndef GDEPTH_SWIGLU
#define GDEPTH_SWIGLU 1
#endif

__device__ __forceinline__ float silu_p(float g) {
    return g / (1.0f + expf(-g));
}

union U4H8 {
    uint4 u;
    h16x8 v;
    h16 h[8];
};

/* exact fp16 of bytes b0,b1 (each < 256) + 1024 */
__device__ __forceinline__ u32 magic2(u32 v, u32 sel) {
    return __builtin_amdgcn_perm(0x64646464u, v, sel);
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */

/* f(integral_constant<int, i>) for i = 0..N-1, in order, unrolled at compile
 * time (register-ring slots need constant indices). */
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

enum { GE_F16 = 0, GE_F32 = 1, GE_SWIGLU = 2, GE_VISION = 3, GE_PART = 4, GE_ROPE = 5 };

/* QuickGELU of the CLIP MLP: x * sigmoid(1.702 x) (dense.metal:63-66). */
__device__ __forceinline__ float quick_gelu(float x) {
    /* hardware exp2 and reciprocal (about 1 ulp each in fp32; the result is
     * rounded to fp16) instead of the full-precision expf and divide */
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.702f * 1.4426950408889634f * x));
}

/* GELU of the SAM MLP, 0.5 x (1 + erf(x / sqrt 2)), with erf from
 * Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), the approximation the
 * reference's SAM kernels use (sam.metal:78-91). */
__device__ __forceinline__ float gelu_erf_as(float x) {
    const float z = x * 0.70710678118654752f;
    const float az = fabsf(z);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * az);
    const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
    const float e = 1.0f - poly * __builtin_amdgcn_exp2f(-1.4426950408889634f * az * az);
    return 0.5f * x * (1.0f + (z < 0.0f ? -e : e));
}

/* Weight piece of one K step (one 64-column quantisation group) for the
 * weight row n = the output column of this lane, lane half h = lane / 32:
 *   Q4: bytes 16h..16h+15 of the group (one uint4); f16 / Q8: columns
 *   32h..32h+31 (Q8 two uint4, f16 four), plus the row's group scale.
 * A K step is four 16-deep MFMA substeps; substep i takes 8 of these
 * weights, at the group columns b_koff(i, h)..+7 (any order of the K sum
 * works as long as the activation operand is read at the same columns):
 *   Q4: i = 0, 1: low nibbles of bytes 8i..8i+7 (columns 16h + 8i ..);
 *       i = 2, 3: high nibbles of the same bytes (columns + 32);
 *   Q8 / f16: columns 32h + 8i ... */
template <int QT>
struct BPiece {
    static constexpr int NV = QT == 4 ? 1 : (QT == 3 ? 2 : 4); /* uint4 loads */
    static constexpr int NW = 4 * NV;                          /* words */
};

template <int QT>
__device__ __forceinline__ u32 b_koff(u32 i, u32 h) {
    return QT == 4 ? ((i & 2u) << 4) + 16u * h + ((i & 1u) << 3) : 32u * h + 8u * i;
}

/* The piece is kept as plain words (no struct or vector copies), so the
 * register ring stays in registers. */
template <int QT>
__device__ __forceinline__ void b_load(u32 (&w)[BPiece<QT>::NW], u32 &sc, const uint8_t *W, const h16 *S, u32 K,
                                       u32 n, u32 g, u32 h, bool with_scale = true, bool packed = false) {
    /* packed (Q4/Q8): the 32-row block's step is one run, half h of row r at
     * (32h + r) * RB/2 */
    constexpr u32 RB = QT == 4 ? 32u : 64u;
    const uint4 *src =
        packed && QT != 1
            ? (const uint4 *)(W + ((size_t)(n / 32u) * (K / 64u) + g) * (32u * RB) + (32u * h + n % 32u) * (RB / 2u))
            : (QT == 4 ? (const uint4 *)(W + (size_t)n * (K / 2u) + g * 32u + 16u * h)
                       : (QT == 3 ? (const uint4 *)(W + (size_t)n * K + g * 64u + 32u * h)
                                  : (const uint4 *)((const h16 *)W + (size_t)n * K + g * 64u + 32u * h)));
#pragma unroll
    for (int v = 0; v < BPiece<QT>::NV; ++v) {
        const uint4 x = src[v];
        w[4 * v] = x.x;
        w[4 * v + 1] = x.y;
        w[4 * v + 2] = x.z;
        w[4 * v + 3] = x.w;
    }
    if (QT != 1 && with_scale) sc = ((const unsigned short *)S)[(size_t)n * (K / 64u) + g];
}

/* The four B operands (8 fp16 each) of a loaded piece: fp16(q * scale), the
 * product of two fp16 values rounded once, as half(float(q) * scale) in
 * gemm_q4.metal:55 (the integer q is exact after the bias subtraction);
 * f16: the values. */
template <int QT>
__device__ __forceinline__ void b_dequant(const u32 (&w)[BPiece<QT>::NW], u32 sc, h16x8 (&b)[4]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h16 sv = __builtin_bit_cast(h16, (unsigned short)sc);
    const h2 sc2 = {sv, sv};
    union {
        h16x8 v;
        u32 d[4];
    } o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (QT == 4) {
            const h2 bb = __builtin_bit_cast(h2, 0x64086408u); /* (1032, 1032) */
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const u32 x = w[2 * (i & 1) + q];
                const u32 nb = (i & 2) ? (x >> 4) & 0x0F0F0F0Fu : x & 0x0F0F0F0Fu;
                o.d[2 * q] = __builtin_bit_cast(u32, (__builtin_bit_cast(h2, magic2(nb, 0x04010400u)) - bb) * sc2);
                o.d[2 * q + 1] = __builtin_bit_cast(u32, (__builtin_bit_cast(h2, magic2(nb, 0x04030402u)) - bb) * sc2);
            }
        } else if (QT == 3) {
            const h2 bb = __builtin_bit_cast(h2, 0x64806480u); /* (1152, 1152) */
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const u32 u = w[2 * i + q] ^ 0x80808080u;
                o.d[2 * q] = __builtin_bit_cast(u32, (__builtin_bit_cast(h2, magic2(u, 0x04010400u)) - bb) * sc2);
                o.d[2 * q + 1] = __builtin_bit_cast(u32, (__builtin_bit_cast(h2, magic2(u, 0x04030402u)) - bb) * sc2);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) o.d[q] = w[4 * i + q];
        }
        b[i] = o.v;
    }
}

struct RopeTabP {
    float f[UOCR_K_HEAD_DIM / 2];
};

/* GE_ROPE destinations: q rows [P][1280], the layer's K / V caches
 * [head][cap][128]; cs holds (cos, sin) of token t's angle t * f[d] at
 * cs[64 t + d]. */
struct RopeDst {
    const float2 *cs;
    h16 *q, *k, *v;
    u32 cap;
};

struct GemmArgs {
    const h16 *A;        /* activations, row stride lda (halves) */
    u32 lda;
    const int32_t *a_idx;  /* grouped: A row of each slot */
    const int32_t *o_idx;  /* grouped: output row of each slot */
    u32 M, N, K;
    uocr_qmat W[3];      /* W[0] (and W[1] for SwiGLU; W[seg] when nseg) */
    u32 nseg;            /* when nonzero, columns [s*nseg, (s+1)*nseg) use W[s] */
    uint64_t w_stride, s_stride; /* grouped: per-expert strides (bytes / halves) */
    const int32_t *tile_e, *tile_s0, *tile_s1, *ntiles; /* grouped tile table */
    void *out;
    u32 ldo;
    const h16 *res;      /* GE_F16: optional residual, row stride ldr */
    u32 ldr;
    const h16 *bias;     /* GE_VISION: per-column bias */
    u32 act;             /* GE_VISION: UOCR_VISION_ACT_* */
    u32 split;           /* GE_VISION: 0, or the width of each of out/out1/out2 */
    void *out1, *out2;
    u32 kst;             /* split-K: K steps per blockIdx.z (0: all of K in one block) */
    u32 sc_lds;          /* the block's scale rows are preloaded into dynamic LDS */
    u32 packed;          /* Q4/Q8 payloads in the GEMM-packed layout */
};

/* Scale rows in LDS: a block's 128 weight rows x K/64 groups are one
 * contiguous region of the scale tensor, loaded once with wide loads instead
 * of one 2-byte load per row per K step (each of which touches a separate
 * cache line).  Used while NMAT x K/64 <= SC_LDS_STEPS (28 KB). */
#define SC_LDS_STEPS 112u

/* C[m][n] = sum_k A[m][k] W[n][k] over one 64 x 128 tile per block.  Wave
 * w owns output columns 32w..32w+31 (its weight rows, dequantised straight
 * into MFMA B operands in registers) for all 64 rows (two 32x32 MFMA
 * tiles); only the activation tile goes through LDS, double-buffered, so a
 * K step has one barrier and LDS carries one activation read per MFMA. */
#ifndef UOCR_GEMM_BLDS
#define UOCR_GEMM_BLDS 1
#endif

template <int QT, int EPI, bool GROUPED, int TMR>
__device__ __forceinline__ void gemm_body(GemmArgs p, u32 bx, u32 by, u32 bz, RopeDst rd = RopeDst{}) {
    constexpr int AQ4 = TMR * (TK / 8) / PB; /* activation pieces (8 halves) per thread per K step */
    static_assert(TMR % 32 == 0 && TMR <= PB && AQ4 * PB == TMR * (TK / 8), "tile rows");
    constexpr int NMAT = EPI == GE_SWIGLU ? 2 : 1;
    constexpr int GD = EPI == GE_SWIGLU ? GDEPTH_SWIGLU : GDEPTH; /* K steps in flight */
    /* f16 with one weight matrix: the block loads each K step's raw weight
     * tile with eight lanes per row (whole 128-byte row pieces) into LDS, and
     * each wavefront reads its 32 rows back in the MFMA operand layout; loads
     * of one row per lane touched a cache line per lane (SAM lin1 with fp16
     * weights 58.4 -> 48.5 us).  The same for Q8 (four lanes per 64-byte
     * piece) measured -4.6% to +3.6% across the SAM / CLIP shapes, the extra
     * 20 KB of LDS costing occupancy at long K, so Q8 keeps the per-lane
     * loads; Q4 rows are 32 bytes per K step. */
    constexpr bool BL = UOCR_GEMM_BLDS && QT == 1 && NMAT == 1;
    constexpr u32 RB = QT == 3 ? 64u : 128u; /* raw bytes per row per K step */
    constexpr u32 LDB = RB + 16u;            /* padded LDS row (bytes) */
    constexpr u32 CPR = RB / 16u;            /* 16-byte pieces per row */
    __shared__ __attribute__((aligned(16))) uint8_t bsm[BL ? 2u * TN * LDB : 16u];
    __shared__ __attribute__((aligned(16))) h16 as[2][TMR * LDA];
    __shared__ int32_t arow[TMR], orow[TMR];
    const u32 t = threadIdx.x, lane = t & 63u, wave = t >> 6, hf = lane >> 5;
    u32 n0 = by * TN, rows = p.M, e = 0, s0 = 0;
    if (GROUPED) {
        if ((int)bx >= *p.ntiles) return;
        e = (u32)p.tile_e[bx];
        s0 = (u32)p.tile_s0[bx];
        rows = (u32)p.tile_s1[bx] - s0;
        if (t < TMR) {
            const u32 s = s0 + min(t, rows - 1u);
            arow[t] = p.a_idx[s];
            orow[t] = p.o_idx[s];
        }
    } else {
        s0 = bx * TMR;
        rows = min((u32)TMR, p.M - s0);
        if (t < TMR) {
            arow[t] = (int32_t)(s0 + min(t, rows - 1u));
            orow[t] = arow[t];
        }
    }
    uocr_qmat W0 = p.W[0], W1 = p.W[1];
    u32 nbase = 0;
    if (p.nseg != 0u) {
        const u32 sgi = n0 / p.nseg;
        W0 = p.W[sgi];
        nbase = sgi * p.nseg;
    }
    const u32 nmax = (p.nseg != 0u ? p.nseg : p.N);
    const uint8_t *wp[2] = {(const uint8_t *)W0.w + (GROUPED ? e * p.w_stride : 0),
                            NMAT == 2 ? (const uint8_t *)W1.w + (GROUPED ? e * p.w_stride : 0) : nullptr};
    const h16 *sp[2] = {(const h16 *)W0.s + (GROUPED ? e * p.s_stride : 0),
                        NMAT == 2 ? (const h16 *)W1.s + (GROUPED ? e * p.s_stride : 0) : nullptr};
    /* this lane's weight row (clamped; columns past N are not stored) */
    const u32 nrow = min(n0 - nbase + 32u * wave + (lane & 31u), nmax - 1u);
    __syncthreads();

    f32x16 acc[NMAT][TMR / 32];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int j = 0; j < TMR / 32; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[m][j][i] = 0.0f;

    /* K steps run GD deep: step s's loads were issued GD steps
     * earlier into a register ring (constant indices only, so the ring stays
     * in registers) */
    /* the lambdas below see plain locals: a reference to the kernel
     * argument struct would copy it to private memory */
    const h16 *Ap = p.A;
    const u32 lda = p.lda, Kd = p.K;
    const bool pk = p.packed != 0u;
    const u32 NT = Kd / TK, kb0 = p.kst != 0u ? bz * p.kst : 0u;
    const u32 NS = p.kst != 0u ? min(p.kst, NT - kb0) : NT;
    u32 ka[GD][AQ4][4]; /* words, not uint4: no struct copies, so they stay in registers */
    u32 kb[GD][NMAT][BPiece<QT>::NW], ks[GD][NMAT];
    extern __shared__ __attribute__((aligned(16))) unsigned short ssc[];
    const bool scl = QT != 1 && p.sc_lds != 0u;
    const u32 lrow0 = n0 - nbase, nvalid = min((u32)TN, nmax - lrow0);
    const u32 lrow = nrow - lrow0; /* this lane's row within the block's scale rows */
    /* this thread's two activation rows, resolved once */
    const h16 *arp[AQ4];
#pragma unroll
    for (int q = 0; q < AQ4; ++q) {
        const u32 idx = t + q * PB;
        arp[q] = Ap + (size_t)arow[idx >> 3] * lda + (size_t)kb0 * TK + 8u * (idx & 7u);
    }
    const uint8_t *bsrc[BPiece<QT>::NV];
    if constexpr (BL) {
        const u32 rowbytes = QT == 3 ? Kd : 2u * Kd;
#pragma unroll
        for (int v = 0; v < BPiece<QT>::NV; ++v) {
            const u32 pidx = t + v * PB, r = pidx / CPR, c = pidx % CPR;
            bsrc[v] = wp[0] + (size_t)min(lrow0 + r, nmax - 1u) * rowbytes + 16u * c;
        }
    }
    auto issue = [&](auto D, u32 st) {
        constexpr int d = decltype(D)::value;
#pragma unroll
        for (int q = 0; q < AQ4; ++q) {
            const uint4 v = *(const uint4 *)(arp[q] + st * TK);
            ka[d][q][0] = v.x;
            ka[d][q][1] = v.y;
            ka[d][q][2] = v.z;
            ka[d][q][3] = v.w;
        }
        if constexpr (BL) {
            /* piece v of this thread: row (t + v PB) / CPR of the block's
             * rows, 16-byte piece (t + v PB) % CPR of its K step */
#pragma unroll
            for (int v = 0; v < BPiece<QT>::NV; ++v) {
                const uint4 x = *(const uint4 *)(bsrc[v] + (size_t)(kb0 + st) * RB);
                kb[d][0][4 * v] = x.x;
                kb[d][0][4 * v + 1] = x.y;
                kb[d][0][4 * v + 2] = x.z;
                kb[d][0][4 * v + 3] = x.w;
            }
            if (!scl) ks[d][0] = ((const unsigned short *)sp[0])[(size_t)nrow * (Kd / 64u) + kb0 + st];
        } else {
#pragma unroll
            for (int m = 0; m < NMAT; ++m) b_load<QT>(kb[d][m], ks[d][m], wp[m], sp[m], Kd, nrow, kb0 + st, hf, !scl, pk);
        }
    };
    auto step = [&](auto D, u32 st) {
        constexpr int d = decltype(D)::value;
        /* keeps the scheduler from hoisting a later step's dequantisation
         * (which waits for that step's loads) into this one */
        __builtin_amdgcn_sched_barrier(0);
        h16 *ab = as[st & 1u];
#pragma unroll
        for (int q = 0; q < AQ4; ++q) {
            const u32 idx = t + q * PB, r = idx >> 3, c8 = idx & 7u;
            *(uint4 *)(ab + r * LDA + 8u * c8) = make_uint4(ka[d][q][0], ka[d][q][1], ka[d][q][2], ka[d][q][3]);
        }
        h16x8 bop[NMAT][4];
        if (scl) {
#pragma unroll
            for (int m = 0; m < NMAT; ++m) ks[d][m] = ssc[(m * TN + lrow) * NT + kb0 + st];
        }
        uint8_t *bb = bsm + (st & 1u) * (BL ? TN * LDB : 0u);
        if constexpr (BL) {
#pragma unroll
            for (int v = 0; v < BPiece<QT>::NV; ++v) {
                const u32 pidx = t + v * PB;
                *(uint4 *)(bb + (pidx / CPR) * LDB + 16u * (pidx % CPR)) =
                    make_uint4(kb[d][0][4 * v], kb[d][0][4 * v + 1], kb[d][0][4 * v + 2], kb[d][0][4 * v + 3]);
            }
        } else {
#pragma unroll
            for (int m = 0; m < NMAT; ++m) b_dequant<QT>(kb[d][m], ks[d][m], bop[m]);
        }
        /* the other buffer's readers (step st - 1) all passed this barrier
         * before anyone writes it again at step st + 1 */
        __syncthreads();
        if constexpr (BL) {
            /* this lane's MFMA piece of its row: bytes RB / 2 * h .. + RB / 2 */
            u32 w[BPiece<QT>::NW];
            const uint8_t *src = bb + (32u * wave + (lane & 31u)) * LDB + (RB / 2u) * hf;
#pragma unroll
            for (int v = 0; v < BPiece<QT>::NV; ++v) {
                const uint4 x = *(const uint4 *)(src + 16u * v);
                w[4 * v] = x.x;
                w[4 * v + 1] = x.y;
                w[4 * v + 2] = x.z;
                w[4 * v + 3] = x.w;
            }
            b_dequant<QT>(w, ks[d][0], bop[0]);
        }
        /* unconditional (past the end it re-reads the last step into a slot
         * no later step consumes): loads issued on every path keep the
         * compiler's load counting exact, so the wait before a step covers
         * only that step's loads and the later steps' stay in flight */
        issue(D, min(st + GD, NS - 1u));
#pragma unroll
        for (u32 i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < TMR / 32; ++j) {
                U4H8 a;
                a.u = *(const uint4 *)(ab + (32u * j + (lane & 31u)) * LDA + b_koff<QT>(i, hf));
#pragma unroll
                for (int m = 0; m < NMAT; ++m) {
                    acc[m][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a.v, bop[m][i], acc[m][j], 0, 0, 0);
                }
            }
        }
    };
    static_for<GD>([&](auto D) { issue(D, min((u32)decltype(D)::value, NS - 1u)); });
    if (scl) {
        /* after the first steps' loads are in flight; rows past nmax are not
         * loaded (their lanes read the last valid row, nrow is clamped) */
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const unsigned short *src = (const unsigned short *)sp[m] + (size_t)lrow0 * NT;
            unsigned short *dst = ssc + m * TN * NT;
            const u32 cnt = nvalid * NT;
            if ((((uintptr_t)src) & 15u) == 0u && cnt % 8u == 0u) {
                for (u32 i = t; i < cnt / 8u; i += PB) ((uint4 *)dst)[i] = ((const uint4 *)src)[i];
            } else {
                for (u32 i = t; i < cnt; i += PB) dst[i] = src[i];
            }
        }
        __syncthreads();
    }
    u32 st = 0;
    for (; st + GD <= NS; st += GD) {
        static_for<GD>([&](auto D) { step(D, st + (u32)decltype(D)::value); });
    }
    static_for<GD>([&](auto D) {
        if (st + (u32)decltype(D)::value < NS) step(D, st + (u32)decltype(D)::value);
    });

    if constexpr (EPI == GE_ROPE) {
        /* The Q | K | V projection with RoPE and the cache scatter as its
         * epilogue: the block's 128 columns are one head of one of the three
         * segments.  The tile is rounded to fp16 (the projection's output
         * type) into LDS, then wavefront w takes rows w, w + 4, ..: lane d
         * rotates the pair (x_d, x_{d+64}) in fp32 by the angle tok * f[d],
         * cos and sin from the prompt's table (q and k; v is copied). */
        static_assert(GROUPED == false && TMR == 64 && TN == UOCR_K_HEAD_DIM, "rope tile");
        constexpr u32 RLD = TN + 8u; /* padded LDS row (halves) */
        static_assert(TMR * RLD <= 2u * TMR * LDA, "rope tile in the activation buffers");
        h16 *tile = &as[0][0];
        const u32 seg = n0 / p.nseg, h = (n0 - seg * p.nseg) / TN, d = lane;
        __syncthreads(); /* every wavefront's last MFMA reads of as[] are done */
#pragma unroll
        for (int j = 0; j < TMR / 32; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const u32 r = 32u * j + 8u * (i / 4) + 4u * hf + (i % 4);
                tile[r * RLD + 32u * wave + (lane & 31u)] = (h16)acc[0][j][i];
            }
        /* the wavefront's cos / sin loads, all in flight across the barrier
         * (issued after the accumulators are staged, so they add no
         * registers to the main loop's) */
        constexpr int RW = TMR / (PB / 64); /* rows per wavefront */
        float2 csr[RW];
        if (seg != 2u) {
#pragma unroll
            for (int k = 0; k < RW; ++k) {
                const u32 r = min(wave + (PB / 64u) * k, rows - 1u);
                csr[k] = rd.cs[(size_t)(s0 + r) * 64u + d];
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < RW; ++k) {
            const u32 r = wave + (PB / 64u) * k;
            if (r >= rows) break;
            const u32 tok = s0 + r;
            const h16 xa = tile[r * RLD + d], xb = tile[r * RLD + d + 64u];
            if (seg == 2u) {
                const size_t ci = ((size_t)h * rd.cap + tok) * UOCR_K_HEAD_DIM + d;
                rd.v[ci] = xa;
                rd.v[ci + 64u] = xb;
                continue;
            }
            const float cs = csr[k].x, sn = csr[k].y;
            const float a = (float)xa, b = (float)xb;
            h16 *dst = seg == 0u ? rd.q + (size_t)tok * UOCR_K_HIDDEN + h * UOCR_K_HEAD_DIM + d
                                 : rd.k + ((size_t)h * rd.cap + tok) * UOCR_K_HEAD_DIM + d;
            dst[0] = (h16)(a * cs - b * sn);
            dst[64] = (h16)(a * sn + b * cs);
        }
        return;
    }

    /* C layout of a 32x32 MFMA tile: lane l, element i -> row 8*(i/4) +
     * 4*(l/32) + i%4, column l%32.  Everything that depends only on the
     * column (output pointer, split routing, bias) is resolved once per lane;
     * rows of a plain GEMM are s0 + r (the row list is only read when
     * grouped). */
    const u32 col = n0 + 32u * wave + (lane & 31u);
    if (col >= p.N) return;
    auto out_row = [&](u32 r) -> size_t { return GROUPED ? (size_t)orow[r] : (size_t)(s0 + r); };
    h16 *vdst = (h16 *)p.out + col;
    size_t vld = p.ldo;
    float bcol = 0.0f;
    if (EPI == GE_VISION) {
        bcol = (float)p.bias[col];
        if (p.split != 0u) {
            const u32 pj = col / p.split;
            vdst = (h16 *)(pj == 0u ? p.out : (pj == 1u ? p.out1 : p.out2)) + (col - pj * p.split);
            vld = p.split;
        }
    }
    const u32 act = p.act;
#pragma unroll
    for (int j = 0; j < TMR / 32; ++j) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const u32 r = 32u * j + 8u * (i / 4) + 4u * hf + (i % 4);
            if (r >= rows) continue;
            const size_t orw = out_row(r);
            if (EPI == GE_F32) {
                ((float *)p.out)[orw * p.ldo + col] = acc[0][j][i];
            } else if (EPI == GE_PART) {
                ((float *)p.out)[((size_t)bz * p.M + orw) * p.ldo + col] = acc[0][j][i];
            } else if (EPI == GE_SWIGLU) {
                ((h16 *)p.out)[orw * p.ldo + col] = (h16)(silu_p(acc[0][j][i]) * acc[NMAT - 1][j][i]);
            } else if (EPI == GE_VISION) {
                float v = acc[0][j][i] + bcol;
                if (act == UOCR_VISION_ACT_QUICKGELU) v = quick_gelu(v);
                else if (act == UOCR_VISION_ACT_GELU_ERF) v = gelu_erf_as(v);
                vdst[orw * vld] = (h16)v;
            } else {
                float v = acc[0][j][i];
                if (p.res != nullptr) v += (float)p.res[orw * p.ldr + col];
                ((h16 *)p.out)[orw * p.ldo + col] = (h16)v;
            }
        }
    }
}

template <int QT, int EPI, bool GROUPED, int TMR>
__global__ __launch_bounds__(PB) void k_gemm(GemmArgs p) {
    gemm_body<QT, EPI, GROUPED, TMR>(p, blockIdx.x, blockIdx.y, blockIdx.z);
}

template <int QT>
__global__ __launch_bounds__(PB) void k_gemm_rope(GemmArgs p, const float2 *cs, h16 *q, h16 *kc, h16 *vc, u32 cap) {
    gemm_body<QT, GE_ROPE, false, TM>(p, blockIdx.x, blockIdx.y, 0u, RopeDst{cs, q, kc, vc, cap});
}

/* cs[64 t + d] = (cos, sin)(t * f[d]) for the P prompt tokens. */
__global__ __launch_bounds__(PB) void k_rope_table(RopeTabP rope, u32 P, float2 *__restrict__ cs) {
    const u32 idx = blockIdx.x * PB + threadIdx.x;
    if (idx >= P * 64u) return;
    const float ang = (float)(idx / 64u) * rope.f[idx % 64u];
    cs[idx] = make_float2(cosf(ang), sinf(ang));
}

/* Two independent GEMMs in one launch: blocks [0, na) run A's tile grid
 * (ax columns of tiles), the rest B's (bx columns).  For GEMMs that read the
 * same input or at least not each other's output, and that each leave most
 * CUs idle or waiting (the router logits beside the shared gate/up, the
 * shared down beside the routed down): one launch overlaps them where a second
 * stream would turn the captured graph into a slower parallel one. */
template <int QA, int EA, bool GA, int QB, int EB, bool GB>
__global__ __launch_bounds__(PB) void k_gemm_pair(GemmArgs a, u32 ax, u32 na, GemmArgs b, u32 bx) {
    const u32 i = blockIdx.x;
    if (i < na) {
        gemm_body<QA, EA, GA, TM>(a, i % ax, i / ax, 0u);
    } else {
        const u32 j = i - na;
        gemm_body<QB, EB, GB, TM>(b, j % bx, j / bx, 0u);
    }
}

/* Split-K epilogue: the z partials summed in order (the result does not
 * depend on block timing), then
 *   RD_VISION: out = f16(act(sum + bias)), split into o0/o1/o2 when split;
 *   RD_F16:    out = f16(sum (+ res)), row stride ldo (res: ldr);
 *   RD_F32:    out = sum (fp32), row stride ldo. */
enum { RD_VISION = 0, RD_F16 = 1, RD_F32 = 2 };
__global__ __launch_bounds__(PB) void k_split_reduce(const float *__restrict__ part, u32 S, u32 M, u32 N, u32 mode,
                                                     const h16 *__restrict__ bias, u32 act, u32 split,
                                                     const h16 *__restrict__ res, u32 ldr, void *__restrict__ o0,
                                                     h16 *__restrict__ o1, h16 *__restrict__ o2, u32 ldo) {
    /* four consecutive columns per thread (N, split, ldo and ldr are
     * multiples of 4, checked by the launcher), so every load is 16 bytes */
    const size_t i = 4u * ((size_t)blockIdx.x * PB + threadIdx.x), MN = (size_t)M * N;
    if (i >= MN) return;
    /* all planes' loads issued before the (ordered) sum; S <= 8 */
    float4 w[8];
#pragma unroll
    for (u32 z = 0; z < 8u; ++z) {
        if (z < S) w[z] = *(const float4 *)(part + z * MN + i);
    }
    float4 v = w[0];
#pragma unroll
    for (u32 z = 1; z < 8u; ++z) {
        if (z < S) {
            v.x += w[z].x;
            v.y += w[z].y;
            v.z += w[z].z;
            v.w += w[z].w;
        }
    }
    const u32 row = (u32)(i / N), col = (u32)(i - (size_t)row * N);
    if (mode == RD_F32) {
        *(float4 *)((float *)o0 + (size_t)row * ldo + col) = v;
        return;
    }
    float r[4] = {v.x, v.y, v.z, v.w};
    union {
        h16 h[4];
        uint2 u;
    } o, rr;
    if (mode == RD_F16) {
        if (res != nullptr) rr.u = *(const uint2 *)(res + (size_t)row * ldr + col);
#pragma unroll
        for (int c = 0; c < 4; ++c) o.h[c] = (h16)(res != nullptr ? r[c] + (float)rr.h[c] : r[c]);
        *(uint2 *)((h16 *)o0 + (size_t)row * ldo + col) = o.u;
        return;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float x = r[c] + (float)bias[col + c];
        if (act == UOCR_VISION_ACT_QUICKGELU) x = quick_gelu(x);
        else if (act == UOCR_VISION_ACT_GELU_ERF) x = gelu_erf_as(x);
        o.h[c] = (h16)x;
    }
    if (split == 0u) {
        *(uint2 *)((h16 *)o0 + (size_t)row * ldo + col) = o.u;
    } else {
        const u32 pj = col / split, lc = col - pj * split;
        *(uint2 *)((pj == 0u ? (h16 *)o0 : (pj == 1u ? o1 : o2)) + (size_t)row * split + lc) = o.u;
    }
}

/* ------------------------------------------------------------------------ */
/* row RMSNorm, RoPE + KV scatter                                            */
/* ------------------------------------------------------------------------ */

/* RMSNorm of one row of 1280 held by a wavefront: lane l holds the 8-half
 * pieces l, l + 64, l + 128 (< 160) in v.  Writes yr = f16(x * inv_rms * w)
 * (norm.metal:12-40), the sum of squares in fp32 in a fixed order (lane
 * pieces in order, then the butterfly), so every caller rounds alike. */
/* The norm weights' pieces of a lane (i = lane + 64q, clamped to the row),
 * loaded at a kernel's start so the tail waits on no further load round. */
__device__ __forceinline__ void norm_w_load(const h16 *__restrict__ w, u32 lane, U4H8 (&wv)[3]) {
#pragma unroll
    for (int q = 0; q < 3; ++q) wv[q].u = ((const uint4 *)w)[min(lane + 64u * q, UOCR_K_HIDDEN / 8u - 1u)];
}

__device__ __forceinline__ void row_norm_tail(U4H8 (&v)[3], u32 lane, const U4H8 (&wv)[3], h16 *__restrict__ yr) {
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        if (lane + 64u * q < UOCR_K_HIDDEN / 8u) {
#pragma unroll
            for (int j = 0; j < 8; ++j) ss = fmaf((float)v[q].h[j], (float)v[q].h[j], ss);
        }
    }
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float inv = 1.0f / sqrtf(ss / (float)UOCR_K_HIDDEN + 1.0e-6f);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const u32 i = lane + 64u * q;
        if (i < UOCR_K_HIDDEN / 8u) {
            U4H8 y;
#pragma unroll
            for (int j = 0; j < 8; ++j) y.h[j] = (h16)(((float)v[q].h[j] * inv) * (float)wv[q].h[j]);
            ((uint4 *)yr)[i] = y.u;
        }
    }
}

/* One wavefront per row of 1280: y = f16(x * inv_rms * w). */
__global__ __launch_bounds__(PB) void k_rows_rmsnorm(const h16 *__restrict__ x, const h16 *__restrict__ w, u32 P,
                                                     h16 *__restrict__ y) {
    const u32 row = blockIdx.x * (PB / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (row >= P) return;
    const h16 *xr = x + (size_t)row * UOCR_K_HIDDEN;
    U4H8 wv[3];
    norm_w_load(w, lane, wv);
    U4H8 v[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const u32 i = lane + 64u * q;
        if (i < UOCR_K_HIDDEN / 8u) v[q].u = ((const uint4 *)xr)[i];
    }
    row_norm_tail(v, lane, wv, y + (size_t)row * UOCR_K_HIDDEN);
}

/* Split-K reduce of a 1280-column fp16 GEMM output with its residual, fused
 * with the RMSNorm that reads it: per row (one wavefront), out = f16(sum of
 * the S planes in order + res) as k_split_reduce (RD_F16) rounds it, then
 * y = rmsnorm(out) * w as k_rows_rmsnorm rounds it. */
__global__ __launch_bounds__(PB) void k_reduce_norm(const float *__restrict__ part, u32 S, u32 M,
                                                    const h16 *__restrict__ res, u32 ldr, h16 *__restrict__ out,
                                                    u32 ldo, const h16 *__restrict__ w, h16 *__restrict__ y) {
    const u32 row = blockIdx.x * (PB / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (row >= M) return;
    const size_t MN = (size_t)M * UOCR_K_HIDDEN;
    /* the first two planes of the row's pieces (and the residual), all in
     * flight before any sum; planes beyond the second are added in order
     * after them */
    float4 pa[3][2], pb2[3][2];
    U4H8 rr[3], wv[3];
    norm_w_load(w, lane, wv);
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const u32 i = min(lane + 64u * q, UOCR_K_HIDDEN / 8u - 1u);
        const float *p0 = part + (size_t)row * UOCR_K_HIDDEN + 8u * i;
#pragma unroll
        for (u32 z = 0; z < 2u; ++z) {
            if (z < S) {
                pa[q][z] = *(const float4 *)(p0 + z * MN);
                pb2[q][z] = *(const float4 *)(p0 + z * MN + 4);
            }
        }
        if (res != nullptr) rr[q].u = *(const uint4 *)(res + (size_t)row * ldr + 8u * i);
    }
    U4H8 v[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const u32 i = lane + 64u * q;
        if (i >= UOCR_K_HIDDEN / 8u) continue;
        const float *p0 = part + (size_t)row * UOCR_K_HIDDEN + 8u * i;
        float4 a = pa[q][0], b = pb2[q][0];
        if (S > 1u) {
            const float4 c = pa[q][1], d = pb2[q][1];
            a.x += c.x;
            a.y += c.y;
            a.z += c.z;
            a.w += c.w;
            b.x += d.x;
            b.y += d.y;
            b.z += d.z;
            b.w += d.w;
        }
        for (u32 z = 2; z < S; ++z) {
            const float4 c = *(const float4 *)(p0 + z * MN), d = *(const float4 *)(p0 + z * MN + 4);
            a.x += c.x;
            a.y += c.y;
            a.z += c.z;
            a.w += c.w;
            b.x += d.x;
            b.y += d.y;
            b.z += d.z;
            b.w += d.w;
        }
        const float r[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) v[q].h[j] = (h16)(res != nullptr ? r[j] + (float)rr[q].h[j] : r[j]);
        *(uint4 *)(out + (size_t)row * ldo + 8u * i) = v[q].u;
    }
    row_norm_tail(v, lane, wv, y + (size_t)row * UOCR_K_HIDDEN);
}

/* ------------------------------------------------------------------------ */
/* causal flash attention over the prompt                                    */
/* ------------------------------------------------------------------------ */

#define AQ 64 /* queries per block */
#define AK 64 /* keys per step */
#define LDQ (UOCR_K_HEAD_DIM + 8)
#define LDV (AK + 8)

/* Block (qt, h): queries q0..q0+63 of head h attend to slots 0..q (causal),
 * fp32 online softmax scaled by 1/sqrt(128), output fp16 into ctx [P][1280]
 * (attention_decode.metal arithmetic per query). */
/* KV split of the causal prefill attention.  Query tile qt (64 queries) sees
 * qt + 1 key tiles; with chunks of CH key tiles it is nsplit(qt) = ceil((qt +
 * 1) / CH) blocks.  Blocks enumerate (qt, head, split) with the split
 * fastest, so the splits of one (qt, head) are consecutive block indices.
 * Each split of a tile with more than one writes its normalised O / l in
 * fp16 (the first half of the O area of its slot) and its row max / sum in
 * fp32 to its own partial slot; k_flash_merge combines them. */
#define FA_PART_FLOATS (AQ * UOCR_K_HEAD_DIM + 2u * AQ)
#define FA_MAX_SPLITS 16u /* splits of one query tile (the merge's weight table) */

__device__ __forceinline__ u32 fa_nsplit(u32 qt, u32 ch) {
    return (qt + ch) / ch;
}

/* first block index of query tile qt (all heads) */
__device__ __forceinline__ u32 fa_tile_base(u32 qt, u32 ch) {
    u32 b = 0;
    for (u32 q = 0; q < qt; ++q) b += UOCR_K_HEADS * fa_nsplit(q, ch);
    return b;
}

/* Wavefront w owns queries q0 + 16w .. + 15 of the block's 64 and keeps
 * everything of them in registers (16x16x32 MFMAs):
 *   S^T = K Q^T per key tile: four 16-key tiles; lane l holds query l % 16
 *   and keys 16t + 4(l / 16) + i (i < 4) of tile t;
 *   the fp32 online softmax per query, its max reduced over the four lanes
 *   that share the query (l, l ^ 16, l ^ 32, l ^ 48), its sum kept per lane
 *   and reduced once at the end;
 *   O^T = V^T P^T: the probabilities stay where S^T left them, because the
 *   B operand's 8 K slots of lane l are chosen as keys {32u + 4(l / 16) + i,
 *   32u + 16 + 4(l / 16) + i} (i < 4) and the A operand (V^T from LDS) is
 *   read at the same keys; lane l holds dims 16d + 4(l / 16) + i of query
 *   l % 16 in O^T tile d.
 * Only the K and V^T tiles go through LDS (two barriers per key tile). */
__global__ __launch_bounds__(PB) void k_flash_attn(const h16 *__restrict__ Q, const h16 *__restrict__ kc,
                                                   const h16 *__restrict__ vc, u32 cap, u32 P,
                                                   h16 *__restrict__ ctx, u32 ch, float *__restrict__ part) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) h16 ks[AK * LDQ];
    __shared__ __attribute__((aligned(16))) h16 vt[UOCR_K_HEAD_DIM * LDV];
    const u32 t = threadIdx.x, lane = t & 63u, wave = t >> 6, qc = lane & 15u, g = lane >> 4;
    /* which (query tile, head, key chunk) this block computes */
    u32 qt = blockIdx.x, h = blockIdx.y, sp = 0, ns = 1;
    if (ch != 0u) {
        u32 b = blockIdx.x;
        qt = 0;
        while (b >= UOCR_K_HEADS * fa_nsplit(qt, ch)) {
            b -= UOCR_K_HEADS * fa_nsplit(qt, ch);
            ++qt;
        }
        ns = fa_nsplit(qt, ch);
        h = b / ns;
        sp = b - h * ns;
    }
    const u32 q0 = qt * AQ;
    const h16 *kh = kc + (size_t)h * cap * 128u, *vh = vc + (size_t)h * cap * 128u;
    const float scale = 0.08838834764831845f;
    /* this lane's query row: B operand pieces of Q^T for the four 32-deep
     * steps over the head dimension */
    const u32 qr = q0 + 16u * wave + qc; /* query index */
    U4H8 qreg[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        qreg[st].u = *(const uint4 *)(Q + (size_t)min(qr, P - 1u) * UOCR_K_HIDDEN + h * 128u + 32u * st + 8u * g);
    }
    f32x4 o[UOCR_K_HEAD_DIM / 16];
#pragma unroll
    for (int d = 0; d < UOCR_K_HEAD_DIM / 16; ++d) o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;
    const u32 qlast = min(q0 + AQ, P) - 1u;
    /* this block's keys: tiles [sp * ch, (sp + 1) * ch) of the causal range */
    const u32 kbeg = ch != 0u ? sp * ch * AK : 0u;
    const u32 klast = ch != 0u ? min(qlast, (sp + 1u) * ch * AK - 1u) : qlast;
    /* next K/V tile in registers (words, so they stay in registers) */
    u32 kr_[4][4], va_[2][4], vb_[2][4];
    auto load_kv = [&](u32 k0n) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32 idx = t + q * PB, r = idx >> 4, c8 = idx & 15u;
            const uint4 v = *(const uint4 *)(kh + (size_t)min(k0n + r, P - 1u) * 128u + 8u * c8);
            kr_[q][0] = v.x;
            kr_[q][1] = v.y;
            kr_[q][2] = v.z;
            kr_[q][3] = v.w;
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const u32 idx = t + q * PB, kp = idx & 31u, c8 = idx >> 5;
            const uint4 a = *(const uint4 *)(vh + (size_t)min(k0n + 2u * kp, P - 1u) * 128u + 8u * c8);
            const uint4 b = *(const uint4 *)(vh + (size_t)min(k0n + 2u * kp + 1u, P - 1u) * 128u + 8u * c8);
            va_[q][0] = a.x;
            va_[q][1] = a.y;
            va_[q][2] = a.z;
            va_[q][3] = a.w;
            vb_[q][0] = b.x;
            vb_[q][1] = b.y;
            vb_[q][2] = b.z;
            vb_[q][3] = b.w;
        }
    };
    load_kv(kbeg);
    for (u32 k0 = kbeg; k0 <= klast; k0 += AK) {
        __syncthreads();
        /* K tile (row-major) and V tile transposed to [dim][key], from the
         * registers loaded one tile ahead.  The transpose goes by key pairs:
         * a thread holds 8 dims of keys 2i and 2i+1 and writes 8 dwords (dim
         * d: key 2i | key 2i+1 << 16); the 32 lanes of a half-wavefront
         * cover consecutive pairs, so each write touches consecutive banks. */
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32 idx = t + q * PB, r = idx >> 4, c8 = idx & 15u;
            *(uint4 *)(ks + r * LDQ + 8u * c8) = make_uint4(kr_[q][0], kr_[q][1], kr_[q][2], kr_[q][3]);
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const u32 idx = t + q * PB, kp = idx & 31u, c8 = idx >> 5;
            u32 *dst = (u32 *)(vt + 8u * c8 * LDV + 2u * kp);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                /* dims 2j and 2j+1: low halves, then high halves */
                dst[(2u * j) * (LDV / 2u)] = __builtin_amdgcn_perm(vb_[q][j], va_[q][j], 0x05040100u);
                dst[(2u * j + 1u) * (LDV / 2u)] = __builtin_amdgcn_perm(vb_[q][j], va_[q][j], 0x07060302u);
            }
        }
        __syncthreads();
        if (k0 + AK <= klast) load_kv(k0 + AK);
        /* S^T: four 16-key tiles x this wavefront's 16 queries */
        float sc[4][4];
        float tm = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                U4H8 a;
                a.u = *(const uint4 *)(ks + (16u * kt + qc) * LDQ + 32u * st + 8u * g);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, qreg[st].v, acc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32 ki = k0 + 16u * kt + 4u * g + i;
                const float v = (ki <= qr && ki < P) ? acc[i] * scale : -INFINITY;
                sc[kt][i] = v;
                tm = fmaxf(tm, v);
            }
        }
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float mnew = fmaxf(m, tm);
        /* every query sees key k0 (k0 <= q0 <= q), so mnew is finite */
        const float corr = m == -INFINITY ? 0.0f : expf(m - mnew);
        l *= corr;
#pragma unroll
        for (int d = 0; d < UOCR_K_HEAD_DIM / 16; ++d) o[d] *= corr;
        m = mnew;
        /* probabilities in fp16, two B operands of 8 keys */
        U4H8 pb[2];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = sc[kt][i] == -INFINITY ? 0.0f : expf(sc[kt][i] - mnew);
                l += e;
                pb[kt >> 1].h[4 * (kt & 1) + i] = (h16)e;
            }
        }
        /* O^T += V^T P^T */
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int d = 0; d < UOCR_K_HEAD_DIM / 16; ++d) {
                const h16 *vr = vt + (16u * d + qc) * LDV + 32u * u + 4u * g;
                U4H8 a;
                const uint2 lo = *(const uint2 *)vr, hi = *(const uint2 *)(vr + 16);
                a.u = make_uint4(lo.x, lo.y, hi.x, hi.y);
                o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, pb[u].v, o[d], 0, 0, 0);
            }
        }
    }
    /* the query's sum over its four lanes */
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const u32 r = 16u * wave + qc; /* row within the tile */
    if (ns > 1u) {
        /* partial of a split tile: O / l in fp16 (a weighted mean of V rows,
         * so within V's range), row max and row sum in fp32 */
        float *po = part + (size_t)blockIdx.x * FA_PART_FLOATS;
        const float li = 1.0f / l;
#pragma unroll
        for (int d = 0; d < UOCR_K_HEAD_DIM / 16; ++d) {
            union {
                h16 hh[4];
                uint2 u;
            } pk;
#pragma unroll
            for (int i = 0; i < 4; ++i) pk.hh[i] = (h16)(o[d][i] * li);
            *(uint2 *)((h16 *)po + r * UOCR_K_HEAD_DIM + 16u * d + 4u * g) = pk.u;
        }
        if (g == 0u) {
            po[AQ * UOCR_K_HEAD_DIM + r] = m;
            po[AQ * UOCR_K_HEAD_DIM + AQ + r] = l;
        }
        return;
    }
    if (qr < P) {
#pragma unroll
        for (int d = 0; d < UOCR_K_HEAD_DIM / 16; ++d) {
            union {
                h16 hh[4];
                uint2 u;
            } pk;
#pragma unroll
            for (int i = 0; i < 4; ++i) pk.hh[i] = (h16)(o[d][i] / l);
            *(uint2 *)(ctx + (size_t)qr * UOCR_K_HIDDEN + h * 128u + 16u * d + 4u * g) = pk.u;
        }
    }
}

/* Merge of the split tiles: block (x, h, z) takes rows 16z..16z+15 of query
 * tile ch + x (every tile from ch on has at least two splits): ctx = sum_s
 * (O_s / l_s) l_s e^(m_s - M) / sum_s l_s e^(m_s - M), M = max_s m_s (split 0
 * holds key 0, so every row has L > 0).  Each thread owns two 4-value pieces
 * of the 16 x 128 block and issues the splits' loads four at a time. */
__global__ __launch_bounds__(PB) void k_flash_merge(const float *__restrict__ part, u32 P, u32 ch,
                                                    h16 *__restrict__ ctx) {
    const u32 qt = ch + blockIdx.x, h = blockIdx.y, r0 = 16u * blockIdx.z, ns = fa_nsplit(qt, ch);
    const float *pb = part + (size_t)(fa_tile_base(qt, ch) + h * ns) * FA_PART_FLOATS;
    __shared__ float wgt[FA_MAX_SPLITS][16], linv[16];
    if (threadIdx.x < 16u) {
        const u32 r = r0 + threadIdx.x;
        /* all of the row's (m, l) loads in flight at once */
        float mv[FA_MAX_SPLITS], lv[FA_MAX_SPLITS];
#pragma unroll
        for (u32 s = 0; s < FA_MAX_SPLITS; ++s) {
            if (s < ns) {
                mv[s] = pb[s * FA_PART_FLOATS + AQ * UOCR_K_HEAD_DIM + r];
                lv[s] = pb[s * FA_PART_FLOATS + AQ * UOCR_K_HEAD_DIM + AQ + r];
            }
        }
        float M = -INFINITY;
#pragma unroll
        for (u32 s = 0; s < FA_MAX_SPLITS; ++s) {
            if (s < ns) M = fmaxf(M, mv[s]);
        }
        float L = 0.0f;
#pragma unroll
        for (u32 s = 0; s < FA_MAX_SPLITS; ++s) {
            if (s < ns) {
                const float w = mv[s] == -INFINITY ? 0.0f : expf(mv[s] - M);
                const float wl = w * lv[s];
                wgt[s][threadIdx.x] = wl; /* the split's O / l times its share */
                L += wl;
            }
        }
        linv[threadIdx.x] = 1.0f / L;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const u32 e4 = threadIdx.x + q * PB;          /* float4 index within the 16 x 128 block */
        const u32 rl = e4 / (UOCR_K_HEAD_DIM / 4u), d = 4u * (e4 % (UOCR_K_HEAD_DIM / 4u));
        const size_t off = (size_t)(r0 + rl) * UOCR_K_HEAD_DIM + d;
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (u32 s0 = 0; s0 < ns; s0 += 4u) {
            float4 v[4];
#pragma unroll
            for (u32 u = 0; u < 4u; ++u) {
                if (s0 + u < ns) {
                    union {
                        h16 hh[4];
                        uint2 u2;
                    } pk;
                    pk.u2 = *(const uint2 *)((const h16 *)(pb + (s0 + u) * FA_PART_FLOATS) + off);
                    v[u] = make_float4((float)pk.hh[0], (float)pk.hh[1], (float)pk.hh[2], (float)pk.hh[3]);
                }
            }
#pragma unroll
            for (u32 u = 0; u < 4u; ++u) {
                if (s0 + u < ns) {
                    const float w = wgt[s0 + u][rl];
                    o.x += w * v[u].x;
                    o.y += w * v[u].y;
                    o.z += w * v[u].z;
                    o.w += w * v[u].w;
                }
            }
        }
        const u32 row = qt * AQ + r0 + rl;
        if (row < P) {
            const float li = linv[rl];
            union {
                h16 hh[4];
                uint2 u;
            } pk;
            pk.hh[0] = (h16)(o.x * li);
            pk.hh[1] = (h16)(o.y * li);
            pk.hh[2] = (h16)(o.z * li);
            pk.hh[3] = (h16)(o.w * li);
            *(uint2 *)(ctx + (size_t)row * UOCR_K_HIDDEN + h * 128u + d) = pk.u;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* MoE routing, buckets, combine                                             */
/* ------------------------------------------------------------------------ */

__device__ __forceinline__ float lane_fp(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

/* One wavefront per token: softmax over its 64 logits, greedy top-6 (ties to
 * the lower id; same key order as the decode router), raw probabilities
 * unless norm_topk. */
__global__ __launch_bounds__(PB) void k_route_rows(const float *__restrict__ logits, u32 P, int norm_topk,
                                                   int32_t *__restrict__ ids, float *__restrict__ wts) {
    const u32 tok = blockIdx.x * (PB / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (tok >= P) return;
    const float lg = logits[(size_t)tok * 64u + lane];
    float mx = lg;
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    const float pe = expf(lg - mx);
    float sum = pe;
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    const float prob = pe / sum;
    const u32 pb = __float_as_uint(prob);
    const unsigned long long key = ((unsigned long long)pb << 32) | (0xffffffffu - lane);
    u32 rank = 0;
#pragma unroll
    for (int j = 0; j < 64; ++j) {
        const unsigned long long kj =
            ((unsigned long long)(u32)__builtin_amdgcn_readlane((int)pb, j) << 32) | (0xffffffffu - (u32)j);
        rank += kj > key ? 1u : 0u;
    }
    float tot = 0.0f;
    float sel[UOCR_K_TOPK];
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        const unsigned long long m = __ballot(rank == (u32)r);
        const u32 l = m != 0ull ? (u32)__builtin_ctzll(m) : 0u;
        sel[r] = __uint_as_float((u32)__builtin_amdgcn_readlane((int)pb, (int)l));
        tot += sel[r];
    }
    if (rank < (u32)UOCR_K_TOPK) {
        ids[tok * UOCR_K_TOPK + rank] = (int32_t)lane;
        wts[tok * UOCR_K_TOPK + rank] = norm_topk ? prob / tot : prob;
    }
}

/* One block builds the expert buckets of all P*6 (token, rank) pairs in
 * LDS: the 64 bucket sizes (LDS atomics), their exclusive scan (offsets),
 * the tile table of the grouped GEMMs (TM rows per tile) and every pair's
 * slot in its bucket (list_tok, list_pair).  The order of pairs inside a
 * bucket does not matter: each pair's row is computed on its own and the
 * combine reads it by pair index.  Nothing is left in global memory that the
 * next routing has to find cleared. */
#define BUCKET_THREADS 1024
__global__ __launch_bounds__(BUCKET_THREADS) void k_bucket_build(const int32_t *__restrict__ ids, u32 P,
                                                                 int32_t *__restrict__ offsets,
                                                                 int32_t *__restrict__ tile_e,
                                                                 int32_t *__restrict__ tile_s0,
                                                                 int32_t *__restrict__ tile_s1,
                                                                 int32_t *__restrict__ ntiles,
                                                                 int32_t *__restrict__ list_tok,
                                                                 int32_t *__restrict__ list_pair) {
    __shared__ int32_t cnt[64], off[65], toff[65], cur[64];
    const u32 t = threadIdx.x, n = P * UOCR_K_TOPK;
    if (t < 64u) {
        cnt[t] = 0;
        cur[t] = 0;
    }
    /* the thread's pairs' ids, all loads in flight at once (up to BUCKET_R
     * per thread; longer prompts loop) */
    constexpr u32 BUCKET_R = 8u;
    const bool inreg = n <= BUCKET_R * BUCKET_THREADS;
    int32_t idr[BUCKET_R];
    if (inreg) {
#pragma unroll
        for (u32 k = 0; k < BUCKET_R; ++k) idr[k] = t + k * BUCKET_THREADS < n ? ids[t + k * BUCKET_THREADS] : -1;
    }
    __syncthreads();
    if (inreg) {
#pragma unroll
        for (u32 k = 0; k < BUCKET_R; ++k) {
            if (idr[k] >= 0) atomicAdd(&cnt[idr[k]], 1);
        }
    } else {
        for (u32 pr = t; pr < n; pr += BUCKET_THREADS) atomicAdd(&cnt[ids[pr]], 1);
    }
    __syncthreads();
    if (t < 64u) {
        /* exclusive scans of the bucket sizes and tile counts: one wavefront,
         * a lane per expert */
        const int32_t c = cnt[t], tl = (c + GTM - 1) / GTM;
        int32_t a = c, b = tl;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int32_t x = __shfl_up(a, o), y = __shfl_up(b, o);
            if ((int)t >= o) {
                a += x;
                b += y;
            }
        }
        off[t] = a - c;
        toff[t] = b - tl;
        if (t == 63u) {
            off[64] = a;
            toff[64] = b;
            *ntiles = b;
        }
    }
    __syncthreads();
    if (t < 64u) {
        offsets[t] = off[t];
        const int32_t c = cnt[t];
        for (int32_t k = 0; k * GTM < c; ++k) {
            const int32_t ti = toff[t] + k;
            tile_e[ti] = (int32_t)t;
            tile_s0[ti] = off[t] + k * GTM;
            tile_s1[ti] = off[t] + min(c, (k + 1) * GTM);
        }
    }
    if (inreg) {
#pragma unroll
        for (u32 k = 0; k < BUCKET_R; ++k) {
            const u32 pr = t + k * BUCKET_THREADS;
            if (idr[k] >= 0) {
                const int32_t slot = off[idr[k]] + atomicAdd(&cur[idr[k]], 1);
                list_tok[slot] = (int32_t)(pr / UOCR_K_TOPK);
                list_pair[slot] = (int32_t)pr;
            }
        }
    } else {
        for (u32 pr = t; pr < n; pr += BUCKET_THREADS) {
            const int32_t e = ids[pr];
            const int32_t slot = off[e] + atomicAdd(&cur[e], 1);
            list_tok[slot] = (int32_t)(pr / UOCR_K_TOPK);
            list_pair[slot] = (int32_t)pr;
        }
    }
}

/* h[t] = f16(sum_r w[t][r] * Y[t*6+r] + shared[t] + res[t]) (decode_gemv_q4.
 * metal:185-224 order: routed sum in fp32, shared already fp16). */
/* the per-pair expert outputs as fp32 (operator API) or fp16 (the prefill,
 * rounded as the reference keeps them) */
__device__ __forceinline__ void y_load8(const float *yr, float (&e)[8]) {
    const float4 a = *(const float4 *)yr, b = *(const float4 *)(yr + 4);
    e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w; e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
}
__device__ __forceinline__ void y_load8(const h16 *yr, float (&e)[8]) {
    U4H8 v;
    v.u = *(const uint4 *)yr;
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = (float)v.h[j];
}

template <typename YT>
__global__ __launch_bounds__(PB) void k_moe_combine(const YT *__restrict__ Y, const float *__restrict__ wts,
                                                    const h16 *__restrict__ shared, const h16 *__restrict__ res, u32 P,
                                                    h16 *__restrict__ out) {
    const u32 idx = blockIdx.x * PB + threadIdx.x;
    if (idx >= P * UOCR_K_HIDDEN) return;
    const u32 t = idx / UOCR_K_HIDDEN, c = idx % UOCR_K_HIDDEN;
    float acc = 0.0f;
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) {
        acc = fmaf(wts[t * UOCR_K_TOPK + r], (float)Y[((size_t)t * UOCR_K_TOPK + r) * UOCR_K_HIDDEN + c], acc);
    }
    out[idx] = (h16)(acc + (float)shared[idx] + (float)res[idx]);
}

/* k_moe_combine fused with the next layer's input RMSNorm: one wavefront
 * per token row, the same per-element arithmetic, then y = rmsnorm(out) * w
 * as k_rows_rmsnorm rounds it. */
template <typename YT>
__global__ __launch_bounds__(PB) void k_moe_combine_norm(const YT *__restrict__ Y, const float *__restrict__ wts,
                                                         const h16 *__restrict__ shared, const h16 *__restrict__ res,
                                                         u32 P, h16 *__restrict__ out, const h16 *__restrict__ w,
                                                         h16 *__restrict__ y) {
    const u32 t = blockIdx.x * (PB / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (t >= P) return;
    float wr[UOCR_K_TOPK];
#pragma unroll
    for (int r = 0; r < UOCR_K_TOPK; ++r) wr[r] = wts[t * UOCR_K_TOPK + r];
    U4H8 wv[3], v[3];
    norm_w_load(w, lane, wv);
    if constexpr (sizeof(YT) == 2) {
        /* fp16 pair rows: every load of the row issued before any sum */
        U4H8 ey[3][UOCR_K_TOPK], sh[3], rs[3];
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            const u32 i = min(lane + 64u * q, UOCR_K_HIDDEN / 8u - 1u);
            const size_t base = (size_t)t * UOCR_K_HIDDEN + 8u * i;
#pragma unroll
            for (int r = 0; r < UOCR_K_TOPK; ++r)
                ey[q][r].u = *(const uint4 *)(Y + ((size_t)t * UOCR_K_TOPK + r) * UOCR_K_HIDDEN + 8u * i);
            sh[q].u = *(const uint4 *)(shared + base);
            rs[q].u = *(const uint4 *)(res + base);
        }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            const u32 i = lane + 64u * q;
            if (i >= UOCR_K_HIDDEN / 8u) continue;
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < UOCR_K_TOPK; ++r) {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = fmaf(wr[r], (float)ey[q][r].h[j], acc[j]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) v[q].h[j] = (h16)(acc[j] + (float)sh[q].h[j] + (float)rs[q].h[j]);
            *(uint4 *)(out + (size_t)t * UOCR_K_HIDDEN + 8u * i) = v[q].u;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            const u32 i = lane + 64u * q;
            if (i >= UOCR_K_HIDDEN / 8u) continue;
            const size_t base = (size_t)t * UOCR_K_HIDDEN + 8u * i;
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int r = 0; r < UOCR_K_TOPK; ++r) {
                float e[8];
                y_load8(Y + ((size_t)t * UOCR_K_TOPK + r) * UOCR_K_HIDDEN + 8u * i, e);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = fmaf(wr[r], e[j], acc[j]);
            }
            U4H8 sh, rs;
            sh.u = *(const uint4 *)(shared + base);
            rs.u = *(const uint4 *)(res + base);
#pragma unroll
            for (int j = 0; j < 8; ++j) v[q].h[j] = (h16)(acc[j] + (float)sh.h[j] + (float)rs.h[j]);
            *(uint4 *)(out + base) = v[q].u;
        }
    }
    row_norm_tail(v, lane, wv, y + (size_t)t * UOCR_K_HIDDEN);
}

/* ------------------------------------------------------------------------ */
/* launchers                                                                 */
/* ------------------------------------------------------------------------ */

static bool pq_ok(u32 q) {
    return q == UOCR_QT_F16 || q == UOCR_QT_Q8 || q == UOCR_QT_Q4;
}

static bool pmat_ok(uocr_qmat m) {
    return m.w != nullptr && pq_ok(m.qtype) && (m.qtype == UOCR_QT_F16 || m.s != nullptr);
}

/* Tile rows of a GEMM.  128-row tiles (each dequantised weight operand
 * feeding four MFMAs instead of two) measured slower at the prefill shapes:
 * 3.83 against 3.17 ms, the grouped gate/up dropping to one wavefront per
 * SIMD; the kernel keeps the template parameter. */
static inline u32 gemm_tm(bool, u32) {
    return (u32)TM;
}

template <int EPI, bool GROUPED, int TMR>
static void gemm_dispatch_tm(hipStream_t st, u32 qt, const GemmArgs &a, dim3 grid, size_t shm) {
    switch (qt) {
        case UOCR_QT_F16: hipLaunchKernelGGL((k_gemm<1, EPI, GROUPED, TMR>), grid, dim3(PB), 0, st, a); break;
        case UOCR_QT_Q8: hipLaunchKernelGGL((k_gemm<3, EPI, GROUPED, TMR>), grid, dim3(PB), shm, st, a); break;
        default: hipLaunchKernelGGL((k_gemm<4, EPI, GROUPED, TMR>), grid, dim3(PB), shm, st, a); break;
    }
}

template <int EPI, bool GROUPED>
static void gemm_dispatch(hipStream_t st, u32 qt, GemmArgs a, dim3 grid, u32 tmr) {
    const u32 nm = EPI == GE_SWIGLU ? 2u : 1u, nt = a.K / TK;
    a.sc_lds = qt != UOCR_QT_F16 && nm * nt <= SC_LDS_STEPS ? 1u : 0u;
    const size_t shm = a.sc_lds ? (size_t)nm * TN * nt * sizeof(unsigned short) : 0;
    (void)tmr;
    gemm_dispatch_tm<EPI, GROUPED, TM>(st, qt, a, grid, shm);
}

/* K splits for a plain GEMM whose tile grid is under one block per CU: the
 * largest power of two <= 8 that keeps the grid in one round of resident
 * blocks (about 512) with at least 5 K steps per split. */
extern "C" uint32_t uocr_gemm_ksplit(uint32_t M, uint32_t N, uint32_t K) {
    const u32 tm = gemm_tm(false, M);
    const u32 blocks = ((M + tm - 1u) / tm) * ((N + TN - 1u) / TN), steps = K / TK;
    if (blocks >= 256u) return 1u;
    u32 s = 1u;
    /* doubling while the split grid stays within 512 blocks and a split keeps
     * 5 K steps, or a split keeps 16: the O projection at P = 932 (150 tiles,
     * 20 steps) takes 2 (4 measured the same GEMM time and a longer reduce),
     * layer 0's dense down (150 tiles, 107 steps) 4 (44.8 -> 36.0 us) */
    while (s < 8u && ((blocks * 2u * s <= 512u && steps / (2u * s) >= 5u) || steps / (2u * s) >= 16u)) s *= 2u;
    return s;
}

static bool gemm_desc_ok(int epi, const uocr_gemm_desc *d) {
    if (d == nullptr || d->A == nullptr || d->out == nullptr || d->N == 0u || d->K == 0u || d->K % 64u != 0u ||
        d->lda % 8u != 0u || !pmat_ok(d->W[0]) || (epi == UOCR_GEMM_SWIGLU && (!pmat_ok(d->W[1]) || d->W[1].qtype != d->W[0].qtype)) ||
        (d->nseg != 0u && (d->nseg % TN != 0u || d->N % d->nseg != 0u || d->N / d->nseg > 3u))) {
        return false;
    }
    for (u32 s = 1; d->nseg != 0u && s < d->N / d->nseg; ++s) {
        if (!pmat_ok(d->W[s]) || d->W[s].qtype != d->W[0].qtype) return false;
    }
    const bool grouped = d->tile_e != nullptr;
    if (grouped ? (d->a_idx == nullptr || d->o_idx == nullptr || d->tile_s0 == nullptr || d->tile_s1 == nullptr ||
                   d->ntiles == nullptr || d->max_tiles == 0u)
                : d->M == 0u) {
        return false;
    }
    return true;
}

static GemmArgs gemm_args(const uocr_gemm_desc *d) {
    GemmArgs a;
    a.A = (const h16 *)d->A;
    a.lda = d->lda;
    a.a_idx = d->a_idx;
    a.o_idx = d->o_idx;
    a.M = d->M;
    a.N = d->N;
    a.K = d->K;
    for (int i = 0; i < 3; ++i) a.W[i] = d->W[i];
    a.nseg = d->nseg;
    a.w_stride = d->w_stride;
    a.s_stride = d->s_stride;
    a.tile_e = d->tile_e;
    a.tile_s0 = d->tile_s0;
    a.tile_s1 = d->tile_s1;
    a.ntiles = d->ntiles;
    a.out = d->out;
    a.ldo = d->ldo;
    a.res = (const h16 *)d->res;
    a.ldr = d->ldr;
    a.bias = (const h16 *)d->bias;
    a.act = d->act;
    a.split = d->split;
    a.out1 = d->out1;
    a.out2 = d->out2;
    a.kst = 0u;
    a.packed = d->packed != 0u && d->W[0].qtype != UOCR_QT_F16 ? 1u : 0u;
    a.sc_lds = 0u;
    return a;
}

extern "C" hipError_t uocr_launch_gemm(hipStream_t st, int epi, const uocr_gemm_desc *d) {
    if (!gemm_desc_ok(epi, d)) return hipErrorInvalidValue;
    const bool grouped = d->tile_e != nullptr;
    GemmArgs a = gemm_args(d);
    const u32 tmr = gemm_tm(grouped, d->M);
    const dim3 grid(grouped ? d->max_tiles : (d->M + tmr - 1u) / tmr, (d->N + TN - 1u) / TN);
    const u32 qt = d->W[0].qtype;
    if (epi == UOCR_GEMM_VISION && (grouped || d->bias == nullptr || d->act > UOCR_VISION_ACT_GELU_ERF ||
                                    (d->split != 0u && (d->N != 3u * d->split || d->out1 == nullptr ||
                                                        d->out2 == nullptr)))) {
        return hipErrorInvalidValue;
    }
    const bool splittable = !grouped && d->ksplit > 1u && d->part != nullptr && d->N % 4u == 0u &&
                            (epi == UOCR_GEMM_VISION ? d->split % 4u == 0u
                                                     : (epi == UOCR_GEMM_F16 || epi == UOCR_GEMM_F32) &&
                                                           d->ldo % 4u == 0u &&
                                                           (d->res == nullptr || d->ldr % 4u == 0u));
    /* norm_w: the F16 output rows also go through the RMSNorm into norm_out
     * (fused into the split-K reduce, else a row-norm launch after the GEMM) */
    const bool want_norm = d->norm_w != nullptr;
    if (want_norm && (epi != UOCR_GEMM_F16 || grouped || d->norm_out == nullptr || d->N != UOCR_K_HIDDEN ||
                      d->ldo != UOCR_K_HIDDEN || (d->res != nullptr && d->ldr % 8u != 0u))) {
        return hipErrorInvalidValue;
    }
    const bool fuse_norm = want_norm && splittable;
    if (splittable) {
        /* split-K: blockIdx.z takes K steps [z*kst, (z+1)*kst) into an fp32
         * partial plane of part, then one ordered reduce applies the
         * epilogue */
        const u32 nt = d->K / TK;
        const u32 kst = (nt + min(d->ksplit, 8u) - 1u) / min(d->ksplit, 8u), S = (nt + kst - 1u) / kst;
        a.kst = kst;
        a.out = d->part;
        a.ldo = d->N;
        gemm_dispatch<GE_PART, false>(st, qt, a, dim3(grid.x, grid.y, S), tmr);
        const size_t mn = (size_t)d->M * d->N;
        const u32 mode = epi == UOCR_GEMM_VISION ? RD_VISION : (epi == UOCR_GEMM_F16 ? RD_F16 : RD_F32);
        if (fuse_norm) {
            hipLaunchKernelGGL(k_reduce_norm, dim3((d->M + 3u) / 4u), dim3(PB), 0, st, (const float *)d->part, S,
                               d->M, (const h16 *)d->res, d->ldr, (h16 *)d->out, d->ldo, (const h16 *)d->norm_w,
                               (h16 *)d->norm_out);
            return hipGetLastError();
        }
        hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((mn / 4u + PB - 1u) / PB)), dim3(PB), 0, st,
                           (const float *)d->part, S, d->M, d->N, mode, (const h16 *)d->bias, d->act, d->split,
                           (const h16 *)d->res, d->ldr, d->out, (h16 *)d->out1, (h16 *)d->out2,
                           epi == UOCR_GEMM_VISION ? d->N : d->ldo);
    } else if (epi == UOCR_GEMM_VISION) {
        gemm_dispatch<GE_VISION, false>(st, qt, a, grid, tmr);
    } else if (epi == UOCR_GEMM_F32) {
        if (grouped) gemm_dispatch<GE_F32, true>(st, qt, a, grid, tmr);
        else gemm_dispatch<GE_F32, false>(st, qt, a, grid, tmr);
    } else if (epi == UOCR_GEMM_SWIGLU) {
        if (grouped) gemm_dispatch<GE_SWIGLU, true>(st, qt, a, grid, tmr);
        else gemm_dispatch<GE_SWIGLU, false>(st, qt, a, grid, tmr);
    } else {
        if (grouped) gemm_dispatch<GE_F16, true>(st, qt, a, grid, tmr);
        else gemm_dispatch<GE_F16, false>(st, qt, a, grid, tmr);
        if (want_norm) {
            hipLaunchKernelGGL(k_rows_rmsnorm, dim3((d->M + 3u) / 4u), dim3(PB), 0, st, (const h16 *)d->out,
                               (const h16 *)d->norm_w, d->M, (h16 *)d->norm_out);
        }
    }
    return hipGetLastError();
}

/* Scales in LDS for a paired GEMM (as gemm_dispatch decides them). */
static size_t gemm_scales(u32 qt, u32 nmat, GemmArgs &a) {
    const u32 nt = a.K / TK;
    a.sc_lds = qt != UOCR_QT_F16 && nmat * nt <= SC_LDS_STEPS ? 1u : 0u;
    return a.sc_lds ? (size_t)nmat * TN * nt * sizeof(unsigned short) : 0;
}

extern "C" hipError_t uocr_launch_gemm_pair(hipStream_t st, int epi_a, const uocr_gemm_desc *da, int epi_b,
                                            const uocr_gemm_desc *db) {
    if (!gemm_desc_ok(epi_a, da) || !gemm_desc_ok(epi_b, db)) return hipErrorInvalidValue;
    static const int on = [] {
        const char *e = getenv("UOCR_HIP_GEMM_PAIR");
        return e == nullptr ? 1 : atoi(e);
    }();
    const u32 qa = da->W[0].qtype, qb = db->W[0].qtype;
    auto simple = [](const uocr_gemm_desc *d) {
        return !(d->ksplit > 1u && d->part != nullptr) && d->norm_w == nullptr && d->nseg == 0u;
    };
    const bool ok = on != 0 && simple(da) && simple(db) && da->tile_e == nullptr;
    const bool router = ok && epi_a == UOCR_GEMM_SWIGLU && epi_b == UOCR_GEMM_F32 && db->tile_e == nullptr &&
                        qb == UOCR_QT_F16;
    const bool experts = ok && epi_a == UOCR_GEMM_F16 && epi_b == UOCR_GEMM_SWIGLU && db->tile_e != nullptr && qa == qb;
    const bool downs = ok && epi_a == UOCR_GEMM_F16 && epi_b == UOCR_GEMM_F32 && db->tile_e != nullptr && qa == qb;
    const bool downs16 = ok && epi_a == UOCR_GEMM_F16 && epi_b == UOCR_GEMM_F16 && db->tile_e != nullptr && qa == qb;
    if (!router && !experts && !downs && !downs16) {
        const hipError_t e = uocr_launch_gemm(st, epi_a, da);
        return e != hipSuccess ? e : uocr_launch_gemm(st, epi_b, db);
    }
    GemmArgs a = gemm_args(da), b = gemm_args(db);
    const size_t sa = gemm_scales(qa, epi_a == UOCR_GEMM_SWIGLU ? 2u : 1u, a);
    const size_t sb = gemm_scales(qb, epi_b == UOCR_GEMM_SWIGLU ? 2u : 1u, b);
    const u32 ax = (da->M + TM - 1u) / TM, na = ax * ((da->N + TN - 1u) / TN);
    const u32 bx = db->tile_e != nullptr ? db->max_tiles : (db->M + TM - 1u) / TM;
    const dim3 grid(na + bx * ((db->N + TN - 1u) / TN));
    const size_t shm = sa > sb ? sa : sb;
    if (router) {
        switch (qa) {
            case UOCR_QT_F16:
                hipLaunchKernelGGL((k_gemm_pair<1, GE_SWIGLU, false, 1, GE_F32, false>), grid, dim3(PB), shm, st, a, ax,
                                   na, b, bx);
                break;
            case UOCR_QT_Q8:
                hipLaunchKernelGGL((k_gemm_pair<3, GE_SWIGLU, false, 1, GE_F32, false>), grid, dim3(PB), shm, st, a, ax,
                                   na, b, bx);
                break;
            default:
                hipLaunchKernelGGL((k_gemm_pair<4, GE_SWIGLU, false, 1, GE_F32, false>), grid, dim3(PB), shm, st, a, ax,
                                   na, b, bx);
                break;
        }
    } else if (downs16) {
        switch (qa) {
            case UOCR_QT_F16:
                hipLaunchKernelGGL((k_gemm_pair<1, GE_F16, false, 1, GE_F16, true>), grid, dim3(PB), shm, st, a, ax, na,
                                   b, bx);
                break;
            case UOCR_QT_Q8:
                hipLaunchKernelGGL((k_gemm_pair<3, GE_F16, false, 3, GE_F16, true>), grid, dim3(PB), shm, st, a, ax, na,
                                   b, bx);
                break;
            default:
                hipLaunchKernelGGL((k_gemm_pair<4, GE_F16, false, 4, GE_F16, true>), grid, dim3(PB), shm, st, a, ax, na,
                                   b, bx);
                break;
        }
    } else if (downs) {
        switch (qa) {
            case UOCR_QT_F16:
                hipLaunchKernelGGL((k_gemm_pair<1, GE_F16, false, 1, GE_F32, true>), grid, dim3(PB), shm, st, a, ax, na,
                                   b, bx);
                break;
            case UOCR_QT_Q8:
                hipLaunchKernelGGL((k_gemm_pair<3, GE_F16, false, 3, GE_F32, true>), grid, dim3(PB), shm, st, a, ax, na,
                                   b, bx);
                break;
            default:
                hipLaunchKernelGGL((k_gemm_pair<4, GE_F16, false, 4, GE_F32, true>), grid, dim3(PB), shm, st, a, ax, na,
                                   b, bx);
                break;
        }
    } else {
        switch (qa) {
            case UOCR_QT_F16:
                hipLaunchKernelGGL((k_gemm_pair<1, GE_F16, false, 1, GE_SWIGLU, true>), grid, dim3(PB), shm, st, a, ax,
                                   na, b, bx);
                break;
            case UOCR_QT_Q8:
                hipLaunchKernelGGL((k_gemm_pair<3, GE_F16, false, 3, GE_SWIGLU, true>), grid, dim3(PB), shm, st, a, ax,
                                   na, b, bx);
                break;
            default:
                hipLaunchKernelGGL((k_gemm_pair<4, GE_F16, false, 4, GE_SWIGLU, true>), grid, dim3(PB), shm, st, a, ax,
                                   na, b, bx);
                break;
        }
    }
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_rows_rmsnorm(hipStream_t st, const uint16_t *x, const uint16_t *w, uint32_t P,
                                               uint16_t *y) {
    if (x == nullptr || w == nullptr || y == nullptr || P == 0u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rows_rmsnorm, dim3((P + 3u) / 4u), dim3(PB), 0, st, (const h16 *)x, (const h16 *)w, P, (h16 *)y);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_rope_table(hipStream_t st, const float *inv_freq, uint32_t P, float *cs) {
    if (inv_freq == nullptr || cs == nullptr || P == 0u) return hipErrorInvalidValue;
    RopeTabP tab;
    for (int i = 0; i < UOCR_K_HEAD_DIM / 2; ++i) tab.f[i] = inv_freq[i];
    hipLaunchKernelGGL(k_rope_table, dim3((P * 64u + PB - 1u) / PB), dim3(PB), 0, st, tab, P, (float2 *)cs);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_gemm_qkv_rope(hipStream_t st, const uocr_gemm_desc *d, const float *cs,
                                                uint16_t *qout, uint16_t *kcache, uint16_t *vcache, uint32_t cap) {
    if (!gemm_desc_ok(UOCR_GEMM_F16, d) || d->tile_e != nullptr || d->nseg != UOCR_K_HIDDEN ||
        d->N != 3u * UOCR_K_HIDDEN || d->M > cap || cs == nullptr || qout == nullptr || kcache == nullptr ||
        vcache == nullptr) {
        return hipErrorInvalidValue;
    }
    GemmArgs a = gemm_args(d);
    const size_t shm = gemm_scales(d->W[0].qtype, 1u, a);
    const float2 *tab = (const float2 *)cs;
    const dim3 grid((d->M + TM - 1u) / TM, d->N / TN);
    switch (d->W[0].qtype) {
        case UOCR_QT_F16:
            hipLaunchKernelGGL(k_gemm_rope<1>, grid, dim3(PB), 0, st, a, tab, (h16 *)qout, (h16 *)kcache,
                               (h16 *)vcache, cap);
            break;
        case UOCR_QT_Q8:
            hipLaunchKernelGGL(k_gemm_rope<3>, grid, dim3(PB), shm, st, a, tab, (h16 *)qout, (h16 *)kcache,
                               (h16 *)vcache, cap);
            break;
        default:
            hipLaunchKernelGGL(k_gemm_rope<4>, grid, dim3(PB), shm, st, a, tab, (h16 *)qout, (h16 *)kcache,
                               (h16 *)vcache, cap);
            break;
    }
    return hipGetLastError();
}

/* Resident blocks of k_flash_attn on the chip (about 80 KB of LDS each: two
 * per CU).  The key chunk is the smallest whose (tile, head, chunk) blocks
 * all fit at once; the longest block then walks ch key tiles instead of all
 * of the last query tile's.  0: one block per (tile, head), no split. */
#ifndef FA_SLOTS
#define FA_SLOTS 512u
#endif

static u32 fa_chunk(u32 P) {
    const u32 nq = (P + AQ - 1u) / AQ;
    for (u32 ch = 1; ch < nq; ++ch) {
        u32 blocks = 0;
        for (u32 q = 0; q < nq; ++q) blocks += UOCR_K_HEADS * ((q + ch) / ch);
        if (blocks <= FA_SLOTS && (nq + ch - 1u) / ch <= FA_MAX_SPLITS) return ch;
    }
    return 0u;
}

extern "C" size_t uocr_flash_attn_ws_bytes(void) {
    return (size_t)FA_SLOTS * FA_PART_FLOATS * sizeof(float);
}

extern "C" hipError_t uocr_launch_flash_attn(hipStream_t st, const uint16_t *q, const uint16_t *kcache,
                                             const uint16_t *vcache, uint32_t cap, uint32_t P, uint16_t *ctx,
                                             float *ws) {
    if (q == nullptr || kcache == nullptr || vcache == nullptr || ctx == nullptr || P == 0u || P > cap) {
        return hipErrorInvalidValue;
    }
    const u32 nq = (P + AQ - 1u) / AQ, ch = ws != nullptr ? fa_chunk(P) : 0u;
    if (ch == 0u) {
        hipLaunchKernelGGL(k_flash_attn, dim3(nq, UOCR_K_HEADS), dim3(PB), 0, st, (const h16 *)q,
                           (const h16 *)kcache, (const h16 *)vcache, cap, P, (h16 *)ctx, 0u, (float *)nullptr);
        return hipGetLastError();
    }
    u32 blocks = 0;
    for (u32 qi = 0; qi < nq; ++qi) blocks += UOCR_K_HEADS * ((qi + ch) / ch);
    hipLaunchKernelGGL(k_flash_attn, dim3(blocks), dim3(PB), 0, st, (const h16 *)q, (const h16 *)kcache,
                       (const h16 *)vcache, cap, P, (h16 *)ctx, ch, ws);
    hipLaunchKernelGGL(k_flash_merge, dim3(nq - ch, UOCR_K_HEADS, AQ / 16u), dim3(PB), 0, st, (const float *)ws, P,
                       ch, (h16 *)ctx);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_route_rows(hipStream_t st, const float *logits, uint32_t P, int norm_topk,
                                             int32_t *ids, float *wts, int32_t *offsets, int32_t *tile_e,
                                             int32_t *tile_s0, int32_t *tile_s1, int32_t *ntiles, int32_t *list_tok,
                                             int32_t *list_pair) {
    if (logits == nullptr || P == 0u || ids == nullptr || wts == nullptr || offsets == nullptr || tile_e == nullptr || tile_s0 == nullptr || tile_s1 == nullptr || ntiles == nullptr ||
        list_tok == nullptr || list_pair == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k_route_rows, dim3((P + 3u) / 4u), dim3(PB), 0, st, logits, P, norm_topk, ids, wts);
    hipLaunchKernelGGL(k_bucket_build, dim3(1), dim3(BUCKET_THREADS), 0, st, (const int32_t *)ids, P, offsets,
                       tile_e, tile_s0, tile_s1, ntiles, list_tok, list_pair);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_moe_combine_norm(hipStream_t st, const float *Y, const float *wts,
                                                   const uint16_t *shared, const uint16_t *res, uint32_t P,
                                                   uint16_t *out, const uint16_t *norm_w, uint16_t *norm_out) {
    if (Y == nullptr || wts == nullptr || shared == nullptr || res == nullptr || out == nullptr || norm_w == nullptr ||
        norm_out == nullptr || P == 0u) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k_moe_combine_norm<float>, dim3((P + 3u) / 4u), dim3(PB), 0, st, Y, wts, (const h16 *)shared,
                       (const h16 *)res, P, (h16 *)out, (const h16 *)norm_w, (h16 *)norm_out);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_moe_combine_norm_h(hipStream_t st, const uint16_t *Y, const float *wts,
                                                     const uint16_t *shared, const uint16_t *res, uint32_t P,
                                                     uint16_t *out, const uint16_t *norm_w, uint16_t *norm_out) {
    if (Y == nullptr || wts == nullptr || shared == nullptr || res == nullptr || out == nullptr || norm_w == nullptr ||
        norm_out == nullptr || P == 0u) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(k_moe_combine_norm<h16>, dim3((P + 3u) / 4u), dim3(PB), 0, st, (const h16 *)Y, wts,
                       (const h16 *)shared, (const h16 *)res, P, (h16 *)out, (const h16 *)norm_w, (h16 *)norm_out);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_moe_combine(hipStream_t st, const float *Y, const float *wts, const uint16_t *shared,
                                              const uint16_t *res, uint32_t P, uint16_t *out) {
    if (Y == nullptr || wts == nullptr || shared == nullptr || res == nullptr || out == nullptr || P == 0u) {
        return hipErrorInvalidValue;
    }
    const u32 n = P * UOCR_K_HIDDEN;
    hipLaunchKernelGGL(k_moe_combine<float>, dim3((n + PB - 1u) / PB), dim3(PB), 0, st, Y, wts, (const h16 *)shared,
                       (const h16 *)res, P, (h16 *)out);
    return hipGetLastError();
}

extern "C" hipError_t uocr_launch_moe_combine_h(hipStream_t st, const uint16_t *Y, const float *wts,
                                                const uint16_t *shared, const uint16_t *res, uint32_t P,
                                                uint16_t *out) {
    if (Y == nullptr || wts == nullptr || shared == nullptr || res == nullptr || out == nullptr || P == 0u) {
        return hipErrorInvalidValue;
    }
    const u32 n = P * UOCR_K_HIDDEN;
    hipLaunchKernelGGL(k_moe_combine<h16>, dim3((n + PB - 1u) / PB), dim3(PB), 0, st, (const h16 *)Y, wts,
                       (const h16 *)shared, (const h16 *)res, P, (h16 *)out);
    return hipGetLastError();
}

/* ---- GEMM-packed weight copies -------------------------------------------- */

/* One 16-byte piece per thread: destination piece i of matrix blockIdx.y. */
template <u32 RB>
__global__ __launch_bounds__(PB) void k_pack_gemm_rows(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                       u32 rows, u32 K, uint64_t stride) {
    const u32 steps = K / 64u, per = 32u * RB / 16u; /* pieces per (32-row block, step) */
    const size_t i = (size_t)blockIdx.x * PB + threadIdx.x, total = (size_t)rows / 32u * steps * per;
    if (i >= total) return;
    const size_t blk = i / per;
    const u32 in = (u32)(i % per), rb = (u32)(blk / steps), g = (u32)(blk % steps);
    const u32 lanes = RB / 2u / 16u;                       /* pieces per lane */
    const u32 l = in / lanes, v = in % lanes, h = l / 32u, r = l % 32u;
    const size_t so = (size_t)(rb * 32u + r) * (K / 64u * RB) + (size_t)g * RB + h * (RB / 2u) + 16u * v;
    const size_t m = (size_t)blockIdx.y * stride;
    *(uint4 *)(dst + m + i * 16u) = *(const uint4 *)(src + m + so);
}

extern "C" hipError_t uocr_launch_pack_gemm_rows(hipStream_t st, uint32_t qtype, const void *src, void *dst,
                                                 uint32_t rows, uint32_t K, uint32_t count, uint64_t stride) {
    if (src == nullptr || dst == nullptr || rows == 0u || rows % 32u != 0u || K == 0u || K % 64u != 0u || count == 0u ||
        (qtype != UOCR_QT_Q4 && qtype != UOCR_QT_Q8)) {
        return hipErrorInvalidValue;
    }
    const size_t pieces = (size_t)rows * (qtype == UOCR_QT_Q4 ? K / 2u : K) / 16u;
    const dim3 grid((unsigned)((pieces + PB - 1u) / PB), count);
    if (qtype == UOCR_QT_Q4) {
        hipLaunchKernelGGL(k_pack_gemm_rows<32u>, grid, dim3(PB), 0, st, (const uint8_t *)src, (uint8_t *)dst, rows, K,
                           stride);
    } else {
        hipLaunchKernelGGL(k_pack_gemm_rows<64u>, grid, dim3(PB), 0, st, (const uint8_t *)src, (uint8_t *)dst, rows, K,
                           stride);
    }
    return hipGetLastError();
}
