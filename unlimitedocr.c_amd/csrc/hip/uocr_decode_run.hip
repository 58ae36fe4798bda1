/*
 * uocr_decode_run.hip - the persistent decode run (k_decode_run): greedy
 * decode steps of the 12-layer decoder carried by 256 resident workgroups,
 * one per CU, with no kernel boundary between stages.
 *
 * Op order and rounding points are the decode step of uocr_metal.m:14299-14518
 * (the same as the per-stage kernels of uocr_kernels.hip):
 *   LM head over the final-normed hidden state -> argmax (NaN rows skipped,
 *   ties to the lowest id, none valid -> 0; lm_head_q4.metal:25-98,
 *   sampling.metal:173-200) -> embedding row -> per layer:
 *   rmsnorm -> q/k/v (f16) -> split-half RoPE (rope.metal:39-70) -> KV slot
 *   write (kv_cache.metal:20-62) -> attention over the live slots
 *   (attention_decode.metal:25-131) -> f16 context -> O + residual (f16) ->
 *   rmsnorm -> layer 0: dense SwiGLU; layers 1-11: router top-6
 *   (moe.metal:12-18, raw probabilities), routed + shared SwiGLU mids (f16),
 *   down-combine f16(sum_r w_r D_r mid_r + f16(shared) + residual)
 *   (decode_gemv_q4.metal:185-224).
 *
 * Stages and the workgroups that run them (b = workgroup index):
 *   LM   all 256: rows [505b, 505b+505) of the LM head, one argmax packet each
 *   QKV  b < 240: 8 (matrix, head, rotation pair) items of 2 rows each
 *   ATT  176 <= b < 256: (head, split) of 10 x 8 over the live KV slots
 *   O    136 <= b < 176: 32 rows of O each, plus the rows' share of the
 *        un-normalised router logits z[e] = sum_i fold[i][e] a[i]
 *   GU   all 256: b < 192 routed (rank b/32, 28 rows of that expert),
 *        b >= 192 the shared experts' 1792 rows (layer 0: 27 dense rows each)
 *   DN   b < 160: 8 output rows each
 * Every block computes the top-6 itself from the O blocks' z partials (summed
 * in a fixed order), so the DN blocks issue their routed down-projection
 * loads as soon as the GU stage knows the experts.
 *
 * Hand-off (see uocr_run.h): packets {tag, 3 words}, device-coherent 16-byte
 * stores into one copy per XCD, device-coherent polls on the block's own
 * copy.  A stage's weight loads are issued before it polls for its inputs.
 * Every wait is bounded: after the model's limit_ticks without its packet a
 * block raises the abort word, every other waiting block sees it within a
 * few polls, and all blocks leave the kernel; the host reports the failure.
 */
#include "uocr_run.h"

#include "uocr_dev.h"

namespace {

typedef uint64_t u64;
#define AS1 __attribute__((address_space(1))) /* global memory */
#define AS4 __attribute__((address_space(4))) /* constant memory: scalar loads */

/* Device view of uocr_run_model: the same layout, read through the constant
 * address space (the descriptor does not change during a run, so its fields
 * come through scalar loads), with global-memory pointer fields (so the
 * weight loads are global, not flat, loads). */
struct RunLayerD {
    const AS1 uint8_t *q, *k, *v, *o;
    const AS1 uint16_t *qs, *ks, *vs, *os;
    const AS1 uint16_t *in_norm, *post_norm;
    const AS1 float *fold, *fold_o;
    const AS1 uint16_t *router;
    const AS1 uint8_t *gate, *up, *down;
    const AS1 uint16_t *gs, *us, *ds;
    const AS1 uint8_t *sg, *su, *sd;
    const AS1 uint16_t *sgs, *sus, *sds;
    const AS1 uint8_t *eg, *eu, *ed;
    const AS1 uint16_t *egs, *eus, *eds;
    uint64_t gu_w_stride, gu_s_stride, dn_w_stride, dn_s_stride;
};
struct RunModelD {
    RunLayerD L[UOCR_RUN_LAYERS];
    const AS1 uint8_t *lm, *emb;
    const AS1 uint16_t *lms, *embs, *final_norm;
    float invf[UOCR_K_HEAD_DIM / 2];
    uint32_t qa, qf, ql, qe;
    uint64_t limit_ticks;
};
static_assert(sizeof(RunModelD) == sizeof(uocr_run_model) && sizeof(RunLayerD) == sizeof(uocr_run_layer),
              "device view of the run model");

template <typename T, typename U>
__device__ __forceinline__ const T *gp(const AS1 U *p) {
    return (const T *)(const AS1 T *)p;
}
__device__ __forceinline__ const h16 *H(const AS1 uint16_t *p) { return gp<h16>(p); }
/* threadIdx.x made opaque to the optimiser at each use, so per-lane values of
 * one stage are recomputed there instead of being hoisted out of the step and
 * layer loops and held in registers through every other stage */
__device__ __forceinline__ u32 tid_() {
    u32 t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

/* Block barrier for data exchanged through LDS by ordinary LDS stores: waits
 * for this wavefront's LDS operations only.  Once a wavefront has issued
 * LDS-direct loads, __syncthreads() also drains every global load in flight
 * (vmcnt(0)), so a barrier placed while polls or weight rows are still
 * arriving would hold the whole block for that round trip. */
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr u32 NB = UOCR_RUN_BLOCKS, NT = UOCR_RUN_THREADS, NREP = UOCR_RUN_REPL;
constexpr u32 HID = UOCR_K_HIDDEN, HDIM = UOCR_K_HEAD_DIM, NHEAD = UOCR_K_HEADS, NEXP = UOCR_K_EXPERTS;
constexpr u32 TOPK = UOCR_K_TOPK, EI = 896u, SI = 1792u, DI = 6848u, VOCAB = 129280u, RING = UOCR_K_RING;

constexpr u32 QKV_BLOCKS = 240u;  /* 1920 items / 8 */
#ifndef UOCR_RUN_ATT_SPLITS
#define UOCR_RUN_ATT_SPLITS 8u
#endif
constexpr u32 ATT_SPLITS = UOCR_RUN_ATT_SPLITS, ATT_BLOCKS = NHEAD * ATT_SPLITS, ATT0 = NB - ATT_BLOCKS;
/* the stages' LDS scratch: the O stage's attention partials at most */
constexpr u32 SCR_BYTES = ATT_BLOCKS * 128u * 2u + ATT_BLOCKS * 12u + 512u * 4u > 24576u
                              ? ((ATT_BLOCKS * 128u * 2u + ATT_BLOCKS * 12u + 512u * 4u + 255u) & ~255u)
                              : 24576u;
#ifndef UOCR_RUN_O_BLOCKS
#define UOCR_RUN_O_BLOCKS 40u
#endif
constexpr u32 O_BLOCKS = UOCR_RUN_O_BLOCKS, O_ROWS = HID / O_BLOCKS, O0 = ATT0 - O_BLOCKS;
static_assert(O_ROWS * O_BLOCKS == HID, "O rows split evenly");
/* O blocks that also publish z partials.  Measured on config 5 (same box,
 * with the store drains): 20 Q4 3,860-3,862 and Q8 3,355-3,361 tok/s
 * against 16 3,812-3,814 and 3,366-3,368, 10 3,794 and 3,354-3,356 (8 and
 * 32, before the drains: both slower than 16). */
#ifndef UOCR_RUN_Z_BLOCKS
#define UOCR_RUN_Z_BLOCKS 20u
#endif
constexpr u32 Z_BLOCKS = UOCR_RUN_Z_BLOCKS, Z_COLS = HID / Z_BLOCKS;
/* UOCR_RUN_Z_SEP 1: the z partials come from Z_BLOCKS blocks below the O
 * blocks (QKV / GU / DN blocks otherwise idle in the O stage), so the O
 * blocks only compute O rows; 0: O blocks j < Z_BLOCKS publish them before
 * their O rows. */
#ifndef UOCR_RUN_Z_SEP
#define UOCR_RUN_Z_SEP 1
#endif
constexpr u32 Z0 = UOCR_RUN_Z_SEP ? O0 - Z_BLOCKS : O0; /* z block j is block Z0 + j */
static_assert(Z0 + Z_BLOCKS <= QKV_BLOCKS, "z blocks hold h from the QKV stage");
constexpr u32 GU_ROUTED = 192u, GU_ROWS = 28u, DGU_ROWS = 27u;
#ifndef UOCR_RUN_EXACT_WEIGHTS
#define UOCR_RUN_EXACT_WEIGHTS 1
#endif
/* exact router logits: GU block b computes quarter b % 4 of logit b / 4 */
constexpr u32 LG_Q = NB / NEXP, LG_COLS = HID / LG_Q;
static_assert(LG_Q * NEXP == NB && LG_COLS % 64u == 0u && LG_COLS / 8u <= 64u, "logit quarters");
constexpr u32 DN_BLOCKS = 160u, DN_ROWS = 8u;
constexpr u32 LM_ROWS = VOCAB / NB;
static_assert(LM_ROWS * NB == VOCAB, "LM rows split evenly");
static_assert(GU_ROUTED * GU_ROWS == TOPK * EI && (NB - GU_ROUTED) * GU_ROWS == SI, "GU rows");
static_assert(NB * DGU_ROWS >= DI, "dense rows");
static_assert(O0 >= 0u && O0 + O_BLOCKS <= QKV_BLOCKS, "O blocks also gather h in the QKV stage");

/* packets per copy */
constexpr u32 PQKV_B = 3u, PQKV = QKV_BLOCKS * PQKV_B;
constexpr u32 PATT_B = 23u, PATT = ATT_BLOCKS * PATT_B;
constexpr u32 PO_A = (O_ROWS + 5u) / 6u, PO_Z = 22u, PO_AR = O_BLOCKS * PO_A, PO = PO_AR + Z_BLOCKS * PO_Z;
/* Tested with 10, 16 and 20 z blocks (one z packet per GU thread); a test
 * build with 32 (two per thread) gave wrong tokens, and its cause was not
 * found, so larger counts are rejected. */
static_assert(Z_BLOCKS * PO_Z <= NT && HID % Z_BLOCKS == 0u, "z blocks: the tested range only");
constexpr u32 PMID_B = 5u, PMID = NB * PMID_B;
constexpr u32 PH_B = 2u, PH = DN_BLOCKS * PH_B;
constexpr u32 PLM = NB;
constexpr u32 PLAYER = PQKV + PATT + PO + PMID + PH;
constexpr u32 CTL_PK = 16u; /* 256 bytes of control words */

__host__ __device__ constexpr u64 off_lm() { return CTL_PK; }
__host__ __device__ constexpr u64 off_layer(u32 l) { return CTL_PK + (u64)PLM * NREP + (u64)l * PLAYER * NREP; }
__host__ __device__ constexpr u64 off_qkv(u32 l) { return off_layer(l); }
__host__ __device__ constexpr u64 off_att(u32 l) { return off_layer(l) + (u64)PQKV * NREP; }
__host__ __device__ constexpr u64 off_o(u32 l) { return off_att(l) + (u64)PATT * NREP; }
__host__ __device__ constexpr u64 off_mid(u32 l) { return off_o(l) + (u64)PO * NREP; }
__host__ __device__ constexpr u64 off_h(u32 l) { return off_mid(l) + (u64)PMID * NREP; }
constexpr u64 ARENA_PK = off_layer(UOCR_RUN_LAYERS);

/* Infinity Cache residency (256 MB) across decode steps: a Q4 LM head (88 MB)
 * with plain loads stays resident beside the shared experts, dense layer 0,
 * the folds and the KV cache; the attention projections (81 MB of Q8) are
 * read non-temporally instead (measured: 3,831 against 3,814 tok/s; the LM
 * head plain with the attention plain too: 3,705).  A Q8 LM head (170 MB)
 * does not fit and is read non-temporally. */
#ifndef UOCR_RUN_LM_NT
#define UOCR_RUN_LM_NT (QL != 4)
#endif
#ifndef UOCR_RUN_ATT_NT
#define UOCR_RUN_ATT_NT true
#endif
#ifndef UOCR_RUN_SLEEP
#define UOCR_RUN_SLEEP 1
#endif

/* stage codes reported on a timeout */
enum { W_LM = 1, W_SEL = 2, W_QKV = 3, W_ATT = 4, W_O = 5, W_GU = 6, W_DN = 7 };

/* Hardware exp2 / reciprocal forms (about 1 ulp in fp32) for the run's
 * softmax, SiLU, router probabilities and norms: with one wavefront per SIMD
 * every instruction on a stage's path costs about 2 ns, and the precise
 * library forms are several times longer.  Each result is rounded to fp16
 * or compared at the 1e-2 margins of the parity contract afterwards. */
__device__ __forceinline__ float fexp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float frcp(float x) {
    return __builtin_amdgcn_rcpf(x);
}
__device__ __forceinline__ float fsilu(float g) {
    return g * frcp(1.0f + fexp(-g));
}

/* ---- device-coherent accesses ------------------------------------------- */

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, 0x7fffffff, 0x00020000);
}
/* sc1 loads are served from the memory side, never from a stale L2 line;
 * the compiler barrier keeps a polling load inside its loop */
__device__ __forceinline__ uint4 cload16(const void *base, u32 off) {
    asm volatile("" ::: "memory");
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc(base), off, 0, 16));
}
__device__ __forceinline__ u32 cload32(const void *base, u32 off) {
    asm volatile("" ::: "memory");
    return __builtin_amdgcn_raw_buffer_load_b32(rsrc(base), off, 0, 16);
}
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void cstore16(void *base, u32 off, uint4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rsrc(base), off, 0, 16);
}
__device__ __forceinline__ void cstore32(void *base, u32 off, u32 v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, rsrc(base), off, 0, 16);
}
__device__ __forceinline__ void cstore_h16(void *base, u32 off, h16 v) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), rsrc(base), off, 0, 16);
}

/* ---- opt-in timeline (builds with -DUOCR_RUN_TIMELINE) ------------------- */

#ifdef UOCR_RUN_TIMELINE
/* s_memrealtime stamps of one chosen step: [block][event], event 2c when
 * stage c's inputs were complete, 2c + 1 when its packets were stored
 * (c = 0: LM head, 1 + 5l + s: stage s of layer l), 127 the step start;
 * 128 + k: points inside the stages of layer 5 and the LM head */
__device__ unsigned long long *g_run_tl;
__device__ int g_run_tl_step;
#define RUN_TL_EVENTS 256u
#define TLR(ev)                                                                                    \
    do {                                                                                           \
        if (R.tl != nullptr && tid_() == 0u) R.tl[blockIdx.x * RUN_TL_EVENTS + (ev)] =             \
            __builtin_amdgcn_s_memrealtime();                                                      \
    } while (0)
#define TLD(l, k)                      \
    do {                               \
        if ((l) == 5u) TLR(128u + (k)); \
    } while (0)
#else
#define TLR(ev) \
    do {        \
    } while (0)
#define TLD(l, k) \
    do {          \
    } while (0)
#endif

/* ---- packet hand-off ---------------------------------------------------- */

struct Run {
    const AS4 RunModelD *M;
    uint4 *pk;
    u32 *ctl;
    h16 *kc, *vc;
    u32 cap, xcc;
    int32_t P;
    int32_t *tokens;
    float *scores;
    h16 *hout;      /* layer 11's output of every step (plain stores) */
    u32 *trace;     /* expert ids [t][11][6] for t < trace_steps, their weights, the router inputs; or NULL */
    u32 trace_steps;
    const int32_t *force; /* teacher-forced ids for t < force_n, or NULL */
    u32 force_n;
    unsigned long long *tl; /* timeline of this step, or NULL */
};

/* Raises the run's abort word with where/step/block; 1. */
__device__ __attribute__((noinline)) int give_up(u32 *ctl, u32 where, u32 step) {
    cstore32(ctl, UOCR_RUN_CTL_WHERE * 4u, where);
    cstore32(ctl, UOCR_RUN_CTL_STEP * 4u, step);
    cstore32(ctl, UOCR_RUN_CTL_BLOCK * 4u, blockIdx.x);
    cstore32(ctl, UOCR_RUN_CTL_ABORT * 4u, 1u);
    return 1;
}

/* Block-wide gather of n packets (logical index i -> physical phys(i)) of
 * the block's copy: sink(i, packet) for each; false when the run aborted.
 * A thread polls all of its packets that are not current yet in one round
 * (one memory round trip per round whatever their number).  Ends with a
 * barrier, so the sinks' LDS writes are visible. */
template <int MAXP, typename Phys, typename Sink>
__device__ __forceinline__ bool gather(const Run &R, const uint4 *region, u32 per_copy, u32 n, u32 tag, u32 where,
                                       u32 step, Phys phys, Sink sink) {
    const uint4 *rep = region + (size_t)R.xcc * per_copy;
    const u32 t = tid_();
    uint4 v[MAXP];
#pragma unroll
    for (int k = 0; k < MAXP; ++k) v[k] = cload16(rep, phys(min(t + (u32)k * NT, n - 1u)) * 16u);
    u32 pend = 0u;
#pragma unroll
    for (int k = 0; k < MAXP; ++k) pend |= (t + (u32)k * NT < n && v[k].x != tag) ? (1u << k) : 0u;
    int bad = 0;
    if (pend != 0u) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (u32 it = 1; pend != 0u; ++it) {
            __builtin_amdgcn_s_sleep(UOCR_RUN_SLEEP);
#pragma unroll
            for (int k = 0; k < MAXP; ++k) {
                if (pend & (1u << k)) v[k] = cload16(rep, phys(t + (u32)k * NT) * 16u);
            }
#pragma unroll
            for (int k = 0; k < MAXP; ++k) {
                if ((pend & (1u << k)) && v[k].x == tag) pend &= ~(1u << k);
            }
            if (pend != 0u && (it & 15u) == 0u) {
                if (cload32(R.ctl, UOCR_RUN_CTL_ABORT * 4u) != 0u ||
                    __builtin_amdgcn_s_memrealtime() - t0 > R.M->limit_ticks) {
                    if (cload32(R.ctl, UOCR_RUN_CTL_ABORT * 4u) == 0u) give_up(R.ctl, where, step);
                    bad = 1;
                    break;
                }
            }
        }
    }
    if (bad == 0) {
#pragma unroll
        for (int k = 0; k < MAXP; ++k) {
            if (t + (u32)k * NT < n) sink(t + (u32)k * NT, v[k]);
        }
    }
    /* readfirstlane: the result is block-uniform, and the compiler must know
     * it, or every loop exit that depends on it turns the layer loop
     * divergent (per-layer pointers then come through vector loads and
     * full waits) */
    return __builtin_amdgcn_readfirstlane(__syncthreads_or(bad)) == 0;
}

/* gather() by wavefront `wave` alone (the others pass straight through):
 * its polls do not queue behind loads the other wavefronts have in flight.
 * The polls are LDS-direct loads into stg ([MAXP][64] packets, 16-byte
 * aligned LDS), so packets in flight take no registers.  No barrier: the
 * caller synchronises before the sinks' LDS writes are read.  The result
 * (false: the run aborted) is uniform in the wavefront. */
template <int MAXP, typename Phys>
__device__ __forceinline__ void gather_wave_issue(const Run &R, const uint4 *region, u32 per_copy, u32 n, u32 wave,
                                                  uint4 *stg, Phys phys) {
    if (__builtin_amdgcn_readfirstlane(tid_() / 64u) != wave) return;
    const __amdgpu_buffer_rsrc_t rs = rsrc(region + (size_t)R.xcc * per_copy);
    const u32 t = tid_() % 64u;
#pragma unroll
    for (int k = 0; k < MAXP; ++k) {
        if (t + (u32)k * 64u < n) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(stg + k * 64), 16u,
                                                     phys(t + (u32)k * 64u) * 16u, 0u, 0u, 16u);
        }
    }
}

/* PRE: gather_wave_issue() has issued the first round of polls into stg. */
template <int MAXP, bool PRE = false, typename Phys, typename Sink>
__device__ __forceinline__ bool gather_wave(const Run &R, const uint4 *region, u32 per_copy, u32 n, u32 tag, u32 where,
                                            u32 step, u32 wave, uint4 *stg, Phys phys, Sink sink, u32 tl_ev = 0u) {
    if (__builtin_amdgcn_readfirstlane(tid_() / 64u) != wave) return true;
    const uint4 *rep = region + (size_t)R.xcc * per_copy;
    const u32 t = tid_() % 64u;
    const __amdgpu_buffer_rsrc_t rs = rsrc(rep);
    u32 pend = 0u;
#pragma unroll
    for (int k = 0; k < MAXP; ++k) pend |= t + (u32)k * 64u < n ? (1u << k) : 0u;
    int bad = 0;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (u32 it = 1;; ++it) {
#pragma unroll
        for (int k = 0; k < MAXP; ++k) {
            if (!(PRE && it == 1u) && (pend & (1u << k))) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void *)(stg + k * 64),
                                                         16u, phys(t + (u32)k * 64u) * 16u, 0u, 0u, 16u);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#ifdef UOCR_RUN_TIMELINE
        /* the completion of the first rounds, and their count (tl_ev + 7) */
        if (tl_ev != 0u && R.tl != nullptr && t == 0u) {
            R.tl[blockIdx.x * RUN_TL_EVENTS + tl_ev + min(it - 1u, 6u)] = __builtin_amdgcn_s_memrealtime();
            R.tl[blockIdx.x * RUN_TL_EVENTS + tl_ev + 7u] = it;
        }
#endif
#pragma unroll
        for (int k = 0; k < MAXP; ++k) {
            if ((pend & (1u << k)) && stg[k * 64 + t].x == tag) pend &= ~(1u << k);
        }
        if (__builtin_amdgcn_readfirstlane(__builtin_amdgcn_ballot_w64(pend != 0u) == 0ull)) break;
        __builtin_amdgcn_s_sleep(1);
        if ((it & 15u) == 0u) {
            if (cload32(R.ctl, UOCR_RUN_CTL_ABORT * 4u) != 0u ||
                __builtin_amdgcn_s_memrealtime() - t0 > R.M->limit_ticks) {
                if (cload32(R.ctl, UOCR_RUN_CTL_ABORT * 4u) == 0u && t == 0u) give_up(R.ctl, where, step);
                bad = 1;
                break;
            }
        }
    }
    bad = __builtin_amdgcn_readfirstlane(bad);
    if (bad == 0) {
#pragma unroll
        for (int k = 0; k < MAXP; ++k) {
            if (t + (u32)k * 64u < n) sink(t + (u32)k * 64u, stg[k * 64 + t]);
        }
    }
    return bad == 0;
}

/* Threads t < npk * NREP store packet t / NREP of the block into copy
 * t % NREP at first + p; payload(p) gives its three words. */
template <typename Pay>
__device__ __forceinline__ void publish(const Run &R, uint4 *region, u32 per_copy, u32 first, u32 npk, u32 tag,
                                        Pay payload) {
    const u32 t = tid_();
    if (t < npk * NREP) {
        const u32 p = t / NREP, r = t % NREP;
        const uint3 d = payload(p);
        cstore16(region, (r * per_copy + first + p) * 16u, make_uint4(tag, d.x, d.y, d.z));
    }
}

/* UOCR_RUN_DRAIN (bit mask: 1 QKV, 2 ATT, 4 O rows, 8 GU (Q8 instance),
 * 16 DN, 32 z partials, 64 LM): after that
 * stage's publish, the storing wavefronts wait for their packet stores to
 * complete before issuing the next stage's loads; loads issued behind
 * device-coherent stores still in flight delay the packets' visibility.
 * Measured on config 5 (same box): 17 gives Q4 3,809-3,817 and Q8
 * 3,351-3,355 tok/s against 3,803 and 3,331 with none; adding ATT (19) the
 * same; adding the O rows (23) Q4 3,818-3,822 but Q8 3,335; the O rows
 * alone cost Q4 0.6%; GU (8) Q8 3,362 against 3,348 but Q4 -0.7%, so the
 * Q8 instance only; z partials (32) Q4 -2.6%, Q8 -2.2%; LM (64) nothing.
 * (The GU stage's publish is followed by the compiler's
 * own waits before the Q4 DN row loads; removing them cost Q4 0.6%.) */
#ifndef UOCR_RUN_DRAIN
#define UOCR_RUN_DRAIN 25
#endif
__device__ __forceinline__ void drain_stores(u32 bit, u32 npk) {
    if ((UOCR_RUN_DRAIN & bit) && __builtin_amdgcn_readfirstlane(tid_() / 64u) * 64u < npk * NREP) {
        __builtin_amdgcn_s_waitcnt(0x0F70); /* vmcnt(0) */
    }
}

__device__ __forceinline__ u32 pack2(h16 a, h16 b) {
    return (u32)__builtin_bit_cast(unsigned short, a) | ((u32)__builtin_bit_cast(unsigned short, b) << 16);
}
__device__ __forceinline__ h16 lo16(u32 w) {
    return __builtin_bit_cast(h16, (unsigned short)(w & 0xffffu));
}
__device__ __forceinline__ h16 hi16(u32 w) {
    return __builtin_bit_cast(h16, (unsigned short)(w >> 16));
}
/* payload of 6 halves v[6p .. 6p+5], zero past n */
__device__ __forceinline__ uint3 pay6(const h16 *v, u32 p, u32 n) {
    h16 e[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) e[j] = 6u * p + j < n ? v[6u * p + j] : (h16)0.0f;
    return make_uint3(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]));
}
/* writes the 6 halves of packet v to dst[0..5], stopping at n - base */
__device__ __forceinline__ void put6(h16 *dst, uint4 v, u32 base, u32 n) {
    const h16 e[6] = {lo16(v.y), hi16(v.y), lo16(v.z), hi16(v.z), lo16(v.w), hi16(v.w)};
#pragma unroll
    for (int j = 0; j < 6; ++j) {
        if (base + j < n) dst[j] = e[j];
    }
}

/* The norm weight's 8 values of thread t < 160 (columns 8t..8t+7), loaded
 * before a stage polls for its inputs. */
__device__ __forceinline__ uint4 norm_piece(const AS1 uint16_t *nw) {
    return gp<uint4>(nw)[min(tid_(), HID / 8u - 1u)];
}

/* RMSNorm of the LDS vector x into xs with the weight piece w of norm_piece
 * (eps 1e-6, fp32 sum of squares, one rounding per element;
 * norm.metal:12-40); returns inv_rms. */
/* Deferred RMSNorm: xs = fp16(x * w) and each wavefront's sum of x^2 in
 * red[wave]; after the caller's barrier rms_inv(red) gives 1 / rms(x), and
 * a dot over xs times it is the dot over the normalised row (the norm is
 * linear in 1 / rms), so the dots do not wait for the block reduction. */
__device__ __forceinline__ void rms_defer(const h16 *x, uint4 w, h16 *xs, float *red, float *x4, float *x8) {
    union h8 {
        uint4 u;
        h16 h[8];
    } xv, wv;
    const u32 t = tid_();
    float ss = 0.0f, ps = 0.0f;
    if (t < HID / 8u) {
        xv.u = ((const uint4 *)x)[t];
        wv.u = w;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float f = (float)xv.h[j];
            ss = fmaf(f, f, ss);
            xv.h[j] = (h16)(f * (float)wv.h[j]);
            ps += (float)xv.h[j];
        }
        ((uint4 *)xs)[t] = xv.u;
    }
    /* the chunk sums of xs for the offset-free dots (LM head) */
    if (x4 != nullptr || x8 != nullptr) piece_sums(ps, t, HID / 8u, x4, x8);
    ss = wave_sum(ss);
    if ((t & 63u) == 0u) red[t >> 6] = ss;
}

/* -bias * (activation sum) of chunk slot j of a lane (chunk sub + LPR j),
 * for chunk_value() */
template <int QT, int LPR, int J>
__device__ __forceinline__ void frag_nx(float (&nx)[J], const float *x4, const float *x8, u32 C, u32 sub) {
    static_assert(QT == 3 || QT == 4, "offset-free dots are Q4/Q8");
#pragma unroll
    for (int j = 0; j < J; ++j) nx[j] = -chunk_bias<QT>() * (QT == 4 ? x4 : x8)[min(sub + LPR * (u32)j, C - 1u)];
}

__device__ __forceinline__ float rms_inv(const float *red) {
    float s = 0.0f;
#pragma unroll
    for (u32 w = 0; w < NT / 64u; ++w) s += red[w];
    return __builtin_amdgcn_rsqf(s / (float)HID + 1.0e-6f);
}

__device__ __forceinline__ float rms_lds(const h16 *x, uint4 w, h16 *xs, float *red) {
    union h8 {
        uint4 u;
        h16 h[8];
    } xv, wv;
    const u32 t = tid_();
    float ss = 0.0f;
    xv.u = ((const uint4 *)x)[min(t, HID / 8u - 1u)];
    if (t < HID / 8u) {
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = fmaf((float)xv.h[j], (float)xv.h[j], ss);
    }
    ss = block_sum(ss, red);
    const float inv = __builtin_amdgcn_rsqf(ss / (float)HID + 1.0e-6f);
    if (t < HID / 8u) {
        wv.u = w;
#pragma unroll
        for (int j = 0; j < 8; ++j) xv.h[j] = (h16)(((float)xv.h[j] * inv) * (float)wv.h[j]);
        ((uint4 *)xs)[t] = xv.u;
    }
    __syncthreads();
    return inv;
}

/* Embedding row tok, columns 8i..8i+7, dequantised as f16(q * scale). */
template <int QE>
__device__ __forceinline__ uint4 embed8(const AS1 uint8_t *EW, const AS1 uint16_t *ES, int32_t tok, u32 i) {
    union h8 {
        uint4 u;
        h16 h[8];
    } o;
    o.u = make_uint4(0u, 0u, 0u, 0u);
    if (tok < 0 || (u32)tok >= VOCAB) return o.u;
    const size_t r = (size_t)tok;
    if (QE == 1) return ((const uint4 *)(gp<h16>(EW) + r * HID))[i];
    const float sc = (float)gp<h16>(ES)[r * (HID / 64u) + i / 8u];
    if (QE == 3) {
        const uint2 v = *(const uint2 *)(gp<uint8_t>(EW) + r * HID + 8u * i);
        const u32 w[2] = {v.x, v.y};
#pragma unroll
        for (int j = 0; j < 8; ++j) o.h[j] = (h16)((float)(int8_t)((w[j / 4] >> (8 * (j % 4))) & 0xffu) * sc);
    } else {
        const u32 j0 = (i % 8u) * 8u;
        const uint2 v = *(const uint2 *)(gp<uint8_t>(EW) + r * (HID / 2u) + (i / 8u) * 32u + (j0 & 31u));
        const u32 w[2] = {v.x, v.y}, sh = j0 < 32u ? 0u : 4u;
#pragma unroll
        for (int j = 0; j < 8; ++j) o.h[j] = (h16)((float)((int)((w[j / 4] >> (8 * (j % 4) + sh)) & 15u) - 8) * sc);
    }
    return o.u;
}

struct Lds {
    h16 *xs, *hres, *outv;
    float *red, *zout, *selw, *zw;
    u32 *selid;
    unsigned long long *keyw;
    uint8_t *scr;
    float *xsum; /* chunk sums of the LM head's activation */
    uint8_t *lgw; /* the GU block's router row and norm weight quarter (2 x 640 bytes) */
    uint4 *dnw;   /* the DN rows' weight chunks: [wavefront][slot][lane] */
};

/* ---- LM head -------------------------------------------------------------- */

template <int QL>
struct LmCfg {
    static constexpr u32 C = chunks_per_row<QL>(HID);
    static constexpr u32 LPR = QL == 4 ? 8u : (QL == 3 ? 16u : 32u);
    static constexpr u32 J = C / LPR;
    static constexpr u32 GPP = NT / LPR;
    static constexpr u32 NPASS = (LM_ROWS + GPP - 1u) / GPP;
    static_assert(J * LPR == C, "LM lanes cover a row");
};

template <int QL>
__device__ __forceinline__ void lm_load(const Run &R, RowFrag<LmCfg<QL>::J> &f, u32 pass) {
    typedef LmCfg<QL> G;
    const u32 grp = tid_() / G::LPR, sub = tid_() % G::LPR;
    const u32 r = blockIdx.x * LM_ROWS + min(pass * G::GPP + grp, LM_ROWS - 1u);
    frag_load<QL, G::LPR, G::J, UOCR_RUN_LM_NT>(f, gp<uint8_t>(R.M->lm) + (size_t)r * 16u * G::C,
                                      H(R.M->lms) + (size_t)r * (HID / 64u), G::C, sub);
}

/* LM head over the hidden state published with htag; publishes the block's
 * argmax key with tag.  The caller issues the loads of passes 0 and 1 into
 * f[0] and f[1]; each pass's dot is followed by the load of the pass two
 * later into the same buffer (10 chunks per lane: 80 KB in flight per CU). */
static_assert(NT % 64u == 0u && NT <= 1024u, "block of whole wavefronts");
constexpr u32 LM_DEPTH = 2u;

template <int QL>
__device__ bool lm_stage(const Run &R, const Lds &S, u32 tag, u32 htag, int32_t step,
                         RowFrag<LmCfg<QL>::J> (&f)[LM_DEPTH]) {
    typedef LmCfg<QL> G;
    const u32 grp = tid_() / G::LPR, sub = tid_() % G::LPR, lane = tid_() & 63u, wave = tid_() >> 6;
    h16 *hres = S.hres;
    const uint4 nwp = norm_piece(R.M->final_norm);
    if (!gather<(PH + NT - 1u) / NT>(R, R.pk + off_h(UOCR_RUN_LAYERS - 1u), PH, PH, htag, W_LM, (u32)step, [](u32 i) { return i; },
                   [&](u32 i, uint4 v) { put6(hres + (i / 2u) * DN_ROWS + (i % 2u) * 6u, v, (i % 2u) * 6u, DN_ROWS); })) {
        return false;
    }
    TLR(0u);
    rms_defer(S.hres, nwp, S.xs, S.red, QL == 4 ? S.xsum : nullptr, QL == 3 ? S.xsum : nullptr);
    __syncthreads();
    TLR(128u + 13u);
    const u32 row0 = blockIdx.x * LM_ROWS;
    float bs = -INFINITY;
    u32 bid = NONE_ID;
    float nx[G::J];
    frag_nx<QL, G::LPR, G::J>(nx, S.xsum, S.xsum, G::C, sub);
    auto finish = [&](const RowFrag<G::J> &fr, u32 pass) {
        const u32 r = pass * G::GPP + grp;
        const float d = group_sum<G::LPR>(frag_dot_u<QL, G::LPR, G::J>(fr, S.xs, nx, G::C, sub));
        if (r < LM_ROWS && !isnan(d) && better(d, row0 + r, bs, bid)) {
            bs = d;
            bid = row0 + r;
        }
    };
#pragma unroll 1
    for (u32 p = 0; p < G::NPASS; p += 2u) {
        finish(f[0], p);
        if (p + 2u < G::NPASS) lm_load<QL>(R, f[0], p + 2u);
        if (p + 1u < G::NPASS) {
            finish(f[1], p + 1u);
            if (p + 3u < G::NPASS) lm_load<QL>(R, f[1], p + 3u);
        }
    }
    TLR(128u + 14u);
#pragma unroll
    for (u32 o = G::LPR; o < 64u; o <<= 1) {
        const float os = __shfl_xor(bs, (int)o);
        const u32 oid = (u32)__shfl_xor((int)bid, (int)o);
        if (better(os, oid, bs, bid)) {
            bs = os;
            bid = oid;
        }
    }
    /* the rows were compared before the positive factor 1 / rms, which
     * scales the winner's logit */
    if (lane == 0u) S.keyw[wave] = argmax_key(bs * rms_inv(S.red), bid);
    __syncthreads();
    unsigned long long k = S.keyw[0];
#pragma unroll
    for (u32 w = 1; w < NT / 64u; ++w) k = S.keyw[w] > k ? S.keyw[w] : k;
    publish(R, R.pk + off_lm(), PLM, blockIdx.x, 1u, tag,
            [&](u32) { return make_uint3((u32)k, (u32)(k >> 32), 0u); });
    drain_stores(64u, 1u);
    TLR(1u);
    return true;
}

/* The token of the step: the largest of the 256 argmax keys (0: no valid
 * row -> token 0).  Every thread receives it. */
__device__ bool select_token(const Run &R, const Lds &S, u32 tag, int32_t step, int32_t &tok, float &score) {
    unsigned long long *kw = S.keyw;
    unsigned long long mine = 0ull;
    if (!gather<(PLM + NT - 1u) / NT>(R, R.pk + off_lm(), PLM, PLM, tag, W_SEL, (u32)step, [](u32 i) { return i; },
                   [&](u32, uint4 v) { mine = ((unsigned long long)v.z << 32) | v.y; })) {
        return false;
    }
    mine = wave_max_u64(mine);
    if ((tid_() & 63u) == 0u) kw[tid_() >> 6] = mine;
    __syncthreads();
    unsigned long long k = kw[0];
#pragma unroll
    for (u32 w = 1; w < NT / 64u; ++w) k = kw[w] > k ? kw[w] : k;
    u32 bi;
    key_winner(k, score, bi);
    tok = bi == NONE_ID ? 0 : (int32_t)bi;
    __syncthreads(); /* keyw is reused */
    return true;
}

/* ---- attention input: q/k/v + RoPE + KV write ---------------------------- */

template <int QA>
struct QkvCfg {
    static constexpr u32 C = chunks_per_row<QA>(HID), LPR = 32u, J = (C + LPR - 1u) / LPR;
};
static_assert(NT / 64u == 8u, "QKV: one (matrix, head, pair) item per wavefront, 8 per block");

template <int QA>
struct QkvFrags {
    RowFrag<QkvCfg<QA>::J> f;
};

/* Item of wavefront w of block b: matrix m = (b % 24) / 8 of q/k/v, head
 * b / 24, rotation pair d = (b % 8) * 8 + w; lanes 0-31 hold row d of the
 * head, lanes 32-63 row d + 64. */
template <int QA>
__device__ __forceinline__ void qkv_load(const Run &R, u32 l, QkvFrags<QA> &F) {
    typedef QkvCfg<QA> G;
    const u32 b = blockIdx.x;
    if (b >= QKV_BLOCKS) return;
    const AS4 RunLayerD &L = R.M->L[l];
    const u32 head = b / 24u, m = (b % 24u) / 8u, lane = tid_() & 63u;
    const u32 d = (b % 8u) * 8u + (tid_() >> 6), sub = lane % 32u;
    const uint8_t *W = gp<uint8_t>(m == 0u ? L.q : (m == 1u ? L.k : L.v));
    const h16 *Sc = m == 0u ? H(L.qs) : (m == 1u ? H(L.ks) : H(L.vs));
    const u32 r = head * HDIM + d + (lane < 32u ? 0u : 64u);
    frag_load<QA, G::LPR, G::J, UOCR_RUN_ATT_NT>(F.f, W + (size_t)r * 16u * G::C, Sc + (size_t)r * (HID / 64u), G::C, sub);
}

/* QKV stage of layer l at decode step t.  Layer 0 selects the token from
 * the LM keys and stages its embedding row as the hidden state. */
template <int QA, int QE>
__device__ bool qkv_stage(const Run &R, const Lds &S, u32 l, int32_t t, u32 tag, QkvFrags<QA> &F) {
    typedef QkvCfg<QA> G;
    const u32 b = blockIdx.x;
    if (b >= QKV_BLOCKS) return true;
    const AS4 RunLayerD &L = R.M->L[l];
    const u32 w = tid_() >> 6, lane = tid_() & 63u;
    const u32 head = b / 24u, m = (b % 24u) / 8u, d = (b % 8u) * 8u + w, sub = lane % 32u;
    const int32_t pos = R.P + t;
    const u32 slot = (u32)(R.P + t % (int32_t)RING);
    float cs = 1.0f, sn = 0.0f;
    if (m < 2u) {
        const float ang = (float)pos * R.M->invf[d];
        cs = cosf(ang);
        sn = sinf(ang);
    }
    h16 *hres = S.hres;
    const uint4 nwp = norm_piece(L.in_norm);
    if (l == 0u) {
        int32_t tok;
        float score;
        if (!select_token(R, S, tag, t, tok, score)) return false;
        if (b == 0u && tid_() == 0u) {
            R.tokens[t] = tok;
            if (R.scores != nullptr) R.scores[t] = score;
        }
        const int32_t etok = R.force != nullptr && (u32)t < R.force_n ? R.force[t] : tok;
        if (tid_() < HID / 8u) ((uint4 *)hres)[tid_()] = embed8<QE>(R.M->emb, R.M->embs, etok, tid_());
        __syncthreads();
    } else {
        if (!gather<(PH + NT - 1u) / NT>(R, R.pk + off_h(l - 1u), PH, PH, tag, W_QKV, (u32)t, [](u32 i) { return i; },
                       [&](u32 i, uint4 v) { put6(hres + (i / 2u) * DN_ROWS + (i % 2u) * 6u, v, (i % 2u) * 6u, DN_ROWS); })) {
            return false;
        }
    }
    TLR(2u * (1u + 5u * l));
    rms_defer(S.hres, nwp, S.xs, S.red, nullptr, nullptr);
    __syncthreads();
    TLD(l, 0u);
    const float dd = group_sum<G::LPR>(frag_dot<QA, G::LPR, G::J>(F.f, S.xs, G::C, sub)) * rms_inv(S.red);
    const float da = lane_f(dd, 0), db = lane_f(dd, 32);
    TLD(l, 1u);
    if (lane == 0u) {
        const h16 a = (h16)da, bb = (h16)db;
        h16 na = a, nb = bb;
        if (m < 2u) {
            const float fa2 = (float)a, fb2 = (float)bb;
            na = (h16)(fa2 * cs - fb2 * sn);
            nb = (h16)(fa2 * sn + fb2 * cs);
        }
        S.outv[w] = na;
        S.outv[8u + w] = nb;
        if (m >= 1u) {
            h16 *cache = (m == 1u ? R.kc : R.vc) + (size_t)l * NHEAD * R.cap * HDIM;
            const u32 off = ((head * R.cap + slot) * HDIM + d) * 2u;
            cstore_h16(cache, off, na);
            cstore_h16(cache, off + 128u, nb);
        }
    }
    __syncthreads();
    TLD(l, 2u);
    publish(R, R.pk + off_qkv(l), PQKV, b * PQKV_B, PQKV_B, tag, [&](u32 p) { return pay6(S.outv, p, 16u); });
    drain_stores(1u, PQKV_B);
    TLR(2u * (1u + 5u * l) + 1u);
    return true;
}

/* ---- attention ------------------------------------------------------------ */

constexpr u32 ATT_NG = NT / 16u; /* 16-lane slot groups per block */
constexpr u32 ATT_PF = 4u;        /* ATT_NG-slot rounds whose K/V are loaded ahead */

struct AttFrags {
    uint4 k[ATT_PF], v[ATT_PF];
};

struct AttPlan {
    u32 i0, i1, cs;
};

__device__ __forceinline__ AttPlan att_plan(const Run &R, int32_t t) {
    const u32 a = blockIdx.x - ATT0, s = a % ATT_SPLITS;
    const u32 live = (u32)min(t + 1, (int32_t)RING);
    const u32 L = (u32)R.P + live;
    const u32 chunk = (L + ATT_SPLITS - 1u) / ATT_SPLITS;
    AttPlan p;
    p.i0 = min(s * chunk, L);
    p.i1 = min(L, p.i0 + chunk);
    p.cs = (u32)(R.P + t % (int32_t)RING);
    return p;
}

/* K/V pieces of rounds [u0, u0 + ATT_PF): slot i0 + g + ATT_NG * u, dims 8p..8p+7;
 * slots past i1 and the current step's slot (taken from the packets) load
 * slot i0 instead (a cache hit, dropped later). */
__device__ __forceinline__ void att_load(const Run &R, u32 l, const AttPlan &pl, u32 u0, AttFrags &F) {
    const u32 a = blockIdx.x - ATT0, head = a / ATT_SPLITS;
    const u32 g = tid_() / 16u, p = tid_() % 16u;
    const size_t lay = (size_t)l * NHEAD * R.cap * HDIM + (size_t)head * R.cap * HDIM;
    const h16 *kb = R.kc + lay, *vb = R.vc + lay;
#pragma unroll
    for (u32 u = 0; u < ATT_PF; ++u) {
        u32 slot = pl.i0 + g + ATT_NG * (u0 + u);
        slot = slot < pl.i1 && slot != pl.cs ? slot : (pl.i1 > pl.i0 ? pl.i0 : 0u);
        F.k[u] = cload16(kb, (slot * HDIM + 8u * p) * 2u);
        F.v[u] = cload16(vb, (slot * HDIM + 8u * p) * 2u);
    }
}

/* Split (head, s) of the attention over slots [i0, i1): online softmax per
 * 16-lane slot group, merged over the block's 16 groups; publishes the
 * normalised accumulator (f16) and (max, sum) (fp32). */
__device__ bool att_stage(const Run &R, const Lds &S, u32 l, int32_t t, u32 tag, AttFrags &F) {
    const u32 b = blockIdx.x;
    if (b < ATT0) return true;
    const u32 a = b - ATT0, head = a / ATT_SPLITS;
    const u32 g = tid_() / 16u, p = tid_() % 16u;
    const AttPlan pl = att_plan(R, t);
    h16 *qn = (h16 *)S.scr, *kn = qn + HDIM, *vn = kn + HDIM; /* [3][128] */
    if (!gather<1>(R, R.pk + off_qkv(l), PQKV, 24u * PQKV_B, tag, W_ATT, (u32)t,
                   [&](u32 i) { return head * 24u * PQKV_B + i; },
                   [&](u32 i, uint4 v) {
                       const u32 blk = i / PQKV_B, k = i % PQKV_B, m = blk / 8u, d0 = (blk % 8u) * 8u;
                       h16 *dst = m == 0u ? qn : (m == 1u ? kn : vn);
                       const h16 e[6] = {lo16(v.y), hi16(v.y), lo16(v.z), hi16(v.z), lo16(v.w), hi16(v.w)};
#pragma unroll
                       for (u32 j = 0; j < 6u; ++j) {
                           const u32 idx = 6u * k + j;
                           if (idx < 16u) dst[idx < 8u ? d0 + idx : d0 + 56u + idx] = e[j];
                       }
                   })) {
        return false;
    }
    TLR(2u * (2u + 5u * l));
    union h8 {
        uint4 u;
        h16 h[8];
    };
    const uint4 qq = ((const uint4 *)qn)[p];
    const float scale = 0.08838834764831845f; /* 1/sqrt(128) */
    float m = -INFINITY, lsum = 0.0f, acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    TLD(l, 3u);
    const u32 nround = (pl.i1 - pl.i0 + ATT_NG - 1u) / ATT_NG;
#pragma unroll 1
    for (u32 u0 = 0;; u0 += ATT_PF) {
        float sc[ATT_PF];
        float mn = m;
#pragma unroll
        for (u32 u = 0; u < ATT_PF; ++u) {
            const u32 slot = pl.i0 + g + ATT_NG * (u0 + u);
            if (slot == pl.cs) {
                F.k[u] = ((const uint4 *)kn)[p];
                F.v[u] = ((const uint4 *)vn)[p];
            }
            float d = dot2(as_h2(qq.x), F.k[u].x, 0.0f);
            d = dot2(as_h2(qq.y), F.k[u].y, d);
            d = dot2(as_h2(qq.z), F.k[u].z, d);
            d = dot2(as_h2(qq.w), F.k[u].w, d);
            sc[u] = slot < pl.i1 ? row16_sum(d) * scale : -INFINITY;
            mn = fmaxf(mn, sc[u]);
        }
        if (mn != -INFINITY) {
            const float corr = fexp(m - mn);
            lsum *= corr;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] *= corr;
#pragma unroll
            for (u32 u = 0; u < ATT_PF; ++u) {
                const float e = fexp(sc[u] - mn);
                lsum += e;
                h8 vv;
                vv.u = F.v[u];
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[j] = fmaf(e, (float)vv.h[j], acc[j]);
            }
            m = mn;
        }
        if (u0 + ATT_PF >= nround) break;
        att_load(R, l, pl, u0 + ATT_PF, F);
    }
    TLD(l, 4u);
    /* merge of the ATT_NG slot groups through LDS in two levels: thread
     * (d, k) merges groups 8k..8k+7 for dim d, then threads d < 128 merge
     * the NT / 128 results */
    constexpr u32 GPK = 8u, NK = ATT_NG / GPK;
    static_assert(NK * HDIM == NT, "ATT merge: one (dim, part) per thread");
    float *gm = (float *)(S.scr + 3u * HDIM * 2u), *gl = gm + ATT_NG, *gacc = gl + ATT_NG; /* gacc [ATT_NG][128] */
    float *pm = gacc + ATT_NG * HDIM, *psum = pm + NK, *pacc = psum + NK;                 /* pacc [NK][128] */
    if (p == 0u) {
        gm[g] = m;
        gl[g] = lsum;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) gacc[g * HDIM + 8u * p + j] = acc[j];
    __syncthreads();
    {
        const u32 d = tid_() % HDIM, k = tid_() / HDIM;
        float M = -INFINITY;
#pragma unroll
        for (u32 q = 0; q < GPK; ++q) M = fmaxf(M, gm[k * GPK + q]);
        float Ls = 0.0f, A = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (u32 q = 0; q < GPK; ++q) {
                const float f = fexp(gm[k * GPK + q] - M);
                Ls = fmaf(gl[k * GPK + q], f, Ls);
                A = fmaf(gacc[(k * GPK + q) * HDIM + d], f, A);
            }
        }
        pacc[k * HDIM + d] = A;
        if (d == 0u) {
            pm[k] = M;
            psum[k] = Ls;
        }
    }
    __syncthreads();
    h16 *outa = (h16 *)(pacc + NK * HDIM);
    float *mlo = (float *)(outa + 132);
    if (tid_() < HDIM) {
        const u32 d = tid_();
        float M = -INFINITY;
#pragma unroll
        for (u32 k = 0; k < NK; ++k) M = fmaxf(M, pm[k]);
        float Ls = 0.0f, A = 0.0f;
        if (M != -INFINITY) {
#pragma unroll
            for (u32 k = 0; k < NK; ++k) {
                const float f = pm[k] == -INFINITY ? 0.0f : fexp(pm[k] - M);
                Ls = fmaf(psum[k], f, Ls);
                A = fmaf(pacc[k * HDIM + d], f, A);
            }
        }
        outa[d] = (h16)(Ls > 0.0f ? A * frcp(Ls) : 0.0f);
        if (d == 0u) {
            mlo[0] = M;
            mlo[1] = Ls;
        }
    }
    __syncthreads();
    TLD(l, 5u);
    publish(R, R.pk + off_att(l), PATT, a * PATT_B, PATT_B, tag, [&](u32 q) {
        return q < PATT_B - 1u ? pay6(outa, q, HDIM) : make_uint3(__float_as_uint(mlo[0]), __float_as_uint(mlo[1]), 0u);
    });
    drain_stores(2u, PATT_B);
    TLR(2u * (2u + 5u * l) + 1u);
    return true;
}

/* ---- O projection + router fold -------------------------------------------- */

template <int QA>
struct OCfg {
    static constexpr u32 C = chunks_per_row<QA>(HID), LPR = 32u;
    static constexpr u32 NG = NT / LPR, RPG = O_ROWS / NG;
    /* a lane group walks its RPG rows' chunks as one list, so every lane
     * holds the same number of chunks */
    static constexpr u32 J = (RPG * C + LPR - 1u) / LPR;
    static_assert(J * LPR == RPG * C, "O chunks split evenly over the lane group");
    static constexpr u32 ZC = Z_COLS / (NT / 64u); /* columns per thread in a z partial */
    static_assert(RPG * NG == O_ROWS && ZC * (NT / 64u) == Z_COLS && (UOCR_RUN_Z_SEP || Z_BLOCKS <= O_BLOCKS),
                  "O rows per group");
};

template <int QA>
struct OFrags {
    RowFrag<OCfg<QA>::J> f;
};

/* z-partial weights of z block j (block Z0 + j; MoE layers): rows
 * [80j, 80j + 80) of fold and of fold_o, two contiguous 20 KB ranges,
 * copied into LDS (zw[0], zw[1]) by LDS-direct loads, so they take no
 * registers while the O stage waits; complete once the issuing thread's
 * later loads have returned (loads return in order). */
constexpr u32 ZW_BYTES = Z_COLS * NEXP * 4u;
static_assert(ZW_BYTES % (64u * 16u) == 0u, "z weights in whole wavefront copies");

__device__ __forceinline__ void o_load_z(const Run &R, u32 l, float *zw) {
    const u32 b = blockIdx.x;
    if (l == 0u || b < Z0 || b >= Z0 + Z_BLOCKS) return;
    const AS4 RunLayerD &L = R.M->L[l];
    const u32 j = b - Z0, wave = __builtin_amdgcn_readfirstlane(tid_() / 64u), lane = tid_() % 64u;
    const AS1 uint8_t *src[2] = {(const AS1 uint8_t *)L.fold + (size_t)j * ZW_BYTES,
                                 (const AS1 uint8_t *)L.fold_o + (size_t)j * ZW_BYTES};
#pragma unroll
    for (u32 a = 0; a < 2u; ++a) {
#pragma unroll
        for (u32 off = wave * 1024u; off < ZW_BYTES; off += NT * 16u) {
            __builtin_amdgcn_global_load_lds((const AS1 void *)(src[a] + off + lane * 16u),
                                             (__attribute__((address_space(3))) void *)((uint8_t *)zw + a * ZW_BYTES + off),
                                             16u, 0, 0);
        }
    }
}

template <int QA>
__device__ __forceinline__ void o_load(const Run &R, u32 l, OFrags<QA> &F) {
    typedef OCfg<QA> G;
    const u32 b = blockIdx.x;
    if (b < O0 || b >= O0 + O_BLOCKS) return;
    const AS4 RunLayerD &L = R.M->L[l];
    const u32 j = b - O0, g = tid_() / 32u, sub = tid_() % 32u;
#pragma unroll
    for (u32 i = 0; i < G::J; ++i) {
        const u32 q = sub + G::LPR * i, k = q / G::C, c = q % G::C;
        const u32 r = j * O_ROWS + g * G::RPG + k;
        const uint8_t *ow = gp<uint8_t>(L.o) + ((size_t)r * G::C + c) * 16u;
        F.f.w[i] = UOCR_RUN_ATT_NT ? __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4v *)ow))
                                   : *(const uint4 *)ow;
        if (QA != 1) F.f.s[i] = H(L.os)[(size_t)r * (HID / 64u) + c / chunks_per_group<QA>()];
    }
}

template <int QA>
__device__ bool o_stage(const Run &R, const Lds &S, u32 l, int32_t t, u32 tag, OFrags<QA> &F) {
    typedef OCfg<QA> G;
    const u32 b = blockIdx.x;
    const bool ob = b >= O0 && b < O0 + O_BLOCKS, zb = l > 0u && b >= Z0 && b < Z0 + Z_BLOCKS;
    if (!ob && !zb) return true;
    const u32 j = b - O0, jz = b - Z0, g = tid_() / 32u, sub = tid_() % 32u;
    h16 *accp = (h16 *)S.scr;                           /* [80][128] */
    float *ml = (float *)(S.scr + ATT_BLOCKS * HDIM * 2u); /* [80][2] */
    float *wk = ml + 2u * ATT_BLOCKS;                     /* [80] */
    float *zq = wk + ATT_BLOCKS;                          /* [NT / 64][64] */
    static_assert(ATT_BLOCKS * HDIM * 2u + ATT_BLOCKS * 12u + NT * 4u <= SCR_BYTES, "O stage LDS");
    static_assert(HDIM % Z_COLS == 0u, "a z block's columns lie in one head");
    /* a z-only block needs the context of its own head only: that head's
     * ATT_SPLITS attention blocks (packets of the other heads are not
     * polled, and their merge is skipped) */
    const bool zonly = !ob;
    const u32 zh = jz * Z_COLS / HDIM, abase = zonly ? zh * ATT_SPLITS : 0u;
    auto att_phys = [=](u32 i) { return abase * PATT_B + i; };
    auto att_sink = [&](u32 i, uint4 v) {
        const u32 a = abase + i / PATT_B, k = i % PATT_B;
        if (k < PATT_B - 1u) {
            put6(accp + a * HDIM + 6u * k, v, 6u * k, HDIM);
        } else {
            ml[2u * a] = __uint_as_float(v.y);
            ml[2u * a + 1u] = __uint_as_float(v.z);
        }
    };
    const bool got = zonly ? gather<(ATT_SPLITS * PATT_B + NT - 1) / NT>(R, R.pk + off_att(l), PATT,
                                                                       ATT_SPLITS * PATT_B, tag, W_O, (u32)t,
                                                                       att_phys, att_sink)
                           : gather<(PATT + NT - 1) / NT>(R, R.pk + off_att(l), PATT, PATT, tag, W_O, (u32)t,
                                                          att_phys, att_sink);
    if (!got) return false;
    TLR(2u * (3u + 5u * l));
    /* merge weights: lanes 8h..8h+7 hold the splits of head h (the same
     * arithmetic as k_attn_out's merge) */
    if (tid_() < ATT_BLOCKS && (!zonly || tid_() / ATT_SPLITS == zh)) {
        const float mk = ml[2u * tid_()], lk = ml[2u * tid_() + 1u];
        float M = mk;
#pragma unroll
        for (u32 o = 1; o < ATT_SPLITS; o <<= 1) M = fmaxf(M, __shfl_xor(M, (int)o));
        const float lf = mk == -INFINITY ? 0.0f : lk * fexp(mk - M);
        wk[tid_()] = lf * frcp(group_sum<ATT_SPLITS>(lf));
    }
    /* the z weights' LDS-direct loads (o_load_z) are complete in every
     * wavefront before the barrier */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    TLD(l, 6u);
    if (tid_() < HID / 8u && (!zonly || tid_() / (HDIM / 8u) == zh)) {
        const u32 hh = tid_() / (HDIM / 8u), d8 = tid_() % (HDIM / 8u);
        float acc[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
#pragma unroll
        for (u32 s = 0; s < ATT_SPLITS; ++s) {
            const float w = wk[hh * ATT_SPLITS + s];
            const uint4 u = ((const uint4 *)(accp + (hh * ATT_SPLITS + s) * HDIM))[d8];
            const u32 uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] = fmaf((float)lo16(uu[q]), w, acc[2 * q]);
                acc[2 * q + 1] = fmaf((float)hi16(uu[q]), w, acc[2 * q + 1]);
            }
        }
        h16x2 r[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) r[q] = h16x2{(h16)acc[2 * q], (h16)acc[2 * q + 1]};
        ((uint4 *)S.xs)[tid_()] = __builtin_bit_cast(uint4, r);
    }
    __syncthreads();
    TLD(l, 7u);
    if (zb) {
        /* the router's pre-norm logits are linear in h and ctx:
         * z = fold^T a = fold^T h + (O^T fold)^T ctx.  This block's partial
         * over columns [Z_COLS jz, + Z_COLS) goes out before the O rows, so
         * the GU stage can choose the experts while the rows are computed. */
        const u32 e = tid_() % 64u, q = tid_() / 64u;
        const float *zf = S.zw, *zo = S.zw + Z_COLS * NEXP;
        /* every operand read before the (ordered) sums, so the LDS round
         * trips overlap */
        float wf[G::ZC], wo[G::ZC], xh[G::ZC], xc[G::ZC];
#pragma unroll
        for (u32 k = 0; k < G::ZC; ++k) {
            const u32 cl = G::ZC * q + k, c = jz * Z_COLS + cl;
            wf[k] = zf[cl * NEXP + e];
            wo[k] = zo[cl * NEXP + e];
            xh[k] = (float)S.hres[c];
            xc[k] = (float)S.xs[c];
        }
        __builtin_amdgcn_sched_barrier(0);
        float z = 0.0f;
#pragma unroll
        for (u32 k = 0; k < G::ZC; ++k) {
            z = fmaf(wf[k], xh[k], z);
            z = fmaf(wo[k], xc[k], z);
        }
        zq[q * 64u + e] = z;
        __syncthreads();
        if (tid_() < 64u) {
            const u32 e2 = tid_();
            float zk[NT / 64u];
#pragma unroll
            for (u32 k = 0; k < NT / 64u; ++k) zk[k] = zq[k * 64u + e2];
            __builtin_amdgcn_sched_barrier(0);
            float zs = 0.0f;
#pragma unroll
            for (u32 k = 0; k < NT / 64u; ++k) zs += zk[k];
            S.zout[e2] = zs;
        }
        __syncthreads();
        publish(R, R.pk + off_o(l), PO, PO_AR + jz * PO_Z, PO_Z, tag, [&](u32 p) {
            const u32 z0 = 3u * p;
            return make_uint3(__float_as_uint(S.zout[z0]), __float_as_uint(z0 + 1u < NEXP ? S.zout[z0 + 1u] : 0.0f),
                              __float_as_uint(z0 + 2u < NEXP ? S.zout[z0 + 2u] : 0.0f));
        });
        drain_stores(32u, PO_Z);
    }
    if (!ob) return true; /* a z block only */
    float part[G::RPG];
#pragma unroll
    for (u32 k = 0; k < G::RPG; ++k) part[k] = 0.0f;
#pragma unroll
    for (u32 i = 0; i < G::J; ++i) {
        const u32 q = sub + G::LPR * i, kq = q / G::C;
        const float d = chunk_dot<QA>(F.f.w[i], S.xs, q % G::C);
        const float v = QA == 1 ? d : d * (float)F.f.s[i];
#pragma unroll
        for (u32 k = 0; k < G::RPG; ++k) part[k] += kq == k ? v : 0.0f;
    }
#pragma unroll
    for (u32 k = 0; k < G::RPG; ++k) {
        const u32 rl = g * G::RPG + k, r = j * O_ROWS + rl;
        const float d = group_sum<G::LPR>(part[k]);
        if (sub == 0u) S.outv[rl] = (h16)(d + (float)S.hres[r]);
    }
    __syncthreads();
    TLD(l, 8u);
    publish(R, R.pk + off_o(l), PO, j * PO_A, PO_A, tag, [&](u32 p) { return pay6(S.outv, p, O_ROWS); });
    drain_stores(4u, PO_A);
    TLR(2u * (3u + 5u * l) + 1u);
    return true;
}

/* ---- gate/up (dense layer 0, routed + shared experts) -------------------- */

template <int QF>
struct GuCfg {
    static constexpr u32 C = chunks_per_row<QF>(HID);
    static constexpr u32 LPR = 16u;
    /* a lane group walks the gate row's C chunks then the up row's as one
     * list of 2C, so every lane holds the same number of chunks */
    static constexpr u32 J = (2u * C + LPR - 1u) / LPR;
    static_assert(J * LPR == 2u * C, "gate and up chunks split evenly over the lane group");
    static constexpr u32 NG = NT / LPR;                 /* lane groups */
    static constexpr u32 RPG = (GU_ROWS + NG - 1u) / NG; /* row pairs per group */
};

template <int QF>
struct GuFrags {
    RowFrag<GuCfg<QF>::J> f[GuCfg<QF>::RPG];
};

template <int QF, bool NTL>
__device__ __forceinline__ void gu_rows(GuFrags<QF> &F, const uint8_t *GW, const h16 *GS, const uint8_t *UW,
                                        const h16 *US, u32 row0, u32 nrows, u32 maxrow) {
    typedef GuCfg<QF> G;
    const u32 grp = tid_() / G::LPR, sub = tid_() % G::LPR;
#pragma unroll
    for (u32 k = 0; k < G::RPG; ++k) {
        /* groups past the last row load nothing (their dots are discarded),
         * which leaves the last wavefront free of loads in the MoE layers */
        if (grp + k * G::NG >= nrows) continue;
        const u32 r = row0 + grp + k * G::NG;
        const u32 rr = min(r, maxrow - 1u);
        const uint8_t *gw = GW + (size_t)rr * 16u * G::C, *uw = UW + (size_t)rr * 16u * G::C;
        const h16 *gs = GS + (size_t)rr * (HID / 64u), *us = US + (size_t)rr * (HID / 64u);
#pragma unroll
        for (u32 j = 0; j < G::J; ++j) {
            const u32 q = sub + G::LPR * j;
            const bool up = q >= G::C;
            const u32 c = up ? q - G::C : q;
            const uint8_t *w = (up ? uw : gw) + 16u * c;
            if (NTL) {
                F.f[k].w[j] = __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4v *)w));
                if (QF != 1) F.f[k].s[j] = __builtin_nontemporal_load((up ? us : gs) + c / chunks_per_group<QF>());
            } else {
                F.f[k].w[j] = *(const uint4 *)w;
                if (QF != 1) F.f[k].s[j] = (up ? us : gs)[c / chunks_per_group<QF>()];
            }
        }
    }
}

/* MoE-layer gate/up rows of block b, GU_ROWS each: blocks < 192 are routed
 * (rank b / 32, rows 28 (b % 32) of that expert), the rest shared.  With
 * UOCR_RUN_O_SHARED=1 the O blocks, which finish their own stage last, take
 * shared slices 0 .. 39 instead (fixed rows, loaded once their O rows are
 * out) and the other blocks, in order, the routed slices and then shared
 * slices 40 ..: measured slower (Q4 3,716 against 3,804 tok/s, Q8 3,308
 * against 3,333).  Returns the routed rank, or -1 with the shared slice. */
#ifndef UOCR_RUN_O_SHARED
#define UOCR_RUN_O_SHARED 0
#endif
__device__ __forceinline__ bool is_o_block(u32 b) {
    return b >= O0 && b < O0 + O_BLOCKS;
}
__device__ __forceinline__ int gu_role(u32 b, u32 &slice) {
    if (!UOCR_RUN_O_SHARED) {
        slice = b < GU_ROUTED ? b % 32u : b - GU_ROUTED;
        return b < GU_ROUTED ? (int)(b / 32u) : -1;
    }
    if (is_o_block(b)) {
        slice = b - O0;
        return -1;
    }
    const u32 n = b < O0 ? b : b - O_BLOCKS;
    if (n < GU_ROUTED) {
        slice = n % 32u;
        return (int)(n / 32u);
    }
    slice = O_BLOCKS + (n - GU_ROUTED);
    return -1;
}
static_assert(NB - O_BLOCKS >= GU_ROUTED && O_BLOCKS * GU_ROWS <= SI, "routed rows on non-O blocks, shared on the rest");

/* Index of block b's first mid in the DN stage's mid vector: layer 0 the
 * dense rows 27 b ..; MoE layers [routed rank 0 | .. | rank 5 | shared]. */
__device__ __forceinline__ u32 mid_base(u32 b, bool moe) {
    if (!moe) return b * DGU_ROWS;
    u32 slice;
    const int rank = gu_role(b, slice);
    return (rank >= 0 ? (u32)rank * EI : TOPK * EI) + slice * GU_ROWS;
}

template <int QF>
__device__ __forceinline__ void gu_load_shared(const Run &R, u32 l, GuFrags<QF> &F) {
    const AS4 RunLayerD &L = R.M->L[l];
    u32 slice;
    if (gu_role(blockIdx.x, slice) < 0) {
        gu_rows<QF, false>(F, gp<uint8_t>(L.sg), H(L.sgs), gp<uint8_t>(L.su), H(L.sus), slice * GU_ROWS, GU_ROWS, SI);
    }
}

/* Loads that do not depend on the router: dense rows (layer 0) or the
 * shared experts' rows of the shared-slice blocks outside the O stage (the O
 * blocks issue theirs in the GU stage). */
template <int QF>
__device__ __forceinline__ void gu_load_static(const Run &R, u32 l, GuFrags<QF> &F) {
    const AS4 RunLayerD &L = R.M->L[l];
    const u32 b = blockIdx.x;
    if (l == 0u) {
        gu_rows<QF, false>(F, gp<uint8_t>(L.gate), H(L.gs), gp<uint8_t>(L.up), H(L.us), b * DGU_ROWS,
                           min(DGU_ROWS, DI - min(b * DGU_ROWS, DI - 1u)), DI);
    } else if (!UOCR_RUN_O_SHARED || !is_o_block(b)) {
        gu_load_shared<QF>(R, l, F);
    }
}

/* A descriptor value read early and made opaque, so the compiler keeps it in
 * a register instead of re-reading it (a scalar load that can miss the
 * scalar cache) where it is used. */
template <typename T>
__device__ __forceinline__ T pin(T v) {
    asm volatile("" : "+s"(v));
    return v;
}

/* Expert slab pointers and strides of one layer, read at the GU stage's
 * start, ahead of the loads that need them. */
struct SlabD {
    const AS1 uint8_t *eg, *eu, *ed, *sd;
    const AS1 uint16_t *egs, *eus, *eds, *sds;
    uint64_t gws, gss, dws, dss;
};

__device__ __forceinline__ SlabD slab_of(const AS4 RunLayerD &L) {
    SlabD d;
    d.eg = pin(L.eg);
    d.eu = pin(L.eu);
    d.ed = pin(L.ed);
    d.sd = pin(L.sd);
    d.egs = pin(L.egs);
    d.eus = pin(L.eus);
    d.eds = pin(L.eds);
    d.sds = pin(L.sds);
    d.gws = pin(L.gu_w_stride);
    d.gss = pin(L.gu_s_stride);
    d.dws = pin(L.dn_w_stride);
    d.dss = pin(L.dn_s_stride);
    return d;
}

/* DN rows: wavefront w of block b owns output row 8b + w.  Its chunks are
 * one list, the 6 routed experts' rows (CR chunks each) then the shared
 * expert's row (CS chunks); lane l holds chunks l, l + 64, ... */
template <int QF>
struct DnCfg {
    static constexpr u32 CR = chunks_per_row<QF>(EI), CS = chunks_per_row<QF>(SI), CT = TOPK * CR + CS;
    static constexpr u32 J = (CT + 63u) / 64u;
    static constexpr u32 CD = chunks_per_row<QF>(DI), JD = (CD + 63u) / 64u;
};
static_assert(NT / 64u == DN_ROWS, "DN: one output row per wavefront");

/* Where the DN rows' 16-byte weight chunks wait for the DN stage (the
 * scales always stay in registers):
 *   - Q4: in registers, loaded once the GU stage's own loads are consumed;
 *   - Q8: in LDS (S.dnw: [wavefront][slot][lane] uint4), by LDS-direct loads
 *     issued during the GU stage right after its gather of a, so the DN
 *     stage polls for the mids with no row loads in flight and finds its
 *     rows resident, and no DN registers are live through the GU stage.
 * Measured on config 5: Q8 3,370 (LDS, early) against 3,199 tok/s (registers,
 * late; the Q8 kernel then spilled 21 VGPRs); Q4 3,810 (registers, late)
 * against 3,736 (LDS, late) and 3,648 (LDS, early). */
template <int QF>
constexpr bool dn_in_lds() {
    return QF == 3;
}
template <int QF>
struct DnFrags {
    uint4 w[dn_in_lds<QF>() ? 1u : DnCfg<QF>::J];
    h16 s[DnCfg<QF>::J];
};

/* layer 0's dense down row uses the same registers: as many chunk slots */
static_assert(DnCfg<4>::JD == DnCfg<4>::J && DnCfg<3>::JD == DnCfg<3>::J, "dense down row fits the DN slots");

__device__ __forceinline__ u32 dn_row() {
    return blockIdx.x * DN_ROWS + (tid_() >> 6);
}

__device__ __forceinline__ void lds16(const void *src, uint4 *dst, bool nt) {
    if (nt) {
        __builtin_amdgcn_global_load_lds((const AS1 void *)src, (__attribute__((address_space(3))) void *)dst, 16u, 0,
                                         2 /* nt */);
    } else {
        __builtin_amdgcn_global_load_lds((const AS1 void *)src, (__attribute__((address_space(3))) void *)dst, 16u, 0,
                                         0);
    }
}

/* Routed down rows of the selected experts (ids in LDS, non-temporal) and
 * the shared down row (plain: it stays in the Infinity Cache). */
template <int QF>
__device__ __forceinline__ void dn_load(const Run &R, const Lds &S, const SlabD &L, DnFrags<QF> &F) {
    typedef DnCfg<QF> G;
    if (blockIdx.x >= DN_BLOCKS) return;
    const u32 c = dn_row(), lane = tid_() & 63u, wave = __builtin_amdgcn_readfirstlane(tid_() >> 6);
    constexpr u32 CPG = chunks_per_group<QF>();
    uint4 *dst = S.dnw + (size_t)wave * G::J * 64u;
#pragma unroll
    for (u32 j = 0; j < G::J; ++j) {
        const u32 q = min(lane + 64u * j, G::CT - 1u);
        if (q < TOPK * G::CR) {
            const u32 r = q / G::CR, cc = q % G::CR, e = S.selid[r];
            const uint8_t *W = gp<uint8_t>(L.ed) + e * L.dws + (size_t)c * 16u * G::CR + 16u * cc;
            if (dn_in_lds<QF>()) {
                lds16(W, dst + j * 64u, true);
            } else {
                F.w[j] = __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4v *)W));
            }
            if (QF != 1) F.s[j] = __builtin_nontemporal_load(H(L.eds) + e * L.dss + (size_t)c * (EI / 64u) + cc / CPG);
        } else {
            const u32 cc = q - TOPK * G::CR;
            const uint8_t *W = gp<uint8_t>(L.sd) + (size_t)c * 16u * G::CS + 16u * cc;
            if (dn_in_lds<QF>()) {
                lds16(W, dst + j * 64u, false);
            } else {
                F.w[j] = *(const uint4 *)W;
            }
            if (QF != 1) F.s[j] = H(L.sds)[(size_t)c * (SI / 64u) + cc / CPG];
        }
    }
}

template <int QF>
__device__ __forceinline__ void dd_load(const Run &R, const Lds &S, DnFrags<QF> &F) {
    typedef DnCfg<QF> G;
    if (blockIdx.x >= DN_BLOCKS) return;
    const AS4 RunLayerD &L = R.M->L[0];
    const u32 c = dn_row(), lane = tid_() & 63u, wave = __builtin_amdgcn_readfirstlane(tid_() >> 6);
    uint4 *dst = S.dnw + (size_t)wave * G::J * 64u;
#pragma unroll
    for (u32 j = 0; j < G::JD; ++j) {
        const u32 q = min(lane + 64u * j, G::CD - 1u);
        const uint8_t *W = gp<uint8_t>(L.down) + (size_t)c * 16u * G::CD + 16u * q;
        if (dn_in_lds<QF>()) {
            lds16(W, dst + j * 64u, false);
        } else {
            F.w[j] = *(const uint4 *)W;
        }
        if (QF != 1) F.s[j] = H(L.ds)[(size_t)c * (DI / 64u) + q / chunks_per_group<QF>()];
    }
}

/* GU stage: gathers the O outputs (a, and the z partials in MoE layers),
 * normalises a, selects the experts (MoE), and computes the block's mids.
 * MoE layers also issue the DN stage's loads (dn) once the experts are known. */
#define UOCR_RUN_DN_EARLY dn_in_lds<QF>()
/* GU's first round of polls for a, per instance: 0 right after the z
 * gather, 1 after the expert choice, 2 after it except in the O blocks.
 * Q8: 1 (3,426-3,430 against 3,394 tok/s with 0); Q4: 0 (3,836-3,846 with 1
 * against 3,906, 2 within the noise) */
#ifndef UOCR_RUN_APRE_Q4
#define UOCR_RUN_APRE_Q4 0
#endif
#ifndef UOCR_RUN_APRE_Q8
#define UOCR_RUN_APRE_Q8 1
#endif
#ifndef UOCR_RUN_Z_ALL_SKIP
#define UOCR_RUN_Z_ALL_SKIP 1 /* Q4: blocks that do not need z skip its gather (2: both instances) */
#endif
#ifndef UOCR_RUN_WAVE_TOPK
#define UOCR_RUN_WAVE_TOPK 1 /* Q8 with 20 z blocks and the store drains: 3,363-3,366 against 3,351-3,353 without it (before them: 3,196 against 3,180) */
#endif
template <int QF>
__device__ bool gu_stage(const Run &R, const Lds &S, u32 l, int32_t t, u32 tag, GuFrags<QF> &F, DnFrags<QF> &dn) {
    typedef GuCfg<QF> G;
    const AS4 RunLayerD &L = R.M->L[l];
    const u32 b = blockIdx.x, grp = tid_() / G::LPR, sub = tid_() % G::LPR;
    const bool moe = l > 0u;
    const SlabD sd = moe ? slab_of(L) : SlabD{};
    float *zpart = (float *)S.scr; /* [Z_BLOCKS][64] */
    h16 *hres = S.hres;
    const uint4 nwp = norm_piece(L.post_norm);
    auto gather_a = [&]() {
        return gather<(PO_AR + NT - 1) / NT>(R, R.pk + off_o(l), PO, PO_AR, tag, W_GU, (u32)t, [](u32 i) { return i; },
                                             [&](u32 i, uint4 v) {
                                                 const u32 j = i / PO_A, k = i % PO_A;
                                                 put6(hres + j * O_ROWS + 6u * k, v, 6u * k, O_ROWS);
                                             });
    };
    float inv;
    if (moe) {
        u32 slice;
        const int rank = gu_role(b, slice);
        /* the O blocks' shared rows, issued now that their O rows are out */
        if (UOCR_RUN_O_SHARED && is_o_block(b)) gu_load_shared<QF>(R, l, F);
        /* the exact router logit's quarter this block owns (expert b / 4,
         * columns [320 (b % 4), + 320)): its router row and norm weight
         * pieces, by wavefront 0 ahead of its polls (used after the dots) */
        if (UOCR_RUN_EXACT_WEIGHTS && __builtin_amdgcn_readfirstlane(tid_() / 64u) == 0u) {
            const u32 lane = tid_() % 64u, e = b / LG_Q, c0 = (b % LG_Q) * LG_COLS;
            if (lane < LG_COLS / 8u) {
                __builtin_amdgcn_global_load_lds((const AS1 void *)(L.router + (size_t)e * HID + c0 + 8u * lane),
                                                 (__attribute__((address_space(3))) void *)S.lgw, 16u, 0, 0);
                __builtin_amdgcn_global_load_lds((const AS1 void *)(L.post_norm + c0 + 8u * lane),
                                                 (__attribute__((address_space(3))) void *)(S.lgw + 2u * LG_COLS), 16u,
                                                 0, 0);
            }
        }
        /* the z partials first (published before the O rows), the top-6 on z
         * (softmax is monotone and inv_rms > 0, so z orders the experts as
         * the probabilities do) and the expert loads; then a and its norm */
        /* z feeds the expert choice only: routed blocks, the DN blocks (their
         * DN stage reads the ids) and the traced block; in the Q4 instance the
         * other shared-row blocks skip its 440 packets (Q4 3,913 against 3,897
         * tok/s; the Q8 instance measured 3,306 against 3,394 with the skip) */
        const bool need_z = !(UOCR_RUN_Z_ALL_SKIP == 2 || (UOCR_RUN_Z_ALL_SKIP == 1 && QF == 4)) ||
                            (rank >= 0 || b < DN_BLOCKS || (R.trace != nullptr && b == 0u) || !UOCR_RUN_EXACT_WEIGHTS);
        if (need_z && !gather<(Z_BLOCKS * PO_Z + NT - 1) / NT>(R, R.pk + off_o(l), PO, Z_BLOCKS * PO_Z, tag, W_GU, (u32)t,
                                                     [](u32 i) { return PO_AR + i; }, [&](u32 i, uint4 v) {
                                                         const u32 j = i / PO_Z, z0 = 3u * (i % PO_Z);
                                                         float *zp = zpart + j * NEXP + z0;
                                                         zp[0] = __uint_as_float(v.y);
                                                         if (z0 + 1u < NEXP) zp[1] = __uint_as_float(v.z);
                                                         if (z0 + 2u < NEXP) zp[2] = __uint_as_float(v.w);
                                                     })) {
            return false;
        }
        TLR(2u * (4u + 5u * l));
        /* the first round of a's polls: issued here (in flight while the
         * experts are chosen), or (UOCR_RUN_APRE_Q4 / _Q8) once they are
         * chosen, still ahead of the expert loads */
        uint4 *stg = (uint4 *)(S.scr + 8192u);
        auto a_pre = [&]() {
            gather_wave_issue<(PO_AR + 63u) / 64u>(R, R.pk + off_o(l), PO, PO_AR, NT / 64u - 1u, stg,
                                                    [](u32 i) { return i; });
#ifdef UOCR_RUN_TIMELINE
            if (l == 5u && R.tl != nullptr && tid_() == NT - 64u)
                R.tl[blockIdx.x * RUN_TL_EVENTS + 128u + 33u] = __builtin_amdgcn_s_memrealtime();
#endif
        };
        constexpr int apre = QF == 4 ? UOCR_RUN_APRE_Q4 : UOCR_RUN_APRE_Q8;
        const bool apre_late = apre == 1 || (apre == 2 && !is_o_block(b));
        if (!apre_late) a_pre();
        /* wavefront 0: z of expert e (lane e) over the Z_BLOCKS partials in a fixed
         * order, then the top-6 */
        TLD(l, 18u);
        /* every wavefront sums z (lane e: expert e, the Z_BLOCKS partials in a fixed
         * order) and takes the top-6 itself, so each issues its expert rows
         * without a barrier; wavefront 0 also leaves the ids in LDS for the
         * later readers (behind the barrier after the gather of a) */
        float z = 0.0f;
        u32 mye = 0u;
        if (need_z && (UOCR_RUN_WAVE_TOPK || tid_() < 64u)) {
            const u32 e = tid_() % 64u;
            /* all partials read before the (ordered) sum: one LDS round trip */
            float zp[Z_BLOCKS];
#pragma unroll
            for (u32 j = 0; j < Z_BLOCKS; ++j) zp[j] = zpart[j * NEXP + e];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (u32 j = 0; j < Z_BLOCKS; ++j) z += zp[j];
            TLD(l, 22u);
            u32 sid[TOPK];
            topk6_ids(z, sid);
            TLD(l, 23u);
            if (tid_() < TOPK) {
#pragma unroll
                for (u32 k = 0; k < TOPK; ++k) {
                    if (e == k) S.selid[k] = sid[k] < NEXP ? sid[k] : 0u;
                }
            }
#pragma unroll
            for (u32 k = 0; k < TOPK; ++k) {
                if (rank == (int)k) mye = sid[k] < NEXP ? sid[k] : 0u;
            }
        }
        /* the last wavefront's polls for a are in flight */
        if (!UOCR_RUN_WAVE_TOPK) lds_barrier();
        if (R.trace != nullptr && b == 0u && (u32)t < R.trace_steps && tid_() < TOPK) {
            R.trace[((size_t)t * 11u + (l - 1u)) * TOPK + tid_()] = S.selid[tid_()];
        }
        if (apre_late) a_pre();
        TLD(l, 9u);
        if (rank >= 0) {
            const u32 e = UOCR_RUN_WAVE_TOPK ? mye : S.selid[rank];
            gu_rows<QF, true>(F, gp<uint8_t>(sd.eg) + e * sd.gws, H(sd.egs) + e * sd.gss, gp<uint8_t>(sd.eu) + e * sd.gws,
                              H(sd.eus) + e * sd.gss, slice * GU_ROWS, GU_ROWS, EI);
        }
        TLD(l, 10u);
#if defined(UOCR_RUN_TIMELINE) && !defined(UOCR_RUN_TL_NOWAIT)
        if (l == 5u && tid_() == 0u) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            TLR(128u + 17u);
        }
#endif
        /* a: polled by the last wavefront, which has no gate/up rows (28 rows
         * of 16 lanes fill wavefronts 0-6), so its polls do not wait behind
         * the expert loads in flight in the others */
        static_assert(GU_ROWS * G::LPR <= NT - 64u && G::RPG == 1u, "the last wavefront holds no GU rows");
        const bool ok_a = gather_wave<(PO_AR + 63u) / 64u, true>(
            R, R.pk + off_o(l), PO, PO_AR, tag, W_GU, (u32)t, NT / 64u - 1u, stg, [](u32 i) { return i; },
            [&](u32 i, uint4 v) {
                const u32 j = i / PO_A, k = i % PO_A;
                put6(hres + j * O_ROWS + 6u * k, v, 6u * k, O_ROWS);
            },
            l == 5u ? 128u + 25u : 0u);
        if (tid_() == NT - 64u) S.red[15] = ok_a ? 1.0f : 0.0f;
#ifdef UOCR_RUN_TIMELINE
        /* the eighth wavefront's gather of a complete (its own stamp) */
        if (l == 5u && R.tl != nullptr && tid_() == NT - 64u)
            R.tl[blockIdx.x * RUN_TL_EVENTS + 128u + 24u] = __builtin_amdgcn_s_memrealtime();
#endif
        /* the other wavefronts' expert rows may still be arriving */
        lds_barrier();
        if (S.red[15] == 0.0f) return false;
        /* the DN stage's rows of the selected experts into LDS, now that no
         * poll of this stage is left behind them */
        if (UOCR_RUN_DN_EARLY) dn_load<QF>(R, S, sd, dn);
        TLD(l, 15u);
        if (R.trace != nullptr && b == 0u && (u32)t < R.trace_steps && tid_() < HID / 8u) {
            uint4 *ta = (uint4 *)(R.trace + 2u * (size_t)R.trace_steps * 11u * TOPK);
            ta[((size_t)t * 11u + (l - 1u)) * (HID / 8u) + tid_()] = ((const uint4 *)S.hres)[tid_()];
        }
        rms_defer(S.hres, nwp, S.xs, S.red, nullptr, nullptr);
        lds_barrier();
        inv = rms_inv(S.red);
        TLD(l, 16u);
        if (!UOCR_RUN_EXACT_WEIGHTS && tid_() < 64u) {
            /* the selection's probabilities: softmax of z * inv_rms (raw, no
             * renormalisation; max-subtracted) */
            const float lg = z * inv;
            const float mx = wave_max_dpp(lg);
            const float pe = fexp(lg - mx);
            const float p = pe * frcp(wave_sum(pe));
            const u32 k = tid_();
            const float ps = __shfl(p, (int)S.selid[min(k, TOPK - 1u)]); /* lane k < 6: p of expert selid[k] */
            if (k < TOPK) S.selw[k] = ps;
        }
    } else {
        if (!gather_a()) return false;
        TLR(2u * (4u + 5u * l));
        if (UOCR_RUN_DN_EARLY) dd_load<QF>(R, S, dn);
        rms_defer(S.hres, nwp, S.xs, S.red, nullptr, nullptr);
        __syncthreads();
        inv = rms_inv(S.red);
    }
    const u32 nrows = moe ? GU_ROWS : min(DGU_ROWS, DI - min(b * DGU_ROWS, DI));
#pragma unroll
    for (u32 k = 0; k < G::RPG; ++k) {
        const u32 r = grp + k * G::NG;
        float pg = 0.0f, pu = 0.0f;
#pragma unroll
        for (u32 j = 0; j < G::J; ++j) {
            const u32 q = sub + G::LPR * j;
            const bool up = q >= G::C;
            const float d = chunk_dot<QF>(F.f[k].w[j], S.xs, up ? q - G::C : q);
            const float v = QF == 1 ? d : d * (float)F.f[k].s[j];
            pg += up ? 0.0f : v;
            pu += up ? v : 0.0f;
        }
        const float dg = group_sum<G::LPR>(pg) * inv;
        const float du = group_sum<G::LPR>(pu) * inv;
        if (sub == 0u && r < nrows) S.outv[r] = (h16)(fsilu(dg) * du);
    }
    constexpr u32 LG_W = 7u, LG_PER = (LG_COLS + LG_W - 1u) / LG_W; /* the 7 row wavefronts' shares */
    if (moe && UOCR_RUN_EXACT_WEIGHTS) {
        /* the reference's router input, rounded as it rounds it:
         * n[c] = f16(a[c] inv w[c]); this block's quarter of logit b / 4 =
         * sum_c R[b / 4][c] n[c] (the experts were chosen from z, the routing
         * weights come from these logits): wavefront w < 7 sums columns
         * [46 w, 46 w + 46) of the quarter, one per lane */
        static_assert(LG_PER <= 64u, "one column per lane");
        const u32 wave = __builtin_amdgcn_readfirstlane(tid_() / 64u), lane = tid_() % 64u;
        if (wave < LG_W) {
            const u32 k = wave * LG_PER + lane;
            float x = 0.0f;
            if (lane < LG_PER && k < LG_COLS) {
                const h16 *rw = (const h16 *)S.lgw, *nw = rw + LG_COLS;
                const h16 n = (h16)(((float)S.hres[(b % LG_Q) * LG_COLS + k] * inv) * (float)nw[k]);
                x = (float)n * (float)rw[k];
            }
            x = wave_sum(x);
            if (lane == 0u) S.zout[wave] = x;
        }
    }
    __syncthreads();
    TLD(l, 11u);
    publish(R, R.pk + off_mid(l), PMID, b * PMID_B, PMID_B, tag, [&](u32 p) {
        uint3 v = pay6(S.outv, p, moe ? GU_ROWS : nrows);
        if (moe && p == PMID_B - 1u && UOCR_RUN_EXACT_WEIGHTS) {
            float q = S.zout[0]; /* mids 28, 29 do not exist: the quarter, its 7 shares in order */
#pragma unroll
            for (u32 w = 1; w < LG_W; ++w) q += S.zout[w];
            v.z = __float_as_uint(q);
        }
        return v;
    });
    drain_stores(dn_in_lds<QF>() ? 8u : 0u, PMID_B); /* Q8 only: Q4 -0.7% */
    TLD(l, 19u);
    if (!UOCR_RUN_DN_EARLY) {
        /* the DN rows after this stage's own loads are consumed */
        if (moe) {
            dn_load<QF>(R, S, sd, dn);
        } else {
            dd_load<QF>(R, S, dn);
        }
    }
    TLD(l, 20u);
    TLR(2u * (4u + 5u * l) + 1u);
    return true;
}

/* DN stage: gathers the mids; MoE: out = f16(sum_r w_r D_r.mid_r + f16(SD.smid)
 * + a); layer 0: out = f16(D.mid + a). */
/* UOCR_RUN_QKV_EARLY: a DN block issues the next layer's QKV rows once its
 * mids are in, so they arrive during its dots; issued after the DN publish
 * (at the top of the next layer), they sat in front of its polls for h. */
#ifndef UOCR_RUN_QKV_EARLY
#define UOCR_RUN_QKV_EARLY 1
#endif
template <int QF, int QA>
__device__ bool dn_stage(const Run &R, const Lds &S, u32 l, int32_t t, u32 tag, DnFrags<QF> &dn, QkvFrags<QA> &qf) {
    typedef DnCfg<QF> G;
    const u32 b = blockIdx.x;
    if (b >= DN_BLOCKS) return true;
    const bool moe = l > 0u;
    const u32 rows_b = moe ? GU_ROWS : DGU_ROWS;
    const u32 nmid = moe ? TOPK * EI + SI : DI;
    h16 *mids = (h16 *)S.scr;
    float *lgp = (float *)(S.scr + (TOPK * EI + SI) * 2u); /* [256] the logit quarters */
    /* the selected experts (this block's GU stage), read before the gather */
    u32 sel[TOPK];
#pragma unroll
    for (u32 r = 0; r < TOPK; ++r) sel[r] = moe ? __builtin_amdgcn_readfirstlane(S.selid[r]) : 0u;
    static_assert((TOPK * EI + SI) * 2u + NB * 4u <= SCR_BYTES, "DN LDS");
    if (!gather<(PMID + NT - 1u) / NT>(R, R.pk + off_mid(l), PMID, PMID, tag, W_DN, (u32)t, [](u32 i) { return i; },
                        [&](u32 i, uint4 v) {
                            const u32 blk = i / PMID_B, k = i % PMID_B, base = mid_base(blk, moe) + 6u * k;
                            if (6u * k < rows_b) put6(mids + base, v, 6u * k, rows_b);
                            if (moe && k == PMID_B - 1u) lgp[blk] = __uint_as_float(v.w);
                            (void)nmid;
                        })) {
        return false;
    }
    TLR(2u * (5u + 5u * l));
#ifdef UOCR_RUN_TIMELINE
    if (l == 5u && tid_() == 0u) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        TLR(128u + 21u);
    }
#endif
    const u32 c = dn_row(), lane = tid_() & 63u, rl = c - b * DN_ROWS;
    /* the rows: registers, or this wavefront's LDS-direct loads */
    if (dn_in_lds<QF>()) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (UOCR_RUN_QKV_EARLY && l + 1u < UOCR_RUN_LAYERS) qkv_load<QA>(R, l + 1u, qf);
    const uint4 *dnw = S.dnw + (size_t)(tid_() >> 6) * G::J * 64u;
    auto dnrow = [&](u32 j) { return dn_in_lds<QF>() ? dnw[j * 64u + tid_() % 64u] : dn.w[dn_in_lds<QF>() ? 0u : j]; };
    float out;
    if (moe) {
        /* routing weights: every wavefront sums the logits (lane e: the four
         * quarters of logit e in order) and takes the raw softmax
         * probabilities of the selected experts (max-subtracted;
         * moe.metal:53-193) */
        float w6[TOPK];
        if (!UOCR_RUN_EXACT_WEIGHTS) {
#pragma unroll
            for (u32 r = 0; r < TOPK; ++r) w6[r] = S.selw[r];
        } else {
            const float4 q4 = ((const float4 *)lgp)[lane];
            const float lg = ((q4.x + q4.y) + q4.z) + q4.w;
            const float mx = wave_max_dpp(lg);
            const float pe = fexp(lg - mx);
            const float p = pe * frcp(wave_sum(pe));
#pragma unroll
            for (u32 r = 0; r < TOPK; ++r) w6[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), (int)sel[r]));
        }
        if (R.trace != nullptr && b == 0u && lane < TOPK && tid_() < 64u && (u32)t < R.trace_steps) {
            float mine = w6[0];
#pragma unroll
            for (u32 r = 1; r < TOPK; ++r) mine = lane == r ? w6[r] : mine;
            R.trace[((size_t)(R.trace_steps + (u32)t) * 11u + (l - 1u)) * TOPK + lane] = __float_as_uint(mine);
        }
        /* routed: sum over chunks of w_r * (scaled chunk dot); the shared
         * expert's sum kept apart (rounded to fp16 before the combine) */
        float acc = 0.0f, sh = 0.0f;
#pragma unroll
        for (u32 j = 0; j < G::J; ++j) {
            const u32 q = lane + 64u * j;
            if (64u * (j + 1u) <= G::CT || q < G::CT) {
                const u32 qq = min(q, G::CT - 1u);
                const bool routed = qq < TOPK * G::CR;
                const u32 r = routed ? qq / G::CR : 0u, cc = routed ? qq % G::CR : qq - TOPK * G::CR;
                const float d = chunk_dot<QF>(dnrow(j), mids + (routed ? r * EI : TOPK * EI), cc);
                const float v = QF == 1 ? d : d * (float)dn.s[j];
                if (q < G::CT) {
                    if (routed) {
                        float wr = w6[0];
#pragma unroll
                        for (u32 k = 1; k < TOPK; ++k) wr = r == k ? w6[k] : wr;
                        acc = fmaf(wr, v, acc);
                    } else {
                        sh += v;
                    }
                }
            }
        }
        acc = wave_sum(acc);
        sh = wave_sum(sh);
        out = acc + (float)(h16)sh + (float)S.hres[c];
    } else {
        float acc = 0.0f;
#pragma unroll
        for (u32 j = 0; j < G::JD; ++j) {
            const u32 q = lane + 64u * j;
            if (64u * (j + 1u) <= G::CD || q < G::CD) {
                const float dj = chunk_dot<QF>(dnrow(j), mids, min(q, G::CD - 1u));
                const float v = QF == 1 ? dj : dj * (float)dn.s[j];
                acc += q < G::CD ? v : 0.0f;
            }
        }
        const float d = wave_sum(acc);
        out = d + (float)S.hres[c];
    }
    TLD(l, 12u);
    if (lane == 0u) {
        S.outv[rl] = (h16)out;
        if (l + 1u == UOCR_RUN_LAYERS) R.hout[c] = (h16)out;
    }
    __syncthreads();
    publish(R, R.pk + off_h(l), PH, b * PH_B, PH_B, tag, [&](u32 p) { return pay6(S.outv, p, DN_ROWS); });
    drain_stores(16u, PH_B);
    TLR(2u * (5u + 5u * l) + 1u);
    return true;
}

/* ---- the run --------------------------------------------------------------- */

struct RunArgs {
    const uocr_run_model *M;
    uint4 *pk;
    h16 *kc, *vc;
    u32 cap;
    int32_t P, t0, n, last;
    u32 tag0;
    int32_t *tokens;
    float *scores;
    h16 *hout;
    u32 *trace;
    u32 trace_steps;
    const int32_t *force;
    u32 force_n;
};

template <int QA, int QF, int QL, int QE>
__global__ __launch_bounds__(NT, 1) void k_decode_run(RunArgs A) {
    __shared__ __attribute__((aligned(16))) h16 xs[HID];
    __shared__ __attribute__((aligned(16))) h16 hres[HID];
    __shared__ __attribute__((aligned(16))) h16 outv[64];
    __shared__ __attribute__((aligned(16))) uint8_t scr[SCR_BYTES];
    __shared__ float red[16], zout[64], selw[8];
    __shared__ __attribute__((aligned(16))) float zw[2u * Z_COLS * NEXP];
    __shared__ u32 selid[8];
    __shared__ unsigned long long keyw[NT / 64u];
    __shared__ float xsum[HID / 16u];
    __shared__ __attribute__((aligned(16))) uint8_t lgw[2u * LG_COLS * 2u];
    /* the DN rows (the Q8 instance; Q4 holds them in registers): with them
     * the block's LDS exceeds half a CU's 160 KB, so no CU can hold two run
     * workgroups whatever the register allocation (the run needs one
     * workgroup on each of the 256 CUs; Q4's 241 VGPRs at 512 threads fill a
     * CU's register file) */
    __shared__ __attribute__((aligned(16))) uint4 dnw[DN_ROWS * DnCfg<QF>::J * 64u];
    Lds S{xs, hres, outv, red, zout, selw, zw, selid, keyw, scr, xsum, lgw, dnw};
    Run R;
    R.M = (const AS4 RunModelD *)A.M;
    R.pk = A.pk;
    R.ctl = (u32 *)A.pk;
    R.kc = A.kc;
    R.vc = A.vc;
    R.cap = A.cap;
    R.xcc = (u32)__builtin_amdgcn_s_getreg(20 | (3 << 11)) % NREP; /* HW_REG_XCC_ID */
    R.P = A.P;
    R.tokens = A.tokens;
    R.scores = A.scores;
    R.hout = A.hout;
    R.trace = A.trace;
    R.trace_steps = A.trace_steps;
    R.force = A.force;
    R.force_n = A.force_n;
    R.tl = nullptr;

    RowFrag<LmCfg<QL>::J> lf[LM_DEPTH];
#pragma unroll 1
    for (int32_t i = 0; i < A.n; ++i) {
        const int32_t t = A.t0 + i;
        const u32 tag = A.tag0 + (u32)i;
#ifdef UOCR_RUN_TIMELINE
        R.tl = t == g_run_tl_step ? g_run_tl : nullptr;
        TLR(127u);
#endif
#pragma unroll
        for (u32 k = 0; k < LM_DEPTH; ++k) lm_load<QL>(R, lf[k], k);
        if (!lm_stage<QL>(R, S, tag, tag - 1u, t, lf)) return;
        if (A.last && i == A.n - 1) {
            if (blockIdx.x == 0u) {
                int32_t tok;
                float score;
                if (!select_token(R, S, tag, t, tok, score)) return;
                if (tid_() == 0u) {
                    R.tokens[t] = tok;
                    if (R.scores != nullptr) R.scores[t] = score;
                }
            }
            return;
        }
        QkvFrags<QA> qf;
#pragma unroll 1
        for (u32 l = 0; l < UOCR_RUN_LAYERS; ++l) {
            /* the DN blocks issued this layer's QKV rows in their DN stage */
            if (!(UOCR_RUN_QKV_EARLY && l > 0u && blockIdx.x < DN_BLOCKS)) qkv_load<QA>(R, l, qf);
            AttFrags af;
            if (blockIdx.x >= ATT0) att_load(R, l, att_plan(R, t), 0u, af);
            if (!qkv_stage<QA, QE>(R, S, l, t, tag, qf)) return;
            OFrags<QA> of;
            o_load<QA>(R, l, of);
            if (!att_stage(R, S, l, t, tag, af)) return;
            GuFrags<QF> gf;
            DnFrags<QF> dn;
            gu_load_static<QF>(R, l, gf);
            o_load_z(R, l, S.zw);
            if (!o_stage<QA>(R, S, l, t, tag, of)) return;
            if (!gu_stage<QF>(R, S, l, t, tag, gf, dn)) return;
            if (!dn_stage<QF, QA>(R, S, l, t, tag, dn, qf)) return;
        }
    }
}

/* Layer 11's output slot of h with the given tag (DN packet layout). */
__global__ __launch_bounds__(NT) void k_run_seed(uint4 *pk, const h16 *__restrict__ h, u32 tag) {
    const u32 t = blockIdx.x * NT + tid_();
    if (t >= PH * NREP) return;
    const u32 p = t % PH, r = t / PH;
    const u32 base = (p / 2u) * DN_ROWS + (p % 2u) * 6u;
    h16 e[6];
#pragma unroll
    for (u32 j = 0; j < 6u; ++j) e[j] = (p % 2u) * 6u + j < DN_ROWS ? h[base + j] : (h16)0.0f;
    pk[off_h(UOCR_RUN_LAYERS - 1u) + (u64)r * PH + p] =
        make_uint4(tag, pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]));
}

/* fold_o[c][e] = sum_r fold[r][e] * O[r][c]: thread (c, e), rows in order. */
template <int QT>
__global__ __launch_bounds__(256) void k_fold_o(const uint8_t *__restrict__ ow, const h16 *__restrict__ os,
                                                const float *__restrict__ fold, float *__restrict__ out) {
    const u32 c = blockIdx.x * 4u + threadIdx.x / 64u, e = threadIdx.x % 64u;
    float acc = 0.0f;
    for (u32 r = 0; r < HID; ++r) {
        float w;
        if (QT == 1) {
            w = (float)((const h16 *)ow)[(size_t)r * HID + c];
        } else if (QT == 3) {
            w = (float)(int8_t)ow[(size_t)r * HID + c] * (float)os[(size_t)r * (HID / 64u) + c / 64u];
        } else {
            const uint8_t byte = ow[(size_t)r * (HID / 2u) + (c / 64u) * 32u + (c % 32u)];
            const int q = (int)((c % 64u) < 32u ? (byte & 15u) : (byte >> 4)) - 8;
            w = (float)q * (float)os[(size_t)r * (HID / 64u) + c / 64u];
        }
        acc = fmaf(fold[(size_t)r * NEXP + e], w, acc);
    }
    out[(size_t)c * NEXP + e] = acc;
}

__global__ void k_run_reset(u32 *ctl) {
    if (tid_() < 64u) ctl[tid_()] = 0u;
}

/* An ordinary launch: the run needs its 256 workgroups resident together
 * (one per CU: 512 threads at 256 VGPRs fill a CU's register file, and the
 * block's LDS is above half a CU's), which an otherwise idle device gives;
 * it uses none of the cooperative launch's grid synchronisation.  A
 * workgroup that never gets a CU shows as a bounded wait that gives up, and
 * the request is served again on the per-step kernels.  (The cooperative
 * launch was replaced because every profiled process that made one ended in
 * a segmentation fault in an exit handler after the profiler's
 * finalisation, while profiled processes without one exited cleanly.) */
template <int QA, int QF, int QL, int QE>
hipError_t launch_run(hipStream_t st, const RunArgs &a) {
    hipLaunchKernelGGL((k_decode_run<QA, QF, QL, QE>), dim3(NB), dim3(NT), 0, st, a);
    return hipGetLastError();
}

}  // namespace

#ifdef UOCR_RUN_TIMELINE
/* Records the stage timeline of decode step `step` into buf
 * (256 x 256 u64, see g_run_tl); NULL stops recording. */
extern "C" __attribute__((visibility("default"))) int uocr_run_timeline(void *buf, int step) {
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_run_tl), &buf, sizeof(buf)) != hipSuccess) return -1;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_run_tl_step), &step, sizeof(step)) != hipSuccess) return -1;
    return hipDeviceSynchronize() == hipSuccess ? 0 : -1;
}
#endif

extern "C" uint64_t uocr_run_arena_bytes(void) {
    return ARENA_PK * 16u;
}

extern "C" int uocr_run_supported(const uocr_run_model *m) {
    if (m == nullptr) return 0;
    return m->qa == UOCR_QT_Q8 && m->ql == m->qf && m->qe == m->qf && (m->qf == UOCR_QT_Q4 || m->qf == UOCR_QT_Q8);
}

extern "C" hipError_t uocr_run_fold_o(hipStream_t st, uint32_t qtype, const void *ow, const uint16_t *os,
                                      const float *fold, float *out) {
    if (ow == nullptr || fold == nullptr || out == nullptr || (qtype != UOCR_QT_F16 && os == nullptr)) {
        return hipErrorInvalidValue;
    }
    const dim3 grid(HID / 4u), block(256u);
    const uint8_t *w = (const uint8_t *)ow;
    const h16 *s = (const h16 *)os;
    switch (qtype) {
    case UOCR_QT_F16: hipLaunchKernelGGL(k_fold_o<1>, grid, block, 0, st, w, s, fold, out); break;
    case UOCR_QT_Q8: hipLaunchKernelGGL(k_fold_o<3>, grid, block, 0, st, w, s, fold, out); break;
    case UOCR_QT_Q4: hipLaunchKernelGGL(k_fold_o<4>, grid, block, 0, st, w, s, fold, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

extern "C" hipError_t uocr_run_seed(hipStream_t st, void *arena, const uint16_t *h, uint32_t tag) {
    if (arena == nullptr || h == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_run_seed, dim3((PH * NREP + NT - 1u) / NT), dim3(NT), 0, st, (uint4 *)arena, (const h16 *)h, tag);
    return hipGetLastError();
}

extern "C" hipError_t uocr_run_reset(hipStream_t st, void *arena) {
    if (arena == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_run_reset, dim3(1), dim3(64), 0, st, (u32 *)arena);
    return hipGetLastError();
}

extern "C" hipError_t uocr_run_launch(hipStream_t st, const uocr_run_model *model, const uocr_run_model *host_model,
                                      void *arena, uint16_t *kc, uint16_t *vc, uint32_t cap, int32_t P, int32_t t0,
                                      int32_t n, int last, uint32_t tag0, int32_t *tokens, float *scores,
                                      uint16_t *hidden, uint32_t *trace, uint32_t trace_steps, const int32_t *force,
                                      uint32_t force_n) {
    if (model == nullptr || host_model == nullptr || arena == nullptr || kc == nullptr || vc == nullptr ||
        tokens == nullptr || hidden == nullptr || (trace == nullptr && trace_steps != 0u) || n <= 0 || n > (int32_t)UOCR_RUN_MAX_STEPS || P <= 0 || t0 < 0 ||
        cap < (uint32_t)P + RING || !uocr_run_supported(host_model)) {
        return hipErrorInvalidValue;
    }
    /* byte offsets of one layer's cache fit the 32-bit buffer offsets */
    if ((uint64_t)NHEAD * cap * HDIM * 2u >= (1ull << 31)) return hipErrorInvalidValue;
    RunArgs a;
    a.M = model;
    a.pk = (uint4 *)arena;
    a.kc = (h16 *)kc;
    a.vc = (h16 *)vc;
    a.cap = cap;
    a.P = P;
    a.t0 = t0;
    a.n = n;
    a.last = last;
    a.tag0 = tag0;
    a.tokens = tokens;
    a.scores = scores;
    a.hout = (h16 *)hidden;
    a.trace = trace;
    a.trace_steps = trace_steps;
    a.force = force_n != 0u ? force : nullptr;
    a.force_n = force_n;
    if (host_model->qf == UOCR_QT_Q4) return launch_run<3, 4, 4, 4>(st, a);
    return launch_run<3, 3, 3, 3>(st, a);
}
