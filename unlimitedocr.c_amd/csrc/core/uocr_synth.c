/* uocr_synth.c - deterministic synthetic .uocr images (see uocr_synth.h). */
#include "uocr_synth.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "uocr_convert.h"
#include "uocr_format.h"
#include "uocr_half.h"

#define ROW_BLOCK 64u

typedef struct synth_tensor {
    uint32_t id, family, projection, qtype, rank, rows, cols;
    int32_t layer, expert;
    uint32_t kind; /* 0 linear weight, 1 norm, 2 router */
    uint64_t w_off, w_bytes, s_off, s_bytes;
} synth_tensor;

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static uint64_t next64(uint64_t *s) {
    *s += 0x9e3779b97f4a7c15ull;
    return mix64(*s);
}

static double unif(uint64_t *s) {
    return ((double)(next64(s) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

static double gauss(uint64_t *s) {
    const double u1 = unif(s), u2 = unif(s);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static uint32_t qtype_for(uint32_t qprofile, uint32_t family) {
    if (qprofile == UOCR_QPROFILE_FP16) return UOCR_TENSOR_F16;
    if (family == UOCR_TENSOR_FAMILY_FINAL_NORM || family == UOCR_TENSOR_FAMILY_LAYER_NORM ||
        family == UOCR_TENSOR_FAMILY_MOE_ROUTER) {
        return UOCR_TENSOR_F16;
    }
    if (qprofile == UOCR_QPROFILE_MIXED_Q8_0 || family == UOCR_TENSOR_FAMILY_LAYER_ATTN) return UOCR_TENSOR_Q8_0;
    return UOCR_TENSOR_Q4_0;
}

static uint32_t add(synth_tensor *t, uint32_t n, uint32_t qprofile, uint32_t id, uint32_t family, uint32_t proj,
                    int32_t layer, int32_t expert, uint32_t rank, uint32_t rows, uint32_t cols, uint32_t kind) {
    synth_tensor *x = &t[n];
    memset(x, 0, sizeof(*x));
    x->id = id;
    x->family = family;
    x->projection = proj;
    x->layer = layer;
    x->expert = expert;
    x->rank = rank;
    x->rows = rows;
    x->cols = cols;
    x->kind = kind;
    x->qtype = qtype_for(qprofile, family);
    return n + 1u;
}

static uint32_t plan(uint32_t qprofile, synth_tensor *t) {
    const uint32_t H = UOCR_HIDDEN_SIZE, V = UOCR_VOCAB_SIZE;
    uint32_t n = 0;
    n = add(t, n, qprofile, UOCR_TID_TOK_EMBED, UOCR_TENSOR_FAMILY_TOK_EMBED, UOCR_TENSOR_PROJ_WEIGHT, -1, -1, 2, V, H, 0);
    n = add(t, n, qprofile, UOCR_TID_LM_HEAD, UOCR_TENSOR_FAMILY_LM_HEAD, UOCR_TENSOR_PROJ_WEIGHT, -1, -1, 2, V, H, 0);
    n = add(t, n, qprofile, UOCR_TID_FINAL_NORM, UOCR_TENSOR_FAMILY_FINAL_NORM, UOCR_TENSOR_PROJ_WEIGHT, -1, -1, 1, 1, H, 1);
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        const int32_t L = (int32_t)l;
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_INPUT_NORM), UOCR_TENSOR_FAMILY_LAYER_NORM, UOCR_TENSOR_PROJ_WEIGHT, L, -1, 1, 1, H, 1);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_POST_ATTN_NORM), UOCR_TENSOR_FAMILY_LAYER_NORM, UOCR_TENSOR_PROJ_WEIGHT, L, -1, 1, 1, H, 1);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_ATTN_Q), UOCR_TENSOR_FAMILY_LAYER_ATTN, UOCR_TENSOR_PROJ_Q, L, -1, 2, H, H, 0);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_ATTN_K), UOCR_TENSOR_FAMILY_LAYER_ATTN, UOCR_TENSOR_PROJ_K, L, -1, 2, H, H, 0);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_ATTN_V), UOCR_TENSOR_FAMILY_LAYER_ATTN, UOCR_TENSOR_PROJ_V, L, -1, 2, H, H, 0);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_ATTN_O), UOCR_TENSOR_FAMILY_LAYER_ATTN, UOCR_TENSOR_PROJ_O, L, -1, 2, H, H, 0);
        if (l == 0u) {
            const uint32_t I = UOCR_DENSE_LAYER0_INTERMEDIATE;
            n = add(t, n, qprofile, uocr_tid_layer(0, UOCR_TID_L_DENSE_GATE), UOCR_TENSOR_FAMILY_LAYER_DENSE_MLP, UOCR_TENSOR_PROJ_GATE, 0, -1, 2, I, H, 0);
            n = add(t, n, qprofile, uocr_tid_layer(0, UOCR_TID_L_DENSE_UP), UOCR_TENSOR_FAMILY_LAYER_DENSE_MLP, UOCR_TENSOR_PROJ_UP, 0, -1, 2, I, H, 0);
            n = add(t, n, qprofile, uocr_tid_layer(0, UOCR_TID_L_DENSE_DOWN), UOCR_TENSOR_FAMILY_LAYER_DENSE_MLP, UOCR_TENSOR_PROJ_DOWN, 0, -1, 2, H, I, 0);
            continue;
        }
        const uint32_t SI = UOCR_MOE_SHARED_INTERMEDIATE, EI = UOCR_MOE_EXPERT_INTERMEDIATE;
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_MOE_ROUTER), UOCR_TENSOR_FAMILY_MOE_ROUTER, UOCR_TENSOR_PROJ_WEIGHT, L, -1, 2, UOCR_ROUTED_EXPERTS, H, 2);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_SHARED_GATE), UOCR_TENSOR_FAMILY_MOE_SHARED, UOCR_TENSOR_PROJ_GATE, L, -1, 2, SI, H, 0);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_SHARED_UP), UOCR_TENSOR_FAMILY_MOE_SHARED, UOCR_TENSOR_PROJ_UP, L, -1, 2, SI, H, 0);
        n = add(t, n, qprofile, uocr_tid_layer(l, UOCR_TID_L_SHARED_DOWN), UOCR_TENSOR_FAMILY_MOE_SHARED, UOCR_TENSOR_PROJ_DOWN, L, -1, 2, H, SI, 0);
        for (uint32_t e = 0; e < UOCR_ROUTED_EXPERTS; ++e) {
            n = add(t, n, qprofile, uocr_tid_expert(l, e, 0), UOCR_TENSOR_FAMILY_MOE_EXPERT, UOCR_TENSOR_PROJ_GATE, L, (int32_t)e, 2, EI, H, 0);
            n = add(t, n, qprofile, uocr_tid_expert(l, e, 1), UOCR_TENSOR_FAMILY_MOE_EXPERT, UOCR_TENSOR_PROJ_UP, L, (int32_t)e, 2, EI, H, 0);
            n = add(t, n, qprofile, uocr_tid_expert(l, e, 2), UOCR_TENSOR_FAMILY_MOE_EXPERT, UOCR_TENSOR_PROJ_DOWN, L, (int32_t)e, 2, H, EI, 0);
        }
    }
    return n;
}

static uint64_t up(uint64_t v, uint64_t a) {
    return (v + a - 1u) / a * a;
}

/* Fills rows [r0, r1) of tensor t. */
static void fill_block(uint8_t *img, const synth_tensor *t, uint32_t r0, uint32_t r1, uint64_t seed) {
    uint64_t s = mix64(seed ^ mix64(((uint64_t)t->id << 20) ^ r0));
    const uint32_t K = t->cols;
    if (t->qtype == UOCR_TENSOR_F16) {
        uint16_t *w = (uint16_t *)(void *)(img + t->w_off);
        for (uint32_t r = r0; r < r1; ++r) {
            for (uint32_t c = 0; c < K; ++c) {
                float v;
                if (t->kind == 1u) {
                    v = (float)(0.8 + 0.4 * unif(&s));
                } else {
                    const uint64_t u = next64(&s);
                    /* Irwin-Hall(4) approximation of N(0,1) */
                    const double g = ((double)(u & 0xffffu) + (double)((u >> 16) & 0xffffu) + (double)((u >> 32) & 0xffffu) +
                                      (double)(u >> 48)) / 65536.0 - 2.0;
                    v = (float)(g * 1.7320508075688772 * (t->kind == 2u ? 0.03 : 0.01));
                }
                w[(size_t)r * K + c] = uocr_half_bits(v);
            }
        }
        return;
    }
    const uint32_t row_bytes = t->qtype == UOCR_TENSOR_Q8_0 ? K : K / 2u;
    uint8_t *w = img + t->w_off + (size_t)r0 * row_bytes;
    const size_t nbytes = (size_t)(r1 - r0) * row_bytes;
    if (t->qtype == UOCR_TENSOR_Q8_0) {
        /* q = ((b * 255) >> 8) - 127 for a uniform byte b: q in [-127, 127] */
        for (size_t i = 0; i < nbytes; i += 8u) {
            uint64_t v = next64(&s);
            for (size_t j = 0; j < 8u && i + j < nbytes; ++j, v >>= 8) {
                w[i + j] = (uint8_t)(int8_t)((int)(((uint32_t)(v & 0xffu) * 255u) >> 8) - 127);
            }
        }
    } else {
        /* q = ((u16 * 15) >> 16) - 7 in [-7, 7] (zero mean), stored as the
         * nibble q + 8; two nibbles per byte, 16 random bits per nibble */
        for (size_t i = 0; i < nbytes; i += 2u) {
            uint64_t v = next64(&s);
            for (size_t j = 0; j < 2u && i + j < nbytes; ++j) {
                const uint32_t lo = (uint32_t)(((v & 0xffffu) * 15u) >> 16) + 1u;
                const uint32_t hi = (uint32_t)((((v >> 16) & 0xffffu) * 15u) >> 16) + 1u;
                w[i + j] = (uint8_t)(lo | (hi << 4));
                v >>= 32;
            }
        }
    }
    uint16_t *sc = (uint16_t *)(void *)(img + t->s_off);
    const uint32_t G = K / UOCR_QGROUP;
    const double div = t->qtype == UOCR_TENSOR_Q8_0 ? 127.0 : 7.0;
    for (uint32_t r = r0; r < r1; ++r) {
        for (uint32_t g = 0; g < G; ++g) sc[(size_t)r * G + g] = uocr_half_bits((float)(fabs(gauss(&s) * 0.02) / div));
    }
}

/* The image of qprofile; with fill, every tensor takes its seeded synthetic
 * values, else the tensor data stays zero (the converter's skeleton). */
static int build_image(uint32_t qprofile, uint64_t seed, int fill, void **out_data, size_t *out_size) {
    if (out_data == NULL || out_size == NULL) return UOCR_ERROR_INVALID_ARGUMENT;
    *out_data = NULL;
    *out_size = 0u;
    if (qprofile != UOCR_QPROFILE_FP16 && qprofile != UOCR_QPROFILE_MIXED_Q8_0 && qprofile != UOCR_QPROFILE_MIXED_Q4) {
        return UOCR_ERROR_INVALID_ARGUMENT;
    }
    const uint32_t max_t = 3u + UOCR_DECODER_LAYERS * (6u + 4u + 3u * UOCR_ROUTED_EXPERTS);
    synth_tensor *t = (synth_tensor *)calloc(max_t, sizeof(synth_tensor));
    if (t == NULL) return UOCR_ERROR_OUT_OF_MEMORY;
    const uint32_t n = plan(qprofile, t);
    const uint64_t dir_off = 512u;
    const uint64_t dir_size = sizeof(uocr_tensor_directory_header) + (uint64_t)n * sizeof(uocr_tensor_entry);
    const uint64_t data_off = up(dir_off + dir_size, UOCR_TENSOR_DATA_ALIGNMENT);
    for (uint32_t i = 0; i < n; ++i) {
        const uint64_t elems = (uint64_t)t[i].rows * t[i].cols;
        if (t[i].qtype == UOCR_TENSOR_F16) {
            t[i].w_bytes = elems * 2u;
        } else {
            t[i].w_bytes = t[i].qtype == UOCR_TENSOR_Q8_0 ? elems : elems / 2u;
            t[i].s_bytes = (uint64_t)t[i].rows * (t[i].cols / UOCR_QGROUP) * 2u;
        }
    }
    /* the reference converter's tensor-data layout (convert.py:928-1036):
     * tensors in id order, payload then scales on 256-byte boundaries; the
     * quantised routed experts of a layer form one group whose payloads are
     * all laid out first, then all its scales */
    uint64_t off = data_off;
    for (uint32_t i = 0; i < n;) {
        uint32_t end = i + 1u;
        if (t[i].family == UOCR_TENSOR_FAMILY_MOE_EXPERT && t[i].qtype != UOCR_TENSOR_F16) {
            while (end < n && t[end].family == UOCR_TENSOR_FAMILY_MOE_EXPERT && t[end].layer == t[i].layer &&
                   t[end].qtype == t[i].qtype) {
                ++end;
            }
        }
        for (uint32_t j = i; j < end; ++j) {
            off = up(off, 256u);
            t[j].w_off = off;
            off += t[j].w_bytes;
        }
        for (uint32_t j = i; j < end; ++j) {
            if (t[j].s_bytes == 0u) continue;
            off = up(off, 256u);
            t[j].s_off = off;
            off += t[j].s_bytes;
        }
        i = end;
    }
    const uint64_t total = up(off, UOCR_FILE_ALIGNMENT);
    uint8_t *img = (uint8_t *)calloc(1, total);
    if (img == NULL) {
        free(t);
        return UOCR_ERROR_OUT_OF_MEMORY;
    }
    uocr_file_header *h = (uocr_file_header *)(void *)img;
    memcpy(h->magic, UOCR_FILE_MAGIC, 4);
    h->version = UOCR_FORMAT_VERSION;
    h->header_size = sizeof(uocr_file_header);
    h->endian_marker = UOCR_ENDIAN_MARKER;
    h->required_alignment = UOCR_FILE_ALIGNMENT;
    h->qprofile = qprofile;
    h->section_count = 3u;
    h->file_size = total;
    h->section_dir_offset = 128u;
    for (int i = 0; fill && i < 32; ++i) h->model_id_hash[i] = (uint8_t)(mix64(seed + (uint64_t)i) & 0xffu);
    uocr_section_entry *sec = (uocr_section_entry *)(void *)(img + 128u);
    sec[0].type = UOCR_SECTION_CONFIG;
    sec[0].offset = 256u;
    sec[0].size = sizeof(uocr_config_record);
    sec[0].alignment = 8u;
    sec[1].type = UOCR_SECTION_TENSOR_DIRECTORY;
    sec[1].offset = dir_off;
    sec[1].size = dir_size;
    sec[1].alignment = 8u;
    sec[2].type = UOCR_SECTION_TENSOR_DATA;
    sec[2].offset = data_off;
    sec[2].size = total - data_off;
    sec[2].alignment = UOCR_TENSOR_DATA_ALIGNMENT;
    const uint32_t cfg[27] = {UOCR_VOCAB_SIZE, UOCR_BPE_VOCAB_SIZE, UOCR_ADDED_TOKEN_COUNT, (uint32_t)UOCR_TOKEN_BOS,
                              (uint32_t)UOCR_TOKEN_EOS, (uint32_t)UOCR_TOKEN_PAD, (uint32_t)UOCR_TOKEN_IMAGE,
                              UOCR_HIDDEN_SIZE, UOCR_DECODER_LAYERS, UOCR_ATTENTION_HEADS, UOCR_KV_HEADS, UOCR_HEAD_DIM,
                              UOCR_ROPE_THETA, UOCR_MAX_POSITIONS, UOCR_GENERATED_RING_WINDOW, UOCR_DENSE_FIRST_LAYERS,
                              UOCR_ROUTED_EXPERTS, UOCR_MOE_TOP_K, UOCR_MOE_EXPERT_INTERMEDIATE, UOCR_MOE_SHARED_EXPERTS,
                              UOCR_DENSE_LAYER0_INTERMEDIATE, UOCR_PROJECTOR_IN_SIZE, UOCR_HIDDEN_SIZE,
                              UOCR_VISION_PATCH_SIZE, UOCR_DOWNSAMPLE_RATIO, UOCR_GLOBAL_VIEW_SIZE, UOCR_LOCAL_VIEW_SIZE};
    memcpy(img + 256u, cfg, sizeof(cfg));
    uocr_tensor_directory_header *dh = (uocr_tensor_directory_header *)(void *)(img + dir_off);
    dh->magic = UOCR_TENSOR_DIR_MAGIC;
    dh->version = UOCR_FORMAT_VERSION;
    dh->entry_size = sizeof(uocr_tensor_entry);
    dh->tensor_count = n;
    uocr_tensor_entry *ents = (uocr_tensor_entry *)(void *)(img + dir_off + sizeof(*dh));
    for (uint32_t i = 0; i < n; ++i) {
        uocr_tensor_entry *e = &ents[i];
        e->id = t[i].id;
        e->family = t[i].family;
        e->layer = t[i].layer;
        e->expert = t[i].expert;
        e->projection = t[i].projection;
        e->usage = UOCR_TENSOR_USAGE_RUNTIME;
        e->qtype = t[i].qtype;
        e->flags = UOCR_TENSOR_FLAG_ROW_MAJOR;
        e->rank = t[i].rank;
        if (t[i].rank == 1u) {
            e->logical_shape[0] = e->physical_shape[0] = t[i].cols;
        } else {
            e->logical_shape[0] = e->physical_shape[0] = t[i].rows;
            e->logical_shape[1] = e->physical_shape[1] = t[i].cols;
        }
        e->payload_offset = t[i].w_off;
        e->payload_size = t[i].w_bytes;
        if (t[i].qtype != UOCR_TENSOR_F16) {
            e->block_size = UOCR_QGROUP;
            e->row_size = t[i].qtype == UOCR_TENSOR_Q8_0 ? t[i].cols : t[i].cols / 2u;
            e->scale_offset = t[i].s_off;
            e->scale_size = t[i].s_bytes;
        }
    }
    if (!fill) {
        free(t);
        *out_data = img;
        *out_size = (size_t)total;
        return UOCR_OK;
    }
    /* value fill: one task per (tensor, 64-row block) */
    uint64_t ntask = 0;
    for (uint32_t i = 0; i < n; ++i) ntask += (t[i].rows + ROW_BLOCK - 1u) / ROW_BLOCK;
    uint32_t *task_t = (uint32_t *)malloc(sizeof(uint32_t) * ntask);
    uint32_t *task_r = (uint32_t *)malloc(sizeof(uint32_t) * ntask);
    if (task_t == NULL || task_r == NULL) {
        free(task_t);
        free(task_r);
        free(t);
        free(img);
        return UOCR_ERROR_OUT_OF_MEMORY;
    }
    uint64_t k = 0;
    for (uint32_t i = 0; i < n; ++i) {
        for (uint32_t r = 0; r < t[i].rows; r += ROW_BLOCK) {
            task_t[k] = i;
            task_r[k] = r;
            ++k;
        }
    }
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t q = 0; q < (int64_t)ntask; ++q) {
        const synth_tensor *x = &t[task_t[q]];
        const uint32_t r0 = task_r[q];
        const uint32_t r1 = r0 + ROW_BLOCK < x->rows ? r0 + ROW_BLOCK : x->rows;
        fill_block(img, x, r0, r1, seed);
    }
    free(task_t);
    free(task_r);
    free(t);
    *out_data = img;
    *out_size = (size_t)total;
    return UOCR_OK;
}

int uocr_synth_model_build(uint32_t qprofile, uint64_t seed, void **out_data, size_t *out_size) {
    return build_image(qprofile, seed, 1, out_data, out_size);
}

int uocr_image_skeleton_build(uint32_t qprofile, void **out_data, size_t *out_size) {
    return build_image(qprofile, 0u, 0, out_data, out_size);
}

int uocr_synth_model_write(const char *path, uint32_t qprofile, uint64_t seed) {
    if (path == NULL) return UOCR_ERROR_INVALID_ARGUMENT;
    void *data = NULL;
    size_t size = 0;
    const int st = uocr_synth_model_build(qprofile, seed, &data, &size);
    if (st != UOCR_OK) return st;
    FILE *f = fopen(path, "wb");
    int ok = f != NULL && fwrite(data, 1, size, f) == size;
    if (f != NULL && fclose(f) != 0) ok = 0;
    free(data);
    return ok ? UOCR_OK : UOCR_ERROR_INTERNAL;
}

void uocr_synth_free(void *data) {
    free(data);
}
