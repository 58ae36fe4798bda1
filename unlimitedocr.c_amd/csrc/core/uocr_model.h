/*
 * uocr_model.h - .uocr reader, validator and decoder tensor binding.
 *
 * Validation follows the reference loader's rules
 * (src/model/uocr_model_file.c:324-1125: header, section directory, config
 * equality with the model constants, optional tokenizer/provenance records,
 * tensor directory with per-qtype size/alignment/range checks and the Q4
 * family allow-list :716-725).  Binding applies the runtime qtype allow-list
 * of the reference GPU backend (src/backend/metal/uocr_metal.m:2728-2763):
 * Q4 only for TOK_EMBED, LM_HEAD, dense MLP, shared and routed experts; Q8
 * also for attention; norms and the router stay fp16.  A tensor outside the
 * allow-list fails at bind time; there is no silent fallback.
 */
#ifndef UOCR_MODEL_H
#define UOCR_MODEL_H

#include <stddef.h>
#include <stdint.h>

#include "uocr_format.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct uocr_model_file {
    const uint8_t *data;
    size_t size;
    uint8_t *owned;                 /* non-NULL when the loader owns the bytes */
    const uocr_file_header *header;
    const uocr_section_entry *sections;
    const uocr_config_record *config;
    const uocr_tensor_entry *tensors;
    uint32_t tensor_count;
    uint64_t tensor_data_bytes;
} uocr_model_file;

int uocr_model_open_path(const char *path, uocr_model_file *out, char *err, size_t err_size);
/* Validates an in-memory image; the caller keeps `data` alive while open. */
int uocr_model_open_memory(const void *data, size_t size, uocr_model_file *out, char *err, size_t err_size);
void uocr_model_close(uocr_model_file *m);
const uocr_tensor_entry *uocr_model_find(const uocr_model_file *m, uint32_t id);
const char *uocr_qprofile_name(uint32_t qprofile);
const char *uocr_qtype_name(uint32_t qtype);

/* One bound decoder tensor: host bytes of payload and scales. */
typedef struct uocr_bound_tensor {
    uint32_t qtype;
    uint32_t rows, cols;
    const uint8_t *w;
    uint64_t w_bytes;
    const uint8_t *s;
    uint64_t s_bytes;
} uocr_bound_tensor;

typedef struct uocr_bound_layer {
    uocr_bound_tensor in_norm, post_norm, q, k, v, o;
    uocr_bound_tensor gate, up, down;               /* layer 0 dense MLP */
    uocr_bound_tensor router, sgate, sup, sdown;    /* MoE layers */
    uocr_bound_tensor egate[UOCR_ROUTED_EXPERTS], eup[UOCR_ROUTED_EXPERTS], edown[UOCR_ROUTED_EXPERTS];
} uocr_bound_layer;

typedef struct uocr_decoder_bindings {
    uocr_bound_tensor embed, lm_head, final_norm;
    uocr_bound_layer layers[UOCR_DECODER_LAYERS];
    uint64_t total_bytes;
} uocr_decoder_bindings;

/* Returns 0 on success, -1 with err set when a decoder tensor is missing, has
 * the wrong shape, or a qtype outside the allow-list. */
int uocr_bind_decoder(const uocr_model_file *m, uocr_decoder_bindings *out, char *err, size_t err_size);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_MODEL_H */
