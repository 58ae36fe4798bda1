/*
 * uocr_synth.h - deterministic synthetic .uocr model builder.
 *
 * Plays the role of the reference's test model writer
 * (tests/uocr_test_model_file.h: tiny valid .uocr files without real
 * weights), at the real decoder shape, so the full decode loop can run and be
 * checked without the 1.8-6.7 GB converted checkpoints.  The image holds a
 * config record equal to the model constants, a sorted tensor directory and
 * page-aligned tensor data for every decoder tensor (no vision tensors).
 *
 * Values: Q8_0 q ~ U[-127,127] with fp16 scales
 * |N(0,0.02)|/127; Q4_0 q ~ U[-7,7] (inside int4 [-8,7], zero mean: a -0.5
 * mean code with positive scales biases every row and the bias compounds
 * through the residual stream) with fp16 scales |N(0,0.02)|/7; fp16 linear weights ~ N(0,0.01); norm weights ~ U[0.8,1.2];
 * router fp16 ~ N(0,0.03).  Every tensor draws from its own stream seeded by
 * (seed, tensor id, row block), so the bytes do not depend on thread count.
 *
 * qprofile: 1 = fp16, 2 = mixed-q8_0 (every quantisable decoder tensor Q8_0),
 * 3 = mixed-q4 (attention Q8_0; embedding, LM head, dense, shared and routed
 * experts Q4_0), as configs/quant-cfg.yaml gates them.
 */
#ifndef UOCR_SYNTH_H
#define UOCR_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#include "unlimitedocr.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Builds the image in a malloc'd buffer (free with uocr_synth_free). */
UOCR_API int uocr_synth_model_build(uint32_t qprofile, uint64_t seed, void **out_data, size_t *out_size);
UOCR_API int uocr_synth_model_write(const char *path, uint32_t qprofile, uint64_t seed);
UOCR_API void uocr_synth_free(void *data);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_SYNTH_H */
