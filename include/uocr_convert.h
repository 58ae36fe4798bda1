/*
 * uocr_convert.h - .uocr decoder image writing: the quantisers and the file
 * skeleton the converter (unlimitedocr.c_amd/uocr_convert.py) fills.
 *
 * The reference converts Hugging Face checkpoints in Python
 * (src/unlimitedocr_c/convert.py); this library carries the two pieces of
 * that path that decide bytes on disk:
 *  - uocr_quantize_rows: fp32 rows -> f16 / Q8_0 / Q4_0 payload + fp16
 *    group-64 scales, bit-identical to convert.py's numpy quantisers
 *    (Q8_0 :2058-2063, Q4_0 _quantize_q4_0_rows :2249-2276, f16 :1992-2016);
 *  - uocr_image_skeleton_build: a zero-filled image with the file header,
 *    config record, tensor directory and the reference's tensor-data layout
 *    (_layout_dry_run_file, convert.py:928-1036: tensors in id order, each
 *    payload then its scales on 256-byte boundaries, except that the routed
 *    experts of a layer keep all payloads back to back followed by all
 *    scales, the slab the runtime binds without copies, convert.py:863).
 */
#ifndef UOCR_CONVERT_H
#define UOCR_CONVERT_H

#include <stddef.h>
#include <stdint.h>

#include "unlimitedocr.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Quantises `rows` rows of `cols` fp32 values (row-major) to qtype 1 (f16:
 * payload fp16 [rows][cols], scales unused), 3 (Q8_0: int8 [rows][cols]) or 4
 * (Q4_0: bytes [rows][cols/2], group-half-split nibbles q + 8), with fp16
 * scales [rows][cols/64] for Q8_0/Q4_0.  cols % 64 == 0 for Q8_0/Q4_0.
 *   Q8_0 (convert.py:2058-2063): s = max|x| / 127 in fp32 (1.0 for an
 *     all-zero group); q = clip(rint(x / s), -127, 127); stored scale fp16(s).
 *   Q4_0 (convert.py:2249-2276): m = the group's first element of largest
 *     |x|; stored scale h = fp16(m / -8); q = clip(rint(x / (h ? h : 1)), -8, 7).
 * rint rounds half to even and fp16 conversion rounds to nearest even, as
 * numpy does.  Returns UOCR_ERROR_INVALID_ARGUMENT for a bad shape or a
 * non-finite input (the reference rejects those tensors). */
UOCR_API int uocr_quantize_rows(uint32_t qtype, const float *src, uint32_t rows, uint32_t cols, void *payload,
                                uint16_t *scales);

/* Zero-filled decoder image for qprofile 1 (fp16), 2 (mixed-q8_0) or 3
 * (mixed-q4) in a malloc'd buffer (free with uocr_synth_free): header,
 * config record, tensor directory (one entry per decoder tensor, qtypes as
 * configs/quant-cfg.yaml gates them) and the tensor-data layout above. */
UOCR_API int uocr_image_skeleton_build(uint32_t qprofile, void **out_data, size_t *out_size);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_CONVERT_H */
