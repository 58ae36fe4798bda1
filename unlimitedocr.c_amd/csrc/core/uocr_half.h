/* uocr_half.h - fp32 -> fp16 bit conversion shared by the image writers. */
#ifndef UOCR_HALF_H
#define UOCR_HALF_H

#include <stdint.h>

/* IEEE binary16 bits of f, rounded to nearest even (subnormals included,
 * overflow to infinity, NaN kept quiet with its sign), as numpy's
 * float32 -> float16 cast. */
uint16_t uocr_half_bits(float f);

#endif /* UOCR_HALF_H */
