/*
 * quantize.h -- GGUF block formats and the quantized matrix-vector entry
 * points (reference include/quantize.h:6-139).
 *
 * Block structs keep the GGUF byte layout exactly (18-byte Q4_0, 34-byte
 * Q8_0).  Q4_0 element order follows the reference: byte qs[j] holds element
 * 2j in its low nibble and element 2j+1 in its high nibble
 * (src/quantize.c:583-588), which is NOT ggml's j / j+16 split.
 *
 * Host pointers in, host pointers out, like the reference; every function
 * that does arithmetic over a matrix (dequantize, dot, gemv) runs on the GPU
 * and returns when the result is in host memory.  vx_fp16_to_fp32 /
 * vx_fp32_to_fp16 / vx_quantize_row_q4_0 / vx_quantized_size are host-side
 * format helpers (bit manipulation for the loader and the GGUF writer).
 *
 * The K-quant, Q4_1/Q5_x/Q8_1 and sparse-column variants of the reference
 * header are not part of the verify path and are not provided.
 */
#ifndef VX_QUANTIZE_H
#define VX_QUANTIZE_H

#include "veltrix.h"

#define QK4_0 32
typedef struct {
    uint16_t d;               /* fp16 scale                                  */
    uint8_t qs[QK4_0 / 2];    /* element 2j: low nibble, 2j+1: high nibble    */
} block_q4_0;

#define QK8_0 32
typedef struct {
    uint16_t d;               /* fp16 scale                                  */
    int8_t qs[QK8_0];
} block_q8_0;

/* Bytes taken by n elements of `type` (reference src/quantize.c:59-86). */
size_t vx_quantized_size(int n, vx_type type);

/* Host format helpers (reference src/quantize.c:17-57, 88-114). */
void vx_quantize_row_q4_0(const float *x, void *y, int n);
uint16_t vx_fp32_to_fp16(float f);
float vx_fp16_to_fp32(uint16_t h);

/* GPU-backed dequantization of n elements (reference src/quantize.c:578-591,
 * 642-651); outputs are multiplied by the synthetic weight scale. */
void vx_dequantize_row_q4_0(const void *x, float *y, int n);
void vx_dequantize_row_q8_0(const void *x, float *y, int n);

/* Process-global multiplier applied by the dequantize entry points
 * (reference src/quantize.c:7-15). Default 1. */
void vx_set_synthetic_weight_scale(float scale);
float vx_get_synthetic_weight_scale(void);

/* dst = sum_i dequant(x)_i * y_i over n elements (reference src/quantize.c:665-678). */
void vx_dot_q4_0(const void *x, const float *y, float *dst, int n);

/* y[rows] = A[rows x cols] . x  with A in Q4_0 blocks, exact Q4_0 arithmetic
 * (reference scalar path src/quantize.c:728-750). */
void vx_gemv_q4_0(const void *restrict A, const float *restrict x,
                  float *restrict y, int rows, int cols);

/* As vx_gemv_q4_0, but y[i] = 0 where |gate[i]| < threshold
 * (reference src/quantize.c:680-704). */
void vx_gemv_q4_0_sparse_rows(const void *restrict A, const float *restrict x,
                              float *restrict y, int rows, int cols,
                              const float *restrict gate, float threshold);

#endif
