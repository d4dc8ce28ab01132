/* sgl/quant.h — int8 per-row quantization and the W8A16 matmul, kept signature-for-signature
 * with the reference (reference include/sgl/quant.h:13-25, src/quant.c:13-89).
 *
 * In this build these run on the GPU (host buffers in, host buffers out).  Semantics:
 *   scale = max|x| / 127 (0 for an all-zero row), q = trunc(x * (1/scale) +- 0.5) clamped to
 *   [-127, 127]; C[m,n] = (sum_k A[m,k] * (float)W[n,k]) * sw[n] + bias[n].
 */
#ifndef SGL_QUANT_H
#define SGL_QUANT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float sgl_quant_row_i8(const float *x, int8_t *out, int n);
void sgl_quant_rows_i8(const float *x, int8_t *out, float *scales, int rows, int dim);
void sgl_dequant_row_i8(const int8_t *q, float scale, float *out, int n);
void sgl_matmul_w8a16(const float *A, const int8_t *W, const float *sw, const float *bias,
                      float *C, int M, int N, int K);

#ifdef __cplusplus
}
#endif

#endif /* SGL_QUANT_H */
