/* sgl/ops.h — the one dense operator on the quantized-linear path: the f32 "NT" matmul every
 * load-time-dequantized weight goes through (reference include/sgl/ops.h:13-14,
 * src/ops.c:243-279).  C[M,N] = A[M,K] * W[N,K]^T + bias[N]; bias may be NULL.
 * Host pointers in and out; the product runs it on the GPU. */
#ifndef SGL_OPS_H
#define SGL_OPS_H

#ifdef __cplusplus
extern "C" {
#endif

void sgl_matmul_nt(const float *A, const float *W, const float *bias, float *C, int M, int N,
                   int K);

#ifdef __cplusplus
}
#endif

#endif /* SGL_OPS_H */
