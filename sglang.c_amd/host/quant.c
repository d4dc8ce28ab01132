/* quant.c — the reference's int8 C API (include/sgl/quant.h) and the dense f32 NT matmul
 * (include/sgl/ops.h), host side, C11.  Host buffers in and out; the arithmetic runs in HIP
 * kernels (csrc/int8.hip, csrc/gemv.hip).
 *   sgl_quant_row(s)_i8 / sgl_dequant_row_i8: reference src/quant.c:13-42, bit-identical.
 *   sgl_matmul_w8a16: reference src/quant.c:44-89, fp32 accumulation of exact int8 codes.
 *   sgl_matmul_nt:    reference src/ops.c:243-279, fp32 accumulation. */
#include <stdlib.h>
#include <string.h>

#include "qhost.h"
#include "sgl/ops.h"
#include "sgl/quant.h"

QH_API float sgl_quant_row_i8(const float *x, int8_t *out, int n) {
  float s = 0.f;
  if (n <= 0) return 0.f;
  if (sglq_quant_rows_i8_host(x, out, &s, 1, n) != 0) {
    QH_ERR("sgl_quant_row_i8: device failure");
    abort(); /* void-returning API: no error channel, like an allocation failure */
  }
  return s;
}

QH_API void sgl_quant_rows_i8(const float *x, int8_t *out, float *scales, int rows, int dim) {
  if (rows <= 0 || dim <= 0) return;
  if (sglq_quant_rows_i8_host(x, out, scales, rows, dim) != 0) {
    QH_ERR("sgl_quant_rows_i8: device failure");
    abort();
  }
}

QH_API void sgl_dequant_row_i8(const int8_t *q, float scale, float *out, int n) {
  if (n <= 0) return;
  if (sglq_dequant_row_i8_host(q, scale, out, n) != 0) {
    QH_ERR("sgl_dequant_row_i8: device failure");
    abort();
  }
}

QH_API void sgl_matmul_w8a16(const float *A, const int8_t *W, const float *sw, const float *bias,
                             float *C, int M, int N, int K) {
  if (M <= 0 || N <= 0) return;
  sglq_plan p;
  int32_t *kmap = NULL, *kinv = NULL;
  memset(&p, 0, sizeof(p));
  p.src = SGLQ_SRC_W8;
  p.kind = SGLQ_KIND_U8;
  p.bits = 8;
  p.zconst = 128;
  p.N = N;
  p.K = K;
  p.G = K;
  p.sc_rows = 1;
  p.sc_cols = N;
  sglq_dev *d = NULL;
  if (qh_plan_groups(&p, 1, NULL, 2, &kmap, &kinv) == 0) d = sglq_build(&p, W, NULL, sw, 0);
  free(kmap);
  free(kinv);
  if (!d || sglq_forward_host(d, A, M, bias, C) != 0) {
    QH_ERR("sgl_matmul_w8a16: device failure");
    abort();
  }
  sglq_free(d);
}

QH_API void sgl_matmul_nt(const float *A, const float *W, const float *bias, float *C, int M,
                          int N, int K) {
  if (M <= 0 || N <= 0) return;
  if (sglq_matmul_nt_host(A, W, bias, C, M, N, K) != 0) {
    QH_ERR("sgl_matmul_nt: device failure");
    abort();
  }
}
