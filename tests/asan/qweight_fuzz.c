/* qweight_fuzz.c — host-side sanitizer run over the create/dequant argument validation
 * (sgl_qlinear_create*, sgl_qweight_dequant*) and sgl_qcfg_from_json, built with
 * -fsanitize=address,undefined by tests/test_host_asan.py.  Shapes are drawn from small,
 * huge and negative values; buffers are dummies that the validation never reads (g_idx, the
 * only host-read array, is passed as NULL).  The device entry points are stand-ins that fail,
 * so every accepted call ends there.  Any sanitizer report is a failure. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sgl/qlinear.h"
#include "sgl/quant.h"
#include "sgl/qweight.h"
#include "sglq_shim.h"

sglq_dev *sglq_build(const sglq_plan *p, const void *w, const void *z, const void *s, int dev) { (void)p; (void)w; (void)z; (void)s; (void)dev; return NULL; }
int sglq_dequant_dev(sglq_dev *d, float *o, void *s) { (void)d; (void)o; (void)s; return -1; }
int sglq_dequant_host(sglq_dev *d, float *o) { (void)d; (void)o; return -1; }
int sglq_forward(sglq_dev *d, const void *a, int t, int64_t m, const float *b, float *c, void *s) { (void)d; (void)a; (void)t; (void)m; (void)b; (void)c; (void)s; return -1; }
int sglq_forward_noalloc(sglq_dev *d, const void *a, int t, int64_t m, const float *b, float *c, void *s) { (void)d; (void)a; (void)t; (void)m; (void)b; (void)c; (void)s; return -1; }
int sglq_forward_host(sglq_dev *d, const float *a, int64_t m, const float *b, float *c) { (void)d; (void)a; (void)m; (void)b; (void)c; return -1; }
void sglq_free(sglq_dev *d) { (void)d; }
int64_t sglq_weight_bytes(const sglq_dev *d) { (void)d; return 0; }
int64_t sglq_N(const sglq_dev *d) { (void)d; return 0; }
int64_t sglq_K(const sglq_dev *d) { (void)d; return 0; }
int sglq_quant_rows_i8_host(const float *x, int8_t *o, float *s, int64_t r, int64_t d) { (void)x; (void)o; (void)s; (void)r; (void)d; return -1; }
int sglq_dequant_row_i8_host(const int8_t *q, float s, float *o, int64_t n) { (void)q; (void)s; (void)o; (void)n; return -1; }
int sglq_matmul_nt_dev_w(const float *a, const float *w, const float *b, float *c, int64_t m, int64_t n, int64_t k, int dev) { (void)a; (void)w; (void)b; (void)c; (void)m; (void)n; (void)k; (void)dev; return -1; }
void *sglq_upload(const void *h, size_t n, int dev) { (void)h; (void)n; (void)dev; return NULL; }
void sglq_release(void *p, int dev) { (void)p; (void)dev; }
int sglq_moe_forward(sglq_dev *const *g, sglq_dev *const *d, int n, const void *h, int t, int64_t T, const int32_t *i, const float *w, int k, float *o, void *s) { (void)g; (void)d; (void)n; (void)h; (void)t; (void)T; (void)i; (void)w; (void)k; (void)o; (void)s; return -1; }
int sglq_moe_router_logits(const float *r, int n, const void *h, int t, int64_t T, int64_t E, float *l, void *s) { (void)r; (void)n; (void)h; (void)t; (void)T; (void)E; (void)l; (void)s; return -1; }
int sglq_moe_route(const float *l, int64_t T, int n, const float *b, int sg, int ng, int tg, int k, int nm, float sc, int32_t *i, float *w, void *s) { (void)l; (void)T; (void)n; (void)b; (void)sg; (void)ng; (void)tg; (void)k; (void)nm; (void)sc; (void)i; (void)w; (void)s; return -1; }
int sglq_moe_shared(sglq_dev *g, sglq_dev *d, const void *h, int t, int64_t T, float *o, void *s) { (void)g; (void)d; (void)h; (void)t; (void)T; (void)o; (void)s; return -1; }
int sglq_mlp_forward(sglq_dev *g, sglq_dev *u, sglq_dev *d, const void *h, int t, int64_t T, float *o, void *s) { (void)g; (void)u; (void)d; (void)h; (void)t; (void)T; (void)o; (void)s; return -1; }
int sglq_quant_rows_i8_dev(const float *x, int8_t *o, float *s, int64_t r, int64_t d, void *st) { (void)x; (void)o; (void)s; (void)r; (void)d; (void)st; return -1; }
int sglq_dequant_rows_i8_dev(const int8_t *q, const float *s, float *o, int64_t r, int64_t d, void *st) { (void)q; (void)s; (void)o; (void)r; (void)d; (void)st; return -1; }

static unsigned long long rs;
static unsigned long long rnd(void) {
  rs ^= rs << 13;
  rs ^= rs >> 7;
  rs ^= rs << 17;
  return rs;
}
static int64_t shape(void) {
  switch (rnd() % 8) {
    case 0: return -(int64_t)(rnd() % 1000);
    case 1: return (int64_t)(rnd() >> 1);           /* up to 2^63 - 1 */
    case 2: return (int64_t)1 << (rnd() % 63);
    case 3: return 0;
    default: return (int64_t)(rnd() % 4096);
  }
}

int main(int argc, char **argv) {
  rs = argc > 1 ? strtoull(argv[1], NULL, 10) * 2654435761ull + 1 : 1;
  static int32_t buf[64];
  static float fbuf[64];
  static uint8_t ubuf[64];
  for (int it = 0; it < 200000; it++) {
    sgl_qcfg c;
    memset(&c, 0, sizeof(c));
    c.method = (int)(rnd() % 6);
    c.bits = (int)(rnd() % 10);
    c.group_size = (int)(rnd() % 3 == 0 ? -1 : (int)(rnd() % 300));
    c.zero_point = (int)(rnd() & 1);
    c.transposed = (int)(rnd() & 1);
    c.v2 = (int)(rnd() & 1);
    c.layout = (int)(rnd() & 1);
    c.offset = (int)(rnd() % 200);
    const int64_t a = shape(), b = shape(), d = shape(), e = shape(), f = shape(), g = shape(),
                  N = shape(), K = shape();
    sgl_qlinear *ql = NULL;
    switch (rnd() % 4) {
      case 0: ql = sgl_qlinear_create(&c, buf, a, b, (rnd() & 1) ? buf : NULL, d, e, fbuf, f, g,
                                      NULL, 0, N, K, 0); break;
      case 1: ql = sgl_qlinear_create_marlin(&c, buf, a, b, (rnd() & 1) ? buf : NULL, d, e, fbuf,
                                             f, g, N, K, 0); break;
      case 2: ql = sgl_qlinear_create_ct(&c, buf, a, b, fbuf, f, g, N, K, 0); break;
      default: ql = sgl_qlinear_create_mxfp4(ubuf, a, b, ubuf, f, g, N, K, 0); break;
    }
    if (ql) sgl_qlinear_destroy(ql);
    if (it % 10 == 0) {
      char js[512];
      const char *keys[] = {"quant_method", "bits", "group_size", "desc_act", "sym", "version",
                            "zero_point", "format", "checkpoint_format", "weight_block_size"};
      const char *vals[] = {"\"gptq\"", "\"awq\"", "\"mxfp4\"", "\"compressed-tensors\"",
                            "4", "8", "-1", "1e300", "true", "null", "[]", "{}", "\"marlin\"",
                            "\"gemv\"", "-9223372036854775808"};
      int n = snprintf(js, sizeof(js), "{\"quantization_config\": {");
      for (int k = 0, m = (int)(rnd() % 6); k < m && n < 400; k++)
        n += snprintf(js + n, sizeof(js) - (size_t)n, "%s\"%s\": %s", k ? ", " : "",
                      keys[rnd() % 10], vals[rnd() % 15]);
      n += snprintf(js + n, sizeof(js) - (size_t)n, "}}");
      sgl_qcfg c2;
      (void)sgl_qcfg_from_json(js, (size_t)n, &c2);
    }
  }
  printf("asan fuzz done\n");
  return 0;
}
