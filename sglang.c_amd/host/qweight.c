/* qweight.c — the reference's quantized-weight C API (include/sgl/qweight.h) and the
 * device-resident sgl_qlinear API (include/sgl/qlinear.h), host side, C11.
 *
 * Each entry point first validates its arguments with the reference's rules and log lines
 * (reference src/qweight.c:28-141, 193-227, 282-303, 334-353) and returns -1 / NULL on a
 * violation.  It then describes the source format and the device layout in a sglq_plan and
 * hands the raw buffers to the HIP shim, which decodes and repacks them on the GPU.  Nothing
 * here touches weight values: all arithmetic runs in the HIP kernels. */
#include <stdlib.h>
#include <string.h>

#include "qhost.h"
#include "sgl/qlinear.h"
#include "sgl/qweight.h"

struct sgl_qlinear {
  sglq_dev *d;
};

QH_API int sgl_q_pack(int bits) { return bits > 0 ? 32 / bits : 0; } /* reference :19 */

static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
static int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

/* Every caller-supplied extent must lie in [0, 2^40) before any shape arithmetic (products of
 * two of them then stay inside int64).  A weight that large could not be resident anyway. */
static int extents_ok(const char *what, const int64_t *v, int n) {
  for (int i = 0; i < n; i++)
    if (v[i] < 0 || v[i] >= ((int64_t)1 << 40)) {
      QH_ERR("%s: extent %lld out of range", what, (long long)v[i]);
      return 0;
    }
  return 1;
}
#define EXTENTS_OK(what, ...) \
  extents_ok(what, (const int64_t[]){__VA_ARGS__}, \
             (int)(sizeof((const int64_t[]){__VA_ARGS__}) / sizeof(int64_t)))

/* Device K positions: groups made contiguous in group order (act-order sorts by g_idx, keeping
 * the original order inside a group), each group padded to a multiple of 32, total padded to a
 * whole number of chunks (spc steps).  kmap[k'] = original k or -1; kinv[k] = k'. */
int qh_plan_groups(sglq_plan *p, int64_t ngroups, const int32_t *gidx, int spc, int32_t **kmap,
                   int32_t **kinv) {
  const int64_t K = p->K;
  int64_t *cnt = (int64_t *)calloc((size_t)ngroups, sizeof(int64_t));
  if (!cnt) return -1;
  for (int64_t k = 0; k < K; k++) cnt[gidx ? gidx[k] : k / p->G]++;
  int64_t gmax = 0;
  for (int64_t g = 0; g < ngroups; g++) gmax = cnt[g] > gmax ? cnt[g] : gmax;
  p->ngroups = ngroups;
  /* one group (per-channel scale): pad it to whole chunks so its scale is applied per chunk */
  p->gp = ngroups == 1 ? round_up(K, 32 * spc) : round_up(gmax, 32);
  p->nsteps = round_up(ngroups * p->gp / 32, spc);
  *kmap = (int32_t *)malloc(sizeof(int32_t) * (size_t)(p->nsteps * 32));
  *kinv = (int32_t *)malloc(sizeof(int32_t) * (size_t)K);
  if (!*kmap || !*kinv) {
    free(cnt);
    free(*kmap);
    free(*kinv);
    *kmap = *kinv = NULL;
    return -1;
  }
  for (int64_t i = 0; i < p->nsteps * 32; i++) (*kmap)[i] = -1;
  for (int64_t g = 0; g < ngroups; g++) cnt[g] = g * p->gp; /* next free slot */
  for (int64_t k = 0; k < K; k++) {
    const int64_t g = gidx ? gidx[k] : k / p->G;
    const int64_t kp = cnt[g]++;
    (*kmap)[kp] = (int32_t)k;
    (*kinv)[k] = (int32_t)kp;
  }
  free(cnt);
  p->kmap = *kmap;
  p->kinv = *kinv;
  return 0;
}

/* ---- AWQ / GPTQ natural layouts: validation of reference src/qweight.c:32-131 ---------- */
static int check_awq_gptq(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                          int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                          int64_t qz_cols, const float *scales, int64_t sc_rows, int64_t sc_cols,
                          const int32_t *g_idx, int64_t g_n, int64_t N, int64_t K,
                          int64_t *ngroups) {
  if (!cfg || !qweight || !scales || N <= 0 || K <= 0) return -1;
  const int bits = cfg->bits ? cfg->bits : 4;
  if (bits != 4 && bits != 8) {
    QH_ERR("quant: %d-bit is not supported (4 or 8 only)", bits);
    return -1;
  }
  if (cfg->method != SGL_Q_AWQ && cfg->method != SGL_Q_GPTQ) {
    QH_ERR("quant: unknown quantization method %d", cfg->method);
    return -1;
  }
  if (cfg->method == SGL_Q_AWQ && bits != 4) {
    QH_ERR("quant: AWQ supports 4-bit only (config says %d)", bits);
    return -1;
  }
  const int pack = 32 / bits;
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  const int has_z = qzeros != NULL;
  if (sc_cols != N) {
    QH_ERR("quant: scales shape [%lld,%lld], expected [%lld,%lld]", (long long)sc_rows,
           (long long)sc_cols, (long long)ceil_div(K, G), (long long)N);
    return -1;
  }
  if (has_z && qz_cols * pack < N) {
    QH_ERR("quant: qzeros packed width %lld*%d < N=%lld", (long long)qz_cols, pack,
           (long long)N);
    return -1;
  }
  if (cfg->method == SGL_Q_AWQ) {
    if (cfg->transposed ? (qw_rows * pack < N || qw_cols != K)
                        : (qw_rows != K || qw_cols * pack < N)) {
      QH_ERR("quant(awq/%s): qweight [%lld,%lld] does not match N=%lld K=%lld",
             cfg->transposed ? "gemv" : "gemm", (long long)qw_rows, (long long)qw_cols,
             (long long)N, (long long)K);
      return -1;
    }
    const int64_t gl = (K - 1) / G;
    if (gl >= sc_rows) {
      QH_ERR("quant(awq): group %lld is beyond the %lld scale rows", (long long)gl,
             (long long)sc_rows);
      return -1;
    }
    if (has_z && gl >= qz_rows) {
      QH_ERR("quant(awq): group %lld is beyond the %lld qzeros rows", (long long)gl,
             (long long)qz_rows);
      return -1;
    }
    *ngroups = gl + 1;
    return 0;
  }
  if (qw_cols != N || qw_rows * pack < K) {
    QH_ERR("quant(gptq): qweight [%lld,%lld] does not match N=%lld K=%lld", (long long)qw_rows,
           (long long)qw_cols, (long long)N, (long long)K);
    return -1;
  }
  if (g_idx && g_n < K) {
    QH_ERR("quant(gptq): g_idx length %lld < K=%lld", (long long)g_n, (long long)K);
    return -1;
  }
  int64_t gmax = 0;
  for (int64_t k = 0; k < K; k++) {
    const int64_t g = g_idx ? (int64_t)g_idx[k] : k / G;
    if (g < 0 || g >= sc_rows) {
      QH_ERR("quant(gptq): row %lld has group %lld, beyond the %lld scale rows", (long long)k,
             (long long)g, (long long)sc_rows);
      return -1;
    }
    if (has_z && g >= qz_rows) {
      QH_ERR("quant(gptq): group %lld is beyond the %lld qzeros rows", (long long)g,
             (long long)qz_rows);
      return -1;
    }
    gmax = g > gmax ? g : gmax;
  }
  *ngroups = gmax + 1;
  return 0;
}

static sglq_dev *build_awq_gptq(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                                int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                                int64_t qz_cols, const float *scales, int64_t sc_rows,
                                int64_t sc_cols, const int32_t *g_idx, int64_t g_n, int64_t N,
                                int64_t K, int dev) {
  int64_t ng = 0;
  if (!EXTENTS_OK("quant", qw_rows, qw_cols, qz_rows, qz_cols, sc_rows, sc_cols, g_n, N, K))
    return NULL;
  if (check_awq_gptq(cfg, qweight, qw_rows, qw_cols, qzeros, qz_rows, qz_cols, scales, sc_rows,
                     sc_cols, g_idx, g_n, N, K, &ng) != 0)
    return NULL;
  const int bits = cfg->bits ? cfg->bits : 4;
  sglq_plan p;
  memset(&p, 0, sizeof(p));
  p.src = cfg->method == SGL_Q_AWQ ? SGLQ_SRC_AWQ : SGLQ_SRC_GPTQ;
  p.kind = bits == 4 ? SGLQ_KIND_U4 : SGLQ_KIND_U8;
  p.bits = bits;
  p.transposed = cfg->method == SGL_Q_AWQ && cfg->transposed;
  p.v2 = cfg->method == SGL_Q_GPTQ && cfg->v2;
  p.has_zero = qzeros != NULL;
  p.zconst = 0;
  p.N = N;
  p.K = K;
  p.G = cfg->group_size > 0 ? cfg->group_size : K;
  p.qw_rows = qw_rows;
  p.qw_cols = qw_cols;
  p.qz_rows = qz_rows;
  p.qz_cols = qz_cols;
  p.sc_rows = ng; /* only the rows any k refers to are uploaded */
  p.sc_cols = sc_cols;
  if (p.has_zero) p.qz_rows = ng;
  const int32_t *gi = (cfg->method == SGL_Q_GPTQ) ? g_idx : NULL;
  int32_t *kmap = NULL, *kinv = NULL;
  if (qh_plan_groups(&p, ng, gi, bits == 4 ? 4 : 2, &kmap, &kinv) != 0) return NULL;
  qh_info("qlinear: %s %d-bit N=%lld K=%lld groups=%lld (padded %lld) steps=%lld",
          p.src == SGLQ_SRC_AWQ ? "AWQ" : "GPTQ", bits, (long long)N, (long long)K,
          (long long)ng, (long long)p.gp, (long long)p.nsteps);
  sglq_dev *d = sglq_build(&p, qweight, qzeros, scales, dev);
  free(kmap);
  free(kinv);
  return d;
}

/* ---- Marlin: validation of reference src/qweight.c:197-227 (+ per-k group checks) ------ */
static sglq_dev *build_marlin(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                              int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                              int64_t qz_cols, const float *scales, int64_t sc_rows,
                              int64_t sc_cols, int64_t N, int64_t K, int dev) {
  if (!cfg || !qweight || !scales || N <= 0 || K <= 0) return NULL;
  if (!EXTENTS_OK("quant(marlin)", qw_rows, qw_cols, qz_rows, qz_cols, sc_rows, sc_cols, N, K))
    return NULL;
  const int bits = cfg->bits ? cfg->bits : 4;
  if (bits != 4 && bits != 8) {
    QH_ERR("quant(marlin): 4/8-bit only (config says %d)", bits);
    return NULL;
  }
  const int pack = 32 / bits;
  if (K % 16 != 0 || N % 64 != 0) {
    QH_ERR("quant(marlin): K=%lld must be a multiple of 16 and N=%lld of 64", (long long)K,
           (long long)N);
    return NULL;
  }
  if (qw_rows != K / 16 || qw_cols * pack < N * 16) {
    QH_ERR("quant(marlin): qweight [%lld,%lld] does not match N=%lld K=%lld (expected "
           "[%lld,%lld])",
           (long long)qw_rows, (long long)qw_cols, (long long)N, (long long)K,
           (long long)(K / 16), (long long)(N * 16 / pack));
    return NULL;
  }
  if (sc_cols != N) {
    QH_ERR("quant(marlin): scales width %lld, expected N=%lld", (long long)sc_cols,
           (long long)N);
    return NULL;
  }
  if (qzeros && (qz_cols * pack < N || qz_rows < sc_rows)) {
    QH_ERR("quant(marlin): qzeros [%lld,%lld] does not match N=%lld / %lld groups",
           (long long)qz_rows, (long long)qz_cols, (long long)N, (long long)sc_rows);
    return NULL;
  }
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  const int64_t gl = (K - 1) / G;
  if (gl >= sc_rows) {
    QH_ERR("quant(marlin): group %lld is beyond the %lld scale rows", (long long)gl,
           (long long)sc_rows);
    return NULL;
  }
  if (qzeros && gl >= qz_rows) {
    QH_ERR("quant(marlin): group %lld is beyond the %lld qzeros rows", (long long)gl,
           (long long)qz_rows);
    return NULL;
  }
  sglq_plan p;
  memset(&p, 0, sizeof(p));
  p.src = SGLQ_SRC_MARLIN;
  p.kind = bits == 4 ? SGLQ_KIND_U4 : SGLQ_KIND_U8;
  p.bits = bits;
  p.has_zero = qzeros != NULL;
  p.zconst = 1 << (bits - 1);
  p.N = N;
  p.K = K;
  p.G = G;
  p.qw_rows = qw_rows;
  p.qw_cols = qw_cols;
  p.qz_rows = gl + 1;
  p.qz_cols = qz_cols;
  p.sc_rows = gl + 1;
  p.sc_cols = sc_cols;
  int32_t *kmap = NULL, *kinv = NULL;
  if (qh_plan_groups(&p, gl + 1, NULL, bits == 4 ? 4 : 2, &kmap, &kinv) != 0) return NULL;
  sglq_dev *d = sglq_build(&p, qweight, qzeros, scales, dev);
  free(kmap);
  free(kinv);
  return d;
}

/* ---- compressed-tensors: validation of reference src/qweight.c:285-303 ----------------- */
static sglq_dev *build_ct(const sgl_qcfg *cfg, const int32_t *wpacked, int64_t rows, int64_t cols,
                          const float *scales, int64_t sc_rows, int64_t sc_cols, int64_t N,
                          int64_t K, int dev) {
  if (!cfg || !wpacked || !scales || N <= 0 || K <= 0) return NULL;
  if (!EXTENTS_OK("quant(ct)", rows, cols, sc_rows, sc_cols, N, K)) return NULL;
  const int bits = cfg->bits ? cfg->bits : 4;
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  const int off = cfg->offset ? cfg->offset : (1 << (bits - 1));
  if (sc_cols != ceil_div(K, G)) {
    QH_ERR("quant(ct): scales [%lld,%lld], expected [%lld,%lld]", (long long)sc_rows,
           (long long)sc_cols, (long long)N, (long long)ceil_div(K, G));
    return NULL;
  }
  if (rows != N) {
    QH_ERR("quant(ct): weight_packed has %lld rows, N=%lld", (long long)rows, (long long)N);
    return NULL;
  }
  if (cols * (bits == 4 ? 8 : 4) < K) {
    QH_ERR("quant(ct): weight_packed [%lld,%lld] cannot hold K=%lld", (long long)rows,
           (long long)cols, (long long)K);
    return NULL;
  }
  /* device-side limits (the zero store is one byte; scales must cover every row) */
  if (off < 0 || off > 255 || sc_rows < N) {
    QH_ERR("quant(ct): offset %d / scale rows %lld not supported on the device", off,
           (long long)sc_rows);
    return NULL;
  }
  sglq_plan p;
  memset(&p, 0, sizeof(p));
  p.src = SGLQ_SRC_CT;
  p.kind = bits == 4 ? SGLQ_KIND_U4 : SGLQ_KIND_U8;
  p.bits = bits == 4 ? 4 : 8;
  p.zconst = off;
  p.N = N;
  p.K = K;
  p.G = G;
  p.qw_rows = rows;
  p.qw_cols = cols;
  p.sc_rows = N;
  p.sc_cols = sc_cols;
  int32_t *kmap = NULL, *kinv = NULL;
  if (qh_plan_groups(&p, ceil_div(K, G), NULL, bits == 4 ? 4 : 2, &kmap, &kinv) != 0)
    return NULL;
  sglq_dev *d = sglq_build(&p, wpacked, NULL, scales, dev);
  free(kmap);
  free(kinv);
  return d;
}

/* ---- MXFP4: validation of reference src/qweight.c:338-353 ------------------------------ */
static sglq_dev *build_mxfp4(const uint8_t *wpacked, int64_t rows, int64_t cols,
                             const uint8_t *scales, int64_t sc_rows, int64_t sc_cols, int64_t N,
                             int64_t K, int dev) {
  if (!wpacked || !scales || N <= 0 || K <= 0) return NULL;
  if (!EXTENTS_OK("quant(mxfp4)", rows, cols, sc_rows, sc_cols, N, K)) return NULL;
  if (rows != N) {
    QH_ERR("quant(mxfp4): weight has %lld rows, N=%lld", (long long)rows, (long long)N);
    return NULL;
  }
  if (cols * 2 < K) {
    QH_ERR("quant(mxfp4): weight [%lld,%lld] cannot hold K=%lld", (long long)rows,
           (long long)cols, (long long)K);
    return NULL;
  }
  const int64_t nb = ceil_div(K, 32);
  if (sc_cols != nb) {
    QH_ERR("quant(mxfp4): scales [%lld,%lld], expected [%lld,%lld]", (long long)sc_rows,
           (long long)sc_cols, (long long)N, (long long)nb);
    return NULL;
  }
  if (sc_rows < N) {
    QH_ERR("quant(mxfp4): %lld scale rows for N=%lld", (long long)sc_rows, (long long)N);
    return NULL;
  }
  sglq_plan p;
  memset(&p, 0, sizeof(p));
  p.src = SGLQ_SRC_MXFP4;
  p.kind = SGLQ_KIND_E2M1;
  p.bits = 4;
  p.N = N;
  p.K = K;
  p.G = 32;
  p.qw_rows = rows;
  p.qw_cols = cols;
  p.sc_rows = N;
  p.sc_cols = sc_cols;
  int32_t *kmap = NULL, *kinv = NULL;
  if (qh_plan_groups(&p, nb, NULL, 4, &kmap, &kinv) != 0) return NULL;
  sglq_dev *d = sglq_build(&p, wpacked, NULL, scales, dev);
  free(kmap);
  free(kinv);
  return d;
}

sglq_dev *qh_build_w8(const int8_t *W, const float *sw, int64_t N, int64_t K, int dev) {
  if (!W || !sw || N <= 0 || K <= 0) return NULL;
  if (!EXTENTS_OK("w8", N, K)) return NULL;
  sglq_plan p;
  memset(&p, 0, sizeof(p));
  p.src = SGLQ_SRC_W8;
  p.kind = SGLQ_KIND_U8;
  p.bits = 8;
  p.zconst = 128; /* codes are stored +128 */
  p.N = N;
  p.K = K;
  p.G = K;
  p.sc_rows = 1;
  p.sc_cols = N;
  int32_t *kmap = NULL, *kinv = NULL;
  if (qh_plan_groups(&p, 1, NULL, 2, &kmap, &kinv) != 0) return NULL;
  sglq_dev *d = sglq_build(&p, W, NULL, sw, dev);
  free(kmap);
  free(kinv);
  return d;
}

/* dequant entry points: build on device 0, dequant there, copy back, release */
static int dequant_via(sglq_dev *d, float *out) {
  if (!d) return -1;
  const int rc = sglq_dequant_host(d, out);
  sglq_free(d);
  return rc;
}

QH_API int sgl_qweight_dequant(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                               int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                               int64_t qz_cols, const float *scales, int64_t sc_rows,
                               int64_t sc_cols, const int32_t *g_idx, int64_t g_n, int64_t N,
                               int64_t K, float *out) {
  if (!out) return -1;
  return dequant_via(build_awq_gptq(cfg, qweight, qw_rows, qw_cols, qzeros, qz_rows, qz_cols,
                                    scales, sc_rows, sc_cols, g_idx, g_n, N, K, 0),
                     out);
}

QH_API int sgl_qweight_dequant_marlin(const sgl_qcfg *cfg, const int32_t *qweight,
                                      int64_t qw_rows, int64_t qw_cols, const int32_t *qzeros,
                                      int64_t qz_rows, int64_t qz_cols, const float *scales,
                                      int64_t sc_rows, int64_t sc_cols, int64_t N, int64_t K,
                                      float *out) {
  if (!out) return -1;
  return dequant_via(build_marlin(cfg, qweight, qw_rows, qw_cols, qzeros, qz_rows, qz_cols,
                                  scales, sc_rows, sc_cols, N, K, 0),
                     out);
}

QH_API int sgl_qweight_dequant_ct(const sgl_qcfg *cfg, const int32_t *wpacked, int64_t rows,
                                  int64_t cols, const float *scales, int64_t sc_rows,
                                  int64_t sc_cols, int64_t N, int64_t K, float *out) {
  if (!out) return -1;
  return dequant_via(build_ct(cfg, wpacked, rows, cols, scales, sc_rows, sc_cols, N, K, 0), out);
}

QH_API int sgl_qweight_dequant_mxfp4(const int32_t *cfg_unused, const uint8_t *wpacked,
                                     int64_t rows, int64_t cols, const uint8_t *scales,
                                     int64_t sc_rows, int64_t sc_cols, int64_t N, int64_t K,
                                     float *out) {
  (void)cfg_unused;
  if (!out) return -1;
  return dequant_via(build_mxfp4(wpacked, rows, cols, scales, sc_rows, sc_cols, N, K, 0), out);
}

/* ---- sgl_qlinear ---------------------------------------------------------------------- */
static sgl_qlinear *wrap(sglq_dev *d) {
  if (!d) return NULL;
  sgl_qlinear *q = (sgl_qlinear *)malloc(sizeof(sgl_qlinear));
  if (!q) {
    sglq_free(d);
    return NULL;
  }
  q->d = d;
  return q;
}

QH_API sgl_qlinear *sgl_qlinear_create(const sgl_qcfg *cfg, const int32_t *qweight,
                                       int64_t qw_rows, int64_t qw_cols, const int32_t *qzeros,
                                       int64_t qz_rows, int64_t qz_cols, const float *scales,
                                       int64_t sc_rows, int64_t sc_cols, const int32_t *g_idx,
                                       int64_t g_n, int64_t N, int64_t K, int dev) {
  if (cfg && cfg->layout == SGL_QLAYOUT_MARLIN)
    return g_idx ? NULL
                 : wrap(build_marlin(cfg, qweight, qw_rows, qw_cols, qzeros, qz_rows, qz_cols,
                                     scales, sc_rows, sc_cols, N, K, dev));
  return wrap(build_awq_gptq(cfg, qweight, qw_rows, qw_cols, qzeros, qz_rows, qz_cols, scales,
                             sc_rows, sc_cols, g_idx, g_n, N, K, dev));
}

QH_API sgl_qlinear *sgl_qlinear_create_marlin(const sgl_qcfg *cfg, const int32_t *qweight,
                                              int64_t qw_rows, int64_t qw_cols,
                                              const int32_t *qzeros, int64_t qz_rows,
                                              int64_t qz_cols, const float *scales,
                                              int64_t sc_rows, int64_t sc_cols, int64_t N,
                                              int64_t K, int dev) {
  return wrap(build_marlin(cfg, qweight, qw_rows, qw_cols, qzeros, qz_rows, qz_cols, scales,
                           sc_rows, sc_cols, N, K, dev));
}

QH_API sgl_qlinear *sgl_qlinear_create_ct(const sgl_qcfg *cfg, const int32_t *wpacked,
                                          int64_t rows, int64_t cols, const float *scales,
                                          int64_t sc_rows, int64_t sc_cols, int64_t N, int64_t K,
                                          int dev) {
  return wrap(build_ct(cfg, wpacked, rows, cols, scales, sc_rows, sc_cols, N, K, dev));
}

QH_API sgl_qlinear *sgl_qlinear_create_mxfp4(const uint8_t *wpacked, int64_t rows, int64_t cols,
                                             const uint8_t *scales, int64_t sc_rows,
                                             int64_t sc_cols, int64_t N, int64_t K, int dev) {
  return wrap(build_mxfp4(wpacked, rows, cols, scales, sc_rows, sc_cols, N, K, dev));
}

QH_API sgl_qlinear *sgl_qlinear_create_w8(const int8_t *W, const float *sw, int64_t N, int64_t K,
                                          int dev) {
  return wrap(qh_build_w8(W, sw, N, K, dev));
}

QH_API int sgl_qlinear_forward(sgl_qlinear *ql, const void *A, int a_dtype, int64_t M,
                               const float *bias, float *C, void *stream) {
  if (!ql || M < 0) return -1;
  if (a_dtype != SGL_QL_F32 && a_dtype != SGL_QL_BF16 && a_dtype != SGL_QL_F16) {
    QH_ERR("qlinear: unknown activation dtype %d", a_dtype);
    return -1;
  }
  if (M == 0) return 0; /* an empty batch: nothing to read or write */
  if (!A || !C) return -1;
  return sglq_forward(ql->d, A, a_dtype, M, bias, C, stream);
}

QH_API int sgl_qlinear_forward_noalloc(sgl_qlinear *ql, const void *A, int a_dtype, int64_t M,
                                       const float *bias, float *C, void *stream) {
  if (!ql || M < 0) return -1;
  if (a_dtype != SGL_QL_F32 && a_dtype != SGL_QL_BF16 && a_dtype != SGL_QL_F16) {
    QH_ERR("qlinear: unknown activation dtype %d", a_dtype);
    return -1;
  }
  if (M == 0) return 0;
  if (!A || !C) return -1;
  return sglq_forward_noalloc(ql->d, A, a_dtype, M, bias, C, stream);
}

QH_API int sgl_qlinear_dequant(sgl_qlinear *ql, float *out, void *stream) {
  if (!ql || !out) return -1;
  return sglq_dequant_dev(ql->d, out, stream);
}

QH_API int64_t sgl_qlinear_out_features(const sgl_qlinear *ql) { return ql ? sglq_N(ql->d) : 0; }
QH_API int64_t sgl_qlinear_in_features(const sgl_qlinear *ql) { return ql ? sglq_K(ql->d) : 0; }
QH_API int64_t sgl_qlinear_weight_bytes(const sgl_qlinear *ql) {
  return ql ? sglq_weight_bytes(ql->d) : 0;
}

QH_API void sgl_qlinear_destroy(sgl_qlinear *ql) {
  if (!ql) return;
  sglq_free(ql->d);
  free(ql);
}

QH_API int sgl_qmoe_forward(sgl_qlinear *const *gate_up, sgl_qlinear *const *down, int n_experts,
                            const void *h, int h_dtype, int64_t T, const int32_t *topk_ids,
                            const float *topk_w, int k, float *out, void *stream) {
  if (!gate_up || !down || n_experts <= 0 || T < 0 || k <= 0) return -1;
  if (T == 0) return 0; /* an empty batch: nothing to read or write */
  if (!h || !topk_ids || !topk_w || !out) return -1;
  sglq_dev **gu = (sglq_dev **)malloc(sizeof(sglq_dev *) * (size_t)n_experts);
  sglq_dev **dn = (sglq_dev **)malloc(sizeof(sglq_dev *) * (size_t)n_experts);
  int rc = -1;
  if (gu && dn) {
    rc = 0;
    for (int e = 0; e < n_experts; e++) {
      if (!gate_up[e] || !down[e]) {
        QH_ERR("qmoe: expert %d has no weights", e);
        rc = -1;
        break;
      }
      gu[e] = gate_up[e]->d;
      dn[e] = down[e]->d;
    }
    if (rc == 0)
      rc = sglq_moe_forward(gu, dn, n_experts, h, h_dtype, T, topk_ids, topk_w, k, out, stream);
  }
  free(gu);
  free(dn);
  return rc;
}

QH_API int sgl_qmoe_router_logits(const float *router_w, int n_experts, const void *h,
                                  int h_dtype, int64_t T, int64_t E, float *logits,
                                  void *stream) {
  if (T < 0) return -1;
  if (T == 0) return 0;
  if (!router_w || !h || !logits) return -1;
  if (h_dtype != SGL_QL_F32 && h_dtype != SGL_QL_BF16 && h_dtype != SGL_QL_F16) {
    QH_ERR("qmoe router: unknown activation dtype %d", h_dtype);
    return -1;
  }
  return sglq_moe_router_logits(router_w, n_experts, h, h_dtype, T, E, logits, stream);
}

QH_API int sgl_qmoe_route(const sgl_qmoe_routing *r, const float *logits, const float *e_bias,
                          int n_experts, int64_t T, int32_t *topk_ids, float *topk_w,
                          void *stream) {
  if (!r || T < 0) return -1;
  if (T == 0) return 0;
  if (!logits || !topk_ids || !topk_w) return -1;
  return sglq_moe_route(logits, T, n_experts, e_bias, r->sigmoid, r->n_group, r->topk_group,
                        r->k, r->norm_topk, r->routed_scale, topk_ids, topk_w, stream);
}

QH_API int sgl_qmoe_shared(sgl_qlinear *gate_up, sgl_qlinear *down, const void *h, int h_dtype,
                           int64_t T, float *out, void *stream) {
  if (!gate_up || !down || T < 0) return -1;
  if (T == 0) return 0;
  if (!h || !out) return -1;
  if (h_dtype != SGL_QL_F32 && h_dtype != SGL_QL_BF16 && h_dtype != SGL_QL_F16) {
    QH_ERR("qmoe shared: unknown activation dtype %d", h_dtype);
    return -1;
  }
  return sglq_moe_shared(gate_up->d, down->d, h, h_dtype, T, out, stream);
}

QH_API int sgl_qmlp_forward(sgl_qlinear *gate, sgl_qlinear *up, sgl_qlinear *down,
                            const void *h, int h_dtype, int64_t T, float *out, void *stream) {
  if (!gate || !down || T < 0) return -1;
  if (T == 0) return 0;
  if (!h || !out) return -1;
  if (h_dtype != SGL_QL_F32 && h_dtype != SGL_QL_BF16 && h_dtype != SGL_QL_F16) {
    QH_ERR("qmlp: unknown activation dtype %d", h_dtype);
    return -1;
  }
  return sglq_mlp_forward(gate->d, up ? up->d : NULL, down->d, h, h_dtype, T, out, stream);
}

QH_API int sgl_quant_rows_i8_dev(const float *x, int8_t *out, float *scales, int64_t rows,
                                 int64_t dim, void *stream) {
  if (rows < 0 || dim < 0) return -1;
  if (rows == 0 || dim == 0) return 0;
  if (!x || !out || !scales) return -1;
  return sglq_quant_rows_i8_dev(x, out, scales, rows, dim, stream);
}

QH_API int sgl_dequant_rows_i8_dev(const int8_t *q, const float *scales, float *out,
                                   int64_t rows, int64_t dim, void *stream) {
  if (rows < 0 || dim < 0) return -1;
  if (rows == 0 || dim == 0) return 0;
  if (!q || !scales || !out) return -1;
  return sglq_dequant_rows_i8_dev(q, scales, out, rows, dim, stream);
}

/* ---- config.json quantization_config (reference src/qweight.c:375-482) ---------------- */
QH_API int sgl_qcfg_from_json(const char *json, size_t len, sgl_qcfg *cfg) {
  if (!cfg) return 0;
  memset(cfg, 0, sizeof(*cfg));
  cfg->method = SGL_Q_NONE;
  if (!json || len == 0) return 0;
  qj *root = qj_parse(json, len);
  if (!root) return 0;
  const qj *qc = qj_get(root, "quantization_config");
  int ok = 0;
  if (!qc || qc->type != QJ_OBJ) goto done;
  const char *method = qj_str(qc, "quant_method", "");
  cfg->bits = qj_int(qc, "bits", 4);
  cfg->group_size = qj_int(qc, "group_size", 128);
  if (!strcmp(method, "awq")) {
    cfg->method = SGL_Q_AWQ;
    cfg->zero_point = qj_bool(qc, "zero_point", 1);
    const char *ver = qj_str(qc, "version", "gemm");
    cfg->transposed = !strcmp(ver, "gemv");
    if (!strcmp(ver, "marlin")) cfg->layout = SGL_QLAYOUT_MARLIN;
  } else if (!strcmp(method, "gptq")) {
    cfg->method = SGL_Q_GPTQ;
    cfg->zero_point = 1;
    cfg->desc_act = qj_bool(qc, "desc_act", 0);
    const char *fmt = qj_str(qc, "format", "gptq");
    if (!strcmp(fmt, "gptq_v2")) {
      cfg->v2 = 1;
    } else if (!strcmp(fmt, "marlin") || !strcmp(fmt, "gptq_marlin")) {
      cfg->layout = SGL_QLAYOUT_MARLIN;
    } else if (fmt[0] && strcmp(fmt, "gptq")) {
      QH_ERR("quant: GPTQ format=%s is not supported (gptq / gptq_v2 / marlin)", fmt);
      cfg->method = SGL_Q_NONE;
      goto done;
    }
  } else if (!strcmp(method, "compressed-tensors")) {
    const char *fmt = qj_str(qc, "format", "");
    const qj *groups = qj_get(qc, "config_groups");
    const qj *g0 = groups && groups->type == QJ_OBJ && groups->count > 0 ? groups->items[0] : NULL;
    const qj *wq = g0 ? qj_get(g0, "weights") : NULL;
    int nb = 4, gsz = 128;
    if (wq && wq->type == QJ_OBJ) {
      nb = qj_int(wq, "num_bits", 4);
      gsz = qj_int(wq, "group_size", 128);
      if (gsz <= 0) gsz = 128;
      if (!qj_bool(wq, "symmetric", 1)) goto done; /* asymmetric CT not handled */
    }
    if (strcmp(fmt, "pack-quantized")) goto done;
    if (nb != 4 && nb != 8) goto done;
    cfg->method = SGL_Q_CT;
    cfg->bits = nb;
    cfg->group_size = gsz;
    cfg->packed_dim = qj_int(qc, "packed_dim", 1);
    cfg->offset = 1 << (nb - 1);
    cfg->zero_point = 0;
  } else if (!strcmp(method, "mxfp4")) {
    cfg->method = SGL_Q_MXFP4;
    cfg->bits = 4;
    cfg->group_size = 32;
    cfg->zero_point = 0;
  } else {
    goto done;
  }
  ok = 1;
  qh_info("quant: method=%d bits=%d group=%d zero_point=%d desc_act=%d layout=%d", cfg->method,
          cfg->bits, cfg->group_size, cfg->zero_point, cfg->desc_act, cfg->layout);
done:
  qj_free(root);
  return ok;
}
