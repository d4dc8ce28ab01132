/* quant.c — the reference's int8 C API (include/sgl/quant.h) and the dense f32 NT matmul
 * (include/sgl/ops.h), host side, C11.  Host buffers in and out; the arithmetic runs in HIP
 * kernels (csrc/int8.hip, csrc/gemv.hip, csrc/gemm.hip) on device 0.
 *   sgl_quant_row(s)_i8 / sgl_dequant_row_i8: reference src/quant.c:13-42, bit-identical.
 *   sgl_matmul_w8a16: reference src/quant.c:44-89, fp32 accumulation of exact int8 codes.
 *   sgl_matmul_nt:    reference src/ops.c:243-279, fp32 accumulation.
 * The weights of the two matmuls are uploaded on first use and kept on the device
 * (include/sgl/qcache.h); later calls move only the activations and the result. */
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "qhost.h"
#include "sgl/ops.h"
#include "sgl/qcache.h"
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

/* ---- device copies of host weights ------------------------------------------------------ */
enum { QC_W8 = 1, QC_F32 = 2 };

typedef struct {
  int kind; /* 0 = free slot */
  const void *w, *s;
  int64_t N, K;
  uint64_t fp;
  sglq_dev *d; /* QC_W8 */
  void *dw;    /* QC_F32: device f32 [N, K] */
  size_t bytes;
  uint64_t tick;
} qc_entry;

#define QC_SLOTS 1024
static qc_entry g_qc[QC_SLOTS];
static pthread_mutex_t g_qc_mu = PTHREAD_MUTEX_INITIALIZER;
static size_t g_qc_bytes;
static uint64_t g_qc_tick;

/* FNV-1a over 64 evenly spaced 8-byte samples, the first and last 64 bytes, and (when given)
 * every byte of `all`. */
static uint64_t qc_fingerprint(const void *w, size_t wbytes, const void *all, size_t abytes) {
  uint64_t h = 1469598103934665603ull;
  const unsigned char *p = (const unsigned char *)w;
#define QC_MIX(b)                  \
  do {                             \
    h ^= (uint64_t)(b);            \
    h *= 1099511628211ull;         \
  } while (0)
  for (size_t i = 0; i < 64 && i < wbytes; i++) QC_MIX(p[i]);
  for (size_t i = wbytes > 64 ? wbytes - 64 : 0; i < wbytes; i++) QC_MIX(p[i]);
  if (wbytes >= 8)
    for (int j = 0; j < 64; j++) {
      const size_t o = (size_t)((wbytes - 8) * (uint64_t)j / 63);
      for (int b = 0; b < 8; b++) QC_MIX(p[o + b]);
    }
  const unsigned char *q = (const unsigned char *)all;
  for (size_t i = 0; i < abytes; i++) QC_MIX(q[i]);
#undef QC_MIX
  return h;
}

static size_t qc_limit(void) {
  const char *v = getenv("SGL_QCACHE_MB");
  const long mb = v ? atol(v) : 16384;
  return (size_t)(mb > 0 ? mb : 16384) << 20;
}

static void qc_drop(qc_entry *e) {
  if (e->kind == QC_W8) sglq_free(e->d);
  if (e->kind == QC_F32) sglq_release(e->dw, 0);
  g_qc_bytes -= e->bytes;
  memset(e, 0, sizeof(*e));
}

/* a free slot after dropping least recently used entries until `bytes` more fit (lock held) */
static qc_entry *qc_make_room(size_t bytes) {
  const size_t lim = qc_limit();
  for (;;) {
    qc_entry *lru = NULL, *freeslot = NULL;
    for (int i = 0; i < QC_SLOTS; i++) {
      if (!g_qc[i].kind) {
        if (!freeslot) freeslot = &g_qc[i];
      } else if (!lru || g_qc[i].tick < lru->tick) {
        lru = &g_qc[i];
      }
    }
    if (freeslot && (g_qc_bytes + bytes <= lim || !lru)) return freeslot;
    if (!lru) return NULL;
    qc_drop(lru);
  }
}

static qc_entry *qc_find(int kind, const void *w, const void *s, int64_t N, int64_t K,
                         uint64_t fp) {
  for (int i = 0; i < QC_SLOTS; i++) {
    qc_entry *e = &g_qc[i];
    if (e->kind == kind && e->w == w && e->s == s && e->N == N && e->K == K) {
      if (e->fp == fp) return e;
      qc_drop(e); /* same buffer, different contents: the old copy is stale */
    }
  }
  return NULL;
}

QH_API int sgl_qcache_release(const void *weight) {
  int n = 0;
  pthread_mutex_lock(&g_qc_mu);
  for (int i = 0; i < QC_SLOTS; i++)
    if (g_qc[i].kind && g_qc[i].w == weight) {
      qc_drop(&g_qc[i]);
      n++;
    }
  pthread_mutex_unlock(&g_qc_mu);
  return n;
}

QH_API int sgl_qcache_clear(void) {
  int n = 0;
  pthread_mutex_lock(&g_qc_mu);
  for (int i = 0; i < QC_SLOTS; i++)
    if (g_qc[i].kind) {
      qc_drop(&g_qc[i]);
      n++;
    }
  pthread_mutex_unlock(&g_qc_mu);
  return n;
}

/* C = bias (or 0) row by row: the reference's result when K <= 0 (an empty sum) */
static void bias_rows(const float *bias, float *C, int M, int N) {
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) C[(size_t)m * N + n] = bias ? bias[n] : 0.f;
}

QH_API void sgl_matmul_w8a16(const float *A, const int8_t *W, const float *sw, const float *bias,
                             float *C, int M, int N, int K) {
  if (M <= 0 || N <= 0) return;
  if (K <= 0) {
    bias_rows(bias, C, M, N);
    return;
  }
  pthread_mutex_lock(&g_qc_mu);
  const uint64_t fp = qc_fingerprint(W, (size_t)N * (size_t)K, sw, (size_t)N * sizeof(float));
  qc_entry *e = qc_find(QC_W8, W, sw, N, K, fp);
  if (!e) {
    sglq_dev *d = qh_build_w8(W, sw, N, K, 0);
    const size_t bytes = d ? (size_t)sglq_weight_bytes(d) : 0;
    if (d && (e = qc_make_room(bytes)) != NULL) {
      *e = (qc_entry){QC_W8, W, sw, N, K, fp, d, NULL, bytes, 0};
      g_qc_bytes += bytes;
    } else {
      sglq_free(d);
    }
  }
  int rc = -1;
  if (e) {
    e->tick = ++g_qc_tick;
    rc = sglq_forward_host(e->d, A, M, bias, C);
  }
  pthread_mutex_unlock(&g_qc_mu);
  if (rc != 0) {
    QH_ERR("sgl_matmul_w8a16: device failure");
    abort();
  }
}

QH_API void sgl_matmul_nt(const float *A, const float *W, const float *bias, float *C, int M,
                          int N, int K) {
  if (M <= 0 || N <= 0) return;
  if (K <= 0) {
    bias_rows(bias, C, M, N);
    return;
  }
  const size_t bytes = (size_t)N * (size_t)K * sizeof(float);
  pthread_mutex_lock(&g_qc_mu);
  const uint64_t fp = qc_fingerprint(W, bytes, NULL, 0);
  qc_entry *e = qc_find(QC_F32, W, NULL, N, K, fp);
  if (!e) {
    void *dw = sglq_upload(W, bytes, 0);
    if (dw && (e = qc_make_room(bytes)) != NULL) {
      *e = (qc_entry){QC_F32, W, NULL, N, K, fp, NULL, dw, bytes, 0};
      g_qc_bytes += bytes;
    } else {
      sglq_release(dw, 0);
    }
  }
  int rc = -1;
  if (e) {
    e->tick = ++g_qc_tick;
    rc = sglq_matmul_nt_dev_w(A, (const float *)e->dw, bias, C, M, N, K, 0);
  }
  pthread_mutex_unlock(&g_qc_mu);
  if (rc != 0) {
    QH_ERR("sgl_matmul_nt: device failure");
    abort();
  }
}
