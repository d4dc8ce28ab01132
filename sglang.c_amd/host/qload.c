/* qload.c — the device-resident load path and a minimal safetensors reader.
 *
 * sgl_qlinear_load is the reference loader's quant_get (reference src/safetensors.c:271-471)
 * with the last step changed: it finds the same tensors under the same names, checks the same
 * dtypes and derives N, K and the layout by the same rules (Marlin shape check with fallback to
 * the natural layout, AWQ gemm/gemv orientation from the shapes, CT weight_shape, MXFP4 two
 * codes per byte), converts the scales to f32 exactly as its bytes_to_f32 does, and then hands
 * the packed buffers to sgl_qlinear_create* where the reference called sgl_qweight_dequant*.
 * Tensors are looked up through a callback with the contract of the reference's
 * sgl_st_get_raw (include/sgl/safetensors.h:53-66), so the reference loader can pass its own
 * context; sgl_qst_* is a single-file reader with the same contract for standalone use.
 */
#define _POSIX_C_SOURCE 200809L
#include "sgl/qload.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "qhost.h"

/* ---- single-file safetensors reader --------------------------------------------------- */

struct sgl_qst {
  void *map;
  size_t size;
  qj *header;
  const char *data;
  size_t data_len;
};

QH_API sgl_qst *sgl_qst_open(const char *path) {
  sgl_qst *st = (sgl_qst *)calloc(1, sizeof(sgl_qst));
  if (!st) return NULL;
  const int fd = open(path, O_RDONLY);
  struct stat sb;
  if (fd < 0 || fstat(fd, &sb) != 0) {
    QH_ERR("safetensors: cannot open %s", path);
    if (fd >= 0) close(fd);
    free(st);
    return NULL;
  }
  st->size = (size_t)sb.st_size;
  if (st->size < 8) {
    QH_ERR("safetensors: %s is too small", path);
    close(fd);
    free(st);
    return NULL;
  }
  st->map = mmap(NULL, st->size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (st->map == MAP_FAILED) {
    QH_ERR("safetensors: cannot map %s", path);
    free(st);
    return NULL;
  }
  uint64_t hlen;  /* little-endian u64 header length, then the JSON header, then the data */
  memcpy(&hlen, st->map, 8);
  if (hlen > st->size - 8) {
    QH_ERR("safetensors: header of %s overruns the file", path);
    sgl_qst_close(st);
    return NULL;
  }
  st->header = qj_parse((const char *)st->map + 8, (size_t)hlen);
  if (!st->header || st->header->type != QJ_OBJ) {
    QH_ERR("safetensors: header of %s is not a JSON object", path);
    sgl_qst_close(st);
    return NULL;
  }
  st->data = (const char *)st->map + 8 + hlen;
  st->data_len = st->size - 8 - (size_t)hlen;
  return st;
}

QH_API int sgl_qst_get_raw(sgl_qst *st, const char *name, const char **dtype, int *ndim,
                           int64_t *dims, const void **bytes, size_t *nbytes) {
  if (!st || !name) return 0;
  const qj *e = qj_get(st->header, name);
  if (!e || e->type != QJ_OBJ) return 0;
  const qj *shape = qj_get(e, "shape"), *offs = qj_get(e, "data_offsets");
  /* tensors of 1-4 dimensions, as the reference's shard_raw (src/safetensors.c:204-221) */
  if (!shape || shape->type != QJ_ARR || !offs || offs->type != QJ_ARR || offs->count != 2 ||
      shape->count < 1 || shape->count > 4)
    return 0;
  const double s = offs->items[0]->num, t = offs->items[1]->num;
  if (offs->items[0]->type != QJ_NUM || offs->items[1]->type != QJ_NUM || !(s >= 0) || s > t ||
      t > (double)st->data_len)
    return 0;
  for (int i = 0; i < shape->count; i++) {  /* whole numbers in [0, 2^40]: no later overflow */
    const qj *d = shape->items[i];
    if (d->type != QJ_NUM || !(d->num >= 0 && d->num <= 1099511627776.0) ||
        d->num != (double)(int64_t)d->num)
      return 0;
  }
  if (dtype) *dtype = qj_str(e, "dtype", "");
  if (ndim) *ndim = shape->count;
  if (dims) {
    for (int i = 0; i < 4; i++) dims[i] = 1;
    for (int i = 0; i < shape->count; i++) dims[i] = (int64_t)shape->items[i]->num;
  }
  if (bytes) *bytes = st->data + (size_t)s;
  if (nbytes) *nbytes = (size_t)(t - s);
  return 1;
}

QH_API void sgl_qst_close(sgl_qst *st) {
  if (!st) return;
  if (st->header) qj_free(st->header);
  if (st->map && st->map != MAP_FAILED) munmap(st->map, st->size);
  free(st);
}

/* ---- quant_get on the device ------------------------------------------------------------ */

typedef struct {
  const char *dtype;
  int ndim;
  int64_t dims[4];
  const void *bytes;
  size_t nbytes;
} qraw;

static int raw_get(sgl_qraw_fn fn, void *ctx, const char *name, qraw *r) {
  memset(r, 0, sizeof(*r));
  for (int i = 0; i < 4; i++) r->dims[i] = 1;
  r->dtype = "";
  if (fn(ctx, name, &r->dtype, &r->ndim, r->dims, &r->bytes, &r->nbytes)) {
    /* a lookup that reports nonsense (dims outside [0, 2^40], 0 or > 4 of them) gets zero
     * dims, which every shape check below rejects, instead of overflowing their products */
    int ok = r->ndim >= 1 && r->ndim <= 4 && r->dtype && r->bytes;
    for (int i = 0; i < 4 && ok; i++) ok = r->dims[i] >= 0 && r->dims[i] <= ((int64_t)1 << 40);
    if (!ok) {
      for (int i = 0; i < 4; i++) r->dims[i] = 0;
      r->ndim = 1;
      r->nbytes = 0;
      if (!r->dtype) r->dtype = "";
    }
    return 1;
  }
  memset(r, 0, sizeof(*r));  /* absent: zero dims, as the reference's memset tensors */
  r->dtype = "";
  return 0;
}

/* aligned copy of little-endian int32 data (the mapped bytes need not be aligned) */
static int32_t *as_i32(const qraw *r, int64_t *n) {
  if (r->nbytes % 4) return NULL;
  int32_t *p = (int32_t *)malloc(r->nbytes ? r->nbytes : 4);
  if (!p) return NULL;
  memcpy(p, r->bytes, r->nbytes);
  if (n) *n = (int64_t)(r->nbytes / 4);
  return p;
}

/* IEEE binary16 -> binary32, exact (subnormals normalised, inf/NaN kept) */
static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 31u;
  uint32_t man = h & 1023u, bits;
  if (ex == 0) {
    if (man == 0) {
      bits = sign;
    } else {  /* subnormal: shift the leading one into place */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while (!(man & 1024u));
      bits = sign | (uint32_t)(127 - 15 - e) << 23 | (man & 1023u) << 13;
    }
  } else if (ex == 31) {
    bits = sign | 0x7F800000u | man << 13;
  } else {
    bits = sign | (ex + 112u) << 23 | man << 13;
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* F32 / F16 / BF16 -> f32, as the reference's bytes_to_f32 (src/safetensors.c:247-268) */
static float *as_f32(const qraw *r, int64_t *n) {
  if (!strcmp(r->dtype, "F32")) {
    if (r->nbytes % 4) return NULL;
    float *p = (float *)malloc(r->nbytes ? r->nbytes : 4);
    if (!p) return NULL;
    memcpy(p, r->bytes, r->nbytes);
    if (n) *n = (int64_t)(r->nbytes / 4);
    return p;
  }
  if (!strcmp(r->dtype, "F16") || !strcmp(r->dtype, "BF16")) {
    if (r->nbytes % 2) return NULL;
    const int64_t cnt = (int64_t)(r->nbytes / 2);
    float *p = (float *)malloc((size_t)(cnt ? cnt : 1) * sizeof(float));
    if (!p) return NULL;
    const int bf = !strcmp(r->dtype, "BF16");
    for (int64_t i = 0; i < cnt; i++) {
      uint16_t h;
      memcpy(&h, (const char *)r->bytes + 2 * i, 2);
      if (bf) {
        const uint32_t b = (uint32_t)h << 16;
        memcpy(&p[i], &b, 4);
      } else {
        p[i] = f16_to_f32(h);
      }
    }
    if (n) *n = cnt;
    return p;
  }
  return NULL;
}

/* Everything quant_get decides before its dequant call.  kind: SGL_QLOAD_*.  Buffers are
 * owned (freed by plan_free); bytes of MXFP4 point into the caller's mapping. */
typedef struct {
  sgl_qload_info info;
  sgl_qcfg cfg;  /* the config the create call gets (layout / orientation as decided) */
  qraw qw, qz, sc, gi;
  int32_t *qwv, *qzv, *giv;
  float *scl;
  int64_t sc_rows, sc_cols, gi_n;
} qplan;

static void plan_free(qplan *p) {
  free(p->qwv);
  free(p->qzv);
  free(p->giv);
  free(p->scl);
}

static int name_of(char *out, size_t cap, const char *base, const char *suffix) {
  const int n = snprintf(out, cap, "%s%s", base, suffix);
  return n > 0 && (size_t)n < cap;
}

/* 1 = planned, 0 = base has no quantized tensors (no log, as quant_get's NULL), -1 = error */
static int plan_load(const sgl_qcfg *cfg, sgl_qraw_fn fn, void *ctx, const char *base,
                     qplan *p) {
  memset(p, 0, sizeof(*p));
  char nm[512];
  if (!cfg || !fn || !base) {
    QH_ERR("qload: missing config, lookup or name");
    return -1;
  }
  p->cfg = *cfg;
  /* compressed-tensors and MXFP4 (reference src/safetensors.c:273-343) */
  if (cfg->method == SGL_Q_CT || cfg->method == SGL_Q_MXFP4) {
    const int ct = cfg->method == SGL_Q_CT;
    if (!name_of(nm, sizeof(nm), base, ct ? ".weight_packed" : ".weight")) return 0;
    if (!raw_get(fn, ctx, nm, &p->qw)) return 0;
    if (!name_of(nm, sizeof(nm), base, ct ? ".weight_scale" : ".scales") ||
        !raw_get(fn, ctx, nm, &p->sc)) {
      QH_ERR("quant: missing %s", nm);
      return -1;
    }
    int64_t N = p->qw.dims[0], K = 0;
    if (ct) {
      qraw ws;
      if (name_of(nm, sizeof(nm), base, ".weight_shape") && raw_get(fn, ctx, nm, &ws) &&
          ws.nbytes >= 16) {
        int64_t d[2];
        memcpy(d, ws.bytes, 16);
        N = d[0];
        K = d[1];
      } else {
        K = p->qw.dims[1] * (cfg->bits == 4 ? 8 : 4);
      }
      p->scl = as_f32(&p->sc, NULL);
      if (!p->scl) {
        QH_ERR("quant: %s scales dtype=%s not supported", base, p->sc.dtype);
        return -1;
      }
    } else {
      K = p->qw.dims[1] * 2;  /* two e2m1 codes per byte */
    }
    p->sc_cols = p->sc.dims[p->sc.ndim - 1];
    p->sc_rows = p->sc.dims[p->sc.ndim - 2 >= 0 ? p->sc.ndim - 2 : 0];
    if (N <= 0 || K <= 0) {
      QH_ERR("quant: %s shape cannot be derived (weight [%lld,%lld])", base,
             (long long)p->qw.dims[0], (long long)p->qw.dims[1]);
      return -1;
    }
    if (ct) {
      p->qwv = as_i32(&p->qw, NULL);
      if (!p->qwv) {
        QH_ERR("quant: %s weight_packed is not int32 data", base);
        return -1;
      }
    }
    p->info.kind = ct ? SGL_QLOAD_CT : SGL_QLOAD_MXFP4;
    p->info.N = N;
    p->info.K = K;
    return 1;
  }

  /* AWQ / GPTQ, natural or Marlin (reference src/safetensors.c:345-456) */
  if (!name_of(nm, sizeof(nm), base, ".qweight") || !raw_get(fn, ctx, nm, &p->qw)) return 0;
  if (strcmp(p->qw.dtype, "I32")) {
    QH_ERR("quant: %s dtype=%s, expected I32", nm, p->qw.dtype);
    return -1;
  }
  if (!name_of(nm, sizeof(nm), base, ".scales") || !raw_get(fn, ctx, nm, &p->sc)) {
    QH_ERR("quant: missing %s.scales", base);
    return -1;
  }
  int has_z = name_of(nm, sizeof(nm), base, ".qzeros") && raw_get(fn, ctx, nm, &p->qz);
  if (!has_z && cfg->zero_point) {
    QH_ERR("quant: zero_point is set but %s.qzeros is missing", base);
    return -1;
  }
  const int has_g = name_of(nm, sizeof(nm), base, ".g_idx") && raw_get(fn, ctx, nm, &p->gi);
  int64_t sc_n = 0;
  p->scl = as_f32(&p->sc, &sc_n);
  if (!p->scl) {
    QH_ERR("quant: %s.scales dtype=%s not supported", base, p->sc.dtype);
    return -1;
  }
  int64_t N = p->sc.dims[p->sc.ndim - 1];
  p->sc_rows = sc_n / (N > 0 ? N : 1);
  p->sc_cols = N;
  const int pack = sgl_q_pack(cfg->bits);
  p->qwv = as_i32(&p->qw, NULL);
  if (!p->qwv || (has_z && !(p->qzv = as_i32(&p->qz, NULL)))) {
    QH_ERR("quant: %s packed tensors are not int32 data", base);
    return -1;
  }
  if (cfg->layout == SGL_QLAYOUT_MARLIN) {
    if (cfg->bits != 4 && cfg->bits != 8) {
      QH_ERR("quant(marlin): %s is in the Marlin layout, which has 4 and 8 bits only "
             "(config bits=%d)", base, cfg->bits);
      return -1;
    }
    const int64_t K_m = p->qw.dims[0] * 16;
    if (K_m > 0 && p->qw.dims[1] * pack == N * 16) {
      p->info.kind = SGL_QLOAD_MARLIN;
      p->info.N = N;
      p->info.K = K_m;
      return 1;
    }
    qh_info("quant: %s declares the Marlin layout but qweight [%lld,%lld] does not fit N=%lld "
            "(pack=%d); reading it in the natural layout", base, (long long)p->qw.dims[0],
            (long long)p->qw.dims[1], (long long)N, pack);
    p->cfg.layout = SGL_QLAYOUT_NATURAL;
  }
  int64_t K = 0;
  if (cfg->method == SGL_Q_AWQ) {
    /* gemm: qweight [K, N/pack]; gemv: [N/pack, K]; a square weight fits both, so the config
     * decides first and the shapes correct it */
    const int gemm_ok = p->qw.dims[1] * pack == N;
    const int gemv_ok = p->qw.dims[0] * pack == N;
    if (!cfg->transposed && gemm_ok) {
      K = p->qw.dims[0];
    } else if ((cfg->transposed || !gemm_ok) && gemv_ok) {
      p->cfg.transposed = 1;
      K = p->qw.dims[1];
    } else {
      QH_ERR("quant(awq): %s qweight [%lld,%lld] does not fit N=%lld (pack=%d)", base,
             (long long)p->qw.dims[0], (long long)p->qw.dims[1], (long long)N, pack);
      return -1;
    }
  } else {
    K = p->qw.dims[0] * pack;
    N = p->qw.dims[1];
  }
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  if (N <= 0 || K <= 0 || p->sc_rows < 1) {
    QH_ERR("quant: %s shape cannot be derived (qweight [%lld,%lld], scales [%lld,%lld])", base,
           (long long)p->qw.dims[0], (long long)p->qw.dims[1], (long long)p->sc_rows,
           (long long)N);
    return -1;
  }
  if (!has_g && p->sc_rows != (K + G - 1) / G) {
    QH_ERR("quant: %s has %lld scale rows, K=%lld / group=%lld needs %lld", base,
           (long long)p->sc_rows, (long long)K, (long long)G, (long long)((K + G - 1) / G));
    return -1;
  }
  if (has_g && !(p->giv = as_i32(&p->gi, &p->gi_n))) {
    QH_ERR("quant: %s.g_idx is not int32 data", base);
    return -1;
  }
  p->info.kind = SGL_QLOAD_NATURAL;
  p->info.N = N;
  p->info.K = K;
  return 1;
}

QH_API int sgl_qlinear_probe(const sgl_qcfg *cfg, sgl_qraw_fn raw, void *ctx, const char *base,
                             sgl_qload_info *info) {
  qplan p;
  const int rc = plan_load(cfg, raw, ctx, base, &p);
  if (rc == 1 && info) {
    *info = p.info;
    info->transposed = p.cfg.transposed;
    info->layout = p.cfg.layout;
  }
  plan_free(&p);
  return rc;
}

QH_API sgl_qlinear *sgl_qlinear_load(sgl_qcfg *cfg, sgl_qraw_fn raw, void *ctx,
                                     const char *base, int64_t *out_N, int64_t *out_K, int dev) {
  qplan p;
  if (plan_load(cfg, raw, ctx, base, &p) != 1) {
    plan_free(&p);
    return NULL;
  }
  sgl_qlinear *ql = NULL;
  const int64_t N = p.info.N, K = p.info.K;
  switch (p.info.kind) {
    case SGL_QLOAD_CT:
      ql = sgl_qlinear_create_ct(&p.cfg, p.qwv, p.qw.dims[0], p.qw.dims[1], p.scl, p.sc_rows,
                                 p.sc_cols, N, K, dev);
      break;
    case SGL_QLOAD_MXFP4:
      ql = sgl_qlinear_create_mxfp4((const uint8_t *)p.qw.bytes, p.qw.dims[0], p.qw.dims[1],
                                    (const uint8_t *)p.sc.bytes, p.sc_rows, p.sc_cols, N, K, dev);
      break;
    case SGL_QLOAD_MARLIN:
      ql = sgl_qlinear_create_marlin(&p.cfg, p.qwv, p.qw.dims[0], p.qw.dims[1], p.qzv,
                                     p.qz.dims[0], p.qz.dims[1], p.scl, p.sc_rows, N, N, K, dev);
      break;
    default:
      ql = sgl_qlinear_create(&p.cfg, p.qwv, p.qw.dims[0], p.qw.dims[1], p.qzv, p.qz.dims[0],
                              p.qz.dims[1], p.scl, p.sc_rows, N, p.giv, p.gi_n, N, K, dev);
      break;
  }
  if (ql) {
    cfg->transposed = p.cfg.transposed;  /* as quant_get updates c->q.transposed */
    if (out_N) *out_N = N;
    if (out_K) *out_K = K;
  }
  plan_free(&p);
  return ql;
}
