/* sgl/qload.h — device-resident load path for quantized linear weights (MI355X / gfx950).
 *
 * The reference's loader turns every AWQ/GPTQ/Marlin/CT/MXFP4 weight into an f32 [N,K] copy
 * at load time (quant_get, reference src/safetensors.c:271-471, called from sgl_st_get at
 * :933-967).  sgl_qlinear_load takes the same tensors and the same decisions but keeps the
 * packed weight: it returns a resident sgl_qlinear (sgl/qlinear.h) instead of the f32 buffer.
 *
 * Tensors are found through a callback with the contract of the reference's sgl_st_get_raw
 * (include/sgl/safetensors.h:53-66): return 1 and a view of the named tensor (dtype string,
 * 1-4 dims, bytes valid while the source is open), or 0 when there is none.  The reference
 * loader passes sgl_st_get_raw and its sgl_st_ctx; sgl_qst_* below is a single-file reader
 * with the same contract.
 */
#ifndef SGL_QLOAD_H
#define SGL_QLOAD_H

#include <stddef.h>
#include <stdint.h>

#include "sgl/qlinear.h"
#include "sgl/qweight.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef int (*sgl_qraw_fn)(void *ctx, const char *name, const char **dtype, int *ndim,
                           int64_t *dims, const void **bytes, size_t *nbytes);

/* which create call a weight takes */
enum { SGL_QLOAD_NATURAL = 0, SGL_QLOAD_MARLIN = 1, SGL_QLOAD_CT = 2, SGL_QLOAD_MXFP4 = 3 };

typedef struct {
  int kind;        /* SGL_QLOAD_* */
  int64_t N, K;    /* out_features, in_features */
  int transposed;  /* AWQ: gemv layout (qweight [N/pack, K]) */
  int layout;      /* SGL_QLAYOUT_* actually used (Marlin falls back when shapes do not fit) */
} sgl_qload_info;

/* Tensors <base>.qweight / .qzeros / .scales / .g_idx (AWQ, GPTQ, Marlin), <base>.weight_packed
 * / .weight_scale / .weight_shape (compressed-tensors), <base>.weight / .scales (MXFP4), looked
 * up and checked as quant_get does.  Returns NULL when base has no quantized tensors (silently,
 * like quant_get) or after one error line.  Like quant_get, an AWQ weight whose shapes only fit
 * the gemv layout sets cfg->transposed.  out_N / out_K (may be NULL) receive the shape. */
sgl_qlinear *sgl_qlinear_load(sgl_qcfg *cfg, sgl_qraw_fn raw, void *ctx, const char *base,
                              int64_t *out_N, int64_t *out_K, int dev);

/* The same lookups and checks without a device: 1 = loadable (info filled), 0 = no quantized
 * tensors under base, -1 = error (logged). */
int sgl_qlinear_probe(const sgl_qcfg *cfg, sgl_qraw_fn raw, void *ctx, const char *base,
                      sgl_qload_info *info);

/* Single-file safetensors reader (read-only mmap).  get_raw follows sgl_qraw_fn with the
 * reader as ctx. */
typedef struct sgl_qst sgl_qst;
sgl_qst *sgl_qst_open(const char *path);
int sgl_qst_get_raw(sgl_qst *st, const char *name, const char **dtype, int *ndim, int64_t *dims,
                    const void **bytes, size_t *nbytes);
void sgl_qst_close(sgl_qst *st);

#ifdef __cplusplus
}
#endif

#endif
