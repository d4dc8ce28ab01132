/* sglq_shim.h — the thin C ABI between the C11 host layer (sglang.c_amd/host, C files) and the HIP
 * kernels (sglang.c_amd/csrc, HIP files).  Plain C types only: no HIP or torch types cross it.
 *
 * The host layer validates arguments exactly like the reference (and logs the reason), builds a
 * sglq_plan describing the source format and the device layout, and calls into here.  Every
 * function returns 0 / a handle on success and -1 / NULL on a HIP error (logged). */
#ifndef SGLQ_SHIM_H
#define SGLQ_SHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* source formats the device decoder understands */
enum {
  SGLQ_SRC_GPTQ = 1,   /* qweight i32 [K/pack, N] */
  SGLQ_SRC_AWQ = 2,    /* qweight i32 [K, N/8] (or [N/8, K] when transposed) */
  SGLQ_SRC_MARLIN = 3, /* qweight i32 [K/16, N*16/pack], 16x64 tiles */
  SGLQ_SRC_CT = 4,     /* weight_packed i32 [N, cols], scales [N, K/G] */
  SGLQ_SRC_MXFP4 = 5,  /* blocks u8 [N, cols], e8m0 u8 [N, ceil(K/32)] */
  SGLQ_SRC_W8 = 6,     /* int8 [N, K], scale f32 [N] */
};

/* device code kinds (what one native nibble/byte means) */
enum {
  SGLQ_KIND_U4 = 0,   /* unsigned 4-bit code, per-(group, column) zero + scale */
  SGLQ_KIND_U8 = 1,   /* unsigned 8-bit code (int8 stored +128), zero + scale */
  SGLQ_KIND_E2M1 = 2, /* e2m1 code with one e8m0 scale per 32 k */
};

enum { SGLQ_DT_F32 = 0, SGLQ_DT_BF16 = 1, SGLQ_DT_F16 = 2 };

typedef struct {
  int src;            /* SGLQ_SRC_* */
  int kind;           /* SGLQ_KIND_* */
  int bits;           /* source bits (4 or 8) */
  int transposed;     /* AWQ gemv layout */
  int v2;             /* GPTQ v2: stored zero + 1 */
  int has_zero;       /* per-(group, column) zeros supplied */
  int zconst;         /* zero used when none is supplied */
  int64_t N, K;       /* logical out/in features */
  int64_t G;          /* effective group size along (original) K */
  int64_t ngroups;    /* real groups */
  int64_t gp;         /* padded group length along the device K (multiple of 32) */
  int64_t nsteps;     /* device K / 32 */
  int64_t qw_rows, qw_cols, qz_rows, qz_cols, sc_rows, sc_cols;
  const int32_t *kmap; /* host [nsteps*32]: original k at each device position, or -1 */
  const int32_t *kinv; /* host [K]: device position of original k */
  const int32_t *gidx; /* host [K] group of original k, or NULL (k / G) */
} sglq_plan;

typedef struct sglq_dev sglq_dev; /* device-resident weight (opaque) */

/* Upload the raw buffers (host pointers; sizes implied by the plan), decode and repack them into
 * the device layout.  qzeros/scales/gidx may be NULL where the plan says so. */
sglq_dev *sglq_build(const sglq_plan *plan, const void *qweight, const void *qzeros,
                     const void *scales, int dev);
/* Same, from buffers already in device memory. */
sglq_dev *sglq_build_device(const sglq_plan *plan, const void *qweight, const void *qzeros,
                            const void *scales, int dev);
void sglq_free(sglq_dev *d);

/* Exact dequant of the device layout back to f32 [N, K] row-major (device pointer out). */
int sglq_dequant_dev(sglq_dev *d, float *out_dev, void *stream);
/* Same, into host memory (synchronous). */
int sglq_dequant_host(sglq_dev *d, float *out_host);

/* C[M,N] = A[M,K] * W^T (+ bias), A in a_dtype, everything in device memory. */
int sglq_forward(sglq_dev *d, const void *A, int a_dtype, int64_t M, const float *bias,
                 float *C, void *stream);
/* Same as sglq_forward with the prefill GEMM's workspace in the library's per-device scratch
 * array (noalloc.hip): allocates nothing; -1 if M rows need more than sglq_scratch_bytes(). */
int sglq_forward_noalloc(sglq_dev *d, const void *A, int a_dtype, int64_t M, const float *bias,
                         float *C, void *stream);
size_t sglq_scratch_bytes(void);
/* Host-pointer convenience (synchronous): uploads A/bias, downloads C. */
int sglq_forward_host(sglq_dev *d, const float *A, int64_t M, const float *bias, float *C);

int64_t sglq_N(const sglq_dev *d);
int64_t sglq_K(const sglq_dev *d);
/* bytes of the device layout that one forward streams (codes + scales + zeros) */
int64_t sglq_weight_bytes(const sglq_dev *d);

/* int8 row quantization on host buffers, computed on the GPU (device 0). */
int sglq_quant_rows_i8_host(const float *x, int8_t *out, float *scales, int64_t rows,
                            int64_t dim);
int sglq_dequant_row_i8_host(const int8_t *q, float scale, float *out, int64_t n);
/* f32 NT matmul with host A / bias / C and a device-resident W (from sglq_upload). */
int sglq_matmul_nt_dev_w(const float *A, const float *dW, const float *bias, float *C,
                         int64_t M, int64_t N, int64_t K, int dev);
/* plain device copies of host buffers (the host layer's weight cache) */
void *sglq_upload(const void *host, size_t bytes, int dev);
void sglq_release(void *dptr, int dev);

/* MoE: routed expert FFN over device-resident experts (see sgl_qmoe_forward). */
int sglq_moe_forward(sglq_dev *const *gate_up, sglq_dev *const *down, int n_exp, const void *h,
                     int h_dtype, int64_t T, const int32_t *topk_ids, const float *topk_w,
                     int k, float *out, void *stream);

/* MoE routing and shared experts on the device (route.hip; see sgl_qmoe_route). */
int sglq_moe_router_logits(const float *router_w, int ne, const void *h, int h_dtype, int64_t T,
                           int64_t E, float *logits, void *stream);
int sglq_moe_route(const float *logits, int64_t T, int ne, const float *bias, int sigmoid,
                   int n_group, int topk_group, int k, int norm, float scale, int32_t *ids,
                   float *wts, void *stream);
int sglq_moe_shared(sglq_dev *gate_up, sglq_dev *down, const void *h, int h_dtype, int64_t T,
                    float *out, void *stream);

int sglq_mlp_forward(sglq_dev *gate, sglq_dev *up, sglq_dev *down, const void *h, int h_dtype,
                     int64_t T, float *out, void *stream);
int sglq_quant_rows_i8_dev(const float *x, int8_t *out, float *scales, int64_t rows,
                           int64_t dim, void *stream);
int sglq_dequant_rows_i8_dev(const int8_t *q, const float *scales, float *out, int64_t rows,
                             int64_t dim, void *stream);

/* Logging hook implemented by the host layer. */
void sglq_log_error(const char *fmt, ...);

#ifdef __cplusplus
}
#endif

#endif /* SGLQ_SHIM_H */
