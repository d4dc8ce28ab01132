/* sgl/qlinear.h — device-resident quantized linear layer (MI355X / gfx950).
 *
 * New entry points with no one-to-one counterpart in the reference: the reference dequantizes
 * AWQ/GPTQ/Marlin/CT/MXFP4 weights to f32 at load time (reference src/safetensors.c:271-471,
 * src/qweight.c) and multiplies the f32 copy with sgl_matmul_nt (reference src/ops.c:243-279),
 * or multiplies int8 weights with sgl_matmul_w8a16 (reference src/quant.c:44-89).  A
 * sgl_qlinear keeps the packed weight resident in HBM instead and runs the multiply on it:
 *
 *   load:     sgl_qlinear_create*  takes the same buffers (and the same validation, error
 *             returns and log lines) as the matching sgl_qweight_dequant* call, so the loader's
 *             quant_get (reference src/safetensors.c:348-457) can pass them through unchanged.
 *   forward:  sgl_qlinear_forward  computes C[M,N] = A[M,K] W^T + bias, where W is exactly the
 *             matrix sgl_qweight_dequant* would have produced; replaces the proj_nt dispatch
 *             (reference src/llama.c:876-884).
 *   checking: sgl_qlinear_dequant  writes that W (f32 [N,K]) to device memory, bit-identical
 *             to the reference dequant.
 *   MoE:      sgl_qmoe_forward     routed expert FFN with the weighted combine of reference
 *             src/deepseek.c:655-677; sgl_qmoe_router_logits + sgl_qmoe_route compute its
 *             routing (:593-633) and sgl_qmoe_shared adds the shared experts (:679-687).
 *
 * All pointers passed to create* are host pointers.  Pointers passed to forward/dequant/moe are
 * device pointers; `stream` is a hipStream_t (NULL = default stream).  A handle is bound to
 * the device it was created on and must not be used by two threads at once, nor by launches on
 * two streams that can overlap: its operand workspace and split-K arrival counters are per
 * handle, so such launches race (order them with events, or give each stream its own handle).
 * Functions return
 * 0 (or a handle) on success and -1 (or NULL) after logging the reason.  A batch of zero rows
 * (M, T or rows = 0) returns 0 at once: its data pointers may be NULL and are not read.
 */
#ifndef SGL_QLINEAR_H
#define SGL_QLINEAR_H

#include <stdint.h>

#include "sgl/qweight.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sgl_qlinear sgl_qlinear;

/* activation element types for forward / MoE */
enum { SGL_QL_F32 = 0, SGL_QL_BF16 = 1, SGL_QL_F16 = 2 };

/* AWQ (gemm / gemv) and GPTQ (incl. act-order g_idx, gptq_v2, 8-bit): same arguments as
 * sgl_qweight_dequant.  A cfg with layout == SGL_QLAYOUT_MARLIN is routed to the Marlin
 * decoder (g_idx must then be NULL, as in the reference). */
sgl_qlinear *sgl_qlinear_create(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                                int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                                int64_t qz_cols, const float *scales, int64_t sc_rows,
                                int64_t sc_cols, const int32_t *g_idx, int64_t g_n, int64_t N,
                                int64_t K, int dev);
/* Marlin layout: same arguments as sgl_qweight_dequant_marlin. */
sgl_qlinear *sgl_qlinear_create_marlin(const sgl_qcfg *cfg, const int32_t *qweight,
                                       int64_t qw_rows, int64_t qw_cols, const int32_t *qzeros,
                                       int64_t qz_rows, int64_t qz_cols, const float *scales,
                                       int64_t sc_rows, int64_t sc_cols, int64_t N, int64_t K,
                                       int dev);
/* compressed-tensors pack-quantized: same arguments as sgl_qweight_dequant_ct. */
sgl_qlinear *sgl_qlinear_create_ct(const sgl_qcfg *cfg, const int32_t *wpacked, int64_t rows,
                                   int64_t cols, const float *scales, int64_t sc_rows,
                                   int64_t sc_cols, int64_t N, int64_t K, int dev);
/* MXFP4: same arguments as sgl_qweight_dequant_mxfp4. */
sgl_qlinear *sgl_qlinear_create_mxfp4(const uint8_t *wpacked, int64_t rows, int64_t cols,
                                      const uint8_t *scales, int64_t sc_rows, int64_t sc_cols,
                                      int64_t N, int64_t K, int dev);
/* W8 per-row int8 (the operands of sgl_matmul_w8a16): W int8 [N,K], sw f32 [N]. */
sgl_qlinear *sgl_qlinear_create_w8(const int8_t *W, const float *sw, int64_t N, int64_t K,
                                   int dev);

/* C[M,N] = A[M,K] * W^T + bias (bias may be NULL).  A is row-major with a_dtype elements,
 * C is f32 row-major.  Any M >= 1. */
int sgl_qlinear_forward(sgl_qlinear *ql, const void *A, int a_dtype, int64_t M,
                        const float *bias, float *C, void *stream);

/* sgl_qlinear_forward that allocates nothing.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * sgl_qlinear_forward; the prefill GEMM (M > 32 rows of f32, M > 24 of 16-bit activations)
 * takes its workspace from a 64 MiB array the library holds on every GPU it runs on, and
 * returns -1 (after a log line) when M rows need more than that (e.g. K = 4096: about 4000
 * f32 rows, 8000 16-bit rows).  All calls on one GPU share that array: calls that can overlap
 * on one GPU (two streams, two threads) race, so order them. */
int sgl_qlinear_forward_noalloc(sgl_qlinear *ql, const void *A, int a_dtype, int64_t M,
                                const float *bias, float *C, void *stream);

/* W as f32 [N,K] into device memory: bit-identical to the reference dequant of the inputs. */
int sgl_qlinear_dequant(sgl_qlinear *ql, float *out, void *stream);

int64_t sgl_qlinear_out_features(const sgl_qlinear *ql);
int64_t sgl_qlinear_in_features(const sgl_qlinear *ql);
/* HBM bytes of the resident weight one forward streams (codes + scales + zeros). */
int64_t sgl_qlinear_weight_bytes(const sgl_qlinear *ql);

void sgl_qlinear_destroy(sgl_qlinear *ql);

/* Routed-expert FFN of one MoE block (reference src/deepseek.c:655-677, fused gate/up):
 * for each token t and slot j < k with e = topk_ids[t*k + j] >= 0:
 *   gu = h_t * gate_up[e]^T ([2*mi]);  a_i = silu(gu_i) * gu_{mi+i};  o = a * down[e]^T ([E]);
 *   out_t += topk_w[t*k + j] * o, slots summed in order j = 0..k-1 (deterministic).
 * gate_up[e] is [2*mi, E], down[e] is [E, mi]; h is [T, E] (h_dtype), out f32 [T, E];
 * topk_ids (int32) / topk_w (f32) are [T, k] device arrays. */
int sgl_qmoe_forward(sgl_qlinear *const *gate_up, sgl_qlinear *const *down, int n_experts,
                     const void *h, int h_dtype, int64_t T, const int32_t *topk_ids,
                     const float *topk_w, int k, float *out, void *stream);

/* Routing of one MoE block on the device (reference src/deepseek.c:593-633; with
 * sgl_qmoe_router_logits, sgl_qmoe_forward and sgl_qmoe_shared the whole block runs on one
 * stream with no host synchronisation). */
typedef struct {
  int sigmoid;        /* 1: sigmoid scores (scoring_func "sigmoid"), 0: softmax */
  int n_group;        /* > 1: group_limited_greedy over n_group equal groups of experts */
  int topk_group;     /* groups kept (1 .. n_group) */
  int k;              /* experts per token */
  int norm_topk;      /* norm_topk_prob: weights / (their sum + 1e-20) when k > 1 */
  float routed_scale; /* routed_scaling_factor */
} sgl_qmoe_routing;

/* logits[t][e] = h_t . router_w[e]: the router product (reference :594, sgl_matmul_nt on the
 * f32 router weight); router_w f32 [n_experts, E], h [T, E] (h_dtype), logits f32 [T,
 * n_experts], all device memory.  fp32 accumulation in another order than the reference's, so
 * logits agree to rounding, not bit for bit.  E at most 16384. */
int sgl_qmoe_router_logits(const float *router_w, int n_experts, const void *h, int h_dtype,
                           int64_t T, int64_t E, float *logits, void *stream);

/* topk_ids int32 [T, k] and topk_w f32 [T, k] from the logits: scores, e_bias (the
 * e_score_correction_bias, may be NULL) added for the choice only, group-limited greedy choice,
 * top-k with ties to the lower index (-1 with weight 0 when fewer than k experts remain),
 * weights from the uncorrected scores.  At most 256 experts and 64 groups. */
int sgl_qmoe_route(const sgl_qmoe_routing *r, const float *logits, const float *e_bias,
                   int n_experts, int64_t T, int32_t *topk_ids, float *topk_w, void *stream);

/* out[t] += the shared experts' SwiGLU MLP of h_t (reference :679-687, added after the routed
 * sum): gate_up [2*sh, E] (gate rows, then up rows), down [E, sh]. */
int sgl_qmoe_shared(sgl_qlinear *gate_up, sgl_qlinear *down, const void *h, int h_dtype,
                    int64_t T, float *out, void *stream);

/* Dense SwiGLU MLP of T rows (reference src/llama.c:1162-1176 mlp_rows with proj_nt):
 * out = (silu(h gate^T) * (h up^T)) down^T, silu(g) = g / (1 + expf(-g)); up == NULL means gate
 * is the fused [2*I, E] weight (gate rows, then up rows).  h [T, E] (h_dtype), out f32 [T, E]. */
int sgl_qmlp_forward(sgl_qlinear *gate, sgl_qlinear *up, sgl_qlinear *down, const void *h,
                     int h_dtype, int64_t T, float *out, void *stream);

/* Device-pointer, stream-ordered twins of sgl_quant_rows_i8 / sgl_dequant_row_i8 (sgl/quant.h,
 * same arithmetic, bit for bit): the int8 KV-cache rows quantized where they are produced
 * (reference src/llama.c:1264-1267, 1485-1488).  x f32 [rows, dim] -> out int8 [rows, dim] +
 * scales f32 [rows]; dequant: out[r][i] = q[r][i] * scales[r]. */
int sgl_quant_rows_i8_dev(const float *x, int8_t *out, float *scales, int64_t rows, int64_t dim,
                          void *stream);
int sgl_dequant_rows_i8_dev(const int8_t *q, const float *scales, float *out, int64_t rows,
                            int64_t dim, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SGL_QLINEAR_H */
