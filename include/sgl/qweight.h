/* sgl/qweight.h — quantized-weight unpack/dequant API (AWQ, GPTQ, Marlin, compressed-tensors,
 * MXFP4), kept signature-for-signature with the reference so that the engine's loader
 * (reference src/safetensors.c:271-471) links against this library unchanged.
 *
 * Replaces: reference include/sgl/qweight.h:38-105 (types and prototypes) and the
 * implementation in reference src/qweight.c:19-482.  In this build every dequant entry point
 * runs on the GPU: the host buffers are uploaded, decoded by a HIP kernel for gfx950 and the
 * f32 [N,K] result is copied back.  Validation and error returns are done on the host in C11
 * and follow the reference's rules (return -1 plus one error log line).
 *
 * Formats (N = out_features, K = in_features, G = group size, pack = 32/bits):
 *   AWQ  (gemm) qweight i32 [K, N/pack]   column n lives in nibble slot AWQ_REV[n&7] of word
 *        (gemv) qweight i32 [N/pack, K]   (cfg->transposed); qzeros i32 [K/G, N/pack] same slots
 *   GPTQ        qweight i32 [K/pack, N]   row k lives in slot k%pack of word row k/pack;
 *               qzeros i32 [K/G, N/pack]  (word n>>3, slot n%pack); g_idx i32 [K] or NULL
 *   scales f32 [K/G, N] for AWQ/GPTQ/Marlin (the loader widens f16 to f32)
 *   dequant: out[n*K + k] = (float)(q - z) * scale[g][n]
 */
#ifndef SGL_QWEIGHT_H
#define SGL_QWEIGHT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference include/sgl/qweight.h:38-44 */
typedef enum {
  SGL_Q_NONE = 0,
  SGL_Q_AWQ = 1,
  SGL_Q_GPTQ = 2,
  SGL_Q_CT = 3,    /* compressed-tensors pack-quantized (W4A16 / W8A16) */
  SGL_Q_MXFP4 = 4, /* e2m1 elements with one e8m0 scale per 32 along K */
} sgl_qmethod;

/* reference include/sgl/qweight.h:45-56 — plain data, same field order */
typedef struct {
  int method;     /* sgl_qmethod */
  int bits;       /* 4 or 8 (0 means 4) */
  int group_size; /* <= 0: one group spans all of K */
  int zero_point; /* AWQ: qzeros present; GPTQ: always 1 */
  int desc_act;   /* GPTQ act-order (g_idx gives non-contiguous groups) */
  int transposed; /* AWQ gemv variant: qweight stored [N/pack, K] */
  int v2;         /* GPTQ gptq_v2: stored zeros are z-1, add 1 when decoding */
  int packed_dim; /* compressed-tensors: packed dimension */
  int offset;     /* compressed-tensors: unsigned-code offset (8 for 4-bit, 128 for 8-bit) */
  int layout;     /* SGL_QLAYOUT_NATURAL or SGL_QLAYOUT_MARLIN */
} sgl_qcfg;

/* reference include/sgl/qweight.h:65-66 */
#define SGL_QLAYOUT_NATURAL 0
#define SGL_QLAYOUT_MARLIN 1

/* Values per 32-bit word (reference src/qweight.c:19). */
int sgl_q_pack(int bits);

/* AWQ / GPTQ natural layouts -> f32 [N,K].  0 on success, -1 on bad config/shape
 * (reference src/qweight.c:28-141). */
int sgl_qweight_dequant(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                        int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                        int64_t qz_cols, const float *scales, int64_t sc_rows, int64_t sc_cols,
                        const int32_t *g_idx, int64_t g_n, int64_t N, int64_t K, float *out);

/* compressed-tensors pack-quantized, weight_packed i32 [N, K/pack], scales f32 [N, K/G]
 * (reference src/qweight.c:282-322). */
int sgl_qweight_dequant_ct(const sgl_qcfg *cfg, const int32_t *wpacked, int64_t rows,
                           int64_t cols, const float *scales, int64_t sc_rows, int64_t sc_cols,
                           int64_t N, int64_t K, float *out);

/* MXFP4: blocks u8 [N, K/2] (low nibble = even k), scales u8 e8m0 [N, ceil(K/32)]
 * (reference src/qweight.c:334-366). */
int sgl_qweight_dequant_mxfp4(const int32_t *cfg_unused, const uint8_t *wpacked, int64_t rows,
                              int64_t cols, const uint8_t *scales, int64_t sc_rows,
                              int64_t sc_cols, int64_t N, int64_t K, float *out);

/* Marlin 16x64 tile layout, 4 or 8 bit, scales/zeros already Marlin-permuted
 * (reference src/qweight.c:193-275). */
int sgl_qweight_dequant_marlin(const sgl_qcfg *cfg, const int32_t *qweight, int64_t qw_rows,
                               int64_t qw_cols, const int32_t *qzeros, int64_t qz_rows,
                               int64_t qz_cols, const float *scales, int64_t sc_rows,
                               int64_t sc_cols, int64_t N, int64_t K, float *out);

/* Fill cfg from config.json text; 1 when a supported quantization_config was recognised
 * (reference src/qweight.c:375-482). */
int sgl_qcfg_from_json(const char *json, size_t len, sgl_qcfg *cfg);

#ifdef __cplusplus
}
#endif

#endif /* SGL_QWEIGHT_H */
