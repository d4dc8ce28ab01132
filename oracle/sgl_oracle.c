/* sgl_oracle.c — CPU restatement of the reference's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP product is compared against:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library (sglang.c_amd) never links, calls or falls back to it.
 *
 * Every function restates one reference function, cited file:line (paths relative to the
 * reference repository), with the same arithmetic in the same order so results are
 * bit-identical when built with the reference's flags (-O2 -march=x86-64-v2 -funroll-loops
 * -fopenmp, reference CMakeLists.txt:30-60).  Symbols carry an orc_ prefix so the oracle and
 * the product can live in one process.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   orc_qweight_dequant*      golden vectors from the compiled reference + inline KATs of
 *                             reference tests/test_qweight.c:130-225 + closed forms
 *   orc_qweight_dequant_marlin reference tests/_marlin_unit.json (4 cases, exact)
 *   orc_qweight_dequant_mxfp4 exhaustive 16 codes x 256 exponents vs ldexp closed form
 *   orc_quant_row(s)_i8       golden vectors + round-half-away / clamp / zero-row edge cases
 *   orc_matmul_w8a16/_nt      golden vectors (bit-exact) + fp64 brute-force dot (tolerance)
 *   orc_moe_ffn               brute-force composition in float64 on tiny expert sets
 *   orc_moe_route             an independent numpy formulation (sorts and masks) on random
 *                             logits, plus hand-built ties, masked groups and k = 1 cases
 *   orc_moe_shared            float64 brute force of the shared SwiGLU MLP
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_ERR(...) (fprintf(stderr, "[oracle] " __VA_ARGS__), fputc('\n', stderr))

typedef struct {
  int method, bits, group_size, zero_point, desc_act, transposed, v2, packed_dim, offset, layout;
} orc_qcfg; /* same field order as reference include/sgl/qweight.h:45-56 */

enum { ORC_AWQ = 1, ORC_GPTQ = 2 };

int orc_q_pack(int bits) { return bits > 0 ? 32 / bits : 0; } /* reference src/qweight.c:19 */

/* reference src/qweight.c:22-26: AWQ stores natural column n in nibble slot rev[n & 7]. */
static const int ORC_AWQ_SLOT[8] = {0, 4, 1, 5, 2, 6, 3, 7};
static inline int orc_code(uint32_t w, int slot, int bits, uint32_t mask) {
  return (int)((w >> (bits * slot)) & mask);
}

/* reference src/qweight.c:28-141 */
int orc_qweight_dequant(const orc_qcfg *cfg, const int32_t *qw, int64_t qw_rows, int64_t qw_cols,
                        const int32_t *qz, int64_t qz_rows, int64_t qz_cols, const float *sc,
                        int64_t sc_rows, int64_t sc_cols, const int32_t *g_idx, int64_t g_n,
                        int64_t N, int64_t K, float *out) {
  if (!cfg || !qw || !sc || !out || N <= 0 || K <= 0) return -1;
  const int bits = cfg->bits ? cfg->bits : 4;
  if (bits != 4 && bits != 8) return ORC_ERR("bits %d", bits), -1;
  if (cfg->method != ORC_AWQ && cfg->method != ORC_GPTQ) return ORC_ERR("method"), -1;
  if (cfg->method == ORC_AWQ && bits != 4) return ORC_ERR("awq bits"), -1;
  const int pack = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  if (sc_cols != N) return ORC_ERR("scales cols"), -1;
  if (qz && qz_cols * pack < N) return ORC_ERR("qzeros cols"), -1;
  if (cfg->method == ORC_AWQ) {
    if (cfg->transposed ? (qw_rows * pack < N || qw_cols != K)
                        : (qw_rows != K || qw_cols * pack < N))
      return ORC_ERR("awq qweight shape"), -1;
    for (int64_t k = 0; k < K; k++) {
      const int64_t g = k / G;
      if (g >= sc_rows) return ORC_ERR("awq group vs scales"), -1;
      if (qz && g >= qz_rows) return ORC_ERR("awq group vs qzeros"), -1;
      for (int64_t n = 0; n < N; n++) {
        const int slot = ORC_AWQ_SLOT[n & 7];
        const uint32_t w = (uint32_t)(cfg->transposed ? qw[(n >> 3) * qw_cols + k]
                                                      : qw[k * qw_cols + (n >> 3)]);
        int q = orc_code(w, slot, bits, mask);
        if (qz) q -= orc_code((uint32_t)qz[g * qz_cols + (n >> 3)], slot, bits, mask);
        out[n * K + k] = (float)q * sc[g * N + n];
      }
    }
    return 0;
  }
  if (qw_cols != N || qw_rows * pack < K) return ORC_ERR("gptq qweight shape"), -1;
  if (g_idx && g_n < K) return ORC_ERR("g_idx short"), -1;
  for (int64_t k = 0; k < K; k++) {
    const int64_t g = g_idx ? (int64_t)g_idx[k] : k / G;
    if (g < 0 || g >= sc_rows) return ORC_ERR("gptq group vs scales"), -1;
    if (qz && g >= qz_rows) return ORC_ERR("gptq group vs qzeros"), -1;
    const int slot = (int)(k % pack);
    for (int64_t n = 0; n < N; n++) {
      int q = orc_code((uint32_t)qw[(k / pack) * qw_cols + n], slot, bits, mask);
      /* zero word index is n>>3 for every bit width (reference src/qweight.c:136) */
      if (qz) q -= orc_code((uint32_t)qz[g * qz_cols + (n >> 3)], (int)(n % pack), bits, mask) +
                   (cfg->v2 ? 1 : 0);
      out[n * K + k] = (float)q * sc[g * N + n];
    }
  }
  return 0;
}

/* reference src/qweight.c:173-191: where natural column n sits in the Marlin-permuted scale row
 * (sidx) and in the interleaved, packed zero row (zcol word, znib slot). */
static void orc_marlin_col(int64_t n, int pack, int64_t *sidx, int64_t *zcol, int *znib) {
  const int64_t f = (n / 64) * 64 + 8 * (n & 7) + ((n % 64) >> 3);
  *sidx = f;
  int pos, gsz;
  if (pack == 8) {
    const int j = (int)(f & 7);
    pos = (j >> 1) + 4 * (j & 1);
    gsz = 8;
  } else {
    const int j = (int)(f & 3);
    pos = ((j & 1) << 1) | (j >> 1);
    gsz = 4;
  }
  const int64_t f2 = gsz * (f / gsz) + pos;
  *zcol = f2 / pack;
  *znib = (int)(f2 % pack);
}

/* reference src/qweight.c:193-275 */
int orc_qweight_dequant_marlin(const orc_qcfg *cfg, const int32_t *qw, int64_t qw_rows,
                               int64_t qw_cols, const int32_t *qz, int64_t qz_rows,
                               int64_t qz_cols, const float *sc, int64_t sc_rows, int64_t sc_cols,
                               int64_t N, int64_t K, float *out) {
  if (!cfg || !qw || !sc || !out || N <= 0 || K <= 0) return -1;
  const int bits = cfg->bits ? cfg->bits : 4;
  if (bits != 4 && bits != 8) return ORC_ERR("marlin bits"), -1;
  const int pack = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  const int qoff = 1 << (bits - 1);
  if (K % 16 != 0 || N % 64 != 0) return ORC_ERR("marlin K/N"), -1;
  if (qw_rows != K / 16 || qw_cols * pack < N * 16) return ORC_ERR("marlin qweight"), -1;
  if (sc_cols != N) return ORC_ERR("marlin scales"), -1;
  if (qz && (qz_cols * pack < N || qz_rows < sc_rows)) return ORC_ERR("marlin qzeros"), -1;
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  const int64_t tile_words = 64 * 16 / pack;
  static const int K8[4] = {0, 8, 1, 9};
  for (int64_t kt = 0; kt < K / 16; kt++)
    for (int64_t nt = 0; nt < N / 64; nt++) {
      const int32_t *tile = qw + kt * qw_cols + nt * tile_words;
      for (int p = 0; p < (int)tile_words; p++) {
        const uint32_t w = (uint32_t)tile[p];
        for (int j = 0; j < pack; j++) {
          int ko, no;
          if (bits == 4) {
            ko = 2 * ((p >> 2) & 3) + ((j & 1) ? 8 : 0) + (j >= 4 ? 1 : 0);
            no = 16 * (p & 3) + (p >> 4) + ((j & 2) ? 8 : 0);
          } else {
            ko = 2 * ((p >> 3) & 3) + K8[j];
            no = 16 * ((p >> 1) & 3) + (p >> 5) + ((p & 1) ? 8 : 0);
          }
          const int64_t k = kt * 16 + ko, n = nt * 64 + no, g = k / G;
          if (g >= sc_rows) return ORC_ERR("marlin group vs scales"), -1;
          int64_t sidx, zcol;
          int znib;
          orc_marlin_col(n, pack, &sidx, &zcol, &znib);
          int q = (int)((w >> (bits * j)) & mask);
          if (qz) {
            if (g >= qz_rows) return ORC_ERR("marlin group vs qzeros"), -1;
            q -= orc_code((uint32_t)qz[g * qz_cols + zcol], znib, bits, mask);
          } else {
            q -= qoff;
          }
          out[n * K + k] = (float)q * sc[g * sc_cols + sidx];
        }
      }
    }
  return 0;
}

/* reference src/qweight.c:282-322 */
int orc_qweight_dequant_ct(const orc_qcfg *cfg, const int32_t *wp, int64_t rows, int64_t cols,
                           const float *sc, int64_t sc_rows, int64_t sc_cols, int64_t N,
                           int64_t K, float *out) {
  (void)sc_rows;
  if (!cfg || !wp || !sc || !out || N <= 0 || K <= 0) return -1;
  const int bits = cfg->bits ? cfg->bits : 4;
  const int64_t G = cfg->group_size > 0 ? cfg->group_size : K;
  const int off = cfg->offset ? cfg->offset : (1 << (bits - 1));
  if (sc_cols != (K + G - 1) / G) return ORC_ERR("ct scales"), -1;
  if (rows != N) return ORC_ERR("ct rows"), -1;
  if (cols * (bits == 4 ? 8 : 4) < K) return ORC_ERR("ct cols"), -1;
  for (int64_t n = 0; n < N; n++) {
    const int32_t *row = wp + n * cols;
    const float *srow = sc + n * sc_cols;
    for (int64_t k = 0; k < K; k++) {
      int code;
      if (bits == 4) {
        const uint8_t b = ((const uint8_t *)row)[k >> 1];
        code = (k & 1) ? (b >> 4) : (b & 0xF);
      } else {
        code = (int)(((uint32_t)row[k >> 2] >> (8 * (k & 3))) & 0xFFu);
      }
      out[n * K + k] = (float)(code - off) * srow[k / G];
    }
  }
  return 0;
}

/* reference src/qweight.c:325-329 (OCP e2m1 code book, bit 3 is the sign) */
static float orc_e2m1(int code) {
  static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  return (code & 8) ? -mag[code & 7] : mag[code & 7];
}

/* reference src/qweight.c:334-366 */
int orc_qweight_dequant_mxfp4(const int32_t *cfg_unused, const uint8_t *wp, int64_t rows,
                              int64_t cols, const uint8_t *sc, int64_t sc_rows, int64_t sc_cols,
                              int64_t N, int64_t K, float *out) {
  (void)cfg_unused;
  (void)sc_rows;
  if (!wp || !sc || !out || N <= 0 || K <= 0) return -1;
  if (rows != N) return ORC_ERR("mxfp4 rows"), -1;
  if (cols * 2 < K) return ORC_ERR("mxfp4 cols"), -1;
  const int64_t nb = (K + 31) / 32;
  if (sc_cols != nb) return ORC_ERR("mxfp4 scales"), -1;
  for (int64_t n = 0; n < N; n++)
    for (int64_t k = 0; k < K; k++) {
      const uint8_t b = wp[n * cols + (k >> 1)];
      const int code = (k & 1) ? (b >> 4) : (b & 0xF);
      const unsigned ex = sc[n * nb + (k >> 5)];
      const float s = ex == 255 ? 0.f : ldexpf(1.0f, (int)ex - 127);
      out[n * K + k] = orc_e2m1(code) * s;
    }
  return 0;
}

/* reference src/quant.c:13-32 */
float orc_quant_row_i8(const float *x, int8_t *out, int n) {
  float maxabs = 0;
  for (int i = 0; i < n; i++) {
    const float a = x[i] < 0 ? -x[i] : x[i];
    if (a > maxabs) maxabs = a;
  }
  if (maxabs <= 0) {
    memset(out, 0, (size_t)n);
    return 0;
  }
  const float scale = maxabs / 127.0f;
  const float inv = 1.0f / scale;
  for (int i = 0; i < n; i++) {
    int v = (int)(x[i] * inv + (x[i] >= 0 ? 0.5f : -0.5f));
    v = v > 127 ? 127 : (v < -127 ? -127 : v);
    out[i] = (int8_t)v;
  }
  return scale;
}

/* reference src/quant.c:34-42 */
void orc_quant_rows_i8(const float *x, int8_t *out, float *scales, int rows, int dim) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++)
    scales[r] = orc_quant_row_i8(x + (size_t)r * dim, out + (size_t)r * dim, dim);
}
void orc_dequant_row_i8(const int8_t *q, float scale, float *out, int n) {
  for (int i = 0; i < n; i++) out[i] = (float)q[i] * scale;
}

/* reference src/quant.c:44-89 (the SSE4.1 branch, which -march=x86-64-v2 selects): 16 k per
 * step into four 4-lane accumulators, multiply then add (no fused multiply-add), lanes combined
 * (a0+a1)+(a2+a3) then (p0+p1)+(p2+p3), scalar tail, scale after the sum. */
void orc_matmul_w8a16(const float *A, const int8_t *W, const float *sw, const float *bias,
                      float *C, int M, int N, int K) {
#pragma omp parallel for
  for (int m = 0; m < M; m++) {
    const float *ar = A + (size_t)m * K;
    for (int n = 0; n < N; n++) {
      const int8_t *wr = W + (size_t)n * K;
      float acc[4][4] = {{0}};
      int k = 0;
      for (; k + 16 <= K; k += 16)
        for (int j = 0; j < 4; j++)
          for (int i = 0; i < 4; i++) {
            const float p = ar[k + 4 * j + i] * (float)wr[k + 4 * j + i];
            acc[j][i] = acc[j][i] + p;
          }
      float part[4];
      for (int i = 0; i < 4; i++) part[i] = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
      float t = (part[0] + part[1]) + (part[2] + part[3]);
      for (; k < K; k++) t += ar[k] * (float)wr[k];
      C[(size_t)m * N + n] = t * sw[n] + (bias ? bias[n] : 0.0f);
    }
  }
}

/* reference src/ops.c:30-51 (AVX2/FMA dot): 32 k per step into four 8-lane fused
 * multiply-add accumulators, combine in float then in double, tail in double. */
__attribute__((target("avx2,fma"))) static double orc_dot_avx2(const float *a, const float *b,
                                                               int K) {
  float acc[4][8] = {{0}};
  int k = 0;
  for (; k + 32 <= K; k += 32)
    for (int j = 0; j < 4; j++)
      for (int i = 0; i < 8; i++)
        acc[j][i] = fmaf(a[k + 8 * j + i], b[k + 8 * j + i], acc[j][i]);
  float p[8];
  for (int i = 0; i < 8; i++) p[i] = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
  double s = ((double)(p[0] + p[1]) + (double)(p[2] + p[3])) +
             ((double)(p[4] + p[5]) + (double)(p[6] + p[7]));
  for (; k < K; k++) s += (double)a[k] * b[k];
  return s;
}

/* reference src/ops.c:57-83 (SSE2 dot, used when the CPU lacks AVX2/FMA) */
static double orc_dot_sse2(const float *a, const float *b, int K) {
  float acc[4][4] = {{0}};
  int k = 0;
  for (; k + 16 <= K; k += 16)
    for (int j = 0; j < 4; j++)
      for (int i = 0; i < 4; i++) {
        const float p = a[k + 4 * j + i] * b[k + 4 * j + i];
        acc[j][i] = acc[j][i] + p;
      }
  float p[4];
  for (int i = 0; i < 4; i++) p[i] = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
  double s = (double)(p[0] + p[1]) + (p[2] + p[3]);
  for (; k < K; k++) s += (double)a[k] * b[k];
  return s;
}

/* reference src/ops.c:94-106 */
static double orc_dot(const float *a, const float *b, int K) {
  static int avx2 = -1;
  if (avx2 < 0) avx2 = (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) ? 1 : 0;
  return avx2 ? orc_dot_avx2(a, b, K) : orc_dot_sse2(a, b, K);
}

/* reference src/ops.c:243-279 with the BLAS branch disabled (SGL_BLAS=0): blocks of 8 rows,
 * parallel over n, each element one independent dot. */
void orc_matmul_nt(const float *A, const float *W, const float *bias, float *C, int M, int N,
                   int K) {
  for (int m0 = 0; m0 < M; m0 += 8) {
    const int me = m0 + 8 < M ? m0 + 8 : M;
#pragma omp parallel for
    for (int n = 0; n < N; n++) {
      const float *wr = W + (size_t)n * K;
      const float b = bias ? bias[n] : 0.0f;
      for (int m = m0; m < me; m++)
        C[(size_t)m * N + n] = (float)orc_dot(A + (size_t)m * K, wr, K) + b;
    }
  }
}

/* Expert FFN + weighted combine of one MoE block, following reference
 * src/deepseek.c:655-677 (fused gate/up path): per token t and slot j in order, expert
 * e = ids[t*k+j]; gu = h_t * Wgu_e^T ([2*mi]); a_i = silu(gu_i) * gu_{mi+i} with
 * silu(g) = g / (1 + expf(-g)) (reference src/ops.c:288-293); o = a * Wdn_e^T ([E]);
 * out_t += w[t*k+j] * o.  Routing is an input.  Negative ids are skipped. */
void orc_moe_ffn(const float *h, int T, int E, int mi, const float *const *w_gu,
                 const float *const *w_dn, const int32_t *ids, const float *wts, int k,
                 float *out) {
  float *gu = (float *)malloc(sizeof(float) * 2 * (size_t)mi);
  float *o = (float *)malloc(sizeof(float) * (size_t)E);
  for (int t = 0; t < T; t++) {
    float *orow = out + (size_t)t * E;
    memset(orow, 0, sizeof(float) * (size_t)E);
    for (int j = 0; j < k; j++) {
      const int e = ids[(size_t)t * k + j];
      if (e < 0) continue;
      orc_matmul_nt(h + (size_t)t * E, w_gu[e], NULL, gu, 1, 2 * mi, E);
      for (int i = 0; i < mi; i++) {
        const float g = gu[i];
        gu[i] = (g / (1.0f + expf(-g))) * gu[mi + i];
      }
      orc_matmul_nt(gu, w_dn[e], NULL, o, 1, E, mi);
      const float w = wts[(size_t)t * k + j];
      for (int i = 0; i < E; i++) orow[i] += w * o[i];
    }
  }
  free(gu);
  free(o);
}

/* Routing of one MoE block, following reference src/deepseek.c:593-633 for each token row of
 * logits ([T][ne], the router product): scores s = sigmoid(logit) (sigmoid = 1) or the softmax
 * of reference src/ops.c:220-231; selection scores ch = s + bias (bias may be NULL); with
 * n_group > 1 (group_limited_greedy), group score = top-1 + top-2 of its ch, the topk_group
 * best groups kept greedily (strictly greater wins, so ties go to the lower index), ch of the
 * others set to -1e30; top-k over ch by the same greedy rule (-1 when nothing beats -1e30);
 * weights = the uncorrected s of the chosen experts, normalised by their double sum + 1e-20
 * when norm && k > 1, then times scale. */
void orc_moe_route(const float *logits, int T, int ne, const float *bias, int sigmoid,
                   int n_group, int topk_group, int k, int norm, float scale, int32_t *ids,
                   float *wts) {
  float *s = (float *)malloc(sizeof(float) * (size_t)ne);
  float *ch = (float *)malloc(sizeof(float) * (size_t)ne);
  float *gs = (float *)malloc(sizeof(float) * (size_t)(n_group > 0 ? n_group : 1));
  int *gsel = (int *)malloc(sizeof(int) * (size_t)(n_group > 0 ? n_group : 1));
  for (int t = 0; t < T; t++) {
    memcpy(s, logits + (size_t)t * ne, sizeof(float) * (size_t)ne);
    if (sigmoid) {
      for (int i = 0; i < ne; i++) s[i] = 1.0f / (1.0f + expf(-s[i]));
    } else {
      float maxv = s[0];
      for (int i = 1; i < ne; i++)
        if (s[i] > maxv) maxv = s[i];
      double sum = 0;
      for (int i = 0; i < ne; i++) {
        s[i] = expf(s[i] - maxv);
        sum += s[i];
      }
      const float inv = (float)(1.0 / sum);
      for (int i = 0; i < ne; i++) s[i] *= inv;
    }
    for (int i = 0; i < ne; i++) ch[i] = s[i] + (bias ? bias[i] : 0.0f);
    if (n_group > 1) {
      const int epg = ne / n_group;
      for (int g = 0; g < n_group; g++) {
        const float *b = ch + (size_t)g * epg;
        float t1 = -1e30f, t2 = -1e30f;
        for (int i = 0; i < epg; i++) {
          if (b[i] > t1) {
            t2 = t1;
            t1 = b[i];
          } else if (b[i] > t2) {
            t2 = b[i];
          }
        }
        gs[g] = epg > 1 ? t1 + t2 : t1;
      }
      for (int g = 0; g < n_group; g++) {
        int best = -1;
        float bv = -1e30f;
        for (int i = 0; i < n_group; i++) {
          int used = 0;
          for (int j = 0; j < g; j++) used |= gsel[j] == i;
          if (!used && gs[i] > bv) {
            bv = gs[i];
            best = i;
          }
        }
        gsel[g] = best;
      }
      for (int i = 0; i < ne; i++) {
        int keep = 0;
        for (int j = 0; j < topk_group; j++) keep |= gsel[j] == i / epg;
        if (!keep) ch[i] = -1e30f;
      }
    }
    int32_t *sel = ids + (size_t)t * k;
    float *sw = wts + (size_t)t * k;
    for (int j = 0; j < k; j++) {
      int best = -1;
      float bv = -1e30f;
      for (int i = 0; i < ne; i++) {
        int used = 0;
        for (int q = 0; q < j; q++) used |= sel[q] == i;
        if (!used && ch[i] > bv) {
          bv = ch[i];
          best = i;
        }
      }
      sel[j] = best;
      sw[j] = best >= 0 ? s[best] : 0.0f;
    }
    if (k > 1 && norm) {
      double tot = 0;
      for (int j = 0; j < k; j++) tot += sw[j];
      tot += 1e-20;
      if (tot != 0)
        for (int j = 0; j < k; j++) sw[j] = (float)(sw[j] / tot);
    }
    for (int j = 0; j < k; j++) sw[j] *= scale;
  }
  free(s);
  free(ch);
  free(gs);
  free(gsel);
}

/* Shared experts of one MoE block, added after the routed sum as reference
 * src/deepseek.c:679-687: out_t += (silu(h_t Wg^T) * (h_t Wu^T)) Wd^T, Wg/Wu [sh][E], Wd [E][sh],
 * each product by orc_matmul_nt (the reference's sgl_matmul_nt). */
void orc_moe_shared(const float *h, int T, int E, int sh, const float *wg, const float *wu,
                    const float *wd, float *out) {
  float *g = (float *)malloc(sizeof(float) * (size_t)sh);
  float *u = (float *)malloc(sizeof(float) * (size_t)sh);
  float *o = (float *)malloc(sizeof(float) * (size_t)E);
  for (int t = 0; t < T; t++) {
    orc_matmul_nt(h + (size_t)t * E, wg, NULL, g, 1, sh, E);
    orc_matmul_nt(h + (size_t)t * E, wu, NULL, u, 1, sh, E);
    for (int i = 0; i < sh; i++) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
    orc_matmul_nt(g, wd, NULL, o, 1, E, sh);
    float *orow = out + (size_t)t * E;
    for (int i = 0; i < E; i++) orow[i] += o[i];
  }
  free(g);
  free(u);
  free(o);
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
