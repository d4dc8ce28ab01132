// build.hip — upload a quantized weight in any supported on-disk layout, decode it on the GPU
// and repack it into the device tile layout (sglq_dev.hpp); plus the exact dequant of that
// layout back to f32 [N, K] (the device twin of the reference's sgl_qweight_dequant*).
//
// Decoding follows the reference's index formulas (cited per kernel); every code, zero and
// scale is moved bit-for-bit, so dequant(device layout) == reference dequant exactly.
#include <string.h>

#include "sglq_dev.hpp"

// reference src/qweight.c:22 — AWQ keeps natural column n in nibble slot AWQ_SLOT[n & 7]
__constant__ int c_awq_slot[8] = {0, 4, 1, 5, 2, 6, 3, 7};

__device__ __forceinline__ uint32_t field(uint32_t w, int slot, int bits) {
  return (w >> (bits * slot)) & ((1u << bits) - 1u);
}

// ---------------------------------------------------------------------------------------
// stage 1: source layout -> dense u8 codes [N, K]
// ---------------------------------------------------------------------------------------

// GPTQ (reference src/qweight.c:132-135): word qw[k/pack][n], k in slot k % pack.
__global__ void k_decode_gptq(const uint32_t *__restrict__ qw, int64_t qw_cols, int64_t N,
                              int64_t K, int bits, uint8_t *__restrict__ out) {
  const int pack = 32 / bits;
  const int64_t rows = (K + pack - 1) / pack;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * N) return;
  const int64_t kw = i / N, n = i % N;
  const uint32_t w = qw[kw * qw_cols + n];
  for (int j = 0; j < pack; j++) {
    const int64_t k = kw * pack + j;
    if (k < K) out[n * K + k] = (uint8_t)field(w, j, bits);
  }
}

// AWQ gemm / gemv (reference src/qweight.c:93-101).
__global__ void k_decode_awq(const uint32_t *__restrict__ qw, int64_t qw_cols, int64_t N,
                             int64_t K, int transposed, uint8_t *__restrict__ out) {
  const int64_t nw_cnt = (N + 7) / 8;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nw_cnt * K) return;
  const int64_t k = i / nw_cnt, nw = i % nw_cnt;
  const uint32_t w = transposed ? qw[nw * qw_cols + k] : qw[k * qw_cols + nw];
  for (int c = 0; c < 8; c++) {
    const int64_t n = nw * 8 + c;
    if (n < N) out[n * K + k] = (uint8_t)field(w, c_awq_slot[c], 4);
  }
}

// Marlin 16(k) x 64(n) tiles (reference src/qweight.c:233-248): word p of a tile, element j.
__global__ void k_decode_marlin(const uint32_t *__restrict__ qw, int64_t qw_cols, int64_t N,
                                int64_t K, int bits, uint8_t *__restrict__ out) {
  const int pack = 32 / bits;
  const int64_t tile_words = 64 * 16 / pack;
  const int64_t words_per_row = (N / 64) * tile_words;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (K / 16) * words_per_row) return;
  const int64_t kt = i / words_per_row, r = i % words_per_row;
  const int64_t nt = r / tile_words;
  const int p = (int)(r % tile_words);
  const uint32_t w = qw[kt * qw_cols + r];
  for (int j = 0; j < pack; j++) {
    int ko, no;
    if (bits == 4) {
      ko = 2 * ((p >> 2) & 3) + ((j & 1) ? 8 : 0) + (j >= 4 ? 1 : 0);
      no = 16 * (p & 3) + (p >> 4) + ((j & 2) ? 8 : 0);
    } else {
      const int k8[4] = {0, 8, 1, 9};
      ko = 2 * ((p >> 3) & 3) + k8[j];
      no = 16 * ((p >> 1) & 3) + (p >> 5) + ((p & 1) ? 8 : 0);
    }
    out[(nt * 64 + no) * K + kt * 16 + ko] = (uint8_t)field(w, j, bits);
  }
}

// compressed-tensors pack-quantized (reference src/qweight.c:304-320): little-endian bytes,
// 4-bit low nibble = even k; 8-bit one byte per k.
__global__ void k_decode_ct(const uint8_t *__restrict__ wp, int64_t cols, int64_t N, int64_t K,
                            int bits, uint8_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * K) return;
  const int64_t n = i / K, k = i % K;
  const uint8_t *row = wp + n * cols * 4;
  uint8_t code;
  if (bits == 4) {
    const uint8_t b = row[k >> 1];
    code = (k & 1) ? (b >> 4) : (b & 0xF);
  } else {
    code = row[k];
  }
  out[i] = code;
}

// MXFP4 (reference src/qweight.c:354-363): byte b of row n holds k = 2b (low) and 2b+1 (high).
__global__ void k_decode_mxfp4(const uint8_t *__restrict__ wp, int64_t cols, int64_t N,
                               int64_t K, uint8_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * K) return;
  const int64_t n = i / K, k = i % K;
  const uint8_t b = wp[n * cols + (k >> 1)];
  out[i] = (k & 1) ? (b >> 4) : (b & 0xF);
}

// W8 (reference src/quant.c:44-89 operand): int8 stored with +128 so every kind is unsigned.
__global__ void k_decode_w8(const int8_t *__restrict__ w, int64_t NK, uint8_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < NK) out[i] = (uint8_t)((int)w[i] + 128);
}

// Per-(group, column) zero and scale.  Zero semantics per format:
//   GPTQ  code(qz[g][n>>3], n % pack) + v2   (reference src/qweight.c:136, incl. the n>>3 word)
//   AWQ   code(qz[g][n>>3], AWQ_SLOT[n&7])   (reference src/qweight.c:98-101)
//   Marlin inverse interleave of reference src/qweight.c:173-191
//   absent: zconst (AWQ/GPTQ 0, Marlin 2^(bits-1), CT offset, W8 128)
struct MetaArgs {
  int src, bits, has_zero, zconst, v2;
  int64_t N, ngroups, qz_cols, sc_cols;
};

__global__ void k_decode_meta(MetaArgs a, const uint32_t *__restrict__ qz,
                              const float *__restrict__ sc, uint16_t *__restrict__ dz,
                              float *__restrict__ ds) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.ngroups * a.N) return;
  const int64_t g = i / a.N, n = i % a.N;
  const int pack = 32 / a.bits;
  int z = a.zconst;
  float s;
  switch (a.src) {
    case SGLQ_SRC_GPTQ:
      if (a.has_zero) z = (int)field(qz[g * a.qz_cols + (n >> 3)], (int)(n % pack), a.bits) + a.v2;
      s = sc[g * a.N + n];
      break;
    case SGLQ_SRC_AWQ:
      if (a.has_zero) z = (int)field(qz[g * a.qz_cols + (n >> 3)], c_awq_slot[n & 7], 4);
      s = sc[g * a.N + n];
      break;
    case SGLQ_SRC_MARLIN: {
      const int64_t f = (n / 64) * 64 + 8 * (n & 7) + ((n % 64) >> 3);
      if (a.has_zero) {
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
        z = (int)field(qz[g * a.qz_cols + f2 / pack], (int)(f2 % pack), a.bits);
      }
      s = sc[g * a.sc_cols + f];
      break;
    }
    case SGLQ_SRC_CT:
      s = sc[n * a.sc_cols + g];
      break;
    default:  // SGLQ_SRC_W8: one group, scale per row
      s = sc[n];
      break;
  }
  dz[i] = (uint16_t)z;  // gptq_v2 8-bit may give 256
  ds[i] = s;
}

__global__ void k_check_f16(const float *__restrict__ s, int64_t n, int *__restrict__ flag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = s[i];
  if ((float)(_Float16)v != v) atomicOr(flag, 1);
  // bit 1: (q - z) * s can leave f16's normal range (|q - z| <= 256)
  const float a = fabsf(v);
  if (!(a == 0.f || (a >= 0x1p-14f && a <= 128.f))) atomicOr(flag, 2);
}

// ---------------------------------------------------------------------------------------
// stage 2: dense codes -> tile layout
// ---------------------------------------------------------------------------------------
__global__ void k_pack_codes(const uint8_t *__restrict__ dc, int64_t N, int64_t K,
                             const int32_t *__restrict__ kmap, int kind, int64_t ntile,
                             int64_t nchunk, u32x4_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ntile * nchunk * 64) return;
  const int lane = (int)(i & 63);
  const int64_t tc = i >> 6;
  const int64_t t = tc / nchunk, c = tc % nchunk;
  const int64_t n = t * 16 + (lane & 15);
  const int kq = lane >> 4;
  uint32_t w[4] = {0, 0, 0, 0};
  if (n < N) {
    const uint8_t *row = dc + n * K;
    if (kind == SGLQ_KIND_U8) {
      for (int j = 0; j < 2; j++)
        for (int b = 0; b < 8; b++) {
          const int64_t kp = (c * 2 + j) * 32 + kq * 8 + b;
          const int32_t k = kmap[kp];
          const uint32_t v = k >= 0 ? row[k] : 0u;
          w[2 * j + (b >> 2)] |= v << (8 * (b & 3));
        }
    } else {
      for (int j = 0; j < 4; j++)
        for (int b = 0; b < 8; b++) {
          const int64_t kp = (c * 4 + j) * 32 + kq * 8 + b;
          const int32_t k = kmap[kp];
          const uint32_t v = k >= 0 ? row[k] : 0u;
          w[j] |= v << (4 * b);
        }
    }
  }
  u32x4_t o = {w[0], w[1], w[2], w[3]};
  out[i] = o;
}

// Per-(tile, column, unit) meta entries (layout in sglq_dev.hpp).  A unit is group u
// (META_GROUP) or step u, whose group is u / spg (META_STEP).  Thread i writes entry i.
__global__ void k_pack_meta(const uint16_t *__restrict__ dz, const float *__restrict__ ds,
                            int64_t N, int64_t ngroups, int64_t ntile, int64_t nmeta,
                            int64_t upg, int f16, void *__restrict__ om) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ntile * 16 * nmeta) return;
  const int64_t t = i / (16 * nmeta), r = i % (16 * nmeta);
  const int64_t u = (r >> 6) * 4 + (r & 3);
  const int64_t n = t * 16 + ((r >> 2) & 15);
  const int64_t g = u / upg;
  float s = 0.f;
  int z = 0;
  if (n < N && g < ngroups) {
    s = ds[g * N + n];
    z = dz[g * N + n];
  }
  const _Float16 zoff = (_Float16)(-1024.0f - (float)z);  // exact: |1024 + z| < 2048
  const uint32_t zb = (uint32_t)__builtin_bit_cast(uint16_t, zoff);
  if (f16) {
    const uint32_t sb = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)s);
    ((uint32_t *)om)[i] = sb | (zb << 16);
  } else {
    ((uint64_t *)om)[i] = (uint64_t)__float_as_uint(s) | ((uint64_t)zb << 32);
  }
}

// e8m0 bytes [N][nb] -> the quad layout of sglq_ebyte (step s of the device K is block s;
// bytes past the last step are 0).  Thread i writes byte i.
__global__ void k_pack_e8m0(const uint8_t *__restrict__ se, int64_t N, int64_t nb, int64_t ntile,
                            int64_t nsteps, int64_t nmeta, uint8_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ntile * 16 * nmeta) return;
  const int64_t t = i / (16 * nmeta), r = i % (16 * nmeta);
  const int64_t s = (r >> 8) * 16 + (r & 15);
  const int64_t n = t * 16 + ((r >> 4) & 15);
  out[i] = (n < N && s < nb && s < nsteps) ? se[n * nb + s] : (uint8_t)0;
}

// largest e8m0 byte of each column (255, the reference's "scale 0" code, ignored; 0 if none)
__global__ void k_col_e8m0_max(const uint8_t *__restrict__ m, int64_t ncol, int64_t nsteps,
                               int64_t nmeta, uint8_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= ncol) return;
  uint32_t mx = 0;
  for (int64_t s = 0; s < nsteps; s++) {
    const uint32_t e = m[sglq_ebyte(i >> 4, (int)(i & 15), s, nmeta)];
    if (e != 255u && e > mx) mx = e;
  }
  out[i] = (uint8_t)mx;
}

// ---------------------------------------------------------------------------------------
// exact dequant of the tile layout: out[n*K + k] = (float)(q - z) * s  (U4/U8)
//                                                = e2m1(q) * (e == 255 ? 0 : 2^(e-127)) (E2M1)
// ---------------------------------------------------------------------------------------
struct DqArgs {
  int kind, scf16, meta_mode;
  int64_t N, K, nchunk, spc, cpg, nmeta, nsteps;
};

__global__ void k_dequant(DqArgs a, const u32x4_t *__restrict__ codes,
                          const void *__restrict__ meta, const int32_t *__restrict__ kinv,
                          float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.N * a.K) return;
  const int64_t n = i / a.K, k = i % a.K;
  const int64_t kp = kinv[k];
  const int64_t s = kp >> 5, c = s / a.spc, j = s % a.spc;
  const int64_t t = n >> 4;
  const int lane = (int)(((kp & 31) >> 3) * 16 + (n & 15));
  const int e = (int)(kp & 7);
  const u32x4_t blk = codes[(t * a.nchunk + c) * 64 + lane];
  if (a.kind == SGLQ_KIND_E2M1) {
    const uint32_t q = (blk[j] >> (4 * e)) & 15u;
    const uint32_t ex = ((const uint8_t *)meta)[sglq_ebyte(t, (int)(n & 15), s, a.nmeta)];
    const float sc = ex == 255 ? 0.f : ldexpf(1.0f, (int)ex - 127);
    out[i] = sglq_e2m1_value(q) * sc;
    return;
  }
  uint32_t q;
  if (a.kind == SGLQ_KIND_U8)
    q = (blk[2 * j + (e >> 2)] >> (8 * (e & 3))) & 255u;
  else
    q = (blk[j] >> (4 * e)) & 15u;
  const int64_t u = a.meta_mode == SGLQ_META_GROUP ? c / a.cpg : s;
  const int64_t mi = sglq_mrow(t, (int)(n & 15), a.nmeta) + sglq_mofs(u);
  float sc;
  uint16_t zb;
  if (a.scf16) {
    const uint32_t m = ((const uint32_t *)meta)[mi];
    sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(m & 0xFFFFu));
    zb = (uint16_t)(m >> 16);
  } else {
    const uint64_t m = ((const uint64_t *)meta)[mi];
    sc = __uint_as_float((uint32_t)m);
    zb = (uint16_t)(m >> 32);
  }
  const int z = (int)(-(float)__builtin_bit_cast(_Float16, zb)) - 1024;
  out[i] = (float)((int)q - z) * sc;  // reference src/qweight.c:102-103, 137-138
}

// ---------------------------------------------------------------------------------------
// host side of the shim
// ---------------------------------------------------------------------------------------
static int64_t src_bytes_qweight(const sglq_plan *p) {
  if (p->src == SGLQ_SRC_MXFP4) return p->qw_rows * p->qw_cols;      // u8
  if (p->src == SGLQ_SRC_W8) return p->N * p->K;                      // i8
  return p->qw_rows * p->qw_cols * 4;                                 // i32
}
static int64_t src_bytes_scales(const sglq_plan *p) {
  if (p->src == SGLQ_SRC_MXFP4) return p->sc_rows * p->sc_cols;      // e8m0
  if (p->src == SGLQ_SRC_W8) return p->N * 4;
  return p->sc_rows * p->sc_cols * 4;
}

static sglq_dev *build_impl(const sglq_plan *p, const void *qw, const void *qz, const void *sc,
                            int dev, int on_device) {
  sglq_dev *d = (sglq_dev *)calloc(1, sizeof(sglq_dev));
  void *b_qw = nullptr, *b_qz = nullptr, *b_sc = nullptr;
  uint8_t *dc = nullptr;
  uint16_t *dz = nullptr;
  float *ds = nullptr;
  int *flag = nullptr;
  hipMemcpyKind kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  const int T = 256;
  if (!d) return nullptr;
  d->dev = dev;
  d->src = p->src;
  d->kind = p->kind;
  d->N = p->N;
  d->K = p->K;
  d->ntile = (p->N + 15) / 16;
  d->nsteps = p->nsteps;
  d->spc = p->kind == SGLQ_KIND_U8 ? 2 : 4;
  d->nchunk = p->nsteps / d->spc;
  d->spg = p->gp / 32;
  d->ngroups = p->ngroups;
  // meta rows are padded (e8m0 rows to 16 bytes, group entries to 4) so that the one-row
  // GEMV reads the entries of consecutive chunks with 16-byte loads; padding entries are zero
  if (p->kind == SGLQ_KIND_E2M1) {
    d->meta_mode = SGLQ_META_E8M0;
    d->nmeta = (d->nsteps + 15) / 16 * 16;
  } else if (d->spg % d->spc == 0) {
    d->meta_mode = SGLQ_META_GROUP;  // every group is cpg whole chunks
    d->cpg = d->spg / d->spc;
    d->nmeta = ((d->nsteps + d->spg - 1) / d->spg + 3) / 4 * 4;
  } else {
    d->meta_mode = SGLQ_META_STEP;
    d->nmeta = (d->nsteps + 3) / 4 * 4;
  }
  d->kident = 1;
  for (int64_t k = 0; k < p->K && d->kident; k++) d->kident = p->kmap[k] == k;
  SGLQ_HIP(hipSetDevice(dev));
  {
    const int64_t qwb = src_bytes_qweight(p), scb = src_bytes_scales(p);
    SGLQ_HIP(hipMalloc(&b_qw, qwb));
    SGLQ_HIP(hipMemcpy(b_qw, qw, qwb, kind));
    SGLQ_HIP(hipMalloc(&b_sc, scb));
    SGLQ_HIP(hipMemcpy(b_sc, sc, scb, kind));
    if (p->has_zero && qz) {
      const int64_t qzb = p->qz_rows * p->qz_cols * 4;
      SGLQ_HIP(hipMalloc(&b_qz, qzb));
      SGLQ_HIP(hipMemcpy(b_qz, qz, qzb, kind));
    }
    const int64_t NK = p->N * p->K;
    SGLQ_HIP(hipMalloc(&dc, NK));
    switch (p->src) {
      case SGLQ_SRC_GPTQ:
        k_decode_gptq<<<sglq_blocks(((p->K + 32 / p->bits - 1) / (32 / p->bits)) * p->N, T), T>>>(
            (const uint32_t *)b_qw, p->qw_cols, p->N, p->K, p->bits, dc);
        break;
      case SGLQ_SRC_AWQ:
        k_decode_awq<<<sglq_blocks(((p->N + 7) / 8) * p->K, T), T>>>(
            (const uint32_t *)b_qw, p->qw_cols, p->N, p->K, p->transposed, dc);
        break;
      case SGLQ_SRC_MARLIN:
        k_decode_marlin<<<sglq_blocks(p->qw_rows * (p->N / 64) * (1024 / (32 / p->bits)), T), T>>>(
            (const uint32_t *)b_qw, p->qw_cols, p->N, p->K, p->bits, dc);
        break;
      case SGLQ_SRC_CT:
        k_decode_ct<<<sglq_blocks(NK, T), T>>>((const uint8_t *)b_qw, p->qw_cols, p->N, p->K,
                                               p->bits, dc);
        break;
      case SGLQ_SRC_MXFP4:
        k_decode_mxfp4<<<sglq_blocks(NK, T), T>>>((const uint8_t *)b_qw, p->qw_cols, p->N, p->K,
                                                  dc);
        break;
      default:
        k_decode_w8<<<sglq_blocks(NK, T), T>>>((const int8_t *)b_qw, NK, dc);
        break;
    }
    SGLQ_HIP(hipGetLastError());
    // kmap / kinv
    SGLQ_HIP(hipMalloc(&d->kmap, p->nsteps * 32 * 4));
    SGLQ_HIP(hipMemcpy(d->kmap, p->kmap, p->nsteps * 32 * 4, hipMemcpyHostToDevice));
    SGLQ_HIP(hipMalloc(&d->kinv, p->K * 4));
    SGLQ_HIP(hipMemcpy(d->kinv, p->kinv, p->K * 4, hipMemcpyHostToDevice));
    SGLQ_HIP(hipMalloc(&d->codes, d->ntile * d->nchunk * 1024));
    k_pack_codes<<<sglq_blocks(d->ntile * d->nchunk * 64, T), T>>>(
        dc, p->N, p->K, d->kmap, p->kind, d->ntile, d->nchunk, d->codes);
    SGLQ_HIP(hipGetLastError());
    if (p->kind == SGLQ_KIND_E2M1) {
      const int64_t nm = d->ntile * 16 * d->nmeta;
      SGLQ_HIP(hipMalloc(&d->meta, nm));
      k_pack_e8m0<<<sglq_blocks(nm, T), T>>>((const uint8_t *)b_sc, p->N, p->sc_cols, d->ntile,
                                             d->nsteps, d->nmeta, (uint8_t *)d->meta);
      SGLQ_HIP(hipGetLastError());
      SGLQ_HIP(hipMalloc(&d->colexp, d->ntile * 16));
      k_col_e8m0_max<<<sglq_blocks(d->ntile * 16, T), T>>>(
          (const uint8_t *)d->meta, d->ntile * 16, d->nsteps, d->nmeta, d->colexp);
      SGLQ_HIP(hipGetLastError());
    } else {
      const int64_t GN = p->ngroups * p->N;
      SGLQ_HIP(hipMalloc(&dz, GN * 2));
      SGLQ_HIP(hipMalloc(&ds, GN * 4));
      MetaArgs ma = {p->src, p->bits, p->has_zero && qz, p->zconst, p->v2,
                     p->N, p->ngroups, p->qz_cols, p->sc_cols};
      k_decode_meta<<<sglq_blocks(GN, T), T>>>(ma, (const uint32_t *)b_qz, (const float *)b_sc,
                                               dz, ds);
      SGLQ_HIP(hipGetLastError());
      SGLQ_HIP(hipMalloc(&flag, 4));
      SGLQ_HIP(hipMemset(flag, 0, 4));
      k_check_f16<<<sglq_blocks(GN, T), T>>>(ds, GN, flag);
      int hflag = 1;
      SGLQ_HIP(hipMemcpy(&hflag, flag, 4, hipMemcpyDeviceToHost));
      d->scf16 = (hflag & 1) == 0;
      d->prescale = hflag == 0;
      const int64_t nm = d->ntile * 16 * d->nmeta;
      SGLQ_HIP(hipMalloc(&d->meta, nm * (d->scf16 ? 4 : 8)));
      k_pack_meta<<<sglq_blocks(nm, T), T>>>(
          dz, ds, p->N, p->ngroups, d->ntile, d->nmeta,
          d->meta_mode == SGLQ_META_GROUP ? 1 : d->spg, d->scf16, d->meta);
      SGLQ_HIP(hipGetLastError());
    }
    SGLQ_HIP(hipDeviceSynchronize());
  }
  if (sglq_gemv_setup(d) != 0) goto fail;
  (void)hipFree(b_qw);
  (void)hipFree(b_qz);
  (void)hipFree(b_sc);
  (void)hipFree(dc);
  (void)hipFree(dz);
  (void)hipFree(ds);
  (void)hipFree(flag);
  return d;
fail:
  (void)hipFree(b_qw);
  (void)hipFree(b_qz);
  (void)hipFree(b_sc);
  (void)hipFree(dc);
  (void)hipFree(dz);
  (void)hipFree(ds);
  (void)hipFree(flag);
  sglq_free(d);
  return nullptr;
}

extern "C" sglq_dev *sglq_build(const sglq_plan *p, const void *qw, const void *qz,
                                const void *sc, int dev) {
  return build_impl(p, qw, qz, sc, dev, 0);
}

extern "C" sglq_dev *sglq_build_device(const sglq_plan *p, const void *qw, const void *qz,
                                       const void *sc, int dev) {
  return build_impl(p, qw, qz, sc, dev, 1);
}

extern "C" void sglq_free(sglq_dev *d) {
  if (!d) return;
  (void)hipSetDevice(d->dev);
  (void)hipFree(d->codes);
  (void)hipFree(d->meta);
  (void)hipFree(d->colexp);
  (void)hipFree(d->gv_part);
  (void)hipFree(d->gv_cnt);
  (void)hipFree(d->kmap);
  (void)hipFree(d->kinv);
  (void)hipFree(d->ws);
  (void)hipFree(d->aux);
  for (int i = 0; i < d->nretired; i++) (void)hipFree(d->retired[i]);
  free(d->retired);
  free(d->moe_tbl);
  free(d);
}

// A buffer outgrown by a larger call is retired, not freed: a HIP graph captured from an
// earlier call on this handle still holds its address, so it stays allocated until
// sglq_free.
static int retire(sglq_dev *d, void *p) {
  if (!p) return 0;
  if (d->nretired == d->cap_retired) {
    const int cap = d->cap_retired ? 2 * d->cap_retired : 8;
    void **r = (void **)realloc(d->retired, sizeof(void *) * (size_t)cap);
    if (!r) return -1;
    d->retired = r;
    d->cap_retired = cap;
  }
  d->retired[d->nretired++] = p;
  return 0;
}

static int grow(sglq_dev *d, void **buf, size_t *have, size_t bytes, const char *what) {
  if (*have >= bytes) return 0;
  void *p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    sglq_log_error("%s allocation of %zu bytes failed", what, bytes);
    return -1;
  }
  if (retire(d, *buf) != 0) {
    (void)hipFree(p);
    sglq_log_error("%s: out of host memory", what);
    return -1;
  }
  *buf = p;
  *have = bytes;
  return 0;
}

int sglq_ws_reserve(sglq_dev *d, size_t bytes) {
  return grow(d, &d->ws, &d->ws_bytes, bytes, "workspace");
}

int sglq_aux_reserve(sglq_dev *d, size_t bytes) {
  return grow(d, &d->aux, &d->aux_bytes, bytes, "auxiliary buffer");
}

extern "C" int sglq_dequant_dev(sglq_dev *d, float *out, void *stream) {
  DqArgs a = {d->kind, d->scf16, d->meta_mode, d->N, d->K, d->nchunk, d->spc, d->cpg,
              d->nmeta, d->nsteps};
  SGLQ_HIP(hipSetDevice(d->dev));
  k_dequant<<<sglq_blocks(d->N * d->K, 256), 256, 0, (hipStream_t)stream>>>(
      a, d->codes, d->meta, d->kinv, out);
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

extern "C" int sglq_dequant_host(sglq_dev *d, float *out_host) {
  float *o = nullptr;
  const size_t bytes = (size_t)(d->N * d->K) * 4;
  SGLQ_HIP(hipSetDevice(d->dev));
  SGLQ_HIP(hipMalloc(&o, bytes));
  if (sglq_dequant_dev(d, o, nullptr) != 0) goto fail;
  SGLQ_HIP(hipMemcpy(out_host, o, bytes, hipMemcpyDeviceToHost));
  (void)hipFree(o);
  return 0;
fail:
  (void)hipFree(o);
  return -1;
}

extern "C" int64_t sglq_N(const sglq_dev *d) { return d->N; }
extern "C" int64_t sglq_K(const sglq_dev *d) { return d->K; }
extern "C" int64_t sglq_weight_bytes(const sglq_dev *d) {
  const int64_t codes = d->ntile * d->nchunk * 1024;
  // entries a forward reads (the row padding is never read)
  const int64_t nm = d->ntile * 16 *
                     (d->meta_mode == SGLQ_META_GROUP ? (d->nsteps + d->spg - 1) / d->spg
                                                      : d->nsteps);
  if (d->kind == SGLQ_KIND_E2M1) return codes + nm;
  return codes + nm * (d->scf16 ? 4 : 8);
}
