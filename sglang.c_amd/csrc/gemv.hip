// gemv.hip — decode-side quantized linear, C[M,N] = A[M,K] * W^T (+ bias), M <= 64 per launch.
//
// The weight is streamed once from HBM in the tile layout (sglq_dev.hpp): each wave loads
// 1 KiB per chunk with one 128-bit load per lane, unpacks the codes in registers straight
// into the B operand of v_mfma_f32_16x16x32_f16 and subtracts the zero exactly in f16
// (q - z is a small integer), so the fp32 MFMA accumulation sees exact weight codes.  The
// per-(group, column) scale is applied in fp32 when a group ends (e8m0 block scale per step
// for MXFP4).  A workgroup owns one 16-column tile; its waves split K and are reduced through
// LDS, so no atomics and a deterministic result.
//
// Activations are prepared once per call by k_prep: gathered through kmap (act-order), scaled
// by an exact per-row power of two so they sit well inside f16 range, and split into f16
// hi + lo parts when they come in as f32 (hi + lo carries ~22 bits, so the f32 input is kept),
// laid out per step exactly as the MFMA A operand wants them.
#include "sglq_dev.hpp"

struct PrepArgs {
  const void *A;
  int dt;
  int64_t lda, K, Kp, M;
  const int32_t *kmap;
  int perm4;  // U4 operand order: element i holds k-offset {0,4,1,5,2,6,3,7}[i]
  int split;
  _Float16 *hi, *lo;
  int *rowexp;
};

__device__ __forceinline__ float load_act(const void *A, int dt, int64_t idx) {
  if (dt == SGLQ_DT_F32) return ((const float *)A)[idx];
  if (dt == SGLQ_DT_F16) return (float)((const _Float16 *)A)[idx];
  const uint32_t b = ((const uint16_t *)A)[idx];
  return __uint_as_float(b << 16);
}

__global__ __launch_bounds__(256) void k_prep(PrepArgs p) {
  const int64_t m = blockIdx.x;
  __shared__ float red[256];
  float amax = 0.f;
  for (int64_t k = threadIdx.x; k < p.K; k += 256)
    amax = fmaxf(amax, fabsf(load_act(p.A, p.dt, m * p.lda + k)));
  red[threadIdx.x] = amax;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  amax = red[0];
  // exact power-of-two row scale: amax * 2^-e lands in [2^13, 2^14)
  const int e = (amax > 0.f && amax <= 3.0e38f) ? ilogbf(amax) - 13 : 0;
  if (threadIdx.x == 0) p.rowexp[m] = e;
  for (int64_t kp = threadIdx.x; kp < p.Kp; kp += 256) {
    const int32_t k = p.kmap[kp];
    const float v = k >= 0 ? ldexpf(load_act(p.A, p.dt, m * p.lda + k), -e) : 0.f;
    const _Float16 h = (_Float16)v;
    const int64_t s = kp >> 5;
    const int r = (int)(kp & 31), kq = r >> 3, o = r & 7;
    const int i = p.perm4 ? 2 * (o & 3) + (o >> 2) : o;
    const int64_t idx = ((s * 4 + kq) * p.M + m) * 8 + i;
    p.hi[idx] = h;
    if (p.split) p.lo[idx] = (_Float16)(v - (float)h);
  }
}

struct GemvArgs {
  const u32x4_t *codes;
  const void *scales;
  const uint8_t *zeros;
  const _Float16 *ahi, *alo;
  const int *rowexp;
  const float *bias;
  float *C;
  int64_t N, M, ldc, nchunk, spg, gpad, m0;
};

union H8 {
  half8_t v;
  uint32_t u[4];
  half2_t h[4];
};

template <int KIND>
__device__ __forceinline__ half8_t unpack(const u32x4_t &w, int j, half2_t zz) {
  H8 r;
  if constexpr (KIND == SGLQ_KIND_U4) {
    const uint32_t x = w[j];
    r.u[0] = (x & 0x000F000Fu) | 0x64006400u;  // 1024 + q, pairs (0,4)
    r.u[1] = ((x >> 4) & 0x000F000Fu) | 0x64006400u;   // (1,5)
    r.u[2] = ((x >> 8) & 0x000F000Fu) | 0x64006400u;   // (2,6)
    r.u[3] = ((x >> 12) & 0x000F000Fu) | 0x64006400u;  // (3,7)
#pragma unroll
    for (int i = 0; i < 4; i++) r.h[i] = r.h[i] + zz;  // exact q - z
  } else if constexpr (KIND == SGLQ_KIND_U8) {
    const uint32_t x0 = w[2 * j], x1 = w[2 * j + 1];
    r.u[0] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);  // 1024 + b0, 1024 + b1
    r.u[1] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
    r.u[2] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
    r.u[3] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
#pragma unroll
    for (int i = 0; i < 4; i++) r.h[i] = r.h[i] + zz;
  } else {
    const uint32_t x = w[j];
    r.h[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 0);
    r.h[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 1);
    r.h[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 2);
    r.h[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 3);
  }
  return r.v;
}

template <int KIND, int MT, bool SPLIT, bool SCF16>
__global__ __launch_bounds__(1024) void k_gemv(GemvArgs a) {
  extern __shared__ float red[];  // [nw][MT*4][64]
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr int CB = 8;
  const int64_t t = blockIdx.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int n16 = lane & 15, kq = lane >> 4;
  const int64_t c0 = a.nchunk * w / nw, c1 = a.nchunk * (w + 1) / nw;
  const int64_t s_last = c1 * SPC - 1;
  float4_t acc[MT], tmp[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) {
    acc[i] = (float4_t){0.f, 0.f, 0.f, 0.f};
    tmp[i] = acc[i];
  }
  const u32x4_t *cp = a.codes + t * a.nchunk * 64 + lane;
  const uint32_t *ep = (const uint32_t *)a.scales + t * a.nchunk * 16 + n16;
  int64_t gcur = -1;
  half2_t zz = {(_Float16)0, (_Float16)0};
  float sc = 0.f;
  for (int64_t cb = c0; cb < c1; cb += CB) {
    u32x4_t wv[CB];
    uint32_t ev[CB];
#pragma unroll
    for (int i = 0; i < CB; i++)
      if (cb + i < c1) {
        wv[i] = __builtin_nontemporal_load(cp + (cb + i) * 64);
        if constexpr (KIND == SGLQ_KIND_E2M1) ev[i] = ep[(cb + i) * 16];
      }
#pragma unroll
    for (int i = 0; i < CB; i++) {
      if (cb + i >= c1) break;
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        const int64_t s = (cb + i) * SPC + j;
        if constexpr (KIND != SGLQ_KIND_E2M1) {
          const int64_t g = s / a.spg;
          if (g != gcur) {
            gcur = g;
            const int64_t mi = (t * a.gpad + g) * 16 + n16;
            sc = SCF16 ? (float)((const _Float16 *)a.scales)[mi] : ((const float *)a.scales)[mi];
            const _Float16 zh = (_Float16)(-1024.0f - (float)a.zeros[mi]);
            zz = (half2_t){zh, zh};
          }
        }
        const half8_t b = unpack<KIND>(wv[i], j, zz);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
          const int64_t m = mt * 16 + n16;
          half8_t av = {0, 0, 0, 0, 0, 0, 0, 0};
          const int64_t ai = ((s * 4 + kq) * a.M + m) * 8;
          if (m < a.M) av = *(const half8_t *)(a.ahi + ai);
          tmp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, tmp[mt], 0, 0, 0);
          if constexpr (SPLIT) {
            half8_t lv = {0, 0, 0, 0, 0, 0, 0, 0};
            if (m < a.M) lv = *(const half8_t *)(a.alo + ai);
            tmp[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lv, b, tmp[mt], 0, 0, 0);
          }
        }
        if constexpr (KIND == SGLQ_KIND_E2M1) {
          const uint32_t ex = (ev[i] >> (8 * j)) & 255u;
          const float ss = ex == 255 ? 0.f : ldexpf(1.0f, (int)ex - 127);
#pragma unroll
          for (int mt = 0; mt < MT; mt++) {
            acc[mt] += ss * tmp[mt];
            tmp[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
          }
        } else if ((s + 1) % a.spg == 0 || s == s_last) {
#pragma unroll
          for (int mt = 0; mt < MT; mt++) {
            acc[mt] += sc * tmp[mt];
            tmp[mt] = (float4_t){0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
  }
  // cross-wave reduction in a fixed order
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int r = 0; r < 4; r++) red[(w * MT * 4 + mt * 4 + r) * 64 + lane] = acc[mt][r];
  __syncthreads();
  for (int idx = threadIdx.x; idx < MT * 4 * 64; idx += blockDim.x) {
    float sum = 0.f;
    for (int ww = 0; ww < nw; ww++) sum += red[ww * MT * 4 * 64 + idx];
    const int e = idx >> 6, l = idx & 63;
    const int64_t m = (e >> 2) * 16 + 4 * (l >> 4) + (e & 3);
    const int64_t n = t * 16 + (l & 15);
    if (m < a.M && n < a.N)
      a.C[(a.m0 + m) * a.ldc + n] = ldexpf(sum, a.rowexp[m]) + (a.bias ? a.bias[n] : 0.f);
  }
}

template <int KIND, int MT, bool SPLIT>
static void launch_kind(const GemvArgs &a, int scf16, int nw, int64_t ntile, hipStream_t st) {
  const size_t lds = (size_t)nw * MT * 4 * 64 * 4;
  if (scf16)
    k_gemv<KIND, MT, SPLIT, true><<<ntile, nw * 64, lds, st>>>(a);
  else
    k_gemv<KIND, MT, SPLIT, false><<<ntile, nw * 64, lds, st>>>(a);
}

template <int KIND>
static void launch_mt(const GemvArgs &a, int mt, bool split, int scf16, int nw, int64_t ntile,
                      hipStream_t st) {
#define SGLQ_L(MTV)                                                  \
  if (split)                                                         \
    launch_kind<KIND, MTV, true>(a, scf16, nw, ntile, st);           \
  else                                                               \
    launch_kind<KIND, MTV, false>(a, scf16, nw, ntile, st);
  switch (mt) {
    case 1: SGLQ_L(1) break;
    case 2: SGLQ_L(2) break;
    case 3: SGLQ_L(3) break;
    default: SGLQ_L(4) break;
  }
#undef SGLQ_L
}

// waves per workgroup: enough that every wave streams at most ~8 KiB of codes
static int pick_waves(int64_t nchunk) {
  int nw = 4;
  while (nw < 16 && nchunk > (int64_t)nw * 8) nw *= 2;
  return nw;
}

extern "C" int sglq_forward(sglq_dev *d, const void *A, int dt, int64_t M, const float *bias,
                            float *C, void *stream) {
  hipStream_t st = (hipStream_t)stream;
  const int64_t Kp = d->nsteps * 32;
  const bool split = dt == SGLQ_DT_F32;
  const int64_t esz = dt == SGLQ_DT_F32 ? 4 : 2;
  const int nw = pick_waves(d->nchunk);
  SGLQ_HIP(hipSetDevice(d->dev));
  for (int64_t m0 = 0; m0 < M; m0 += 64) {
    const int64_t mb = M - m0 < 64 ? M - m0 : 64;
    const size_t half_elems = (size_t)(Kp * mb);
    const size_t need = half_elems * 2 * (split ? 2 : 1) + 64 * 4 + 256;
    if (sglq_ws_reserve(d, need) != 0) return -1;
    _Float16 *hi = (_Float16 *)d->ws;
    _Float16 *lo = hi + half_elems;
    int *rowexp = (int *)((char *)d->ws + half_elems * 2 * (split ? 2 : 1));
    PrepArgs pa = {(const char *)A + m0 * d->K * esz, dt, d->K, d->K, Kp, mb, d->kmap,
                   d->kind == SGLQ_KIND_U4, split, hi, lo, rowexp};
    k_prep<<<(unsigned)mb, 256, 0, st>>>(pa);
    SGLQ_HIP(hipGetLastError());
    GemvArgs ga = {d->codes, d->scales, d->zeros, hi, lo, rowexp, bias, C,
                   d->N, mb, d->N, d->nchunk, d->spg, d->gpad, m0};
    const int mt = (int)((mb + 15) / 16);
    switch (d->kind) {
      case SGLQ_KIND_U4: launch_mt<SGLQ_KIND_U4>(ga, mt, split, d->scf16, nw, d->ntile, st); break;
      case SGLQ_KIND_U8: launch_mt<SGLQ_KIND_U8>(ga, mt, split, d->scf16, nw, d->ntile, st); break;
      default: launch_mt<SGLQ_KIND_E2M1>(ga, mt, split, 0, nw, d->ntile, st); break;
    }
    SGLQ_HIP(hipGetLastError());
  }
  return 0;
fail:
  return -1;
}

extern "C" int sglq_forward_host(sglq_dev *d, const float *A, int64_t M, const float *bias,
                                 float *C) {
  float *dA = nullptr, *dB = nullptr, *dC = nullptr;
  SGLQ_HIP(hipSetDevice(d->dev));
  SGLQ_HIP(hipMalloc(&dA, (size_t)(M * d->K) * 4));
  SGLQ_HIP(hipMalloc(&dC, (size_t)(M * d->N) * 4));
  SGLQ_HIP(hipMemcpy(dA, A, (size_t)(M * d->K) * 4, hipMemcpyHostToDevice));
  if (bias) {
    SGLQ_HIP(hipMalloc(&dB, (size_t)d->N * 4));
    SGLQ_HIP(hipMemcpy(dB, bias, (size_t)d->N * 4, hipMemcpyHostToDevice));
  }
  if (sglq_forward(d, dA, SGLQ_DT_F32, M, dB, dC, nullptr) != 0) goto fail;
  SGLQ_HIP(hipMemcpy(C, dC, (size_t)(M * d->N) * 4, hipMemcpyDeviceToHost));
  (void)hipFree(dA);
  (void)hipFree(dB);
  (void)hipFree(dC);
  return 0;
fail:
  (void)hipFree(dA);
  (void)hipFree(dB);
  (void)hipFree(dC);
  return -1;
}
