// gemm.hip — prefill-side quantized linear, C[M,N] = A[M,K] * W^T (+ bias) for M > 16.
//
// Launches:
//   k_prep_rows (or k_rowexp + k_prep_a)  the A operands, once per call: per row an exact
//             power of two that puts max|a| in [2^13, 2^14), then f16 hi (+ lo for f32 inputs)
//             in the layout [piece][step][kq][Mpad][8], gathered through kmap (act-order);
//             rows M..Mpad are zero.
//   k_gemm_lds  weights whose codes prescale exactly enough into f16 (groups with f16 scales in
//             [2^-14, 128], and MXFP4): each workgroup unpacks its weight tile once per stage
//             into LDS next to the A operands, through a ring of LDS buffers, and its waves run
//             v_mfma_f32_16x16x32_f16 from there.  Small M splits the stages over K, and
//             k_splitk_reduce adds the slices in order.
//   k_gemm_dma  the same weights, dense, where enough 128-row tiles exist (K <= 4096): wide
//             tiles (192 or 384 columns), codes unpacked in registers once per workgroup,
//             A operands copied global -> LDS through a four-deep ring.
//   k_gemm_breg  the same weights in the grouped (MoE) launches, 64-row expert blocks: the A
//             operands through LDS, each wave's codes unpacked in registers (one wave per
//             weight tile there, so LDS would buy no reuse); same products as k_gemm_lds.
//   k_gemm    every other weight: each wave loads its own codes straight into registers,
//             unpacks exact f16 (q - z) and applies the group scales in fp32 per chunk or step.
// MXFP4 block scales are folded into the fp4 -> f16 conversion relative to a per-column
// exponent (exact for every block within 2^23 of the column's largest), applied at the end.
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "sglq_dev.hpp"

namespace {


__device__ __forceinline__ float act_at(const void *A, int dt, int64_t i) {
  if (dt == SGLQ_DT_F32) return ((const float *)A)[i];
  const uint32_t b = ((const uint16_t *)A)[i];
  if (dt == SGLQ_DT_BF16) return __uint_as_float(b << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

__device__ __forceinline__ constexpr int kofs4(int i) { return (i >> 1) + 4 * (i & 1); }

// A operands for the GEMM, in two launches.  Source row of Aop row m:
//   MODE 0  A[m]                           (dense)
//   MODE 1  A[rowmap[m]], zero if < 0       (MoE: token of each expert-sorted row)
//   MODE 2  a_k = silu(A[m][k]) * A[m][kcols + k], A f32 (MoE: SwiGLU of the gate/up product,
//           silu(g) = g / (1 + e^-g) as reference src/deepseek.c:662-663, sglq_silu)
// k_rowexp: one wave per row finds its largest |a| and the exact power of two that puts it in
// [2^13, 2^14).  k_prep_a: workgroups of 16 rows x 64 items write the scaled f16 operands with
// consecutive threads on consecutive rows of one 16-B item (Aop keeps the rows of an item
// contiguous, so the stores coalesce).  vec: identity kmap with 16-byte aligned rows (8
// elements load as one or two 128-bit loads).
template <int MODE>
__device__ __forceinline__ int64_t prep_src(const int32_t *rowmap, int M, int m) {
  if (m >= M) return -1;
  if constexpr (MODE == 1) return rowmap[m];
  return m;
}

template <int MODE>
__device__ __forceinline__ float prep_value(const void *A, int dt, int64_t rb, int kcols, int k) {
  if constexpr (MODE == 2) {
    const float g = ((const float *)A)[rb + k];
    return sglq_silu(g) * ((const float *)A)[rb + kcols + k];
  } else {
    return act_at(A, dt, rb + k);
  }
}

// exponent e with |a| / 2^e in [2^13, 2^14) for the row's largest finite |a| = mx (0 for rows
// of zeros, infinities or NaNs only)
__device__ __forceinline__ int row_exponent(float mx) {
  return (mx > 0.f && mx <= 3.0e38f) ? ilogbf(mx) - 13 : 0;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_rowexp(const void *__restrict__ A, int dt, int64_t lda,
                                                int M, int Mpad, int K, int nsteps,
                                                const int32_t *__restrict__ kmap,
                                                const int32_t *__restrict__ rowmap, int kcols,
                                                int vec, int *__restrict__ rowexp) {
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (m >= Mpad) return;
  const int64_t src = prep_src<MODE>(rowmap, M, m);
  float mx = 0.f;
  if (src >= 0) {
    const int64_t rb = src * lda;
    if (MODE != 2 && vec) {
      // 8 elements per lane per 128-bit load, eight loads in flight at a time
      const int nv = K / 8;
      for (int v0 = 0; v0 < nv; v0 += 512) {
        uint4 raw[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int vi = min(v0 + lane + 64 * j, nv - 1);
          raw[j] = dt == SGLQ_DT_F32 ? *(const uint4 *)((const float *)A + rb + vi * 8)
                                     : *(const uint4 *)((const uint16_t *)A + rb + vi * 8);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
          if (v0 + lane + 64 * j >= nv) continue;
          const uint32_t wd[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
          if (dt == SGLQ_DT_F32) {
#pragma unroll
            for (int i = 0; i < 4; i++) mx = fmaxf(mx, fabsf(__uint_as_float(wd[i])));
            const uint4 hi4 = *(const uint4 *)((const float *)A + rb + (v0 + lane + 64 * j) * 8 + 4);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(__uint_as_float(hi4.x)), fabsf(__uint_as_float(hi4.y))),
                                 fmaxf(fabsf(__uint_as_float(hi4.z)), fabsf(__uint_as_float(hi4.w)))));
          } else {
#pragma unroll
            for (int i = 0; i < 8; i++) {
              const uint32_t hb = (wd[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
              const float x = dt == SGLQ_DT_BF16 ? __uint_as_float(hb << 16)
                                                 : (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
              mx = fmaxf(mx, fabsf(x));
            }
          }
        }
      }
      for (int k = nv * 8 + lane; k < K; k += 64) mx = fmaxf(mx, fabsf(act_at(A, dt, rb + k)));
    } else {
      for (int kp = lane; kp < nsteps * 32; kp += 64) {
        const int k = kmap ? kmap[kp] : (kp < K ? kp : -1);
        if (k >= 0) mx = fmaxf(mx, fabsf(prep_value<MODE>(A, dt, rb, kcols, k)));
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) rowexp[m] = row_exponent(mx);
}

template <int MODE>
__global__ __launch_bounds__(256) void k_prep_a(const void *__restrict__ A, int dt, int64_t lda,
                                                int M, int Mpad, int K, int nsteps,
                                                const int32_t *__restrict__ kmap,
                                                const int32_t *__restrict__ rowmap, int kcols,
                                                int perm4, int split, int vec,
                                                half8_t *__restrict__ aop,
                                                const int *__restrict__ rowmax,
                                                int *__restrict__ rowexp) {
  const int nitems = nsteps * 4;  // it = step * 4 + kq
  const int64_t plane = (int64_t)nitems * Mpad;  // 16-B items per piece
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int u = threadIdx.x + 256 * q;
    const int r = u & 15, it = blockIdx.y * 64 + (u >> 4);
    const int m = blockIdx.x * 16 + r;
    if (it >= nitems) continue;
    const int64_t src = prep_src<MODE>(rowmap, M, m);
    int e;
    if (rowmax) {  // row maxima from the producing kernel: the exponent is derived here
      e = row_exponent(__int_as_float(rowmax[m]));
      if (it == 0) rowexp[m] = e;
    } else {
      e = rowexp[m];
    }
    float v[8];
    if (src < 0) {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = 0.f;
    } else {
      const int64_t rb = src * lda;
      const int kb = it * 8;
      if (MODE != 2 && vec && kb + 8 <= K) {
        float raw[8];
        if (dt == SGLQ_DT_F32) {
          const float4 *p = (const float4 *)((const float *)A + rb + kb);
          const float4 x = p[0], y = p[1];
          raw[0] = x.x; raw[1] = x.y; raw[2] = x.z; raw[3] = x.w;
          raw[4] = y.x; raw[5] = y.y; raw[6] = y.z; raw[7] = y.w;
        } else {
          const uint4 x = *(const uint4 *)((const uint16_t *)A + rb + kb);
          const uint32_t wd[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const uint32_t hb = (wd[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
            raw[i] = dt == SGLQ_DT_BF16 ? __uint_as_float(hb << 16)
                                        : (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
          }
        }
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = raw[perm4 ? kofs4(i) : i];
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int kp = kb + (perm4 ? kofs4(i) : i);
          const int k = kmap ? kmap[kp] : (kp < K ? kp : -1);
          v[i] = k >= 0 ? prep_value<MODE>(A, dt, rb, kcols, k) : 0.f;
        }
      }
    }
    half8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x = ldexpf(v[i], -e);
      const _Float16 h = (_Float16)x;
      hi[i] = h;
      lo[i] = (_Float16)(x - (float)h);
    }
    aop[(int64_t)it * Mpad + m] = hi;
    if (split) aop[plane + (int64_t)it * Mpad + m] = lo;
  }
}

// k_prep_rows: both steps in one pass for dense or gathered rows (MODE 0/1): 16-byte loads
// for an identity kmap and 16-byte aligned rows, element gathers through kmap otherwise.  A workgroup owns R whole rows (R divides 256 and Mpad):
// thread u takes row u % R and items (u + 256 j) / R, holds up to IT items of that row in
// registers, the row maximum is reduced over the workgroup, and the scaled operands are
// written from registers, so A is read once and there is no second launch.  Consecutive
// threads write consecutive rows of one item (R x 16 contiguous bytes).  Bit-identical to
// k_rowexp + k_prep_a (the maximum is order-independent and the scaling is the same).
template <int MODE, int IT>
__global__ __launch_bounds__(256) void k_prep_rows(const void *__restrict__ A, int dt,
                                                   int64_t lda, int M, int Mpad, int K,
                                                   int nitems, const int32_t *__restrict__ kmap,
                                                   const int32_t *__restrict__ rowmap, int R, int xcd, int perm4, int split,
                                                   half8_t *__restrict__ aop,
                                                   int *__restrict__ rowexp) {
  __shared__ float red[4][16];
  // 16-B items of 8 consecutive rows share a 128-B line: with xcd set (Mpad % 64 == 0, R <= 8)
  // the 8 / R workgroups of one line run on one XCD (workgroups go round-robin over the 8
  // XCDs), so that XCD's L2 assembles the line before it is written back
  int blk = blockIdx.x;
  if (xcd) {
    const int G = 8 / R, x = blk & 7, t = blk >> 3;
    blk = (t / G) * 8 * G + x * G + t % G;
  }
  const int u = threadIdx.x, r = u % R, m = blk * R + r;
  const int64_t src = prep_src<MODE>(rowmap, M, m);
  const int64_t rb = src * lda;
  float v[IT][8];
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < IT; j++) {
    const int it = (u + 256 * j) / R, kb = it * 8;
    float raw[8];
    if (kmap) {  // act-order: element i of the item is A[kmap[kb + i]] (-1: padding)
      int4 k0 = make_int4(-1, -1, -1, -1), k1 = k0;
      if (src >= 0 && it < nitems) {
        k0 = *(const int4 *)(kmap + kb);
        k1 = *(const int4 *)(kmap + kb + 4);
      }
      const int kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
      for (int i = 0; i < 8; i++) raw[i] = kk[i] >= 0 ? act_at(A, dt, rb + kk[i]) : 0.f;
    } else if (src >= 0 && it < nitems && kb + 8 <= K) {
      if (dt == SGLQ_DT_F32) {
        const float4 *p = (const float4 *)((const float *)A + rb + kb);
        const float4 x = p[0], y = p[1];
        raw[0] = x.x; raw[1] = x.y; raw[2] = x.z; raw[3] = x.w;
        raw[4] = y.x; raw[5] = y.y; raw[6] = y.z; raw[7] = y.w;
      } else {
        const uint4 x = *(const uint4 *)((const uint16_t *)A + rb + kb);
        const uint32_t wd[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const uint32_t hb = (wd[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
          raw[i] = dt == SGLQ_DT_BF16 ? __uint_as_float(hb << 16)
                                      : (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++)
        raw[i] = (src >= 0 && it < nitems && kb + i < K) ? act_at(A, dt, rb + kb + i) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      v[j][i] = raw[perm4 ? kofs4(i) : i];
      mx = fmaxf(mx, fabsf(raw[i]));
    }
  }
  // row maximum: lanes u, u ^ o (o >= R) share a row; then the four waves through LDS
  for (int o = 32; o >= R; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  const int w = u >> 6, lane = u & 63;
  if (lane < R) red[w][lane] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][r], red[1][r]), fmaxf(red[2][r], red[3][r]));
  const int e = row_exponent(mx);
  if (u < R) rowexp[m] = e;
  const int64_t plane = (int64_t)nitems * Mpad;
#pragma unroll
  for (int j = 0; j < IT; j++) {
    const int it = (u + 256 * j) / R;
    if (it >= nitems) continue;
    half8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x = ldexpf(v[j][i], -e);
      const _Float16 h = (_Float16)x;
      hi[i] = h;
      lo[i] = (_Float16)(x - (float)h);
    }
    aop[(int64_t)it * Mpad + m] = hi;
    if (split) aop[plane + (int64_t)it * Mpad + m] = lo;
  }
}

struct GemmArgs {
  // dense: one weight; grouped (MoE): weight pointers per expert, picked per row block
  const u32x4_t *codes;
  const void *meta;
  const uint8_t *colexp;  // E2M1: per-column reference exponent (largest e8m0 of the column)
  const u32x4_t *const *codes_e;
  const void *const *meta_e;
  const uint8_t *const *colexp_e;
  const int4 *segs;       // grouped: per row block {expert, first row, rows, -}
  const int *nseg;        // grouped: number of row blocks (device scalar)
  const half8_t *aop;    // [np][nsteps][4][Mpad]
  const int *rowexp;
  const float *bias;
  float *C;
  int64_t ldc;
  int M, Mpad, N, ntile, nchunk, nsteps, nmeta, cpg, nbn;
  int nbm, xmap;  // dense: row blocks; 1 = XCD-aware tile order (see k_gemm)
  float *part;    // k_gemm_lds split over K: unscaled partial sums [gridDim.y][M][N], else null
  int swiglu;     // k_gemm_lds grouped: mi > 0 = C gets silu(gate) * up, [rows][mi] (see there)
  int *rowmax;    // with swiglu: per row, bits of the largest |C| (atomic max, preset to 0)
  int epi;        // k_gemm_breg: 1 = whole-row epilogue through LDS, 0 = per-lane stores
};

union H8 {
  half8_t v;
  uint32_t u[4];
  half2_t h[4];
};

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(o));
  return r;
}

template <int KIND>
__device__ __forceinline__ half8_t unpack_b(const u32x4_t &w, int j, half2_t zA, half2_t zB,
                                            float fsc) {
  H8 r;
  if constexpr (KIND == SGLQ_KIND_U4) {
    const uint32_t x = w[j], y = x >> 8;
    r.u[0] = and_or(x, 0x000F000Fu, 0x64006400u);
    r.u[1] = and_or(x, 0x00F000F0u, 0x54005400u);
    r.u[2] = and_or(y, 0x000F000Fu, 0x64006400u);
    r.u[3] = and_or(y, 0x00F000F0u, 0x54005400u);
    r.h[0] = r.h[0] + zA;
    r.h[1] = r.h[1] + zB;
    r.h[2] = r.h[2] + zA;
    r.h[3] = r.h[3] + zB;
  } else if constexpr (KIND == SGLQ_KIND_U8) {
    const uint32_t x0 = w[2 * j], x1 = w[2 * j + 1];
    r.u[0] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);
    r.u[1] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
    r.u[2] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
    r.u[3] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
#pragma unroll
    for (int i = 0; i < 4; i++) r.h[i] = r.h[i] + zA;
  } else {
    const uint32_t x = w[j];
    r.h[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, fsc, 0);
    r.h[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, fsc, 1);
    r.h[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, fsc, 2);
    r.h[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, fsc, 3);
  }
  return r.v;
}

template <bool SCF16>
using meta_t = typename std::conditional<SCF16, uint32_t, uint64_t>::type;

template <bool SCF16>
__device__ __forceinline__ void decode_meta(meta_t<SCF16> m, float &sc, half2_t &zA,
                                            half2_t &zB) {
  uint32_t zb;
  if constexpr (SCF16) {
    sc = (float)__builtin_bit_cast(_Float16, (uint16_t)(m & 0xFFFFu));
    zb = m >> 16;
  } else {
    sc = __uint_as_float((uint32_t)m);
    zb = (uint32_t)(m >> 32) & 0xFFFFu;
  }
  const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)zb);
  zA = (half2_t){z, z};
  const _Float16 z2 = z + (_Float16)960.0f;
  zB = (half2_t){z2, z2};
}

// 2^(e - ref) as f32 (0 for the reference's e == 255 "no scale" code and for underflow)
__device__ __forceinline__ float e8m0_rel(uint32_t e, int ref) {
  const int d = (int)e - ref + 127;
  return (e == 255u || d <= 0) ? 0.f : __uint_as_float((uint32_t)d << 23);
}

// Non-temporal 128-bit load through a global (not flat) pointer: weights are streamed once.
__device__ __forceinline__ u32x4_t ldg_nt(const u32x4_t *p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4_t *)p);
}
template <class T>
__device__ __forceinline__ T ldg(const T *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}

// Prefill GEMM.  PS ("prescaled"): the group scale is multiplied into the f16 weight in the
// unpack ((q - z) exact, then one f16 rounding of (q - z) * s) and the MFMAs accumulate C
// directly; used when every scale is an f16 value whose products stay normal f16.  Otherwise
// (f32 scales, per-step groups) the exact form keeps per-chunk partial sums and applies the
// fp32 scale to them.  MXFP4 always accumulates directly (scales folded exactly).  MB 16-row
// blocks per wave: the workgroup covers 32*MB rows x BN columns with 2 x 2 waves.
template <int KIND, bool SPLIT, bool SCF16, bool STEPM, int BN, bool PS, int MB>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr int NP = SPLIT ? 2 : 1;
  constexpr int TN = BN / 32;  // 16-column tiles per wave
  constexpr int BMR = 32 * MB; // rows per workgroup
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr bool DIRECT = PS || E2M1;       // accumulate C directly (no per-chunk partials)
  constexpr int ITEMS = NP * SPC * 4 * BMR; // 16-B A items per chunk
  constexpr int IPT = ITEMS / 256;          // per thread
  constexpr int RPI = 256 / BMR;            // item rows per 256 threads (1 or 2)
  extern __shared__ half8_t s_a[];          // [2][NP][SPC][4][BMR]

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int wm = w & 1, wn = w >> 1;
  const int n16 = lane & 15, kq = lane >> 4;
  // Tile order.  Workgroup i runs on XCD i % 8, and each XCD has its own L2.  With xmap the
  // row blocks are dealt to XCDs so that one XCD's workgroups share few activation row
  // blocks (kept in its L2) while the weight columns stream through: nbm >= 8 gives XCD x the
  // row blocks x, x+8, ...; nbm < 8 gives each row block 8/nbm XCDs that split the columns.
  int bn, bm;
  if (a.xmap) {
    const int x = (int)(blockIdx.x & 7), l = (int)(blockIdx.x >> 3);
    if (a.nbm >= 8) {
      bm = x + 8 * (l / a.nbn);
      bn = l % a.nbn;
    } else {
      const int r = 8 / a.nbm;
      bm = x % a.nbm;
      bn = x / a.nbm + r * l;
    }
    if (bm >= a.nbm || bn >= a.nbn) return;
  } else {
    bn = (int)(blockIdx.x % (unsigned)a.nbn);
    bm = (int)(blockIdx.x / (unsigned)a.nbn);
  }
  int m0 = bm * BMR, mend = a.M;
  const u32x4_t *codes = a.codes;
  const void *meta = a.meta;
  const uint8_t *colexp = a.colexp;
  if (a.segs) {  // grouped: row block bm of the expert-sorted rows
    if (bm >= *a.nseg) return;
    const int4 sg = a.segs[bm];
    m0 = sg.y;
    mend = sg.y + sg.z;
    codes = a.codes_e[sg.x];
    meta = a.meta_e[sg.x];
    if constexpr (KIND == SGLQ_KIND_E2M1) colexp = a.colexp_e[sg.x];
  }

  // A tile of chunk c, item q of this thread: row tid % BMR, slot r = q * RPI + tid / BMR with
  // r = (p * SPC + j) * 4 + kq'
  const int64_t plane = (int64_t)a.nsteps * 4 * a.Mpad;
  const int64_t cstride = (int64_t)SPC * 4 * a.Mpad;  // items per chunk along the K steps
  const half8_t *abase = a.aop + m0 + (tid % BMR) + (int64_t)(tid / BMR) * a.Mpad;
  auto a_off = [&](int q) -> int64_t {  // uniform part of item q's offset
    const int r = q * RPI;
    const int p = r / (SPC * 4), sj = r % (SPC * 4);
    return p * plane + (int64_t)sj * a.Mpad;
  };
  half8_t areg[IPT];
  auto load_a = [&](int c) {
#pragma unroll
    for (int q = 0; q < IPT; q++) areg[q] = ldg(abase + a_off(q) + c * cstride);
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int q = 0; q < IPT; q++) s_a[buf * ITEMS + tid + 256 * q] = areg[q];
  };

  // weights of this wave: tiles t0 .. t0+TN-1
  const int t0 = bn * (BN / 16) + wn * TN;
  using MT = typename std::conditional<E2M1, uint32_t, meta_t<SCF16>>::type;
  constexpr int NMV = STEPM ? SPC : 1;
  const u32x4_t *bptr[TN];
  const MT *mptr[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int t = min(t0 + j, a.ntile - 1);
    bptr[j] = codes + (int64_t)t * a.nchunk * 64 + lane;
    mptr[j] = (const MT *)meta + sglq_mrow(t, n16, E2M1 ? a.nmeta / 4 : a.nmeta);
  }
  u32x4_t bw[TN];
  MT bm_[TN][NMV];
  int cref[TN];
  u32x4_t bw2[TN];
  MT bm2[TN][NMV];
  // weights of chunk c (clamped to the last chunk: valid memory, never used past the end)
  auto load_b = [&](int c, u32x4_t (&w_)[TN], MT (&m_)[TN][NMV]) {
    c = min(c, a.nchunk - 1);
    const int g = c / a.cpg;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      w_[j] = ldg_nt(bptr[j] + c * 64);
      if constexpr (E2M1) {
        m_[j][0] = ldg((const uint32_t *)mptr[j] + sglq_mofs(c));
      } else if constexpr (STEPM) {
#pragma unroll
        for (int s = 0; s < SPC; s++) m_[j][s] = ldg(mptr[j] + sglq_mofs(c * SPC + s));
      } else {
        m_[j][0] = ldg(mptr[j] + sglq_mofs(g));
      }
    }
  };
  if constexpr (E2M1) {
#pragma unroll
    for (int j = 0; j < TN; j++) cref[j] = colexp[min(t0 + j, a.ntile - 1) * 16 + n16];
  }

  float4_t acc[MB][TN];
  float4_t tmp[DIRECT ? 1 : MB][DIRECT ? 1 : TN];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
  if constexpr (!DIRECT) {
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) tmp[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
  }

  // weights are loaded two chunks ahead (HBM latency), activations one chunk ahead (L2)
  load_a(0);
  load_b(0, bw, bm_);
  load_b(1, bw2, bm2);
  store_a(0);
  __syncthreads();
  for (int c = 0; c < a.nchunk; c++) {
    const int buf = c & 1;
    u32x4_t cw[TN];
    MT cm[TN][NMV];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      cw[j] = bw[j];
      bw[j] = bw2[j];
#pragma unroll
      for (int s = 0; s < NMV; s++) {
        cm[j][s] = bm_[j][s];
        bm_[j][s] = bm2[j][s];
      }
    }
    if (c + 1 < a.nchunk) {
      load_a(c + 1);
      load_b(c + 2, bw2, bm2);
    }
    const half8_t *sa = s_a + buf * ITEMS + wm * (16 * MB) + n16;
    float sc[TN];
    half2_t zA[TN], zB[TN], s2[TN];
    if constexpr (!E2M1 && !STEPM) {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        decode_meta<SCF16>(cm[j][0], sc[j], zA[j], zB[j]);
        if constexpr (PS) {
          const _Float16 hs = (_Float16)sc[j];
          s2[j] = (half2_t){hs, hs};
        }
      }
    }
#pragma unroll
    for (int s = 0; s < SPC; s++) {
      half8_t b[TN];
#pragma unroll
      for (int j = 0; j < TN; j++) {
        float fsc = 1.f;
        if constexpr (STEPM) decode_meta<SCF16>(cm[j][s], sc[j], zA[j], zB[j]);
        if constexpr (E2M1) fsc = e8m0_rel((cm[j][0] >> (8 * s)) & 255u, cref[j]);
        b[j] = unpack_b<KIND>(cw[j], s, zA[j], zB[j], fsc);
        if constexpr (PS && !E2M1) {
          H8 u;
          u.v = b[j];
#pragma unroll
          for (int h = 0; h < 4; h++) u.h[h] = u.h[h] * s2[j];
          b[j] = u.v;
        }
      }
#pragma unroll
      for (int i = 0; i < MB; i++) {
        half8_t av[NP];
#pragma unroll
        for (int p = 0; p < NP; p++) av[p] = sa[((p * SPC + s) * 4 + kq) * BMR + i * 16];
#pragma unroll
        for (int j = 0; j < TN; j++) {
#pragma unroll
          for (int p = 0; p < NP; p++) {
            if constexpr (DIRECT)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p], b[j], acc[i][j], 0, 0, 0);
            else
              tmp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p], b[j], tmp[i][j], 0, 0, 0);
          }
        }
      }
      if constexpr (STEPM && !DIRECT) {
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < TN; j++) {
            acc[i][j] += sc[j] * tmp[i][j];
            tmp[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    if constexpr (!STEPM && !DIRECT) {
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
          acc[i][j] += sc[j] * tmp[i][j];
          tmp[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};
        }
    }
    if (c + 1 < a.nchunk) {
      store_a(buf ^ 1);
      __syncthreads();
    }
  }

  // epilogue: lane holds rows 4*kq + r of each 16-row block, column n16 of each tile.  MXFP4
  // sums take the column exponent.
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int n = (t0 + j) * 16 + n16;
    if (n >= a.N) continue;
    const float bv = a.bias ? a.bias[n] : 0.f;
    const int ce = E2M1 ? cref[j] - 127 : 0;
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * (16 * MB) + i * 16 + 4 * kq + r;
        if (m < mend) a.C[(int64_t)m * a.ldc + n] = ldexpf(acc[i][j][r], a.rowexp[m] + ce) + bv;
      }
    }
  }
}

// Epilogue of the LDS kernels.  The lane holds rows mr0 + 16 i + 4 kq + r (i < MB) and
// column n16 of each of its TN tiles, the wave's tiles being the wn-th TN of the workgroup's
// NT16 (column block bn).  Three forms: the MoE gate/up SwiGLU (C = silu(g) * u with the row
// maxima of |C|), raw partial sums of a split over K, or C scaled by the row and column
// exponents plus the bias.
template <int MB, int TN, int NT16, bool E2M1>
__device__ __forceinline__ void lds_epilogue(const GemmArgs &a, const float4_t (&acc)[MB][TN],
                                             int mr0, int mend, int bn, int wn,
                                             const uint8_t *colexp, int n16, int kq) {
  if (a.swiglu) {
    // MoE gate/up: C[m][n] = silu(g) * u with g, u the gate and up outputs (sglq_silu,
    // g / (1 + e^-g) as reference src/deepseek.c:662-663), and the row maxima of |C|
    const int tg = bn * (NT16 / 2) + wn * (TN / 2), mi = a.swiglu;
    float rmx[MB][4];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
      for (int r = 0; r < 4; r++) rmx[i][r] = 0.f;
#pragma unroll
    for (int pj = 0; pj < TN / 2; pj++) {
      const int n = (tg + pj) * 16 + n16;
      if (n >= mi) continue;
      const int ceg = E2M1 ? (int)colexp[n] - 127 : 0;
      const int ceu = E2M1 ? (int)colexp[n + mi] - 127 : 0;
#pragma unroll
      for (int i = 0; i < MB; i++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = mr0 + i * 16 + 4 * kq + r;
          if (m < mend) {
            const float g = ldexpf(acc[i][2 * pj][r], a.rowexp[m] + ceg);
            const float u = ldexpf(acc[i][2 * pj + 1][r], a.rowexp[m] + ceu);
            const float v = sglq_silu(g) * u;
            a.C[(int64_t)m * a.ldc + n] = v;
            rmx[i][r] = fmaxf(rmx[i][r], fabsf(v));
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float x = rmx[i][r];
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));  // the row's 16 lanes
        const int m = mr0 + i * 16 + 4 * kq + r;
        if (n16 == 0 && m < mend) atomicMax(&a.rowmax[m], __float_as_int(x));
      }
    }
    return;
  }
  const int t0 = bn * NT16 + wn * TN;
  if (a.part) {  // split over K: raw partial sums, scaled by k_splitk_reduce
    float *pp = a.part + (int64_t)blockIdx.y * a.M * a.N;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = (t0 + j) * 16 + n16;
      if (n >= a.N) continue;
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = mr0 + i * 16 + 4 * kq + r;
          if (m < mend) pp[(int64_t)m * a.N + n] = acc[i][j][r];
        }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int n = (t0 + j) * 16 + n16;
    if (n >= a.N) continue;
    const float bv = a.bias ? a.bias[n] : 0.f;
    const int ce = E2M1 ? (int)colexp[min(t0 + j, a.ntile - 1) * 16 + n16] - 127 : 0;
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = mr0 + i * 16 + 4 * kq + r;
        if (m < mend) a.C[(int64_t)m * a.ldc + n] = ldexpf(acc[i][j][r], a.rowexp[m] + ce) + bv;
      }
    }
  }
}

// Prefill GEMM with the weight tile dequantized once per workgroup into LDS (the "direct"
// formats: prescaled U4/U8 groups and MXFP4).  (64 WMW) x BN tile, 2 WMW waves (WMW along M x 2
// along N, each 64 x BN/2), pipelined over stages of two MFMA steps through a ring of NBUF LDS
// buffers.  Each stage's A operands are copied and its weight codes unpacked (each code once
// per workgroup, not once per wave) into a buffer while the MFMAs read another one; blockIdx.y
// selects a slice of the stages when the call is split over K.
template <int KIND, int NP, int BN, int SSX, int WMW, int NBUF, int MB, int RS>
__global__ __launch_bounds__(128 * WMW, 2) void k_gemm_lds(GemmArgs a) {
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr int SS = SSX < SPC ? SSX : SPC;  // MFMA steps per stage
  constexpr int HPC = SPC / SS;         // stages per chunk
  constexpr int NTH = 128 * WMW;        // threads: WMW waves along M x 2 along N
  constexpr int BMR = 16 * MB * WMW;   // rows: WMW waves of MB 16-row blocks
  constexpr int NT16 = BN / 16;         // weight tiles per workgroup
  constexpr int TN = NT16 / 2;          // per wave
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr int AITEMS = NP * SS * 4 * BMR;  // 16-B A items per stage
  constexpr int AIPT = AITEMS / NTH;
  constexpr int BITEMS = NT16 * SS * 64;     // 16-B weight operands per stage
  constexpr int PB = NT16 * 64 / NTH;        // (tile, lane) code words per thread
  extern __shared__ half8_t s_lds[];         // [NBUF][AITEMS] A, then [NBUF][BITEMS] B
  half8_t *s_a = s_lds;
  half8_t *s_b = s_lds + NBUF * AITEMS;

  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int wm = w % WMW, wn = w / WMW;
  const int n16 = lane & 15, kq = lane >> 4;
  int bn, bm;
  if (a.xmap) {
    const int x = (int)(blockIdx.x & 7), l = (int)(blockIdx.x >> 3);
    if (a.nbm >= 8) {
      bm = x + 8 * (l / a.nbn);
      bn = l % a.nbn;
    } else {
      const int r = 8 / a.nbm;
      bm = x % a.nbm;
      bn = x / a.nbm + r * l;
    }
    if (bm >= a.nbm || bn >= a.nbn) return;
  } else {
    bn = (int)(blockIdx.x % (unsigned)a.nbn);
    bm = (int)(blockIdx.x / (unsigned)a.nbn);
  }
  int m0 = bm * BMR, mend = a.M;
  const u32x4_t *codes = a.codes;
  const void *meta = a.meta;
  const uint8_t *colexp = a.colexp;
  if (a.segs) {  // grouped: row block bm of the expert-sorted rows
    if (bm >= *a.nseg) return;
    const int4 sg = a.segs[bm];
    m0 = sg.y;
    mend = sg.y + sg.z;
    codes = a.codes_e[sg.x];
    meta = a.meta_e[sg.x];
    if constexpr (E2M1) colexp = a.colexp_e[sg.x];
  }
  // split over K (blockIdx.y): this workgroup's stages [st0, st1)
  const int nstage = a.nsteps / SS;
  const int st0 = (int)((int64_t)nstage * blockIdx.y / gridDim.y);
  const int st1 = (int)((int64_t)nstage * (blockIdx.y + 1) / gridDim.y);

  // ---- activations: item q of this thread is row tid % BMR, slot r = RPI q + tid / BMR with
  // r = (p * SS + s) * 4 + kq'
  constexpr int RPI = NTH / BMR;  // 2
  const int64_t plane = (int64_t)a.nsteps * 4 * a.Mpad;
  const half8_t *abase = a.aop + m0 + (tid % BMR) + (int64_t)(tid / BMR) * a.Mpad;
  auto load_a = [&](int st, half8_t(&areg)[AIPT]) {
#pragma unroll
    for (int q = 0; q < AIPT; q++) {
      const int r = RPI * q;  // + tid / BMR (in abase)
      const int p = r / (SS * 4), sj = r % (SS * 4);
      areg[q] = ldg(abase + p * plane + ((int64_t)st * SS * 4 + sj) * a.Mpad);
    }
  };
  auto store_a = [&](int buf, const half8_t(&areg)[AIPT]) {
#pragma unroll
    for (int q = 0; q < AIPT; q++) s_a[buf * AITEMS + tid + NTH * q] = areg[q];
  };

  // ---- weights: thread handles (tile tb, lane lb) = (p / 64, p % 64) for p = tid + 256 q
  using MT = typename std::conditional<E2M1, uint32_t, uint32_t>::type;  // f16 scale | zero
  const u32x4_t *bsrc[PB];
  const uint32_t *msrc[PB];
  int cref[PB];
#pragma unroll
  for (int q = 0; q < PB; q++) {
    const int pp = tid + NTH * q, tb = pp >> 6, lb = pp & 63;
    int t;
    if (a.swiglu) {  // a wave's tiles alternate gate tile g, up tile g + mi / 16
      const int jj = tb % TN, mt = a.swiglu / 16;
      t = min(bn * (NT16 / 2) + (tb / TN) * (TN / 2) + jj / 2, mt - 1) + (jj & 1) * mt;
    } else {
      t = min(bn * NT16 + tb, a.ntile - 1);
    }
    bsrc[q] = codes + (int64_t)t * a.nchunk * 64 + lb;
    msrc[q] = (const uint32_t *)meta + sglq_mrow(t, lb & 15, E2M1 ? a.nmeta / 4 : a.nmeta);
    if constexpr (E2M1) cref[q] = colexp[t * 16 + (lb & 15)];
  }
  auto load_b = [&](int st, u32x4_t(&breg)[PB], MT(&mreg)[PB]) {
    const int c = st / HPC, h = st % HPC;
    const int g = c / a.cpg;
#pragma unroll
    for (int q = 0; q < PB; q++) {
      if constexpr (KIND == SGLQ_KIND_U8) {
        breg[q] = ldg_nt(bsrc[q] + c * 64);
      } else if constexpr (SS == SPC) {
        breg[q] = ldg_nt(bsrc[q] + c * 64);
      } else {  // the two words of this half chunk
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t x = ldg((const u32x2_t *)((const uint32_t *)(bsrc[q] + c * 64) + 2 * h));
        breg[q] = (u32x4_t){x[0], x[1], 0u, 0u};
      }
      if constexpr (E2M1)
        mreg[q] = ldg(msrc[q] + sglq_mofs(c)) >> (8 * SS * h);  // e8m0 bytes of the stage's steps
      else
        mreg[q] = ldg(msrc[q] + sglq_mofs(g));
    }
  };
  auto store_b = [&](int buf, const u32x4_t(&breg)[PB], const MT(&mreg)[PB]) {
#pragma unroll
    for (int q = 0; q < PB; q++) {
      const int pp = tid + NTH * q, tb = pp >> 6, lb = pp & 63;
      float sc;
      half2_t zA = {0, 0}, zB = {0, 0}, s2 = {0, 0};
      if constexpr (!E2M1) {
        decode_meta<true>(mreg[q], sc, zA, zB);
        const _Float16 hs = (_Float16)sc;
        s2 = (half2_t){hs, hs};
      }
#pragma unroll
      for (int s = 0; s < SS; s++) {
        float fsc = 1.f;
        if constexpr (E2M1) fsc = e8m0_rel((mreg[q] >> (8 * s)) & 255u, cref[q]);
        H8 u;
        u.v = unpack_b<KIND>(breg[q], s, zA, zB, fsc);
        if constexpr (!E2M1) {
#pragma unroll
          for (int hh = 0; hh < 4; hh++) u.h[hh] = u.h[hh] * s2;
        }
        s_b[buf * BITEMS + (tb * SS + s) * 64 + lb] = u.v;
      }
    }
  };

  float4_t acc[MB][TN];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // all operands of one stage are read from LDS before its MFMAs, so the reads overlap each
  // other and the MFMAs wait once
  auto compute = [&](int buf) {
    const half8_t *sa = s_a + buf * AITEMS + wm * (16 * MB) + n16;
    const half8_t *sb = s_b + buf * BITEMS + wn * TN * SS * 64 + lane;
    half8_t bv[SS][TN], av[SS][NP][MB];
#pragma unroll
    for (int s = 0; s < SS; s++) {
#pragma unroll
      for (int j = 0; j < TN; j++) bv[s][j] = sb[(j * SS + s) * 64];
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < MB; i++) av[s][p][i] = sa[((p * SS + s) * 4 + kq) * BMR + i * 16];
    }
#pragma unroll
    for (int s = 0; s < SS; s++)
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < MB; i++)
#pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(av[s][p][i], bv[s][j], acc[i][j], 0, 0, 0);
  };

  // One register set and NBUF LDS buffers in a ring.  NBUF = 2: iteration r loads stage r + 1,
  // multiplies stage r, then writes stage r + 1 into the other buffer.  NBUF = 3: iteration r
  // writes stage r + 1 (loaded during iteration r - 1) into buffer (r + 1) % 3, loads stage
  // r + 2 and multiplies stage r, so the loads of a stage have a whole iteration in flight.
  // One barrier per iteration; the loop body is uniform (past the end it reloads the last
  // stage into a buffer nobody reads).
  if constexpr (RS == 2) {
    // Two register sets, two LDS buffers: iteration r loads stage r + 2 into one set while the
    // other holds stage r + 1 (loaded one iteration earlier), multiplies stage r and then writes
    // stage r + 1 into the other buffer, so each stage's loads have two iterations in flight.
    // Unrolled by two so that each set is named at compile time.
    half8_t a0[AIPT], a1[AIPT];
    u32x4_t b0[PB], b1[PB];
    MT mr0[PB], mr1[PB];
    auto step = [&](int st, int p, half8_t(&al)[AIPT], u32x4_t(&bl)[PB], MT(&ml)[PB],
                    const half8_t(&as)[AIPT], const u32x4_t(&bs)[PB], const MT(&ms)[PB]) {
      const int nx = min(st + 2, st1 - 1);  // past the end: a harmless reload
      load_a(nx, al);
      load_b(nx, bl, ml);
      __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the MFMAs
      compute(p);
      store_a(p ^ 1, as);
      store_b(p ^ 1, bs, ms);
      __builtin_amdgcn_iglp_opt(1);  // let the scheduler interleave LDS traffic with MFMAs
      __syncthreads();
    };
    load_a(st0, a0);
    load_b(st0, b0, mr0);
    load_a(min(st0 + 1, st1 - 1), a1);
    load_b(min(st0 + 1, st1 - 1), b1, mr1);
    store_a(0, a0);
    store_b(0, b0, mr0);
    __syncthreads();
    int st = st0;
    for (; st + 2 <= st1; st += 2) {
      step(st, 0, a0, b0, mr0, a1, b1, mr1);
      step(st + 1, 1, a1, b1, mr1, a0, b0, mr0);
    }
    if (st < st1) step(st, 0, a0, b0, mr0, a1, b1, mr1);
  } else {
  half8_t ar[AIPT];
  u32x4_t br[PB];
  MT mr[PB];
  load_a(st0, ar);
  load_b(st0, br, mr);
  store_a(0, ar);
  store_b(0, br, mr);
  if constexpr (NBUF == 3) {
    load_a(min(st0 + 1, st1 - 1), ar);
    load_b(min(st0 + 1, st1 - 1), br, mr);
  }
  __syncthreads();
  int bc = 0;  // buffer of stage r
  for (int st = st0; st < st1; st++) {
    const int bn1 = bc == NBUF - 1 ? 0 : bc + 1;
    if constexpr (NBUF == 3) {
      store_a(bn1, ar);
      store_b(bn1, br, mr);
    }
    const int nx = min(st + NBUF - 1, st1 - 1);
    load_a(nx, ar);
    load_b(nx, br, mr);
    __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of the MFMAs
    compute(bc);
    if constexpr (NBUF == 2) {
      store_a(bn1, ar);
      store_b(bn1, br, mr);
    }
    __syncthreads();
    bc = bn1;
  }
  }

  lds_epilogue<MB, TN, NT16, E2M1>(a, acc, m0 + wm * (16 * MB), mend, bn, wn, colexp, n16, kq);
}

template <int MBW, int TN, bool E2M1, int RP, int WN>
__device__ void wide_epilogue(const GemmArgs &a, const float4_t (&acc)[MBW][TN], float *stg,
                              int m0, int mend, int bn, int w, int n16, int kq,
                              const uint8_t *colexp);
template <int MBW, int TN, bool E2M1, int RP, int WN>
__device__ void swiglu_epilogue(const GemmArgs &a, const float4_t (&acc)[MBW][TN], float *stg,
                                int m0, int mend, int bn, int w, int n16, int kq,
                                const uint8_t *colexp);

// Prefill GEMM for row blocks of at most 64 rows (dense M <= 64, MoE expert blocks) on the
// direct formats: the same 64 x 128 tile, operands and epilogue as k_gemm_lds<.., 128, .., 1,
// .., 4, ..>, but each weight tile feeds a single wave there, so a trip through LDS buys no
// reuse.  Here each of the WN waves (TN = 8 / WN tiles each) loads its own codes straight into
// registers, D chunks ahead in a ring, and unpacks them there with the same prescale ((q - z)
// exact in f16, then one f16 rounding of the product with the f16 group scale; MXFP4 through
// the scaled fp4 conversion), so the products are bit-identical to k_gemm_lds.  Only the A
// operands (64 rows, one chunk per stage) go through a double-buffered LDS ring, one chunk
// ahead in registers.  blockIdx.y selects a slice of the chunks when the call is split over K.
// MINB: waves per SIMD the register budget must allow.
template <int KIND, int NP, int WN, int TN, int D, int MINB = 2>
__global__ __launch_bounds__(64 * WN, MINB) void k_gemm_breg(GemmArgs a) {
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr int MB = 4, BMR = 64, NT16 = WN * TN, NTH = 64 * WN;
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr int AITEMS = NP * SPC * 4 * BMR;  // 16-B A items per chunk
  constexpr int AIPT = AITEMS / NTH;
  extern __shared__ half8_t s_a[];  // [2][AITEMS]

  const int tid = threadIdx.x, wn = tid >> 6, lane = tid & 63;
  const int n16 = lane & 15, kq = lane >> 4;
  int bn, bm;
  if (a.xmap) {
    const int x = (int)(blockIdx.x & 7), l = (int)(blockIdx.x >> 3);
    if (a.nbm >= 8) {
      bm = x + 8 * (l / a.nbn);
      bn = l % a.nbn;
    } else {
      const int r = 8 / a.nbm;
      bm = x % a.nbm;
      bn = x / a.nbm + r * l;
    }
    if (bm >= a.nbm || bn >= a.nbn) return;
  } else {
    bn = (int)(blockIdx.x % (unsigned)a.nbn);
    bm = (int)(blockIdx.x / (unsigned)a.nbn);
  }
  int m0 = bm * BMR, mend = a.M;
  const u32x4_t *codes = a.codes;
  const void *meta = a.meta;
  const uint8_t *colexp = a.colexp;
  if (a.segs) {  // grouped: row block bm of the expert-sorted rows
    if (bm >= *a.nseg) return;
    const int4 sg = a.segs[bm];
    m0 = sg.y;
    mend = sg.y + sg.z;
    codes = a.codes_e[sg.x];
    meta = a.meta_e[sg.x];
    if constexpr (E2M1) colexp = a.colexp_e[sg.x];
  }
  const int c0 = (int)((int64_t)a.nchunk * blockIdx.y / gridDim.y);
  const int c1 = (int)((int64_t)a.nchunk * (blockIdx.y + 1) / gridDim.y);

  // ---- A operands of chunk c: item q of this thread is row tid % 64, slot WN q + tid / 64
  // with slot = (p * SPC + s) * 4 + kq'
  const int64_t plane = (int64_t)a.nsteps * 4 * a.Mpad;
  const half8_t *abase = a.aop + m0 + lane + (int64_t)wn * a.Mpad;
  auto load_a = [&](int c, half8_t(&ar)[AIPT]) {
#pragma unroll
    for (int q = 0; q < AIPT; q++) {
      const int r = WN * q, p = r / (SPC * 4), sj = r % (SPC * 4);
      ar[q] = ldg(abase + p * plane + ((int64_t)c * SPC * 4 + sj) * a.Mpad);
    }
  };
  auto store_a = [&](int buf, const half8_t(&ar)[AIPT]) {
#pragma unroll
    for (int q = 0; q < AIPT; q++) s_a[buf * AITEMS + tid + NTH * q] = ar[q];
  };

  // ---- this wave's weight tiles
  const u32x4_t *bsrc[TN];
  const uint32_t *msrc[TN];
  int cref[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) {
    int t;
    if (a.swiglu) {  // a wave's tiles alternate gate tile g, up tile g + mi / 16
      const int mt = a.swiglu / 16;
      t = min(bn * (NT16 / 2) + wn * (TN / 2) + j / 2, mt - 1) + (j & 1) * mt;
    } else {
      t = min(bn * NT16 + wn * TN + j, a.ntile - 1);
    }
    bsrc[j] = codes + (int64_t)t * a.nchunk * 64 + lane;
    msrc[j] = (const uint32_t *)meta + sglq_mrow(t, n16, E2M1 ? a.nmeta / 4 : a.nmeta);
    cref[j] = E2M1 ? colexp[t * 16 + n16] : 0;
  }
  auto load_b = [&](int c, u32x4_t(&bw)[TN], uint32_t(&bm_)[TN]) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
      bw[j] = ldg_nt(bsrc[j] + c * 64);
      // e8m0 bytes | group meta
      bm_[j] = E2M1 ? ldg(msrc[j] + sglq_mofs(c)) : ldg(msrc[j] + sglq_mofs(c / a.cpg));
    }
  };

  float4_t acc[MB][TN];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, const u32x4_t(&cw)[TN], const uint32_t(&cm)[TN]) {
    const half8_t *sa = s_a + buf * AITEMS + n16;
    half2_t zA[TN], zB[TN], s2[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      zA[j] = zB[j] = s2[j] = (half2_t){0, 0};
      if constexpr (!E2M1) {
        float sc;
        decode_meta<true>(cm[j], sc, zA[j], zB[j]);
        const _Float16 hs = (_Float16)sc;
        s2[j] = (half2_t){hs, hs};
      }
    }
#pragma unroll
    for (int s = 0; s < SPC; s++) {
      half8_t av[NP][MB];
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < MB; i++) av[p][i] = sa[((p * SPC + s) * 4 + kq) * BMR + i * 16];
      // each unpacked weight fragment feeds its MB (x NP) MFMAs at once, so one fragment is
      // live at a time (fewer registers: three workgroups per CU)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const float fsc = E2M1 ? e8m0_rel((cm[j] >> (8 * s)) & 255u, cref[j]) : 1.f;
        H8 u;
        u.v = unpack_b<KIND>(cw[j], s, zA[j], zB[j], fsc);
        if constexpr (!E2M1) {
#pragma unroll
          for (int hh = 0; hh < 4; hh++) u.h[hh] = u.h[hh] * s2[j];
        }
#pragma unroll
        for (int p = 0; p < NP; p++)
#pragma unroll
          for (int i = 0; i < MB; i++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p][i], u.v, acc[i][j], 0, 0, 0);
      }
    }
  };

  // Chunk k of the slice: its codes were loaded D chunks earlier into ring slot k % D (the
  // loop is unrolled by D so every slot is named at compile time); its A operands sit in LDS
  // buffer k & 1.  An iteration multiplies chunk k from its ring slot, refills the slot with
  // chunk k + D, then writes chunk k + 1's A operands (loaded one iteration earlier) into the
  // other buffer and loads chunk k + 2's.  Loads past the slice reload its last chunk (valid
  // memory, never used).
  u32x4_t bq[D][TN];
  uint32_t mq[D][TN];
  half8_t ar[AIPT];
  const int nc = c1 - c0;
#pragma unroll
  for (int u = 0; u < D; u++) load_b(min(c0 + u, c1 - 1), bq[u], mq[u]);
  load_a(c0, ar);
  store_a(0, ar);
  load_a(min(c0 + 1, c1 - 1), ar);
  __syncthreads();
  for (int kb = 0; kb < nc; kb += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int k = kb + u;
      if (k < nc) {
        // multiply from the ring slot, then refill it: D sets of codes live, not D + 1
        // (copying a slot out before its refill cost the registers of a third workgroup per
        // CU; config 5 prefill 174-177 -> 163-174 us with the third)
        compute(k & 1, bq[u], mq[u]);
        load_b(min(c0 + k + D, c1 - 1), bq[u], mq[u]);
        store_a((k + 1) & 1, ar);
        load_a(min(c0 + k + 2, c1 - 1), ar);
        __syncthreads();
      }
    }
  }
  if (a.epi) {  // whole rows through LDS (the A buffers are free after the loop's barrier)
    constexpr int COLS = 16 * NT16, RP = 16;
    static_assert(RP * COLS * 4 <= 2 * AITEMS * 16, "k_gemm_breg: epilogue staging");
    if (a.swiglu)
      swiglu_epilogue<MB, TN, E2M1, RP, WN>(a, acc, (float *)s_a, m0, mend, bn, wn, n16, kq,
                                            colexp);
    else
      wide_epilogue<MB, TN, E2M1, RP, WN>(a, acc, (float *)s_a, m0, mend, bn, wn, n16, kq,
                                          colexp);
    return;
  }
  lds_epilogue<MB, TN, NT16, E2M1>(a, acc, m0, mend, bn, wn, colexp, n16, kq);
}

// Epilogue of the dense register-B kernels: the tile goes through LDS (16, 8 or 4 rows at a
// time) so that consecutive threads store consecutive 16-byte pieces of whole rows of C (or of
// the K-split partials), instead of each lane storing 4-byte values of four rows.  C[m][n] =
// 2^(rowexp[m] + ce[n]) acc + bias[n]; partials are stored unscaled.  stg: at least
// RP x 64 TN floats of LDS, free for this use (every wave is past its last LDS read).
template <int MBW, int TN, bool E2M1, int RP, int WN>
__device__ void wide_epilogue(const GemmArgs &a, const float4_t (&acc)[MBW][TN], float *stg,
                              int m0, int mend, int bn, int w, int n16, int kq,
                              const uint8_t *colexp) {
  // wave w holds every 16-row block i < MBW of column group w; pass (i, h) stages rows
  // h RP .. h RP + RP - 1 of block i
  constexpr int COLS = 16 * WN * TN, C4 = COLS / 4, ITEMS = RP * C4, NTH = 64 * WN;
  const int tid = threadIdx.x;
  const int nb = bn * COLS;
  float *out = a.part ? a.part + (int64_t)blockIdx.y * a.M * a.N : a.C;
  const int64_t ld = a.part ? a.N : a.ldc;
  const bool vec = ((uintptr_t)out % 16 == 0) && (ld % 4 == 0) && (a.N % 4 == 0);
#pragma unroll
  for (int i = 0; i < MBW; i++) {
#pragma unroll
    for (int h = 0; h < 16 / RP; h++) {
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int row = 4 * kq + r - h * RP;
          if (row >= 0 && row < RP)
            stg[row * COLS + (w * TN + j) * 16 + n16] = acc[i][j][r];
        }
      __syncthreads();
      for (int e = tid; e < ITEMS; e += NTH) {
        const int row = e / C4, c4 = e % C4;
        const int m = m0 + 16 * i + h * RP + row, n = nb + 4 * c4;
        if (m >= mend || n >= a.N) continue;
        float4_t v = *(const float4_t *)(stg + row * COLS + 4 * c4);
        if (!a.part) {
          const int re = a.rowexp[m];
#pragma unroll
          for (int u = 0; u < 4; u++) {
            const int nn = min(n + u, a.N - 1);
            const int ce = E2M1 ? (int)colexp[nn] - 127 : 0;
            v[u] = ldexpf(v[u], re + ce) + (a.bias ? a.bias[nn] : 0.f);
          }
        }
        float *o = out + (int64_t)m * ld + n;
        if (vec) {
          *(float4_t *)o = v;
        } else {
#pragma unroll
          for (int u = 0; u < 4; u++)
            if (n + u < a.N) o[u] = v[u];
        }
      }
      __syncthreads();
    }
  }
}

// Epilogue of the grouped gate/up launch (MoE, k_gemm_breg with the SwiGLU): wave w's tile
// pairs (2p, 2p + 1) hold gate tile g and up tile g + mi / 16 of the same columns, so
// silu(g) * u is formed in registers (reference src/deepseek.c:662-663), staged through LDS RP
// rows at a time and stored as whole rows of C [rows][mi]; the row maxima of |C| go to
// a.rowmax (one atomic max per row and wave) for the next prep.
template <int MBW, int TN, bool E2M1, int RP, int WN>
__device__ void swiglu_epilogue(const GemmArgs &a, const float4_t (&acc)[MBW][TN], float *stg,
                                int m0, int mend, int bn, int w, int n16, int kq,
                                const uint8_t *colexp) {
  constexpr int HC = 8 * WN * TN, C4 = HC / 4, ITEMS = RP * C4, NTH = 64 * WN;
  const int tid = threadIdx.x, mi = a.swiglu, nb = bn * HC;
  const bool vec = ((uintptr_t)a.C % 16 == 0) && (a.ldc % 4 == 0) && (mi % 4 == 0);
  float rmx[MBW][4];
#pragma unroll
  for (int i = 0; i < MBW; i++)
#pragma unroll
    for (int r = 0; r < 4; r++) rmx[i][r] = 0.f;
#pragma unroll
  for (int i = 0; i < MBW; i++) {
#pragma unroll
    for (int h = 0; h < 16 / RP; h++) {
#pragma unroll
      for (int pj = 0; pj < TN / 2; pj++) {
        const int col = (w * (TN / 2) + pj) * 16 + n16, n = nb + col;
        const int ceg = E2M1 ? (int)colexp[min(n, mi - 1)] - 127 : 0;
        const int ceu = E2M1 ? (int)colexp[min(n, mi - 1) + mi] - 127 : 0;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int row = 4 * kq + r - h * RP, m = m0 + 16 * i + 4 * kq + r;
          if (row < 0 || row >= RP) continue;
          float v = 0.f;
          if (n < mi && m < mend) {
            const float g = ldexpf(acc[i][2 * pj][r], a.rowexp[m] + ceg);
            const float u = ldexpf(acc[i][2 * pj + 1][r], a.rowexp[m] + ceu);
            v = sglq_silu(g) * u;
          }
          stg[row * HC + col] = v;
          rmx[i][r] = fmaxf(rmx[i][r], fabsf(v));
        }
      }
      __syncthreads();
      for (int e = tid; e < ITEMS; e += NTH) {
        const int row = e / C4, c4 = e % C4;
        const int m = m0 + 16 * i + h * RP + row, n = nb + 4 * c4;
        if (m >= mend || n >= mi) continue;
        const float4_t v = *(const float4_t *)(stg + row * HC + 4 * c4);
        float *o = a.C + (int64_t)m * a.ldc + n;
        if (vec) {
          *(float4_t *)o = v;
        } else {
#pragma unroll
          for (int u = 0; u < 4; u++)
            if (n + u < mi) o[u] = v[u];
        }
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < MBW; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float x = rmx[i][r];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));  // the row's 16 lanes
      const int m = m0 + 16 * i + 4 * kq + r;
      if (n16 == 0 && m < mend) atomicMax(&a.rowmax[m], __float_as_int(x));
    }
  }
}

// Tile of k_gemm_dma's workgroup.  Workgroups go round-robin over the 8 XCDs
// (blockIdx.x & 7); each XCD takes a contiguous run of tiles in row-block-major order, so it
// holds few row blocks and its L2 keeps their A rows.  (Column-block-major order, where each
// XCD reads its weights once, and row-block pairs measured the same at M = 512 and 2048.)
__device__ __forceinline__ bool wide_tile(const GemmArgs &a, int &bm, int &bn) {
  const int total = a.nbm * a.nbn, per = (total + 7) >> 3;
  const int idx = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (idx >= total) return false;
  bm = idx / a.nbn;
  bn = idx % a.nbn;
  return true;
}

// s_waitcnt that waits until at most n vector memory operations of this wave are outstanding
// (expcnt and lgkmcnt left alone): gfx9 encoding, vmcnt in bits 3:0 and 15:14
#define SGLQ_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x70 | 0xF00)

// Dense prefill GEMM on the direct formats, deep asynchronous pipeline.  A workgroup of WN
// waves covers 16 MB rows x 16 WN TN columns; wave w owns weight tiles WN TN bn + TN w + j
// (j < TN) over all rows, so each code is loaded and unpacked once per workgroup, in
// registers, and only the A operands go through LDS:
//   * A operands go global -> LDS directly (global_load_lds_dwordx4, no registers) into a
//     ring of four buffers, issued three chunks ahead of their use;
//   * codes and meta of a chunk are loaded into a 4-deep register ring four chunks ahead;
//   * the loop body is four chunks, so every buffer and register set is named statically;
//     chunks past the end compute with zero scales (adding exact zeros);
//   * one barrier per chunk, after this wave's own copies of the chunk have landed (an
//     explicit vmcnt wait: the copies of the next chunks stay in flight);
//   * VALU work does not issue in the shadow of the same wave's MFMAs on gfx950 (measured with
//     k_mfma_valu), so the unpack is kept to one pass per workgroup, and with 4 waves (one per
//     SIMD) the A fragments of a chunk are read up front and the unpack of step s + 1 is
//     interleaved with step s's MFMAs (SCHED); 8 waves (two per SIMD) overlap each other, and
//     so do two workgroups of 64-row tiles (MINB = 2 waves per SIMD, A fragments per step).
// Products are those of k_gemm_lds (same prescale and unpack); the epilogue stores whole rows.
template <int KIND, int NP, int TN, int MB, bool SCHED, int WN, int MINB = 1>
__global__ __launch_bounds__(64 * WN, MINB) void k_gemm_dma(GemmArgs a) {
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr int BMR = 16 * MB;
  constexpr int NT16 = WN * TN;
  constexpr int SLOTS = NP * SPC * 4;  // 16-B A slots (piece, step, kq) per chunk
  constexpr int AITEMS = SLOTS * BMR;  // 16-B A items per chunk
  constexpr int NTH = 64 * WN;       // WN waves along N
  constexpr int MBW = MB;            // 16-row blocks per wave (all rows of the tile)
  constexpr int AIPT = AITEMS / NTH;  // copies per thread per chunk
  constexpr int RPI = NTH / BMR;
  static_assert(AITEMS % NTH == 0 && NTH % BMR == 0, "k_gemm_dma: row tile");
  // four separately declared buffers: the compiler then tells the copies into one buffer from
  // reads of another and does not wait for every outstanding copy before an LDS read
  __shared__ half8_t sA0[AITEMS], sA1[AITEMS], sA2[AITEMS], sA3[AITEMS];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = tid >> 6;  // column group
  const int n16 = lane & 15, kq = lane >> 4;
  int bm, bn;
  if (!wide_tile(a, bm, bn)) return;
  const int m0 = bm * BMR, mend = a.M;
  const int c0 = (int)((int64_t)a.nchunk * blockIdx.y / gridDim.y);
  const int c1 = (int)((int64_t)a.nchunk * (blockIdx.y + 1) / gridDim.y);

  // copy q of this thread: LDS item tid + 256 q = row tid % BMR of slot RPI q + tid / BMR; the
  // 64 lanes of a wave fill 1 KiB of LDS from 1 KiB of consecutive rows
  const int64_t plane = (int64_t)a.nsteps * 4 * a.Mpad;
  const half8_t *abase = a.aop + m0 + (tid % BMR) + (int64_t)(tid / BMR) * a.Mpad;
  auto copy_a = [&](int c, half8_t *buf) {
    const int cc = min(c, c1 - 1);
#pragma unroll
    for (int q = 0; q < AIPT; q++) {
      const int r = RPI * q, p = r / (SPC * 4), sj = r % (SPC * 4);
      const half8_t *g = abase + p * plane + ((int64_t)cc * SPC * 4 + sj) * a.Mpad;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)g,
                                       (__attribute__((address_space(3))) void *)(buf + NTH * q + 64 * (tid >> 6)),
                                       16, 0, 0);
    }
  };

  const u32x4_t *bsrc[TN];
  const uint32_t *msrc[TN];
  int cref[TN];
#pragma unroll
  for (int j = 0; j < TN; j++) {
    const int t = min(bn * NT16 + w * TN + j, a.ntile - 1);
    bsrc[j] = a.codes + (int64_t)t * a.nchunk * 64 + lane;
    msrc[j] = (const uint32_t *)a.meta + sglq_mrow(t, n16, E2M1 ? a.nmeta / 4 : a.nmeta);
    cref[j] = 0;
    if constexpr (E2M1) cref[j] = a.colexp[t * 16 + n16];
  }
  struct BSet {
    u32x4_t code[TN];
    uint32_t meta[TN];
    bool live;
  };
  // chunks past the end reload the last chunk and compute with scale 0 (exact zero weights);
  // the flag is applied where the values are used, so no load is waited for early
  auto load_b = [&](int c, BSet &b) {
    b.live = c < c1;
    const int cc = min(c, c1 - 1);
    const int u = E2M1 ? cc : cc / a.cpg;
#pragma unroll
    for (int j = 0; j < TN; j++) {
      b.code[j] = ldg_nt(bsrc[j] + (int64_t)cc * 64);
      b.meta[j] = ldg(msrc[j] + sglq_mofs(u));
    }
  };

  float4_t acc[MBW][TN];
#pragma unroll
  for (int i = 0; i < MBW; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = (float4_t){0.f, 0.f, 0.f, 0.f};

  // one chunk: every A fragment of the chunk is read from LDS first (one LDS wait per chunk),
  // then step s's MFMAs run while step s + 1's weights are unpacked; sched_group_barrier
  // interleaves them (one MFMA, then up to two VALU), so the unpack issues in the MFMA shadow
  auto unpack = [&](const BSet &b, int s, const half2_t(&zA)[TN], const half2_t(&zB)[TN],
                    const half2_t(&s2)[TN], half8_t(&bv)[TN]) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
      float fsc = 1.f;
      if constexpr (E2M1)
        fsc = b.live ? e8m0_rel((b.meta[j] >> (8 * s)) & 255u, cref[j]) : 0.f;
      H8 u;
      u.v = unpack_b<KIND>(b.code[j], s, zA[j], zB[j], fsc);
      if constexpr (!E2M1) {
#pragma unroll
        for (int hh = 0; hh < 4; hh++) u.h[hh] = u.h[hh] * s2[j];
      }
      bv[j] = u.v;
    }
  };
  auto compute = [&](const half8_t *buf, const BSet &b) {
    half2_t zA[TN], zB[TN], s2[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      zA[j] = zB[j] = s2[j] = (half2_t){0, 0};
      if constexpr (!E2M1) {
        float sc;
        decode_meta<true>(b.meta[j], sc, zA[j], zB[j]);
        const _Float16 hs = b.live ? (_Float16)sc : (_Float16)0.f;
        s2[j] = (half2_t){hs, hs};
      }
    }
    const half8_t *sa = buf + kq * BMR + n16;
    // SCHED: every A fragment of the chunk up front; otherwise per step (fewer registers)
    constexpr int AS = SCHED ? SPC : 1;
    half8_t av[AS][NP][MBW];
    auto read_a = [&](int s) {
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < MBW; i++)
          av[SCHED ? s : 0][p][i] = sa[(p * SPC + s) * 4 * BMR + i * 16];
    };
    if constexpr (SCHED) {
#pragma unroll
      for (int s = 0; s < SPC; s++) read_a(s);
    }
    half8_t bv0[TN], bv1[TN];
    unpack(b, 0, zA, zB, s2, bv0);
    if constexpr (SCHED) __builtin_amdgcn_sched_barrier(0);  // the LDS reads stay first
#pragma unroll
    for (int s = 0; s < SPC; s++) {
      half8_t(&cur)[TN] = (s & 1) ? bv1 : bv0;
      half8_t(&nxt)[TN] = (s & 1) ? bv0 : bv1;
      if constexpr (!SCHED) read_a(s);
      if (s + 1 < SPC) unpack(b, s + 1, zA, zB, s2, nxt);
      const int sa_ = SCHED ? s : 0;
#pragma unroll
      for (int p = 0; p < NP; p++)
#pragma unroll
        for (int i = 0; i < MBW; i++)
#pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(av[sa_][p][i], cur[j], acc[i][j], 0, 0, 0);
      if constexpr (SCHED) {
#pragma unroll
        for (int x = 0; x < NP * MBW * TN; x++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // then up to two VALU
        }
      }
    }
  };

  // issue order per chunk k: [wait for own copies of k, barrier] copies of k + 3, codes of
  // k + 4 (after chunk k's codes are consumed).  At the top of chunk k the operations issued
  // after the copies of k are: codes k+1, copies k+1, codes k+2, copies k+2, codes k+3.
  constexpr int AFTER = 2 * AIPT + 3 * 2 * TN;
  static_assert(AFTER <= 63, "k_gemm_dma: vmcnt range");
  BSet b0, b1, b2, b3;
  load_b(c0, b0);
  copy_a(c0, sA0);
  load_b(c0 + 1, b1);
  copy_a(c0 + 1, sA1);
  load_b(c0 + 2, b2);
  copy_a(c0 + 2, sA2);
  load_b(c0 + 3, b3);
  auto chunk = [&](int k, half8_t *cur, half8_t *nxt3, BSet &b) {
    SGLQ_WAIT_VMCNT(AFTER);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    copy_a(k + 3, nxt3);
    __builtin_amdgcn_sched_barrier(0);
    compute(cur, b);
    __builtin_amdgcn_sched_barrier(0);
    load_b(k + 4, b);
  };
  for (int k = c0; k < c1; k += 4) {
    chunk(k, sA0, sA3, b0);
    chunk(k + 1, sA1, sA0, b1);
    chunk(k + 2, sA2, sA1, b2);
    chunk(k + 3, sA3, sA2, b3);
  }
  SGLQ_WAIT_VMCNT(0);  // no copy may land in LDS after the workgroup ends
  (void)mend;
  __syncthreads();
  constexpr int RP = 16 * 16 * NT16 * 4 <= AITEMS * 16 ? 16
                     : 8 * 16 * NT16 * 4 <= AITEMS * 16 ? 8 : 4;
  static_assert(RP * 16 * NT16 * 4 <= AITEMS * 16, "k_gemm_dma: epilogue staging");
  wide_epilogue<MBW, TN, E2M1, RP, WN>(a, acc, (float *)sA0, m0, mend, bn, w, n16, kq,
                                       a.colexp);
}

// Sum of the K-split partials of k_gemm_lds in slice order (deterministic), then the row and
// column exponents and the bias: C[m][n] = 2^(rowexp[m] + ce[n]) * sum_z part[z][m][n] + bias[n]
__global__ __launch_bounds__(256) void k_splitk_reduce(const float *__restrict__ part, int nz,
                                                       int M, int N,
                                                       const int *__restrict__ rowexp,
                                                       const uint8_t *__restrict__ colexp,
                                                       const float *__restrict__ bias,
                                                       float *__restrict__ C, int64_t ldc) {
  const int n = (int)(blockIdx.x * 256 + threadIdx.x), m = (int)blockIdx.y;
  if (n >= N) return;
  const int64_t plane = (int64_t)M * N, o = (int64_t)m * N + n;
  // slices added in order, 8 loads in flight at a time (one at a time, each waiting for its
  // predecessor, the pass was latency-bound)
  float s = 0.f;
  for (int z0 = 0; z0 < nz; z0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = z0 + u < nz ? part[(z0 + u) * plane + o] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (z0 + u < nz) s = z0 + u == 0 ? v[u] : s + v[u];
  }
  const int ce = colexp ? (int)colexp[n] - 127 : 0;
  C[(int64_t)m * ldc + n] = ldexpf(s, rowexp[m] + ce) + (bias ? bias[n] : 0.f);
}

template <int KIND, int NP, int BN, int SSX, int WMW, int NBUF, int MB = 4, int RS = 1>
void launch_lds1(const GemmArgs &a, dim3 grid, hipStream_t st) {
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr int SS = SSX < SPC ? SSX : SPC;
  // LDS: NBUF x (A: NP pieces x SS steps x 4 x rows, B: BN/16 tiles x SS steps x 64) x 16 B
  constexpr size_t lds =
      (size_t)NBUF * (NP * SS * 4 * 16 * MB * WMW + (BN / 16) * SS * 64) * 16;
  if constexpr (lds > 160 * 1024) {
    // too big with two A pieces: the same tile with 2-step stages and two buffers (fits)
    static_assert(SSX != 2 || NBUF != 2, "k_gemm_lds tile exceeds the LDS");
    launch_lds1<KIND, NP, BN, 2, WMW, 2, MB, RS>(a, grid, st);
  } else {
    auto f = k_gemm_lds<KIND, NP, BN, SSX, WMW, NBUF, MB, RS>;
    static unsigned long long raised = 0;
    sglq_raise_lds((const void *)f, 160 * 1024, &raised);
    f<<<grid, 128 * WMW, lds, st>>>(a);
  }
}

// tile configurations of k_gemm_lds (rows x columns per workgroup).  All stages are two MFMA
// steps; each stage's loads are issued two iterations ahead through two register sets (a
// single set measured 3-5% slower at every M, larger per-wave tiles and 3-buffer rings slower
// still: the kernel waits on memory and LDS latency with 2 waves per SIMD, not on bandwidth).
enum { LDS_64x128 = 0, LDS_128x64 = 1, LDS_256x128 = 2 };
int lds_rows(int cfg) { return cfg == LDS_256x128 ? 256 : cfg == LDS_128x64 ? 128 : 64; }
int lds_cols(int cfg) { return cfg == LDS_128x64 ? 64 : 128; }

// k_gemm_breg for the grouped (MoE) launches, codes 2 chunks ahead (3-4 chunks measured 2-8%
// slower).  On k_gemm_lds's 64 x 128 tile it measured 105.7 us (gate/up with the SwiGLU
// epilogue) and 69.9 us (down, f32 operands) at the DeepSeek shapes, against 123.2 and 114.3
// us for k_gemm_lds; the wave layouts below improve on that.  (Dense calls of at most 64 rows
// measured 21.7 us on k_gemm_lds against 22.6 on this kernel at M = 64, [11008, 4096]; they
// now take k_gemm_dma.)
template <int KIND, int NP, int WN, int TN, int MINB = 2>
void launch_breg1(const GemmArgs &a, dim3 grid, hipStream_t st) {
  constexpr int D = 2;
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr size_t lds = (size_t)2 * NP * SPC * 4 * 64 * 16;
  static unsigned long long raised = 0;
  auto f = k_gemm_breg<KIND, NP, WN, TN, D, MINB>;
  sglq_raise_lds((const void *)f, 160 * 1024, &raised);
  f<<<grid, 64 * WN, lds, st>>>(a);
}
// Wave layout of the grouped launches, from a sweep at the DeepSeek shapes (64 experts, 48
// rows each on average): one A piece (bf16 rows, gate/up with the SwiGLU epilogue) 4 waves of
// 4 tiles (256 columns: 96.6 us; 4 x 2 103.7, 8 x 2 101.8, 8 x 4 103.8); two pieces (f32 rows,
// down) 8 waves of 2 tiles (55.8 us; 4 x 2 69.9, 4 x 4 64.0, 8 x 4 59.0).  Wider workgroups
// re-stage each expert block's A operands for fewer column blocks.
static void breg_shape(int np, int &wn, int &tn) {
  wn = np == 1 ? 4 : 8;
  tn = np == 1 ? 4 : 2;
}
template <int KIND, int NP>
void launch_breg(const GemmArgs &a, dim3 grid, hipStream_t st) {
  // one piece of int codes: three waves per SIMD (three workgroups per CU: 168 registers, the
  // grid's row blocks in about one round).  MXFP4 codes keep two (three would spill).
  if constexpr (NP == 1)
    launch_breg1<KIND, NP, 4, 4, KIND != SGLQ_KIND_E2M1 ? 3 : 2>(a, grid, st);
  else
    launch_breg1<KIND, NP, 8, 2>(a, grid, st);
}

template <int KIND, int NP>
void launch_lds(const GemmArgs &a, int cfg, dim3 grid, hipStream_t st) {
  switch (cfg) {
    // 64 x 128 with f32 operands (two A pieces) does not fit two register sets in 256 VGPRs
    case LDS_64x128: launch_lds1<KIND, NP, 128, 2, 1, 2, 4, NP == 1 ? 2 : 1>(a, grid, st); break;
    case LDS_256x128: launch_lds1<KIND, NP, 128, 2, 4, 2, 4, 2>(a, grid, st); break;
    default: launch_lds1<KIND, NP, 64, 2, 2, 2, 4, 2>(a, grid, st); break;
  }
}

template <int KIND, int NP, int TN, int MB, int WN>
void launch_dma1(const GemmArgs &a, dim3 grid, hipStream_t st) {
  // 4 waves (one per SIMD): every A fragment of a chunk read up front, scheduled interleave;
  // 8 waves (two per SIMD): A fragments read per step (register budget of two waves)
  k_gemm_dma<KIND, NP, TN, MB, WN == 4, WN><<<grid, 64 * WN, 0, st>>>(a);
}
// shapes of k_gemm_dma: 128 rows x 192 columns (4 waves) or x 384 columns (8 waves); two A
// pieces (f32 rows) use 64-row tiles, the largest whose four A buffers fit the LDS
template <int KIND, int NP>
void launch_dma(const GemmArgs &a, int mb, int wn, bool occ2, dim3 grid, hipStream_t st) {
  if constexpr (NP == 1) {
    if (mb == 4 && occ2)  // 64-row tiles beyond 64 rows, two workgroups per CU
      k_gemm_dma<KIND, NP, 3, 4, false, 4, 2><<<grid, 256, 0, st>>>(a);
    else if (mb == 4)  // up to 64 rows
      launch_dma1<KIND, NP, 3, 4, 4>(a, grid, st);
    else if (wn == 8)
      launch_dma1<KIND, NP, 3, 8, 8>(a, grid, st);
    else
      launch_dma1<KIND, NP, 3, 8, 4>(a, grid, st);
  } else {
    if (wn == 8)
      launch_dma1<KIND, NP, 3, 4, 8>(a, grid, st);
    else
      launch_dma1<KIND, NP, 3, 4, 4>(a, grid, st);
  }
}

template <int KIND, bool SPLIT, bool SCF16, bool STEPM, bool PS, int MB>
void launch_bn(const GemmArgs &a, int bn, unsigned grid, size_t lds, hipStream_t st) {
  // LDS beyond 64 KiB must be enabled per kernel once (160 KiB on gfx950)
  static unsigned long long raised128 = 0, raised64 = 0;
  if (bn == 128) {
    auto f = k_gemm<KIND, SPLIT, SCF16, STEPM, 128, PS, MB>;
    sglq_raise_lds((const void *)f, 160 * 1024, &raised128);
    f<<<grid, 256, lds, st>>>(a);
  } else {
    auto f = k_gemm<KIND, SPLIT, SCF16, STEPM, 64, PS, MB>;
    sglq_raise_lds((const void *)f, 160 * 1024, &raised64);
    f<<<grid, 256, lds, st>>>(a);
  }
}

// variant: 0 exact (per-chunk partials), 1 prescaled MB=4, 2 prescaled MB=8
template <int KIND, bool SPLIT>
void launch_meta(const GemmArgs &a, int scf16, int stepm, int variant, int bn, unsigned grid,
                 size_t lds, hipStream_t st) {
  if constexpr (KIND == SGLQ_KIND_E2M1) {
    if (variant == 2)
      launch_bn<KIND, SPLIT, true, false, true, 8>(a, bn, grid, lds, st);
    else
      launch_bn<KIND, SPLIT, true, false, true, 4>(a, bn, grid, lds, st);
  } else {
    if (variant == 2) {
      launch_bn<KIND, SPLIT, true, false, true, 8>(a, bn, grid, lds, st);
    } else if (variant == 1) {
      launch_bn<KIND, SPLIT, true, false, true, 4>(a, bn, grid, lds, st);
    } else if (scf16) {
      if (stepm)
        launch_bn<KIND, SPLIT, true, true, false, 4>(a, bn, grid, lds, st);
      else
        launch_bn<KIND, SPLIT, true, false, false, 4>(a, bn, grid, lds, st);
    } else {
      if (stepm)
        launch_bn<KIND, SPLIT, false, true, false, 4>(a, bn, grid, lds, st);
      else
        launch_bn<KIND, SPLIT, false, false, false, 4>(a, bn, grid, lds, st);
    }
  }
}

template <int KIND>
void launch_split(const GemmArgs &a, bool split, int scf16, int stepm, int variant, int bn,
                  unsigned grid, size_t lds, hipStream_t st) {
  if (split)
    launch_meta<KIND, true>(a, scf16, stepm, variant, bn, grid, lds, st);
  else
    launch_meta<KIND, false>(a, scf16, stepm, variant, bn, grid, lds, st);
}

}  // namespace

int sglq_prep_a(const sglq_dev *d, int mode, const void *A, int dt, int64_t lda, int64_t M,
                int64_t Mpad, const int32_t *rowmap, int kcols, int split, void *aop,
                int *rowexp, hipStream_t st, const int *rowmax) {
  const int32_t *kmap = d->kident ? nullptr : d->kmap;
  const int perm4 = d->kind == SGLQ_KIND_U4;
  const int64_t esz = dt == SGLQ_DT_F32 ? 4 : 2;
  const int vec = kmap == nullptr && (uintptr_t)A % 16 == 0 && (lda * esz) % 16 == 0;
  const dim3 pgrid((unsigned)(Mpad / 16), (unsigned)((d->nsteps * 4 + 63) / 64));
  if (!rowmax && mode != 2 && (vec || kmap) && Mpad % 16 == 0) {
    // one pass: one row per workgroup (measured fastest at M = 64..2048 against 2..16 rows),
    // at most 16 items (128 elements) per thread
    const int64_t nitems = d->nsteps * 4;
    const int R = 1;
    const int64_t need = (R * nitems + 255) / 256;
    if (need <= 16) {
      const unsigned grid = (unsigned)(Mpad / R);
      const int xcd = Mpad % 64 == 0 && R <= 8;
#define SGLQ_PREP_ROWS(MODE, IT)                                                               \
  k_prep_rows<MODE, IT><<<grid, 256, 0, st>>>(A, dt, lda, (int)M, (int)Mpad, (int)d->K,        \
                                              (int)nitems, kmap, rowmap, R, xcd, perm4, split, \
                                              (half8_t *)aop, rowexp)
#define SGLQ_PREP_ROWS_IT(MODE)         \
  if (need <= 2)                         \
    SGLQ_PREP_ROWS(MODE, 2);             \
  else if (need <= 4)                    \
    SGLQ_PREP_ROWS(MODE, 4);             \
  else if (need <= 8)                    \
    SGLQ_PREP_ROWS(MODE, 8);             \
  else                                   \
    SGLQ_PREP_ROWS(MODE, 16)
      if (mode == 0) {
        SGLQ_PREP_ROWS_IT(0);
      } else {
        SGLQ_PREP_ROWS_IT(1);
      }
#undef SGLQ_PREP_ROWS_IT
#undef SGLQ_PREP_ROWS
      SGLQ_HIP(hipGetLastError());
      return 0;
    }
  }
#define SGLQ_PREP(MODE)                                                                       \
  if (!rowmax)                                                                                  \
    k_rowexp<MODE><<<(unsigned)((Mpad + 3) / 4), 256, 0, st>>>(                                 \
        A, dt, lda, (int)M, (int)Mpad, (int)d->K, (int)d->nsteps, kmap, rowmap, kcols, vec,     \
        rowexp);                                                                                \
  k_prep_a<MODE><<<pgrid, 256, 0, st>>>(A, dt, lda, (int)M, (int)Mpad, (int)d->K, (int)d->nsteps, \
                                        kmap, rowmap, kcols, perm4, split, vec, (half8_t *)aop,   \
                                        rowmax, rowexp)
  if (mode == 0) {
    SGLQ_PREP(0);
  } else if (mode == 1) {
    SGLQ_PREP(1);
  } else {
    SGLQ_PREP(2);
  }
#undef SGLQ_PREP
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

size_t sglq_aop_bytes(const sglq_dev *d, int64_t Mpad, int split) {
  return (size_t)(split ? 2 : 1) * d->nsteps * 4 * Mpad * 16;
}

// Rows per workgroup of the dense GEMM.  (The 256-row prescaled variant, MB = 8, needs one
// wave per SIMD and measured slower than two 128-row workgroups per CU; it stays instantiated
// for tuning but is not selected.)
// weights the LDS-dequant kernel takes: MXFP4, and groups whose f16 scales prescale the codes
static bool lds_direct(const sglq_dev *d) {
  const bool direct = d->kind == SGLQ_KIND_E2M1 ||
                      (d->prescale && d->meta_mode == SGLQ_META_GROUP);
  return direct && (d->kind == SGLQ_KIND_E2M1 || d->scf16);
}

bool sglq_gemm_lds_direct(const sglq_dev *d) { return lds_direct(d); }

// k_gemm_lds tiling of a dense call: 64 x 128 tiles for M <= 64, 128 x 64 below M = 1024, then
// 256 x 128; and a split over K (deterministic, reduced in slice order) when the tiles alone
// leave the 256 CUs under one workgroup each.  Every slice keeps at least 8 stages.
struct LdsPlan {
  int cfg, nz;
};
static LdsPlan lds_plan(const sglq_dev *d, int64_t M) {
  LdsPlan p;
  p.cfg = M <= 64 ? LDS_64x128 : M >= 1024 ? LDS_256x128 : LDS_128x64;
  const int64_t tiles = (M + lds_rows(p.cfg) - 1) / lds_rows(p.cfg) *
                        ((d->N + lds_cols(p.cfg) - 1) / lds_cols(p.cfg));
  const int64_t nstage = d->nsteps / 2;
  p.nz = 1;
  if (tiles < 256) {
    p.nz = (int)std::min<int64_t>((512 + tiles - 1) / tiles, std::min<int64_t>(16, nstage / 8));
    if (p.nz < 1) p.nz = 1;
  }
  return p;
}

// k_gemm_dma plan of a dense call.  Taken where it measured faster than k_gemm_lds: K of at
// most 4096, and either at most 64 rows (below) or enough tiles to give most CUs one
// workgroup without a split over K (no partial sums).  8 waves (384 columns) when that
// alone gives 200 tiles, else 4 waves (192 columns).  Measured (graph replay, GPTQ int4 g128 [11008, 4096], bf16 rows, incl. the A
// prep): M = 512 95.5 -> 86.5 us, 1024 175 -> 139 us, 2048 289 -> 274 us.  At K = 11008 and
// where a split over K is needed it measured slower, so those stay on k_gemm_lds.
// SGLQ_GEMM_DMA=0 keeps every call on k_gemm_lds (A/B measurement).
struct WidePlan {
  int use, mb, wn, nz;  // wn waves along N, nz slices of K (partials added by k_splitk_reduce)
  int occ2;             // 64-row tiles of more than 64 rows: two waves per SIMD (see below)
};
static WidePlan wide_plan(const sglq_dev *d, int64_t M, int np) {
  WidePlan p = {0, np == 1 ? 8 : 4, 4, 1, 0};
  static int env = -1, small = -1;
  if (env < 0) {
    const char *e = getenv("SGLQ_GEMM_DMA");
    env = e ? atoi(e) : 1;
    const char *s = getenv("SGLQ_GEMM_DMA_SMALL");  // rows 17-64 (A/B measurement)
    small = s ? atoi(s) : 1;
  }
  if (!env || !lds_direct(d) || d->K > 4096) return p;
  if (M <= 64) {
    // one 64-row block: 192-column tiles with K cut into nz slices for about 232 workgroups.
    // [11008, 4096] bf16 against k_gemm_lds: M = 25 36.9 -> 32.2 us, 48 39.1 -> 35.4, 64
    // 40.2 -> 37.3 (A prep and slice sums included); at K = 11008 it measured slower (M = 64
    // 43.5 -> 54.6), as does every K > 4096 below.
    if (!small) return p;
    p.mb = 4;
    const int64_t tiles = (d->N + 191) / 192;
    p.nz = (int)std::max<int64_t>(1, std::min<int64_t>(d->nchunk / 4, (256 + tiles / 2) / tiles));
    p.use = 1;
    return p;
  }
  const int64_t bmr = 16 * p.mb, nbm = (M + bmr - 1) / bmr;
  // MXFP4 codes spill in the 8-wave tile (256 registers): it pays only from about twice as
  // many tiles ([8192, 4096] bf16: M = 2048 284.3 -> 254.8 us on 4 waves, M = 4096 452.6 us
  // on 8 against 477.0 on 4)
  const int64_t min8 = d->kind == SGLQ_KIND_E2M1 ? 400 : 200;
  if (nbm * ((d->N + 383) / 384) >= min8) {
    p.use = 1;
    p.wn = 8;
  } else if (nbm * ((d->N + 191) / 192) >= 200) {
    p.use = 1;
  } else if (np == 1 && ((M + 63) / 64) * ((d->N + 191) / 192) >= 170) {
    // too few 128-row tiles but enough 64-row ones: 64 x 192 tiles with the A fragments read
    // per step (186 registers), so two workgroups share a CU and one wave's unpack runs
    // beside the other's MFMAs.  [11008, 4096] bf16 against k_gemm_lds: M = 160 69.1 -> 58.0
    // us, 256 69.3 -> 60.4, 320 87.3 -> 80.6, 384 88.4 -> 83.0.  With fewer tiles it measured
    // slower (M = 128: 47.7 -> 56.4; [4096, 4096] M = 256: 39.8 -> 55.4), as it did in place
    // of the 128-row tiles (M = 512: 83.8 -> 89.5).
    p.use = 1;
    p.mb = 4;
    p.occ2 = 1;
  }
  return p;
}

int64_t sglq_gemm_rows(const sglq_dev *d, int split) {
  (void)d;
  (void)split;
  return 128;
}

int sglq_gemm_run(const sglq_dev *d, const sglq_group *grp, const void *aop,
                  const int *rowexp, int64_t M, int64_t Mpad, int64_t nblk, int split,
                  const float *bias, float *C, int64_t ldc, float *part, hipStream_t st) {
  const bool direct = d->kind == SGLQ_KIND_E2M1 ||
                      (d->prescale && d->meta_mode == SGLQ_META_GROUP);
  // grouped row blocks hold at most 128 rows of one expert: 128-row tiles there
  const int variant = !direct ? 0 : 1;
  const int bmr = variant == 2 ? 256 : 128;
  // 128-column tiles unless that leaves the chip under-filled
  int bn = 128;
  if (nblk * ((d->N + 127) / 128) < 512 || d->meta_mode == SGLQ_META_STEP) bn = 64;
  const int nbn = (int)((d->N + bn - 1) / bn);
  const size_t lds = (size_t)2 * (split ? 2 : 1) * d->spc * 4 * bmr * 16;
  GemmArgs a;
  memset(&a, 0, sizeof(a));
  a.codes = d->codes;
  a.meta = d->meta;
  a.colexp = d->colexp;
  if (grp) {
    a.codes_e = (const u32x4_t *const *)grp->codes;
    a.meta_e = grp->meta;
    a.colexp_e = grp->colexp;
    a.segs = (const int4 *)grp->segs;
    a.nseg = grp->nseg;
    a.swiglu = grp->swiglu;
    a.rowmax = grp->rowmax;
  }
  a.aop = (const half8_t *)aop;
  a.rowexp = rowexp;
  a.bias = bias;
  a.C = C;
  a.ldc = ldc;
  a.M = (int)M;
  a.Mpad = (int)Mpad;
  a.N = (int)d->N;
  a.ntile = (int)d->ntile;
  a.nchunk = (int)d->nchunk;
  a.nsteps = (int)d->nsteps;
  a.nmeta = (int)d->nmeta;
  a.cpg = d->cpg > 0 ? (int)d->cpg : 1;
  a.nbn = nbn;
  a.nbm = (int)nblk;
  unsigned grid = (unsigned)(nblk * nbn);
  if (!grp && ((nblk >= 8 && nblk % 8 == 0) || (nblk < 8 && 8 % nblk == 0))) {
    a.xmap = 1;
    const int64_t per_xcd = nblk >= 8 ? (nblk / 8) * nbn : (nbn + 8 / nblk - 1) / (8 / nblk);
    grid = (unsigned)(8 * per_xcd);
  }

  const int stepm = d->meta_mode == SGLQ_META_STEP;
  if (grp && grp->swiglu && (!lds_direct(d) || grp->swiglu % 16 != 0)) {
    sglq_log_error("grouped GEMM: the fused SwiGLU needs the LDS kernel and mi %% 16 == 0");
    return -1;
  }
  if (!grp) {
    const WidePlan wp = wide_plan(d, M, split ? 2 : 1);
    if (wp.use) {
      const int64_t bmr = 16 * wp.mb, cols = 48 * wp.wn;
      if (wp.nz > 1 && !part) {
        sglq_log_error("prefill GEMM: no workspace for the split over K");
        return -1;
      }
      a.nbm = (int)((M + bmr - 1) / bmr);
      a.nbn = (int)((d->N + cols - 1) / cols);
      a.part = wp.nz > 1 ? part : nullptr;
      a.xmap = 0;
      const dim3 grid2((unsigned)(8 * ((a.nbm * a.nbn + 7) / 8)), (unsigned)wp.nz);
      switch (d->kind) {
        case SGLQ_KIND_U4:
          if (split) launch_dma<SGLQ_KIND_U4, 2>(a, wp.mb, wp.wn, wp.occ2, grid2, st);
          else launch_dma<SGLQ_KIND_U4, 1>(a, wp.mb, wp.wn, wp.occ2, grid2, st);
          break;
        case SGLQ_KIND_U8:
          if (split) launch_dma<SGLQ_KIND_U8, 2>(a, wp.mb, wp.wn, wp.occ2, grid2, st);
          else launch_dma<SGLQ_KIND_U8, 1>(a, wp.mb, wp.wn, wp.occ2, grid2, st);
          break;
        default:
          if (split) launch_dma<SGLQ_KIND_E2M1, 2>(a, wp.mb, wp.wn, wp.occ2, grid2, st);
          else launch_dma<SGLQ_KIND_E2M1, 1>(a, wp.mb, wp.wn, wp.occ2, grid2, st);
          break;
      }
      SGLQ_HIP(hipGetLastError());
      if (wp.nz > 1) {
        k_splitk_reduce<<<dim3((unsigned)((d->N + 255) / 256), (unsigned)M), 256, 0, st>>>(
            part, wp.nz, (int)M, (int)d->N, rowexp,
            d->kind == SGLQ_KIND_E2M1 ? d->colexp : nullptr, bias, C, ldc);
        SGLQ_HIP(hipGetLastError());
      }
      return 0;
    }
  }
  // direct formats with f16-exact scales: the LDS-dequant kernel
  if (lds_direct(d)) {
    const LdsPlan pl = grp ? LdsPlan{LDS_64x128, 1} : lds_plan(d, M);
    if (pl.nz > 1 && !part) {
      sglq_log_error("prefill GEMM: no workspace for the split over K");
      return -1;
    }
    int gwn = 0, gtn = 0;
    if (grp) breg_shape(split ? 2 : 1, gwn, gtn);
    const int cbm = grp ? 64 : lds_rows(pl.cfg), cbn = grp ? 16 * gwn * gtn : lds_cols(pl.cfg);
    // grouped: row blocks of one expert each (at most 64 rows); dense: the rows of M
    const int64_t nbm2 = grp ? nblk : (M + cbm - 1) / cbm;
    a.nbn = (int)((d->N + cbn - 1) / cbn);
    if (a.swiglu) a.nbn = (int)((a.swiglu / 16 + cbn / 32 - 1) / (cbn / 32));  // gate tiles / 2
    a.nbm = (int)nbm2;
    a.xmap = 0;
    a.part = pl.nz > 1 ? part : nullptr;
    unsigned gx = (unsigned)(nbm2 * a.nbn);
    if (!grp && ((nbm2 >= 8 && nbm2 % 8 == 0) || (nbm2 < 8 && 8 % nbm2 == 0))) {
      a.xmap = 1;
      const int64_t per = nbm2 >= 8 ? (nbm2 / 8) * a.nbn : (a.nbn + 8 / nbm2 - 1) / (8 / nbm2);
      gx = (unsigned)(8 * per);
    }
    const dim3 grid2(gx, (unsigned)pl.nz);
    if (grp) {  // expert row blocks of at most 64 rows: codes unpacked in registers
      static int epi = -1;
      if (epi < 0) {
        const char *e = getenv("SGLQ_BREG_EPI");  // 0: per-lane stores (A/B measurement)
        epi = e ? atoi(e) : 1;
      }
      a.epi = epi;
      switch (d->kind) {
        case SGLQ_KIND_U4:
          if (split) launch_breg<SGLQ_KIND_U4, 2>(a, grid2, st);
          else launch_breg<SGLQ_KIND_U4, 1>(a, grid2, st);
          break;
        case SGLQ_KIND_U8:
          if (split) launch_breg<SGLQ_KIND_U8, 2>(a, grid2, st);
          else launch_breg<SGLQ_KIND_U8, 1>(a, grid2, st);
          break;
        default:
          if (split) launch_breg<SGLQ_KIND_E2M1, 2>(a, grid2, st);
          else launch_breg<SGLQ_KIND_E2M1, 1>(a, grid2, st);
          break;
      }
      SGLQ_HIP(hipGetLastError());
      return 0;
    }
    switch (d->kind) {
      case SGLQ_KIND_U4:
        if (split) launch_lds<SGLQ_KIND_U4, 2>(a, pl.cfg, grid2, st);
        else launch_lds<SGLQ_KIND_U4, 1>(a, pl.cfg, grid2, st);
        break;
      case SGLQ_KIND_U8:
        if (split) launch_lds<SGLQ_KIND_U8, 2>(a, pl.cfg, grid2, st);
        else launch_lds<SGLQ_KIND_U8, 1>(a, pl.cfg, grid2, st);
        break;
      default:
        if (split) launch_lds<SGLQ_KIND_E2M1, 2>(a, pl.cfg, grid2, st);
        else launch_lds<SGLQ_KIND_E2M1, 1>(a, pl.cfg, grid2, st);
        break;
    }
    SGLQ_HIP(hipGetLastError());
    if (pl.nz > 1) {
      k_splitk_reduce<<<dim3((unsigned)((d->N + 255) / 256), (unsigned)M), 256, 0, st>>>(
          part, pl.nz, (int)M, (int)d->N, rowexp,
          d->kind == SGLQ_KIND_E2M1 ? d->colexp : nullptr, bias, C, ldc);
      SGLQ_HIP(hipGetLastError());
    }
    return 0;
  }
  switch (d->kind) {
    case SGLQ_KIND_U4:
      launch_split<SGLQ_KIND_U4>(a, split, d->scf16, stepm, variant, bn, grid, lds, st);
      break;
    case SGLQ_KIND_U8:
      launch_split<SGLQ_KIND_U8>(a, split, d->scf16, stepm, variant, bn, grid, lds, st);
      break;
    default:
      launch_split<SGLQ_KIND_E2M1>(a, split, 1, 0, variant, bn, grid, lds, st);
      break;
  }
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

// Workspace of a prefill GEMM of M rows: A operands, row exponents, split-K partials.
static void gemm_ws_layout(const sglq_dev *d, int dt, int64_t M, int64_t *Mpad_out,
                           size_t *aop_bytes, size_t *o_part, size_t *part_bytes) {
  const int split = dt == SGLQ_DT_F32;
  // rows of A operands: whole row tiles of the LDS kernel's tiling (it reads no further), else
  // whole 128- and 256-row blocks
  const WidePlan wp = wide_plan(d, M, split ? 2 : 1);
  const int64_t rt = wp.use ? std::max<int64_t>(16 * wp.mb, lds_rows(lds_plan(d, M).cfg))
                    : lds_direct(d) ? lds_rows(lds_plan(d, M).cfg) : 256;
  const int64_t Mpad = (M + rt - 1) / rt * rt;
  *Mpad_out = Mpad;
  *aop_bytes = sglq_aop_bytes(d, Mpad, split);
  *o_part = (*aop_bytes + (size_t)Mpad * sizeof(int) + 255) / 256 * 256;
  const int nz = wp.use ? wp.nz : lds_direct(d) ? lds_plan(d, M).nz : 0;
  *part_bytes = (size_t)nz * M * d->N * sizeof(float);
}

size_t sglq_gemm_ws_bytes(const sglq_dev *d, int dt, int64_t M) {
  int64_t Mpad;
  size_t aop_bytes, o_part, part_bytes;
  gemm_ws_layout(d, dt, M, &Mpad, &aop_bytes, &o_part, &part_bytes);
  return o_part + part_bytes + 256;
}

int sglq_gemm_ws(const sglq_dev *d, const void *A, int dt, int64_t lda, int64_t M,
                 const float *bias, float *C, int64_t ldc, void *ws, hipStream_t st) {
  const int split = dt == SGLQ_DT_F32;
  const int64_t bmr = sglq_gemm_rows(d, split);
  int64_t Mpad;
  size_t aop_bytes, o_part, part_bytes;
  gemm_ws_layout(d, dt, M, &Mpad, &aop_bytes, &o_part, &part_bytes);
  void *aop = ws;
  int *rowexp = (int *)((char *)ws + aop_bytes);
  float *part = part_bytes > (size_t)M * d->N * sizeof(float) ? (float *)((char *)ws + o_part)
                                                              : nullptr;
  if (sglq_prep_a(d, 0, A, dt, lda, M, Mpad, nullptr, 0, split, aop, rowexp, st) != 0)
    return -1;
  return sglq_gemm_run(d, nullptr, aop, rowexp, M, Mpad, (Mpad + bmr - 1) / bmr, split, bias, C,
                       ldc, part, st);
}

int sglq_gemm(sglq_dev *d, const void *A, int dt, int64_t lda, int64_t M, const float *bias,
              float *C, int64_t ldc, hipStream_t st) {
  if (sglq_ws_reserve(d, sglq_gemm_ws_bytes(d, dt, M)) != 0) return -1;
  return sglq_gemm_ws(d, A, dt, lda, M, bias, C, ldc, d->ws, st);
}
