// gemv_row.hip — one-row decode GEMV (M = 1) with a lean issue budget.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gemv_ops.hpp"

using namespace sglq;

namespace {

// ---------------------------------------------------------------------------------------
// One-row decode GEMV (k_gemv_row).  Same operands and arithmetic as k_gemv_wave for one
// identity-order, 16-byte aligned row (exact q - z in f16, scale in fp32 per chunk, f16 hi + lo
// activations under a per-wave power of two), laid out so that few instructions besides the
// multiply itself are issued:
//   * a wave takes one K slice of CPW chunks on TPW tiles: the slice of activations is staged
//     once (per wave, in its own LDS rows) and every A operand read from LDS feeds TPW MFMAs;
//   * the workgroup geometry is fixed per launch (NW waves; ks = 1 << ksl slices per tile
//     group, NW / ks tile groups per workgroup), so tile, slice and chunk indices are shifts
//     of the wave index, kept in scalar registers;
//   * code, meta and activation addresses are one scalar base per wave plus one per-lane
//     offset; the meta entries of four consecutive chunks of a column are one 16-byte load
//     (quad meta layout);
//   * the MXFP4 block scale relative to the column's largest is folded into the conversion
//     (v_cvt_scalef32_pk_f16_fp4), so all steps share one accumulator and the column scale
//     2^(colexp - 127) is applied once.
// ---------------------------------------------------------------------------------------
struct RowArgs {
  const u32x4_t *codes;
  const void *meta;
  const uint8_t *colexp;
  const void *A;
  const float *bias;
  float *C;
  int N, K, ntile, nchunk, nmeta, cpg, ksl, adt;
  // grouped MoE decode launches (GRP 1 gate/up, GRP 2 down) of nid / slots tokens read
  // straight from the routing: blockIdx.y = pair j = (token j / slots, slot j % slots), expert
  // ids[j] (pairs with ids[j] outside [0, nexp) are empty); C row j is written (ldc).  GRP 1
  // reads token row j / slots of A (lda); GRP 2 reads silu(A[j][k]) * A[j][kcols + k] of the
  // f32 gate/up rows (lda), and the last pair to finish a tile writes, for every token t,
  // cout[t][n] (ldo) = sum over its slots s of cw[t slots + s] * C[t slots + s][n], in order.
  const u32x4_t *const *codes_e;
  const void *const *meta_e;
  const int32_t *ids;
  const float *cw;
  float *cout;
  int *cnt;
  int64_t lda, ldc, ldo;
  int nid, nexp, kcols, slots;
};

// 32 zero bytes: the activation item of a lane whose item lies past K (or past the wave's
// chunks) is read from here, so no per-element masking is needed
__device__ const u32x4_t g_zero_item[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};

typedef __attribute__((address_space(1))) const u32x4_t GU4;

template <int KIND, int CPW, int TPW, int DT, bool SCF16, bool MV, int NW, int GRP = 0>
__global__ __launch_bounds__(NW * 64) void k_gemv_row(RowArgs a) {
  static_assert(GRP < 2 || DT == SGLQ_DT_F32, "SwiGLU rows are f32");
  static_assert(GRP == 0 || (TPW == 1 && KIND != SGLQ_KIND_E2M1), "grouped: one tile per wave");
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr int NP = DT == SGLQ_DT_BF16 ? 1 : 2;     // f16 operand rows: hi (+ lo)
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;  // MFMA steps per chunk
  constexpr int IPW = CPW * SPC * 4;                 // 8-element items of a wave's slice
  constexpr int NQ = (IPW + 63) / 64;                // items per lane
  constexpr int RS = IPW + 4;                        // LDS row stride (rows 64 B apart)
  using MT = typename std::conditional<E2M1, uint32_t, meta_t<SCF16>>::type;
  extern __shared__ half8_t s_op[];                  // [NW waves][NP][RS]
  __shared__ float s_sum[NW][TPW][16];

  const int lane = (int)threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int ks = 1 << a.ksl;
  // GRP 3: one tile per workgroup, wave w = (routing slot w >> ksl, K slice); otherwise
  // wave w >> ksl takes tile group blockIdx.x * (NW >> ksl) + (w >> ksl)
  const int tg = GRP == 3 ? (int)blockIdx.x : (int)blockIdx.x * (NW >> a.ksl) + (w >> a.ksl);
  const int t0 = tg * TPW;                                        // its first tile
  const int sl = w & (ks - 1);
  const int c0 = sl * CPW;
  // GRP 3: this wave's slot and whether it is routed (an empty slot's waves stream the first
  // routed expert's chunk 0 and contribute zero)
  int slot = 0, e3 = -1, e3first = -1;
  if constexpr (GRP == 3) {
    slot = w >> a.ksl;
    for (int j = 0; j < a.nid; j++) {
      const bool v = a.ids[j] >= 0 && a.ids[j] < a.nexp;
      if (v && e3first < 0) e3first = a.ids[j];
      if (j == slot && v) e3 = a.ids[j];
    }
  }
  // chunks of this wave (0 for a wave past the last tile or chunk: it streams chunk 0 of the
  // last tile and contributes zero)
  const int nch = t0 < a.ntile && c0 < a.nchunk && (GRP != 3 || e3 >= 0)
                      ? min(CPW, a.nchunk - c0)
                      : 0;
  const int cb = nch > 0 ? c0 : 0;
  const int n16 = lane & 15, kq = lane >> 4;
  // grouped: this workgroup's routing slot and its expert's weights
  const u32x4_t *codes = a.codes;
  const void *meta = a.meta;
  const char *arow = (const char *)a.A;
  float *crow = a.C;
  int ns = 0;
  if constexpr (GRP == 3) {
    if (e3first < 0) {  // no routed slot: the combined row is zero
      const int n = t0 * 16 + n16;
      if (w == 0 && kq == 0 && t0 < a.ntile && n < a.N) a.cout[n] = 0.f;
      return;
    }
    const int e = e3 >= 0 ? e3 : e3first;
    codes = a.codes_e[e];
    meta = a.meta_e[e];
    arow += (int64_t)slot * a.lda * 4;
  } else if constexpr (GRP != 0) {
    for (int j = 0; j < a.nid; j++) ns += a.ids[j] >= 0 && a.ids[j] < a.nexp;
    const int y = (int)blockIdx.y, e = y < a.nid ? a.ids[y] : -1;
    if (GRP == 2 && ns == 0) {  // no routed pair: the combined rows are zero
      if (y == 0 && sl == 0 && kq == 0) {
#pragma unroll
        for (int u = 0; u < TPW; u++) {
          const int n = (t0 + u) * 16 + n16;
          if (t0 + u < a.ntile && n < a.N)
            for (int t = 0; t < a.nid / a.slots; t++) a.cout[t * a.ldo + n] = 0.f;
        }
      }
      return;
    }
    if (e < 0 || e >= a.nexp) return;  // workgroup-uniform
    codes = a.codes_e[e];
    meta = a.meta_e[e];
    if (GRP == 2)
      arow += (int64_t)y * a.lda * 4;
    else
      arow += (int64_t)(y / a.slots) * a.lda * (DT == SGLQ_DT_F32 ? 4 : 2);
    crow += (int64_t)y * a.ldc;
  }
  int tl[TPW];  // tiles, clamped to the last (valid memory; results past it are not stored)
#pragma unroll
  for (int u = 0; u < TPW; u++) tl[u] = min(t0 + u, a.ntile - 1);

  // ---- loads: activations, meta, codes (all issued before any is used)
  constexpr int RW = DT == SGLQ_DT_F32 ? 2 : 1;  // 128-bit words per 8-element item
  constexpr int RU = GRP >= 2 ? RW : 0;          // and as many of the up half (SwiGLU rows)
  u32x4_t raw[NQ][RW + RU];
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    const int it = 64 * q + lane;
    const int k = (cb * SPC * 4 + it) * 8;
    const bool ok = nch > 0 && it < IPW && k < a.K;
    // global address space on both sides of the select keeps these global (not flat) loads,
    // which the staging can wait for without waiting for the weights behind them
    const GU4 *p = ok ? (const GU4 *)(arow + (int64_t)k * (RW * 2)) : (const GU4 *)g_zero_item;
#pragma unroll
    for (int i = 0; i < RW; i++) raw[q][i] = p[i];
    if constexpr (GRP >= 2) {
      const GU4 *pu = ok ? (const GU4 *)(arow + ((int64_t)a.kcols + k) * 4)
                         : (const GU4 *)g_zero_item;
#pragma unroll
      for (int i = 0; i < RW; i++) raw[q][RW + i] = pu[i];
    }
  }
  MT mv[TPW][CPW];  // meta entry (e8m0 bytes of four steps) of every chunk
  uint32_t cexp[TPW];
#pragma unroll
  for (int u = 0; u < TPW; u++) {
    cexp[u] = 0;
    if constexpr ((E2M1 || MV) && CPW % 4 == 0) {
      // one entry (word) per chunk, quads of four chunks contiguous per column: 16-byte loads
      // (32 for 8-byte entries) of the quads cb/4 .. , clamped to the row
      constexpr int ESZ = sizeof(MT);
      const int64_t nm = E2M1 ? a.nmeta / 4 : a.nmeta;  // entries per column
      const MT *mp = (const MT *)meta + sglq_mrow(tl[u], n16, nm);
      const int q0 = cb >> 2, qlast = (int)(nm >> 2) - 1;
#pragma unroll
      for (int v = 0; v < CPW / 4; v++) {
        const u32x4_t *qp = (const u32x4_t *)(mp + (int64_t)min(q0 + v, qlast) * 64);
        if constexpr (ESZ == 4) {
          const u32x4_t x = qp[0];
#pragma unroll
          for (int j = 0; j < 4; j++) mv[u][4 * v + j] = x[j];
        } else {
          const u32x4_t x0 = qp[0], x1 = qp[1];
          mv[u][4 * v] = (uint64_t)x0[0] | ((uint64_t)x0[1] << 32);
          mv[u][4 * v + 1] = (uint64_t)x0[2] | ((uint64_t)x0[3] << 32);
          mv[u][4 * v + 2] = (uint64_t)x1[0] | ((uint64_t)x1[1] << 32);
          mv[u][4 * v + 3] = (uint64_t)x1[2] | ((uint64_t)x1[3] << 32);
        }
      }
    } else {
      // groups of cpg chunks (or slices not aligned to quads): the entry of chunk cb + i is
      // group (cb + i) / cpg, found with scalar arithmetic
      const int cpg = E2M1 ? 1 : a.cpg;
      const MT *mp = (const MT *)meta + sglq_mrow(tl[u], n16, E2M1 ? a.nmeta / 4 : a.nmeta);
      int g = cb / cpg, r = cb - g * cpg;
#pragma unroll
      for (int i = 0; i < CPW; i++) {
        mv[u][i] = mp[sglq_mofs(g)];
        if (++r == cpg && i + 1 < nch) {
          r = 0;
          g++;
        }
      }
    }
    if constexpr (E2M1) cexp[u] = a.colexp[tl[u] * 16 + n16];
  }
  u32x4_t wv[TPW][CPW];
  {
    const int last = nch > 0 ? nch - 1 : 0;
#pragma unroll
    for (int u = 0; u < TPW; u++) {
      const u32x4_t *cp = codes + ((int64_t)tl[u] * a.nchunk + cb) * 64 + lane;
#pragma unroll
      for (int i = 0; i < CPW; i++) wv[u][i] = __builtin_nontemporal_load(cp + min(i, last) * 64);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // the whole batch of loads stays ahead of the staging

  // ---- staging: row maximum over the slice, one power of two per wave, f16 hi (+ lo)
  auto decode = [&](int q, float (&v)[8]) {
#pragma unroll
    for (int o = 0; o < 8; o++) {
      if constexpr (GRP >= 2)  // silu(gate) * up (reference src/deepseek.c:662-663)
        v[o] = sglq_silu(__uint_as_float(raw[q][o >> 2][o & 3])) *
               __uint_as_float(raw[q][RW + (o >> 2)][o & 3]);
      else if constexpr (DT == SGLQ_DT_F32)
        v[o] = __uint_as_float(raw[q][o >> 2][o & 3]);
      else if constexpr (DT == SGLQ_DT_F16)
        v[o] = f16_bits((raw[q][0][o >> 1] >> (16 * (o & 1))) & 0xFFFFu);
      else
        v[o] = bf16_bits((raw[q][0][o >> 1] >> (16 * (o & 1))) & 0xFFFFu);
    }
  };
  // |x| compared as integers (the order of non-negative floats); rows of 16 lanes by DPP
  // rotations, then the four rows through scalar registers
  uint32_t mb = 0;
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    float v[8];
    decode(q, v);
    float m = 0.f;
#pragma unroll
    for (int o = 0; o < 8; o++) m = fmaxf(m, fabsf(v[o]));
    mb = max(mb, __float_as_uint(m));
  }
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x128, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x124, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x122, 0xF, 0xF, false));
  mb = max(mb, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mb, 0x121, 0xF, 0xF, false));
  mb = max(max((uint32_t)__builtin_amdgcn_readlane((int)mb, 0),
               (uint32_t)__builtin_amdgcn_readlane((int)mb, 16)),
           max((uint32_t)__builtin_amdgcn_readlane((int)mb, 32),
               (uint32_t)__builtin_amdgcn_readlane((int)mb, 48)));
  // the power of two that puts the slice maximum in [2^13, 2^14) (denormal maxima count as
  // 2^-127; zero, inf and NaN slices keep 0)
  const int bex = (int)(mb >> 23);
  const int e = (mb == 0 || bex == 255) ? 0 : bex - 127 - 13;
  half8_t *base = s_op + w * NP * RS;
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    const int it = 64 * q + lane;
    if (IPW % 64 != 0 && it >= IPW) continue;
    float v[8];
    decode(q, v);
    half8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x = ldexpf(v[KIND == SGLQ_KIND_U4 ? kofs4(i) : i], -e);
      const _Float16 h = (_Float16)x;
      hi[i] = h;
      lo[i] = (_Float16)(x - (float)h);
    }
    base[it] = hi;
    if constexpr (NP == 2) base[RS + it] = lo;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- multiply: the lanes of column n16 < NP carry operand row n16 (hi, lo); the other lanes
  // read row NP - 1 again, so product rows NP .. 15 hold copies that are never used.  Each
  // operand read feeds the MFMAs of all TPW tiles.
  const half8_t *opp = base + min(n16, NP - 1) * RS + kq;
  float f[TPW];
  float4_t acc[TPW][2];
#pragma unroll
  for (int u = 0; u < TPW; u++) {
    f[u] = 0.f;
    acc[u][0] = acc[u][1] = (float4_t){0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int i = 0; i < CPW; i++) {
    if (i < nch) {  // wave-uniform
      float sc[TPW];
      half2_t zA[TPW], zB[TPW];
      float4_t tc[TPW];
#pragma unroll
      for (int u = 0; u < TPW; u++) {
        sc[u] = 0.f;
        zA[u] = zB[u] = (half2_t){0, 0};
        if constexpr (!E2M1) decode_meta<SCF16>(mv[u][i], sc[u], zA[u], zB[u]);
        tc[u] = E2M1 ? acc[u][i & 1] : (float4_t){0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        const half8_t op = opp[(i * SPC + j) * 4];
#pragma unroll
        for (int u = 0; u < TPW; u++) {
          half8_t b;
          if constexpr (E2M1) {
            // block scale relative to the column's largest, folded into the conversion (exact
            // down to 2^-24 of the column's largest block; smaller blocks flush)
            const uint32_t ex = (mv[u][i] >> (8 * j)) & 255u;
            const int rel = (int)ex - (int)cexp[u];
            const float bs =
                (ex == 255u || rel < -60) ? 0.f : __uint_as_float((uint32_t)(127 + rel) << 23);
            H8 r;
            r.h[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[u][i][j], bs, 0);
            r.h[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[u][i][j], bs, 1);
            r.h[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[u][i][j], bs, 2);
            r.h[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[u][i][j], bs, 3);
            b = r.v;
          } else {
            b = unpack<KIND>(wv[u][i], j, zA[u], zB[u]);
          }
          tc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(op, b, tc[u], 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < TPW; u++) {
        if constexpr (E2M1)
          acc[u][i & 1] = tc[u];
        else  // rows 0 (hi) and 1 (lo) of this chunk, scaled
          f[u] = fmaf(sc[u], NP == 2 ? tc[u][0] + tc[u][1] : tc[u][0], f[u]);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < TPW; u++) {
    if constexpr (E2M1) {
      const float4_t s2 = acc[u][0] + acc[u][1];
      // 2^(colexp - 127) and the wave's power of two in one exponent
      f[u] = ldexpf(NP == 2 ? s2[0] + s2[1] : s2[0], (int)cexp[u] - 127 + e);
    } else {
      f[u] = ldexpf(f[u], e);
    }
  }

  if constexpr (GRP == 3) {
    // every slot's slices, then out[n] = ((0 + w0 o0) + w1 o1) + ... in slot order, each o the
    // slot's slices added in slice order, as k_moe_combine (reference src/deepseek.c:675-676)
    if (kq == 0) s_sum[w][0][n16] = f[0];
    __syncthreads();
    const int n = t0 * 16 + n16;
    if (w != 0 || kq != 0 || t0 >= a.ntile || n >= a.N) return;
    float out = 0.f;
    for (int j = 0; j < a.nid && j < (NW >> a.ksl); j++) {
      if (a.ids[j] < 0 || a.ids[j] >= a.nexp) continue;
      float o = s_sum[j << a.ksl][0][n16];
      for (int q = 1; q < ks; q++) o += s_sum[(j << a.ksl) + q][0][n16];
      out = __fadd_rn(out, __fmul_rn(a.cw[j], o));
    }
    a.cout[n] = out;
    return;
  }
  // ---- K slices of a tile group added in slice order, then bias and store (lanes 0-15)
  if (ks > 1) {
    if (kq == 0) {
#pragma unroll
      for (int u = 0; u < TPW; u++) s_sum[w][u][n16] = f[u];
    }
    __syncthreads();
    if (sl != 0) return;
    if (kq == 0) {
#pragma unroll
      for (int u = 0; u < TPW; u++) {
        float sum = s_sum[w][u][n16];
        for (int q = 1; q < ks; q++) sum += s_sum[w + q][u][n16];
        f[u] = sum;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < TPW; u++) {
    const int n = (t0 + u) * 16 + n16;
    if (kq != 0 || t0 + u >= a.ntile || n >= a.N) continue;
    if constexpr (GRP == 2)  // read back by another workgroup's combine: written through
      __hip_atomic_store(&crow[n], f[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      crow[n] = f[u] + (GRP == 0 && a.bias ? a.bias[n] : 0.f);
  }
  if constexpr (GRP == 2) {
    // fused combine: the stores above are acknowledged before the arrival, and the last slot
    // of the tile adds the rows ((0 + w0 o0) + w1 o1) + ... in slot order, as k_moe_combine
    // (reference src/deepseek.c:675-676)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int t = t0;
    if (t >= a.ntile) return;
    int last = 0;
    if (lane == 0)
      last = __hip_atomic_fetch_add(&a.cnt[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             ns - 1;
    last = __shfl(last, 0);
    if (!last) return;
    const int n = t * 16 + n16;
    if (lane < 16 && n < a.N) {
      for (int tok = 0; tok < a.nid / a.slots; tok++) {
        const int jb = tok * a.slots;
        float sum = 0.f;
        for (int j0 = 0; j0 < a.slots; j0 += 8) {
          float wj[8], vj[8];
          bool lj[8];
#pragma unroll
          for (int u = 0; u < 8; u++) {
            const int j = jb + j0 + u;
            lj[u] = j0 + u < a.slots && a.ids[j] >= 0 && a.ids[j] < a.nexp;
            wj[u] = lj[u] ? a.cw[j] : 0.f;
            vj[u] = lj[u] ? __hip_atomic_load(&a.C[(int64_t)j * a.ldc + n], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : 0.f;
          }
#pragma unroll
          for (int u = 0; u < 8; u++)
            if (lj[u]) sum = __fadd_rn(sum, __fmul_rn(wj[u], vj[u]));
        }
        a.cout[tok * a.ldo + n] = sum;
      }
    }
    if (lane == 0) __hip_atomic_store(&a.cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int KIND, int CPW, int TPW, int NW, int DT>
void launch_row3(const RowArgs &a, bool scf16, bool mv, dim3 grid, size_t lds, hipStream_t st) {
  if constexpr (KIND == SGLQ_KIND_E2M1) {
    k_gemv_row<KIND, CPW, TPW, DT, true, false, NW><<<grid, NW * 64, lds, st>>>(a);
  } else {
    if (scf16 && mv)
      k_gemv_row<KIND, CPW, TPW, DT, true, true, NW><<<grid, NW * 64, lds, st>>>(a);
    else if (scf16)
      k_gemv_row<KIND, CPW, TPW, DT, true, false, NW><<<grid, NW * 64, lds, st>>>(a);
    else if (mv)
      k_gemv_row<KIND, CPW, TPW, DT, false, true, NW><<<grid, NW * 64, lds, st>>>(a);
    else
      k_gemv_row<KIND, CPW, TPW, DT, false, false, NW><<<grid, NW * 64, lds, st>>>(a);
  }
}

template <int KIND, int CPW, int TPW, int NW>
void launch_row2(const RowArgs &a, int dt, bool scf16, bool mv, dim3 grid, size_t lds,
                 hipStream_t st) {
  if (dt == SGLQ_DT_F32)
    launch_row3<KIND, CPW, TPW, NW, SGLQ_DT_F32>(a, scf16, mv, grid, lds, st);
  else if (dt == SGLQ_DT_F16)
    launch_row3<KIND, CPW, TPW, NW, SGLQ_DT_F16>(a, scf16, mv, grid, lds, st);
  else
    launch_row3<KIND, CPW, TPW, NW, SGLQ_DT_BF16>(a, scf16, mv, grid, lds, st);
}

// Chunks per wave, tiles per wave and waves per workgroup of a k_gemv_row launch (the
// instantiated set).
template <int KIND>
bool launch_row(const RowArgs &a, int cpw, int tpw, int nw, int dt, bool scf16, bool mv,
                dim3 grid, size_t lds, hipStream_t st) {
#define SGLQ_ROW_CASE(C, T, W)                                   \
  if (cpw == C && tpw == T && nw == W) {                          \
    launch_row2<KIND, C, T, W>(a, dt, scf16, mv, grid, lds, st); \
    return true;                                                  \
  }
  SGLQ_ROW_CASE(1, 1, 8)
  SGLQ_ROW_CASE(2, 1, 8)
  SGLQ_ROW_CASE(4, 1, 8)
  SGLQ_ROW_CASE(8, 1, 8)
  SGLQ_ROW_CASE(12, 1, 8)
  SGLQ_ROW_CASE(16, 1, 8)
  SGLQ_ROW_CASE(1, 1, 16)
  SGLQ_ROW_CASE(2, 1, 16)
  SGLQ_ROW_CASE(4, 1, 16)
  SGLQ_ROW_CASE(8, 1, 16)
#undef SGLQ_ROW_CASE
  return false;
}

// grouped one-token launch: f16 scales, one group per chunk (quad meta loads from 4 chunks),
// 8 waves, cpw chunks per wave
template <int KIND, int GRP, int DT>
bool launch_row_grp2(const RowArgs &a, int cpw, dim3 grid, size_t lds, hipStream_t st) {
  switch (cpw) {
    case 1: k_gemv_row<KIND, 1, 1, DT, true, false, 8, GRP><<<grid, 512, lds, st>>>(a); return true;
    case 2: k_gemv_row<KIND, 2, 1, DT, true, false, 8, GRP><<<grid, 512, lds, st>>>(a); return true;
    case 4: k_gemv_row<KIND, 4, 1, DT, true, true, 8, GRP><<<grid, 512, lds, st>>>(a); return true;
    case 8: k_gemv_row<KIND, 8, 1, DT, true, true, 8, GRP><<<grid, 512, lds, st>>>(a); return true;
    default: return false;
  }
}
// GRP 3: 16 waves, up to 8 slots x 2 K slices of one tile
template <int KIND, int C, bool MV>
void launch_row_grp3c(const RowArgs &a, dim3 grid, size_t lds, hipStream_t st) {
  auto f = k_gemv_row<KIND, C, 1, SGLQ_DT_F32, true, MV, 16, 3>;
  // dynamic LDS beyond 64 KiB is enabled per kernel and device; the request must leave room
  // for the kernel's static LDS (the slice sums) within the 160 KiB of a workgroup, so it is
  // exactly this launch's size, raised again when a larger one comes
  static size_t raised[64];
  int dev = 0;
  if (lds > 64 * 1024 && hipGetDevice(&dev) == hipSuccess &&
      (dev >= 64 || lds > raised[dev]) &&
      hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) == hipSuccess &&
      dev < 64)
    raised[dev] = lds;
  f<<<grid, 1024, lds, st>>>(a);
}
template <int KIND>
bool launch_row_grp3(const RowArgs &a, int cpw, dim3 grid, size_t lds, hipStream_t st) {
  switch (cpw) {
    case 1: launch_row_grp3c<KIND, 1, false>(a, grid, lds, st); return true;
    case 2: launch_row_grp3c<KIND, 2, false>(a, grid, lds, st); return true;
    case 4: launch_row_grp3c<KIND, 4, true>(a, grid, lds, st); return true;
    case 8: launch_row_grp3c<KIND, 8, true>(a, grid, lds, st); return true;
    default: return false;
  }
}
template <int KIND>
bool launch_row_grp(const RowArgs &a, int grp, int dt, int cpw, dim3 grid, size_t lds,
                    hipStream_t st) {
  if (grp == 3) return launch_row_grp3<KIND>(a, cpw, grid, lds, st);
  if (grp == 2) return launch_row_grp2<KIND, 2, SGLQ_DT_F32>(a, cpw, grid, lds, st);
  if (dt == SGLQ_DT_F32) return launch_row_grp2<KIND, 1, SGLQ_DT_F32>(a, cpw, grid, lds, st);
  if (dt == SGLQ_DT_F16) return launch_row_grp2<KIND, 1, SGLQ_DT_F16>(a, cpw, grid, lds, st);
  return launch_row_grp2<KIND, 1, SGLQ_DT_BF16>(a, cpw, grid, lds, st);
}

}  // namespace

// Grouped MoE decode launch on k_gemv_row (see RowArgs).  The weights and rows it takes:
// f16 group scales, one group per chunk, K within 8 waves of at most 8 chunks, 16-byte
// aligned rows (grp 2: f32 gate/up rows with 4-element aligned halves and arrival counters).
int sglq_gemv_row_grouped_ok(const sglq_dev *d, int grp, const void *A, int dt, int64_t lda,
                             int kcols) {
  if (d->kind == SGLQ_KIND_E2M1 || !d->kident || d->K % 8 != 0 || !d->scf16 ||
      d->meta_mode != SGLQ_META_GROUP || d->cpg != 1 || d->nchunk > 64)
    return 0;
  const int64_t esz = dt == SGLQ_DT_F32 ? 4 : 2;
  if ((uintptr_t)A % 16 != 0 || (lda * esz) % 16 != 0) return 0;
  if (grp == 2 && (dt != SGLQ_DT_F32 || kcols % 4 != 0 || !d->gv_cnt)) return 0;
  if (const char *e = getenv("SGLQ_GEMV_ROW"))
    if (atoi(e) == 0) return 0;
  return 1;
}

// 1 = launched, 0 = not applicable (sglq_gemv_row_grouped_ok), -1 = launch error.
int sglq_gemv_row_grouped(const sglq_dev *d, const void *const *codes_e,
                          const void *const *meta_e, const int32_t *ids, int npairs, int slots,
                          int nexp, int grp, const void *A, int dt, int64_t lda, int kcols,
                          float *C, int64_t ldc, const float *cw, float *cout, int64_t ldo,
                          hipStream_t st) {
  if (!sglq_gemv_row_grouped_ok(d, grp == 3 ? 2 : grp, A, dt, lda, kcols) ||
      (grp >= 2 && !cout))
    return 0;
  const int64_t nc = d->nchunk;
  // grp 3 (one token, at most 8 slots, K within two slices of 8 chunks): two K slices per slot
  if (grp == 3 && (npairs > 8 || npairs != slots || nc > 16)) return 0;
  const int ways = grp == 3 ? 2 : 8;  // K slices per workgroup row of waves
  int cpw = 0;
  for (int c : {1, 2, 4, 8})
    if (!cpw && ways * c >= nc) cpw = c;
  if (!cpw) return 0;
  if (const char *ov = getenv("SGLQ_ROW_PLAN")) {  // "cpw,..." (measurement override, grp 1)
    const int c = atoi(ov);
    if (grp == 1 && (c == 1 || c == 2 || c == 4 || c == 8) && ways * c >= nc) cpw = c;
  }
  int ksl = 0;
  while ((1 << ksl) * cpw < nc && (2 << ksl) <= ways) ksl++;
  if (grp == 3) ksl = 1;
  RowArgs a;
  memset(&a, 0, sizeof(a));
  a.A = A;
  a.C = C;
  a.N = (int)d->N;
  a.K = (int)d->K;
  a.ntile = (int)d->ntile;
  a.nchunk = (int)nc;
  a.nmeta = (int)d->nmeta;
  a.cpg = 1;
  a.ksl = ksl;
  a.adt = dt;
  a.codes_e = (const u32x4_t *const *)codes_e;
  a.meta_e = meta_e;
  a.ids = ids;
  a.nid = npairs;
  a.slots = slots;
  a.nexp = nexp;
  a.lda = lda;
  a.ldc = ldc;
  a.ldo = ldo;
  a.kcols = kcols;
  a.cw = cw;
  a.cout = cout;
  a.cnt = d->gv_cnt;
  const int tpg = grp == 3 ? 1 : 8 >> ksl;
  const dim3 grid((unsigned)((d->ntile + tpg - 1) / tpg), grp == 3 ? 1u : (unsigned)npairs);
  const int np = dt == SGLQ_DT_BF16 && grp == 1 ? 1 : 2;
  const int spc = d->kind == SGLQ_KIND_U8 ? 2 : 4;
  const size_t lds = (size_t)(grp == 3 ? 16 : 8) * np * (cpw * spc * 4 + 4) * 16;
  const bool ok = d->kind == SGLQ_KIND_U8
                      ? launch_row_grp<SGLQ_KIND_U8>(a, grp, dt, cpw, grid, lds, st)
                      : launch_row_grp<SGLQ_KIND_U4>(a, grp, dt, cpw, grid, lds, st);
  if (!ok) return 0;
  SGLQ_HIP(hipGetLastError());
  return 1;
fail:
  return -1;
}

// 1 = launched, 0 = this weight / row takes the general kernels, -1 = launch error
int sglq_gemv_row(const sglq_dev *d, const void *A, int dt, const float *bias, float *C,
                  hipStream_t st) {
  if (!d->kident || d->K % 8 != 0 || (uintptr_t)A % 16 != 0) return 0;
  if (d->kind != SGLQ_KIND_E2M1 && d->meta_mode != SGLQ_META_GROUP) return 0;
  const int64_t nc = d->nchunk;
  // plan: one tile per wave; 8 waves per workgroup up to 32 chunks, 16 beyond; the fewest
  // chunks per wave that let the workgroup's waves cover K.  Measured (graph replay, rotated
  // weights, one box): [11008, 4096] 4 chunks x 8 waves 7.3 us (2 x 16: 8.3, 8 x 8: 8.5);
  // [4096, 11008] 8 x 16 8.1 us (12 x 8: 8.6); MXFP4 [8192, 8192] 4 x 16 8.8 us (8 x 8: 9.1);
  // two or four tiles per wave (one operand read feeding several MFMAs) measured 15-40% slower.
  static const int cs[] = {1, 2, 4, 8, 12, 16};
  int cpw = 0, tpw = 1;
  int nw = nc <= 32 ? 8 : 16;
  for (int i = 0; i < 6 && !cpw; i++)
    if (nw * cs[i] >= nc && (nw == 8 || cs[i] <= 8)) cpw = cs[i];
  if (!cpw) return 0;  // K beyond the longest slices
  if (const char *ov = getenv("SGLQ_ROW_PLAN")) {  // "cpw,tpw,waves" (measurement override)
    int c = 0, t = 0, w = 0;
    if (sscanf(ov, "%d,%d,%d", &c, &t, &w) == 3 && c > 0 && t > 0 && (w == 8 || w == 16)) {
      cpw = c;
      tpw = t;
      nw = w;
    }
  }
  int ksl = 0;
  while ((1 << ksl) * cpw < nc && (2 << ksl) <= nw) ksl++;
  if ((1 << ksl) * cpw < nc) return 0;
  RowArgs a;
  a.codes = d->codes;
  a.meta = d->meta;
  a.colexp = d->colexp;
  a.A = A;
  a.bias = bias;
  a.C = C;
  a.N = (int)d->N;
  a.K = (int)d->K;
  a.ntile = (int)d->ntile;
  a.nchunk = (int)nc;
  a.nmeta = (int)d->nmeta;
  a.cpg = d->cpg > 0 ? (int)d->cpg : 1;
  a.ksl = ksl;
  a.adt = dt;
  const int np = dt == SGLQ_DT_BF16 ? 1 : 2;
  const bool mv = d->kind != SGLQ_KIND_E2M1 && d->cpg == 1 && cpw % 4 == 0;
  const int tpg = (nw >> ksl) * tpw;  // tiles per workgroup
  const dim3 grid((unsigned)((d->ntile + tpg - 1) / tpg));
  const int spc = d->kind == SGLQ_KIND_U8 ? 2 : 4;
  const size_t lds = (size_t)nw * np * (cpw * spc * 4 + 4) * 16;
  bool ok;
  switch (d->kind) {
    case SGLQ_KIND_U4:
      ok = launch_row<SGLQ_KIND_U4>(a, cpw, tpw, nw, dt, d->scf16, mv, grid, lds, st);
      break;
    case SGLQ_KIND_U8:
      ok = launch_row<SGLQ_KIND_U8>(a, cpw, tpw, nw, dt, d->scf16, mv, grid, lds, st);
      break;
    default:
      ok = launch_row<SGLQ_KIND_E2M1>(a, cpw, tpw, nw, dt, true, false, grid, lds, st);
      break;
  }
  if (!ok) return 0;
  SGLQ_HIP(hipGetLastError());
  return 1;
fail:
  return -1;
}
