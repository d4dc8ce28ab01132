// gemv_row.hip — one-row decode GEMV (M = 1) with a lean issue budget.
#include "gemv_ops.hpp"

using namespace sglq;

namespace {

// ---------------------------------------------------------------------------------------
// One-row decode GEMV with a lean issue budget (k_gemv_row).  Same operands and arithmetic as
// k_gemv_wave for one identity-order, 16-byte aligned row (exact q - z in f16, scale in fp32
// per chunk, f16 hi + lo activations under a per-wave power of two), with the work laid out so
// that almost every instruction is the multiply itself:
//   * the wave geometry is fixed (8 waves; ks = 1 << ksl K slices of CPW chunks per tile,
//     8 / ks tiles per workgroup), so tile, slice and chunk indices are shifts of the wave
//     index, kept in scalar registers;
//   * code, meta and activation addresses are one scalar base per wave plus one per-lane
//     offset; meta entries of consecutive chunks come in 16-byte loads (meta rows are padded
//     to 4 entries, e8m0 rows to 16 bytes);
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
};

// 32 zero bytes: the activation item of a lane whose item lies past K (or past the wave's
// chunks) is read from here, so no per-element masking is needed
__device__ const u32x4_t g_zero_item[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};

typedef __attribute__((address_space(1))) const u32x4_t GU4;

template <int KIND, int CPW, int DT, bool SCF16, bool MV>
__global__ __launch_bounds__(512) void k_gemv_row(RowArgs a) {
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr int NP = DT == SGLQ_DT_BF16 ? 1 : 2;     // f16 operand rows: hi (+ lo)
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;  // MFMA steps per chunk
  constexpr int IPW = CPW * SPC * 4;                 // 8-element items of a wave's slice
  static_assert(IPW % 64 == 0 || 64 % IPW == 0, "items per lane");
  constexpr int NQ = (IPW + 63) / 64;                // items per lane
  constexpr int RS = IPW + 4;                        // LDS row stride (rows 64 B apart)
  using MT = typename std::conditional<E2M1, uint32_t, meta_t<SCF16>>::type;
  extern __shared__ half8_t s_op[];                  // [8 waves][NP][RS]
  __shared__ float s_sum[8][16];

  const int lane = (int)threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int ks = 1 << a.ksl;
  const int t = (int)blockIdx.x * (8 >> a.ksl) + (w >> a.ksl);
  const int sl = w & (ks - 1);
  const int tl = t < a.ntile ? t : a.ntile - 1;
  const int c0 = sl * CPW;
  // chunks of this wave (0 for a wave past the last tile or chunk: it streams chunk 0 of its
  // tile and contributes zero)
  const int nch = t < a.ntile && c0 < a.nchunk ? min(CPW, a.nchunk - c0) : 0;
  const int cb = nch > 0 ? c0 : 0;
  const int n16 = lane & 15, kq = lane >> 4;

  // ---- loads: activations, meta, codes (all issued before any is used)
  constexpr int RW = DT == SGLQ_DT_F32 ? 2 : 1;  // 128-bit words per 8-element item
  u32x4_t raw[NQ][RW];
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    const int it = 64 * q + lane;
    const int k = (cb * SPC * 4 + it) * 8;
    const bool ok = nch > 0 && it < IPW && k < a.K;
    // global address space on both sides of the select keeps these global (not flat) loads,
    // which the staging can wait for without waiting for the weights behind them
    const GU4 *p = ok ? (const GU4 *)((const char *)a.A + (int64_t)k * (RW * 2))
                      : (const GU4 *)g_zero_item;
#pragma unroll
    for (int i = 0; i < RW; i++) raw[q][i] = p[i];
  }
  MT mv[CPW];  // meta entry (e8m0 bytes of four steps) of every chunk
  uint32_t cexp = 0;
  const int64_t mrow = ((int64_t)tl * 16 + n16) * a.nmeta;
  if constexpr (E2M1) {
    // e8m0 bytes of this column's steps cb*4 .. (16-byte loads; rows are 16-byte multiples)
    const uint8_t *eb = (const uint8_t *)a.meta + mrow + cb * 4;
    if constexpr (CPW % 4 == 0) {
      const int nv = (a.nmeta - cb * 4) / 16;  // 16-byte words left in the row (>= 1)
#pragma unroll
      for (int i = 0; i < CPW / 4; i++) {
        const u32x4_t v = ((const u32x4_t *)eb)[min(i, nv - 1)];
#pragma unroll
        for (int j = 0; j < 4; j++) mv[4 * i + j] = v[j];
      }
    } else {
#pragma unroll
      for (int i = 0; i < CPW; i++) mv[i] = ((const uint32_t *)eb)[min(i, max(nch, 1) - 1)];
    }
    cexp = a.colexp[tl * 16 + n16];
  } else if constexpr (MV) {
    // one entry per chunk (cpg == 1), rows padded to 4 entries: 16-byte loads
    const u32x4_t *mp = (const u32x4_t *)((const MT *)a.meta + mrow + cb);
    constexpr int PER = 16 / sizeof(MT);
    const int nv = (a.nmeta - cb) / PER;  // 16-byte words left in the row (>= 1)
#pragma unroll
    for (int i = 0; i < (CPW + PER - 1) / PER; i++) {
      const u32x4_t v = mp[min(i, nv - 1)];
      if constexpr (SCF16) {
#pragma unroll
        for (int j = 0; j < 4; j++)
          if (4 * i + j < CPW) mv[4 * i + j] = v[j];
      } else {
#pragma unroll
        for (int j = 0; j < 2; j++)
          if (2 * i + j < CPW) mv[2 * i + j] = (uint64_t)v[2 * j] | ((uint64_t)v[2 * j + 1] << 32);
      }
    }
  } else {
    // groups of cpg chunks: entry of chunk cb + i is (cb + i) / cpg (scalar arithmetic)
    const MT *mp = (const MT *)a.meta + mrow;
    int g = cb / a.cpg, r = cb - g * a.cpg;
#pragma unroll
    for (int i = 0; i < CPW; i++) {
      mv[i] = mp[g];
      if (++r == a.cpg && i + 1 < nch) {
        r = 0;
        g++;
      }
    }
  }
  u32x4_t wv[CPW];
  {
    const u32x4_t *cp = a.codes + ((int64_t)tl * a.nchunk + cb) * 64 + lane;
    const int last = nch > 0 ? nch - 1 : 0;
#pragma unroll
    for (int i = 0; i < CPW; i++) wv[i] = __builtin_nontemporal_load(cp + min(i, last) * 64);
  }
  __builtin_amdgcn_sched_barrier(0);  // the whole batch of loads stays ahead of the staging

  // ---- staging: row maximum over the slice, one power of two per wave, f16 hi (+ lo)
  auto decode = [&](int q, float (&v)[8]) {
#pragma unroll
    for (int o = 0; o < 8; o++) {
      if constexpr (DT == SGLQ_DT_F32)
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
    if (IPW < 64 && it >= IPW) continue;
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
  // read row NP - 1 again, so product rows NP .. 15 hold copies that are never used
  const half8_t *opp = base + min(n16, NP - 1) * RS + kq;
  float f = 0.f;
  float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < CPW; i++) {
    if (i < nch) {  // wave-uniform
      float sc = 0.f;
      half2_t zA = {0, 0}, zB = {0, 0};
      if constexpr (!E2M1) decode_meta<SCF16>(mv[i], sc, zA, zB);
      float4_t tc = (E2M1 && (i & 1)) ? acc1 : acc0;
      if constexpr (!E2M1) tc = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        const half8_t op = opp[(i * SPC + j) * 4];
        half8_t b;
        if constexpr (E2M1) {
          // block scale relative to the column's largest, folded into the conversion (exact
          // down to 2^-24 of the column's largest block; smaller blocks flush)
          const uint32_t ex = (mv[i] >> (8 * j)) & 255u;
          const int rel = (int)ex - (int)cexp;
          const float bs =
              (ex == 255u || rel < -60) ? 0.f : __uint_as_float((uint32_t)(127 + rel) << 23);
          H8 r;
          r.h[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[i][j], bs, 0);
          r.h[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[i][j], bs, 1);
          r.h[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[i][j], bs, 2);
          r.h[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(wv[i][j], bs, 3);
          b = r.v;
        } else {
          b = unpack<KIND>(wv[i], j, zA, zB);
        }
        tc = __builtin_amdgcn_mfma_f32_16x16x32_f16(op, b, tc, 0, 0, 0);
      }
      if constexpr (E2M1) {
        if (i & 1)
          acc1 = tc;
        else
          acc0 = tc;
      } else {
        // rows 0 (hi) and 1 (lo) of this chunk, scaled
        f = fmaf(sc, NP == 2 ? tc[0] + tc[1] : tc[0], f);
      }
    }
  }
  if constexpr (E2M1) {
    const float4_t s2 = acc0 + acc1;
    // 2^(colexp - 127) and the wave's power of two in one exponent
    f = ldexpf(NP == 2 ? s2[0] + s2[1] : s2[0], (int)cexp - 127 + e);
  } else {
    f = ldexpf(f, e);
  }

  // ---- K slices of a tile added in slice order, then bias and store (lanes 0-15: kq == 0)
  const int n = tl * 16 + n16;
  if (ks == 1) {
    if (kq == 0 && t < a.ntile && n < a.N) a.C[n] = f + (a.bias ? a.bias[n] : 0.f);
    return;
  }
  if (kq == 0) s_sum[w][n16] = f;
  __syncthreads();
  if (sl != 0 || kq != 0 || t >= a.ntile || n >= a.N) return;
  float sum = s_sum[w][n16];
  for (int q = 1; q < ks; q++) sum += s_sum[w + q][n16];
  a.C[n] = sum + (a.bias ? a.bias[n] : 0.f);
}

template <int KIND, int CPW, int DT>
void launch_row3(const RowArgs &a, bool scf16, bool mv, dim3 grid, size_t lds, hipStream_t st) {
  if constexpr (KIND == SGLQ_KIND_E2M1) {
    k_gemv_row<KIND, CPW, DT, true, false><<<grid, 512, lds, st>>>(a);
  } else {
    if (scf16 && mv)
      k_gemv_row<KIND, CPW, DT, true, true><<<grid, 512, lds, st>>>(a);
    else if (scf16)
      k_gemv_row<KIND, CPW, DT, true, false><<<grid, 512, lds, st>>>(a);
    else if (mv)
      k_gemv_row<KIND, CPW, DT, false, true><<<grid, 512, lds, st>>>(a);
    else
      k_gemv_row<KIND, CPW, DT, false, false><<<grid, 512, lds, st>>>(a);
  }
}

template <int KIND, int CPW>
void launch_row2(const RowArgs &a, int dt, bool scf16, bool mv, dim3 grid, size_t lds,
                 hipStream_t st) {
  if (dt == SGLQ_DT_F32)
    launch_row3<KIND, CPW, SGLQ_DT_F32>(a, scf16, mv, grid, lds, st);
  else if (dt == SGLQ_DT_F16)
    launch_row3<KIND, CPW, SGLQ_DT_F16>(a, scf16, mv, grid, lds, st);
  else
    launch_row3<KIND, CPW, SGLQ_DT_BF16>(a, scf16, mv, grid, lds, st);
}

// Chunks per wave for k_gemv_row: U4 / E2M1 chunks hold 16 items, U8 chunks 8; a slice must be
// a whole number of 64-item passes or a power-of-two fraction of one.
template <int KIND>
bool launch_row(const RowArgs &a, int cpw, int dt, bool scf16, bool mv, dim3 grid, size_t lds,
                hipStream_t st) {
  if constexpr (KIND == SGLQ_KIND_U8) {
    switch (cpw) {
      case 2: launch_row2<KIND, 2>(a, dt, scf16, mv, grid, lds, st); return true;
      case 4: launch_row2<KIND, 4>(a, dt, scf16, mv, grid, lds, st); return true;
      case 8: launch_row2<KIND, 8>(a, dt, scf16, mv, grid, lds, st); return true;
      case 16: launch_row2<KIND, 16>(a, dt, scf16, mv, grid, lds, st); return true;
      default: return false;
    }
  } else {
    switch (cpw) {
      case 1: launch_row2<KIND, 1>(a, dt, scf16, mv, grid, lds, st); return true;
      case 2: launch_row2<KIND, 2>(a, dt, scf16, mv, grid, lds, st); return true;
      case 4: launch_row2<KIND, 4>(a, dt, scf16, mv, grid, lds, st); return true;
      case 8: launch_row2<KIND, 8>(a, dt, scf16, mv, grid, lds, st); return true;
      case 12: launch_row2<KIND, 12>(a, dt, scf16, mv, grid, lds, st); return true;
      case 16: launch_row2<KIND, 16>(a, dt, scf16, mv, grid, lds, st); return true;
      default: return false;
    }
  }
}

}  // namespace

// 1 = launched, 0 = this weight / row takes the general kernels, -1 = launch error
int sglq_gemv_row(const sglq_dev *d, const void *A, int dt, const float *bias, float *C,
             hipStream_t st) {
  if (!d->kident || d->K % 8 != 0 || (uintptr_t)A % 16 != 0) return 0;
  if (d->kind != SGLQ_KIND_E2M1 && d->meta_mode != SGLQ_META_GROUP) return 0;
  if (d->kind == SGLQ_KIND_E2M1 && d->nmeta % 16 != 0) return 0;
  const int64_t nc = d->nchunk;
  static const int c4[] = {1, 2, 4, 8, 12, 16}, c8[] = {2, 4, 8, 16};
  const int *cs = d->kind == SGLQ_KIND_U8 ? c8 : c4;
  const int ncs = d->kind == SGLQ_KIND_U8 ? 4 : 6;
  int cpw = 0;
  for (int i = 0; i < ncs && !cpw; i++)
    if (8 * cs[i] >= nc) cpw = cs[i];
  if (!cpw) return 0;  // K beyond 8 slices of the longest
  int ksl = 0;
  while ((1 << ksl) * cpw < nc && ksl < 3) ksl++;
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
  const bool mv = d->kind != SGLQ_KIND_E2M1 && d->cpg == 1 && d->nmeta % 4 == 0 && cpw % 4 == 0;
  const int tpg = 8 >> ksl;
  const dim3 grid((unsigned)((d->ntile + tpg - 1) / tpg));
  const int spc = d->kind == SGLQ_KIND_U8 ? 2 : 4;
  const size_t lds = (size_t)8 * np * (cpw * spc * 4 + 4) * 16;
  bool ok;
  switch (d->kind) {
    case SGLQ_KIND_U4: ok = launch_row<SGLQ_KIND_U4>(a, cpw, dt, d->scf16, mv, grid, lds, st); break;
    case SGLQ_KIND_U8: ok = launch_row<SGLQ_KIND_U8>(a, cpw, dt, d->scf16, mv, grid, lds, st); break;
    default: ok = launch_row<SGLQ_KIND_E2M1>(a, cpw, dt, true, false, grid, lds, st); break;
  }
  if (!ok) return 0;
  SGLQ_HIP(hipGetLastError());
  return 1;
fail:
  return -1;
}

