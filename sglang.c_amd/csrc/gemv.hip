// gemv.hip — decode-side quantized linear, C[M,N] = A[M,K] * W^T (+ bias) for M <= 16.
//
// Work split: a workgroup stages one K range of the activations in LDS and its ks x tpg waves
// split that range into ks slices of CPW chunks over tpg 16-column tiles; the slices of a tile
// are added through LDS in slice order.  When K is longer than one workgroup's range (large M
// shrinks the staging budget), the ranges of one column group leave fp32 partial sums in a
// per-handle buffer and the last workgroup to arrive (an arrival counter) adds them in K order.
// No atomics touch C, so the result is deterministic, and every counter is back at zero when a
// launch ends.
//
// Weight codes are streamed once with one 128-bit non-temporal load per lane per chunk, all
// of a wave's chunks issued before any is consumed and before the activation staging.  Codes
// are unpacked in registers straight into the B operand of v_mfma_f32_16x16x32_f16 with the
// zero subtracted exactly in f16 (q - z is a small integer), so the fp32 MFMA accumulation sees
// exact weight codes.  The group scale is applied in fp32 per chunk (per step for MXFP4's e8m0
// block scales and for group sizes that are not whole chunks).
//
// Activations: each workgroup finds, per row, the largest |a| over its K range and scales the
// row by an exact power of two so it sits well inside f16 range; f32 inputs are split into f16
// hi + lo parts (about 22 significant bits), bf16/f16 inputs fit one f16 part.  The power of
// two is undone exactly on the result.
#include <stdlib.h>
#include <string.h>

#include "gemv_ops.hpp"

using namespace sglq;

namespace {

struct GemvArgs {
  const u32x4_t *codes;
  const void *meta;
  const void *A;
  const int32_t *kmap;  // device position -> original k; nullptr = identity on [0, K)
  const float *bias;
  float *C;
  float *part;  // [S][M][N]
  int *cnt;     // [ncg]
  int64_t lda, ldc;
  int N, K, M, adt, ntile, nchunk, nmeta, cpg, S, ncg, ks, tpg;
  // grouped (MoE decode): blockIdx.y picks a row segment {expert, first row, rows, -} whose
  // expert supplies the weights; rows are read as A row r (amode 0), A row rowmap[r] (amode 1)
  // or silu(A[r][k]) * A[r][kcols + k] of an f32 A (amode 2); C row r is written
  const int4 *segs;
  const int *nseg;
  const u32x4_t *const *codes_e;
  const void *const *meta_e;
  const int32_t *rowmap;
  int amode, kcols;
  uint32_t ipr_magic;  // ceil(2^32 / items per row)
  // one-token MoE down projection with the combine fused (k_gemv_wave GRP 2): the last segment
  // of a tile to finish writes cout[n] = sum over slots j of cw[j] * C[cpos[j]][n], in slot order
  const int32_t *cpos;
  const float *cw;
  float *cout;
  int ck;
  // one token: slot j is segment {ids[j], row j, 1 row} if 0 <= ids[j] < nexp (segs, nseg,
  // rowmap and cpos unused; the token row is A row 0)
  const int32_t *ids;
  int nid, nexp;
};


__device__ __forceinline__ float act1(const void *A, int dt, int64_t i) {
  if (dt == SGLQ_DT_F32) return ((const float *)A)[i];
  const uint32_t b = ((const uint16_t *)A)[i];
  return dt == SGLQ_DT_BF16 ? bf16_bits(b) : f16_bits(b);
}

// Activations of source row `row` at device positions kp .. kp+7 (0 outside [0, K) and in
// padding), one element at a time (the general path: act-order gather, unaligned rows,
// K % 8 != 0, SwiGLU rows).
__device__ __forceinline__ float swiglu_at(const GemvArgs &a, int64_t rb, int k) {
  const float g = ((const float *)a.A)[rb + k];  // silu as reference src/deepseek.c:662-663
  return sglq_silu(g) * ((const float *)a.A)[rb + a.kcols + k];
}

__device__ __forceinline__ void load8(const GemvArgs &a, int64_t row, int kp, float v[8]) {
  const int64_t rb = row * a.lda;
  if (a.amode == 2) {
#pragma unroll
    for (int o = 0; o < 8; o++) {
      const int k = a.kmap ? a.kmap[kp + o] : (kp + o < a.K ? kp + o : -1);
      v[o] = k >= 0 ? swiglu_at(a, rb, k) : 0.f;
    }
    return;
  }
  if (a.kmap == nullptr) {
#pragma unroll
    for (int o = 0; o < 8; o++) v[o] = kp + o < a.K ? act1(a.A, a.adt, rb + kp + o) : 0.f;
  } else {
#pragma unroll
    for (int o = 0; o < 8; o++) {
      const int k = a.kmap[kp + o];
      v[o] = k >= 0 ? act1(a.A, a.adt, rb + k) : 0.f;
    }
  }
}


// Split-K epilogue of a decode GEMV workgroup whose partial sums are stored: the last
// workgroup of the column group (the last wave of the tile when a.ks > 1, after the other
// slices' waves have left) adds the partials in K order into C and re-arms the counter.
__device__ __forceinline__ void gemv_splitk_tail(const GemvArgs &a, int M, int sidx, int cg,
                                                 int t, bool tvalid, int tid, int lane, int nthr,
                                                 int &s_last) {
  // ---- split-K over workgroups: the last workgroup of this column group adds the partials in
  // K order.  Partials are device-scope stores/loads, so no cache write-back or invalidate is
  // needed; waiting for the stores' acknowledgement before the arrival increment orders them.
  // (Only the ks == 0 waves are still running here.)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // partials of (row r, column nn) added in K order; eight loads are in flight at a time
  // (one at a time, each waiting for its predecessor, they made the reduction latency-bound)
  auto sum_parts = [&](int r, int nn) -> float {
    const float *pp = a.part + (int64_t)r * a.N + nn;
    const int64_t ss = (int64_t)M * a.N;
    float sum = 0.f;
    int s0 = 0;
    for (; s0 + 8 <= a.S; s0 += 8) {
      float v[8];
#pragma unroll
      for (int q = 0; q < 8; q++)
        v[q] = __hip_atomic_load(pp + (s0 + q) * ss, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int q = 0; q < 8; q++) sum += v[q];
    }
    for (; s0 < a.S; s0++)
      sum += __hip_atomic_load(pp + s0 * ss, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return sum;
  };
  if (a.ks > 1) {
    // the ks != 0 waves have left, so no workgroup barrier is possible: arrivals are counted
    // per tile, by its ks == 0 wave
    if (!tvalid) return;
    int last = 0;
    if (lane == 0)
      last = __hip_atomic_fetch_add(&a.cnt[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             a.S - 1;
    last = __shfl(last, 0);
    if (!last) return;
    for (int idx = lane; idx < M * 16; idx += 64) {
      const int r = idx >> 4, nn = t * 16 + (idx & 15);
      if (tvalid && nn < a.N)
        a.C[r * a.ldc + nn] = sum_parts(r, nn) + (a.bias ? a.bias[nn] : 0.f);
    }
    if (lane == 0) __hip_atomic_store(&a.cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(&a.cnt[cg], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             a.S - 1;
  __syncthreads();
  if (!s_last) return;
  const int ncol = a.tpg * 16;
  for (int idx = tid; idx < M * ncol; idx += nthr) {
    const int r = idx / ncol, nn = cg * ncol + idx % ncol;
    if (nn < a.N) a.C[r * a.ldc + nn] = sum_parts(r, nn) + (a.bias ? a.bias[nn] : 0.f);
  }
  if (tid == 0) __hip_atomic_store(&a.cnt[cg], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave's weights for CPW chunks of one tile (meta entries, then codes), every address
// clamped into the weight so the loads are straight-line code issued before any use, and the
// product of those chunks with the A operands of chunk i, step j at arow_p[(i * SPC + j) * 4]
// (NP == 2: the lo part at lo_off further).  Chunks past the end (c0 + i >= nchunk) run on a
// zero scale.
template <int KIND, int CPW, bool SCF16, bool STEPM>
struct WaveWeights {
  static constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  static constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  static constexpr int NMV = E2M1 ? CPW : (STEPM ? CPW * SPC : CPW);
  using MT = typename std::conditional<E2M1, uint32_t, meta_t<SCF16>>::type;
  MT mv[NMV];
  u32x4_t wv[CPW];

  __device__ __forceinline__ void load(const GemvArgs &a, const u32x4_t *codes, const void *meta,
                                       int tl, int n16, int lane, int c0) {
    const int clast = a.nchunk - 1;
    if constexpr (E2M1) {
      const uint32_t *ep = (const uint32_t *)meta + sglq_mrow(tl, n16, a.nmeta / 4);
#pragma unroll
      for (int i = 0; i < CPW; i++) mv[i] = ep[sglq_mofs(min(c0 + i, clast))];
    } else if constexpr (STEPM) {
      const MT *mp = (const MT *)meta + sglq_mrow(tl, n16, a.nmeta);
#pragma unroll
      for (int i = 0; i < CPW * SPC; i++)
        mv[i] = mp[sglq_mofs(min(c0 * SPC + i, clast * SPC + SPC - 1))];
    } else {
      const MT *mp = (const MT *)meta + sglq_mrow(tl, n16, a.nmeta);
      const int cc = min(c0, clast);
      int g = cc / a.cpg, r = cc - g * a.cpg;
      const int glast = clast / a.cpg;
#pragma unroll
      for (int i = 0; i < CPW; i++) {
        mv[i] = mp[sglq_mofs(min(g, glast))];
        if (++r == a.cpg) {
          r = 0;
          g++;
        }
      }
    }
    const u32x4_t *cp = codes + (int64_t)tl * a.nchunk * 64 + lane;
#pragma unroll
    for (int i = 0; i < CPW; i++) wv[i] = __builtin_nontemporal_load(cp + min(c0 + i, clast) * 64);
  }

  template <int NP>
  __device__ __forceinline__ float4_t multiply(const GemvArgs &a, const half8_t *arow_p,
                                               int lo_off, int c0) const {
    auto read_ops = [&](int i, half8_t (&op)[SPC * NP]) {
#pragma unroll
      for (int j = 0; j < SPC; j++) {
        op[j] = arow_p[(i * SPC + j) * 4];
        if constexpr (NP == 2) op[SPC + j] = arow_p[lo_off + (i * SPC + j) * 4];
      }
    };
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    float4_t pacc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    half8_t opc[SPC * NP], opn[SPC * NP];
    read_ops(0, opc);
  #pragma unroll
    for (int i = 0; i < CPW; i++) {
      const bool live = c0 + i < a.nchunk;
      if (i + 1 < CPW) read_ops(i + 1, opn);
      float sc = 0.f;
      half2_t zA = {0, 0}, zB = {0, 0};
      if constexpr (!E2M1 && !STEPM) {
        decode_meta<SCF16>(mv[i], sc, zA, zB);
        sc = live ? sc : 0.f;
      }
  #pragma unroll
      for (int j = 0; j < SPC; j++) {
        if constexpr (!E2M1 && STEPM) {
          decode_meta<SCF16>(mv[i * SPC + j], sc, zA, zB);
          sc = live ? sc : 0.f;
        }
        const half8_t b = unpack<KIND>(wv[i], j, zA, zB);
        // even and odd chunks accumulate in separate registers: two independent MFMA chains
        float4_t &tc = pacc[i & 1];
        tc = __builtin_amdgcn_mfma_f32_16x16x32_f16(opc[j], b, tc, 0, 0, 0);
        if constexpr (NP == 2)
          tc = __builtin_amdgcn_mfma_f32_16x16x32_f16(opc[SPC + j], b, tc, 0, 0, 0);
        if constexpr (E2M1 || STEPM) {
          if constexpr (E2M1) {
            const uint32_t ex = (mv[i] >> (8 * j)) & 255u;
            sc = (ex == 255u || !live) ? 0.f : ldexpf(1.0f, (int)ex - 127);  // ref qweight.c:361
          }
          acc += sc * tc;
          tc = (float4_t){0.f, 0.f, 0.f, 0.f};
        }
      }
      if constexpr (!E2M1 && !STEPM) {
        acc += sc * pacc[i & 1];
        pacc[i & 1] = (float4_t){0.f, 0.f, 0.f, 0.f};
      }
  #pragma unroll
      for (int q = 0; q < SPC * NP; q++) opc[q] = opn[q];
    }
    return acc;
  }
};

// SPL: 0 = 16-bit activations (one f16 part); 1 = f32 activations as f16 hi + lo, two MFMAs per
// step; 2 = f32 activations with at most 8 rows: the lo rows sit right below the hi rows in the
// staging area (rows M .. 2M-1), so one MFMA covers both and row r + M is added to row r at the
// end.
// AM (activations): 0 = staged element by element (act-order gather, unaligned rows, K % 8,
// SwiGLU rows); 1 = 128-bit loads (FAST) with two items per thread held from before the weight
// loads; 2 = FAST holding eight (several rows over a long range: items loaded after the
// weights would only arrive with them, and be loaded twice).
template <int KIND, int CPW, int SPL, bool SCF16, bool STEPM, int AM>
__global__ __launch_bounds__(512) void k_gemv(GemvArgs a) {
  constexpr bool FAST = AM != 0;
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr bool E2M1 = KIND == SGLQ_KIND_E2M1;
  constexpr bool SPLIT = SPL != 0, FOLD = SPL == 2;
  constexpr int NP = SPL == 1 ? 2 : 1;  // MFMAs per step
  constexpr int RW = SPLIT ? 2 : 1;  // 128-bit words per 8-element activation item
  constexpr int KEEP = AM == 2 ? 8 : 2;  // items per thread held in registers across the passes
  constexpr bool KEEPDEC = AM != 2;       // hold them decoded (else raw, decoded twice)
  extern __shared__ half8_t s_act[];  // [NP][M][RS] activation operands, then [waves][64] acc
  __shared__ unsigned s_amax[16];
  __shared__ int s_exp[16];
  __shared__ int s_last;

  const int nthr = blockDim.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int cg = (int)(blockIdx.x % (unsigned)a.ncg), sidx = (int)(blockIdx.x / (unsigned)a.ncg);
  const int tt = w / a.ks, ks = w - tt * a.ks;     // tile within the group, K slice
  const int cw0 = sidx * a.ks * CPW;              // first chunk of the workgroup's K range
  const int c0 = cw0 + ks * CPW;                  // first chunk of this wave
  const int ncw = min(a.ks * CPW, a.nchunk - cw0);  // chunks in the workgroup's range
  const int kp0 = cw0 * SPC * 32;
  int M = a.M, row0 = 0;
  const u32x4_t *codes = a.codes;
  const void *meta = a.meta;
  if (a.segs) {
    if ((int)blockIdx.y >= *a.nseg) return;
    const int4 sg = a.segs[blockIdx.y];
    row0 = sg.y;
    M = min(sg.z, a.M);  // the staging holds a.M rows (the host cuts blocks to that)
    codes = a.codes_e[sg.x];
    meta = a.meta_e[sg.x];
  }
  // source row of activation row m (m < M)
  auto src_row = [&](int m) -> uint32_t {
    const int r = row0 + m;
    return a.amode == 1 ? (uint32_t)a.rowmap[r] : (uint32_t)r;
  };
  // it / IPR for it < 2^16 as one multiply-high by the host's ceil(2^32 / IPR)
  auto row_of = [&](int it) { return (int)__umulhi((uint32_t)it, a.ipr_magic); };
  const int IPR = a.ks * CPW * SPC * 4;           // 8-element activation items per row
  const int RS = IPR + 1;                         // LDS row stride (+1 spreads rows over banks)
  const int items = M * IPR;
  const int t = cg * a.tpg + tt;
  const bool tvalid = t < a.ntile;
  const int tl = min(t, a.ntile - 1);  // waves past the last tile load valid memory, unused
  const int n16 = lane & 15, kq = lane >> 4;

  // ---- activation items: the first KEEP per thread are loaded before the weight loads
  // (vmcnt retires in order, so they can be consumed while the weights are still in flight).
  // FAST items are one (16-bit) or two (f32) 128-bit loads from a clamped, always-valid
  // address with no branch; decoding to f32 happens at first use.
  if (tid < 16) s_amax[tid] = 0u;
  struct Raw {
    u32x4_t q[RW];
    bool ok;
  };
  auto item_kp = [&](int r) { return kp0 + (r >> 2) * 32 + (r & 3) * 8; };
  auto load_raw = [&](int it, Raw &x) {
    const int m = row_of(it), r = it - m * IPR;
    const int kp = item_kp(r);
    x.ok = it < items && (r >> 2) < ncw * SPC && (!FAST || kp < a.K);
    if constexpr (FAST) {
      // element offset in 32 bits (the host keeps the activation block under 2^31 elements)
      const uint32_t off = src_row(min(m, M - 1)) * (uint32_t)a.lda + (x.ok ? kp : 0);
      const u32x4_t *p = (const u32x4_t *)((const char *)a.A + off * (SPLIT ? 4 : 2));
#pragma unroll
      for (int i = 0; i < RW; i++) x.q[i] = p[i];
    }
  };
  auto decode_raw = [&](int it, const Raw &x, float (&v)[8]) {
#pragma unroll
    for (int o = 0; o < 8; o++) v[o] = 0.f;
    if (!x.ok) return;
    if constexpr (FAST) {
      if constexpr (SPLIT) {
#pragma unroll
        for (int o = 0; o < 8; o++) v[o] = __uint_as_float(x.q[o >> 2][o & 3]);
      } else if (a.adt == SGLQ_DT_BF16) {
#pragma unroll
        for (int o = 0; o < 8; o++) v[o] = bf16_bits((x.q[0][o >> 1] >> (16 * (o & 1))) & 0xFFFFu);
      } else {
#pragma unroll
        for (int o = 0; o < 8; o++) v[o] = f16_bits((x.q[0][o >> 1] >> (16 * (o & 1))) & 0xFFFFu);
      }
    } else {
      const int m = row_of(it);
      load8(a, src_row(m), item_kp(it - m * IPR), v);
    }
  };
  auto amax_item = [&](int it, const float (&v)[8]) {
    float mx = 0.f;
#pragma unroll
    for (int o = 0; o < 8; o++) mx = fmaxf(mx, fabsf(v[o]));
    atomicMax(&s_amax[row_of(it)], __float_as_uint(mx));
  };
  // the same for item it = (first item of the wave) + lane, called by every lane (items past
  // the end carry zeros): a wave whose items all lie in one row (the usual case: rows hold a
  // multiple of 64 items) reduces across its lanes first and makes one LDS atomic, not 64 on
  // one address
  auto amax_wave = [&](int it, const float (&v)[8]) {
    const int base = it - lane, last = min(base + 63, items - 1);
    if (base >= items) return;
    float mx = 0.f;
#pragma unroll
    for (int o = 0; o < 8; o++) mx = fmaxf(mx, fabsf(v[o]));
    const int ma = row_of(base);
    if (ma == row_of(last)) {
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      if (lane == 0) atomicMax(&s_amax[ma], __float_as_uint(mx));
    } else if (it < items) {
      atomicMax(&s_amax[row_of(it)], __float_as_uint(mx));
    }
  };
  auto store_item = [&](int it, const float (&v)[8]) {
    const int m = row_of(it), r = it - m * IPR;
    const int e = s_exp[m];
    half8_t hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x = ldexpf(v[KIND == SGLQ_KIND_U4 ? kofs4(i) : i], -e);
      const _Float16 h = (_Float16)x;
      hi[i] = h;
      lo[i] = (_Float16)(x - (float)h);
    }
    s_act[m * RS + r] = hi;
    if constexpr (SPLIT) s_act[(M + m) * RS + r] = lo;
  };
  Raw keep[KEEP];
#pragma unroll
  for (int j = 0; j < KEEP; j++) load_raw(tid + nthr * j, keep[j]);

  // ---- this wave's weight loads (meta, then codes), all issued before the activation
  // staging so their HBM latency overlaps it.  Chunk indices are clamped into [0, nchunk)
  // (valid memory; chunks past the wave's range are never accumulated), so the loads are
  // straight-line code.
  WaveWeights<KIND, CPW, SCF16, STEPM> WW;
  WW.load(a, codes, meta, tl, n16, lane, c0);
  __builtin_amdgcn_sched_barrier(0);  // keep the whole batch of loads ahead of the staging

  // ---- stage the activations: per-row max |a| -> exact power-of-two scale -> f16 operands
  __syncthreads();  // s_amax cleared
  float kv[KEEPDEC ? KEEP : 1][8];
#pragma unroll
  for (int j = 0; j < KEEP; j++) {
    float v[8];
    decode_raw(tid + nthr * j, keep[j], v);
    if constexpr (AM == 2)
      amax_wave(tid + nthr * j, v);
    else if (tid + nthr * j < items)
      amax_item(tid + nthr * j, v);
    if constexpr (KEEPDEC) {
#pragma unroll
      for (int o = 0; o < 8; o++) kv[j][o] = v[o];
    }
  }
  for (int it = tid + nthr * KEEP; it < items; it += nthr) {
    Raw x;
    float v[8];
    load_raw(it, x);
    decode_raw(it, x, v);
    amax_item(it, v);
  }
  __syncthreads();
  if (tid < M) {
    const float mx = __uint_as_float(s_amax[tid]);
    s_exp[tid] = (mx > 0.f && mx <= 3.0e38f) ? ilogbf(mx) - 13 : 0;  // max in [2^13, 2^14)
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < KEEP; j++) {
    if (tid + nthr * j >= items) continue;
    if constexpr (KEEPDEC) {
      store_item(tid + nthr * j, kv[KEEPDEC ? j : 0]);
    } else {
      float v[8];
      decode_raw(tid + nthr * j, keep[j], v);
      store_item(tid + nthr * j, v);
    }
  }
  for (int it = tid + nthr * KEEP; it < items; it += nthr) {
    Raw x;
    float v[8];
    load_raw(it, x);
    decode_raw(it, x, v);
    store_item(it, v);
  }
  __syncthreads();

  // ---- multiply: chunks past the wave's range (c0 + i >= nchunk) run on zero activations
  // with a zero scale, which keeps the code straight-line and every load ahead of its use.
  // Lanes of rows >= M read row M-1 instead: an A row only feeds the same row of the
  // product, and rows >= M are never written.
  const half8_t *arow_p = s_act + min(n16, (FOLD ? 2 * M : M) - 1) * RS + ks * CPW * SPC * 4 + kq;
  float4_t acc = WW.template multiply<NP>(a, arow_p, M * RS, c0);

  // ---- K slices of one tile are added in slice order through LDS (reusing the staging area)
  if (a.ks > 1) {
    float4_t *red = (float4_t *)s_act;
    __syncthreads();  // every wave is done reading activations
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (ks != 0) return;
    acc = red[w * 64 + lane];
    for (int q = 1; q < a.ks; q++) acc += red[(w + q) * 64 + lane];
  }

  if constexpr (FOLD) {
    // row r (hi part) += row r + M (lo part); row rr of this column sits in lane
    // 16 (rr / 4) + n16, element rr % 4, and (i + M) % 4 is the same for every lane
    float4_t f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pr = 4 * kq + i + M, e = (i + M) & 3;
      const float v = e == 0 ? acc[0] : e == 1 ? acc[1] : e == 2 ? acc[2] : acc[3];
      f[i] = acc[i] + __shfl(v, ((pr >> 2) & 3) * 16 + n16);
    }
    acc = f;
  }

  // lane holds rows 4*kq + i of column n (v_mfma_f32_16x16x32 C layout)
  const int n = t * 16 + n16;
  if (tvalid && n < a.N) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = 4 * kq + i;
      if (r < M) {
        const float v = ldexpf(acc[i], s_exp[r]);
        if (a.S == 1)
          a.C[(int64_t)(row0 + r) * a.ldc + n] = v + (a.bias ? a.bias[n] : 0.f);
        else  // device-scope store: written through to the level all XCDs share
          __hip_atomic_store(&a.part[((int64_t)sidx * M + r) * a.N + n], v, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (a.S == 1) return;

  gemv_splitk_tail(a, M, sidx, cg, t, tvalid, tid, lane, nthr, s_last);
}

// Decode GEMV of one row (or MR = 2 rows) with wave-private activation staging: fast
// activations (identity kmap, 16-byte aligned rows), one K slice of CPW chunks per wave (the
// host launches CPW = 4, 8 and 12, the slice lengths of the one-row plan).
// GRP 1 and 2 (MoE decode, segments of at most MR rows): blockIdx.y picks the segment, whose
// expert supplies the weights; the row is A row r (amode 0), A row rowmap[r] (amode 1), or
// with GRP 2 silu(A[r][k]) * A[r][kcols + k] of an f32 A; C row r is written.  Each wave
// stages every row of its segment, so this pays while most segments hold one row.  (The segment
// lookups cost the one-row launches 0.8 us when they were runtime branches, so GRP is a
// template parameter.)  Each wave loads only its own slice of the rows, takes each row's largest |a| over that
// slice with lane shuffles, and stages the scaled f16 operands in an LDS area of its own, so no
// workgroup barrier or LDS atomic comes before the multiply.  The power of two belongs to the
// (wave, row) pair and is undone exactly on the wave's sums, before the slices of a tile are
// added in slice order; everything after that is as in k_gemv.
// Measured against k_gemv at M = 1 (graph replay, f32 activations): [11008, 4096] 10.2 -> 8.5
// us, [4096, 11008] 11.6 -> 10.5 us (int4 g128), W8 [4864, 896] 4.6 -> 3.9 us.  At 2-4 rows it
// measured slower or equal (on four tiles per slice each tile repeats the staging; on one tile
// per workgroup every workgroup reads the whole block of rows), so it runs one row, or two
// rows over K of 17-32 chunks (one workgroup range), where it measured faster.
template <int KIND, int CPW, int SPL, bool SCF16, bool STEPM, int GRP, int MR>
__global__ __launch_bounds__(512) void k_gemv_wave(GemvArgs a) {
  static_assert(MR == 1 || MR == 2 || MR == 4, "rows per launch or segment");
  constexpr bool SWI = GRP == 2;
  static_assert(!SWI || SPL == 2, "SwiGLU rows are f32");
  constexpr int SPC = KIND == SGLQ_KIND_U8 ? 2 : 4;
  constexpr bool FOLD = SPL == 2;                  // f32: hi rows [0, M), lo rows [M, 2M)
  constexpr int RW = FOLD ? 2 : 1;                 // 128-bit words per 8-element item (and
                                                   // as many again for the up half with SWI)
  constexpr int IPR = CPW * SPC * 4;               // items per row of a wave's slice
  // a row's items must be whole 64-item passes, or a pass whole rows (the row maximum is
  // reduced per pass, then over the passes of a row)
  static_assert(IPR % 64 == 0 || 64 % IPR == 0, "slice length");
  constexpr int RS = IPR + 1;                      // LDS row stride (+1 spreads rows over banks)
  constexpr int LPR = IPR >= 64 ? 64 : IPR;        // lanes of one pass that hold the same row
  constexpr int QPR = IPR >= 64 ? IPR / 64 : 1;    // passes per row
  constexpr int NQ = (MR * IPR + 63) / 64;         // passes of 64 items over MR rows
  extern __shared__ half8_t s_act[];  // [waves][RA][RS] operands, then [waves][64] sums
  __shared__ int s_e[8][MR];
  __shared__ int s_last;

  const int nthr = blockDim.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int cg = (int)(blockIdx.x % (unsigned)a.ncg), sidx = (int)(blockIdx.x / (unsigned)a.ncg);
  const int tt = w / a.ks, ks = w - tt * a.ks;
  const int c0 = (sidx * a.ks + ks) * CPW;  // first chunk of this wave
  int M = a.M, row0 = 0;
  const u32x4_t *codes = a.codes;
  const void *meta = a.meta;
  int ns = 0;
  if constexpr (GRP != 0) {
    int4 sg;
    bool live;
    if (a.ids) {  // one token: slot blockIdx.y, its expert straight from the routing
      for (int j = 0; j < a.nid; j++) ns += a.ids[j] >= 0 && a.ids[j] < a.nexp;
      const int y = (int)blockIdx.y, e = y < a.nid ? a.ids[y] : -1;
      live = e >= 0 && e < a.nexp;
      sg = make_int4(e, y, 1, 0);
    } else {
      ns = *a.nseg;
      live = (int)blockIdx.y < ns;
      if (live) {
        sg = a.segs[blockIdx.y];
        sg.z = min(sg.z, min(MR, a.M));  // the staging holds these rows (the host cuts blocks)
      }
    }
    if (GRP == 2 && a.cout && ns == 0) {
      // no routed slot: the combined row is zero
      const int n = (cg * a.tpg) * 16 + lane;
      if (blockIdx.y == 0 && w == 0 && lane < 16 && n < a.N) a.cout[n] = 0.f;
      return;
    }
    if (!live) return;
    row0 = sg.y;
    M = sg.z;
    codes = a.codes_e[sg.x];
    meta = a.meta_e[sg.x];
  }
  const int RA = FOLD ? 2 * M : M;
  const int t = cg * a.tpg + tt;
  const bool tvalid = t < a.ntile;
  const int tl = min(t, a.ntile - 1);
  const int n16 = lane & 15, kq = lane >> 4;
  const int kp0 = c0 * SPC * 32;
  const int nit = M * IPR;

  // ---- this wave's activation items (item it = 64 q + lane: row it / IPR, 8 elements at
  // k = kp0 + 8 (it % IPR)), then its weights; all loads issued before any is used
  u32x4_t raw[NQ][SWI ? 2 * RW : RW];
  bool ok[NQ];
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    const int it = 64 * q + lane, m = it / IPR, kp = kp0 + (it - m * IPR) * 8;
    ok[q] = it < nit && kp < a.K;
    if (64 * q < nit) {  // wave-uniform
      // element offset in 32 bits (the host keeps the activation block under 2^31 elements)
      const int r = row0 + min(m, M - 1);
      const uint32_t src =
          GRP == 1 && a.amode == 1 ? (a.ids ? 0u : (uint32_t)a.rowmap[r]) : (uint32_t)r;
      const uint32_t off = src * (uint32_t)a.lda + (ok[q] ? kp : 0);
      const u32x4_t *p = (const u32x4_t *)((const char *)a.A + off * (FOLD ? 4 : 2));
#pragma unroll
      for (int i = 0; i < RW; i++) raw[q][i] = p[i];
      if constexpr (SWI) {
        const u32x4_t *pu = (const u32x4_t *)((const float *)a.A + off + a.kcols);
#pragma unroll
        for (int i = 0; i < RW; i++) raw[q][RW + i] = pu[i];
      }
    }
  }
  WaveWeights<KIND, CPW, SCF16, STEPM> WW;
  WW.load(a, codes, meta, tl, n16, lane, c0);
  __builtin_amdgcn_sched_barrier(0);  // keep the whole batch of loads ahead of the staging

  auto decode = [&](int q, float (&v)[8]) {
#pragma unroll
    for (int o = 0; o < 8; o++) {
      float x;
      if constexpr (SWI) {
        const float g = __uint_as_float(raw[q][o >> 2][o & 3]);  // reference deepseek.c:662-663
        x = sglq_silu(g) * __uint_as_float(raw[q][RW + (o >> 2)][o & 3]);
      } else if constexpr (FOLD)
        x = __uint_as_float(raw[q][o >> 2][o & 3]);
      else if (a.adt == SGLQ_DT_BF16)
        x = bf16_bits((raw[q][0][o >> 1] >> (16 * (o & 1))) & 0xFFFFu);
      else
        x = f16_bits((raw[q][0][o >> 1] >> (16 * (o & 1))) & 0xFFFFu);
      v[o] = ok[q] ? x : 0.f;
    }
  };
  // ---- per-row max |a| over the slice: lanes of one row in a pass, then the passes of a row
  float mq[NQ];
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    mq[q] = 0.f;
    if (64 * q >= nit) continue;
    float v[8];
    decode(q, v);
#pragma unroll
    for (int o = 0; o < 8; o++) mq[q] = fmaxf(mq[q], fabsf(v[o]));
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) mq[q] = fmaxf(mq[q], __shfl_xor(mq[q], o));
  }
  half8_t *base = s_act + w * RA * RS;
#pragma unroll
  for (int q = 0; q < NQ; q++) {
    if (64 * q >= nit) continue;
    float mx = 0.f;
#pragma unroll
    for (int u = 0; u < QPR; u++) mx = fmaxf(mx, mq[q - q % QPR + u]);
    const int e = (mx > 0.f && mx <= 3.0e38f) ? ilogbf(mx) - 13 : 0;  // max in [2^13, 2^14)
    const int it = 64 * q + lane, m = it / IPR, r = it - m * IPR;
    if (it >= nit) continue;
    if (r == 0) s_e[w][m] = e;
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
    base[m * RS + r] = hi;
    if constexpr (FOLD) base[(M + m) * RS + r] = lo;
  }
  // the staging area and s_e[w] are this wave's own: a wavefront-scope fence orders its LDS
  // stores before the reads of other lanes of the wave
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- multiply (lanes of rows >= RA read row RA - 1; those product rows are never written)
  const half8_t *arow_p = base + min(n16, RA - 1) * RS + kq;
  float4_t acc = WW.template multiply<1>(a, arow_p, 0, c0);
  if constexpr (FOLD) {
    // row r (hi part) += row r + M (lo part), as in k_gemv
    float4_t f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int pr = 4 * kq + i + M, e = (i + M) & 3;
      const float v = e == 0 ? acc[0] : e == 1 ? acc[1] : e == 2 ? acc[2] : acc[3];
      f[i] = acc[i] + __shfl(v, ((pr >> 2) & 3) * 16 + n16);
    }
    acc = f;
  }
  // undo this wave's power of two of row 4 kq + i
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * kq + i;
    acc[i] = r < M ? ldexpf(acc[i], s_e[w][r < MR ? r : 0]) : 0.f;
  }

  // ---- K slices of one tile are added in slice order through LDS (reusing the staging area)
  if (a.ks > 1) {
    float4_t *red = (float4_t *)s_act;
    __syncthreads();  // every wave is done reading its operands
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (ks != 0) return;
    acc = red[w * 64 + lane];
    for (int q = 1; q < a.ks; q++) acc += red[(w + q) * 64 + lane];
  }
  const int n = t * 16 + n16;
  if (tvalid && n < a.N) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = 4 * kq + i;
      if (r < M) {
        float *dst = &a.C[(int64_t)(row0 + r) * a.ldc + n];
        if (GRP == 2 && a.cout)  // read back by another workgroup's combine
          __hip_atomic_store(dst, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else if (a.S == 1)
          *dst = acc[i] + (a.bias ? a.bias[n] : 0.f);
        else  // device-scope store: written through to the level all XCDs share
          __hip_atomic_store(&a.part[((int64_t)sidx * M + r) * a.N + n], acc[i],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if constexpr (GRP == 2) {
    if (a.cout) {
      // fused combine (one K range, one live wave per workgroup here): the stores above are
      // acknowledged before the arrival, and the last segment of the tile reads them back
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0);
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      if (!tvalid) return;
      int last = 0;
      if (lane == 0)
        last = __hip_atomic_fetch_add(&a.cnt[t], 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == ns - 1;
      last = __shfl(last, 0);
      if (!last) return;
      if (lane < 16 && n < a.N) {
        // ((0 + w0 o0) + w1 o1) + ... in slot order, as k_moe_combine (reference
        // src/deepseek.c:675-676)
        // (8 slots at a time: rows and weights, then products, loaded before any is added)
        float sum = 0.f;
        for (int j0 = 0; j0 < a.ck; j0 += 8) {
          int rj[8];
          float wj[8], vj[8];
#pragma unroll
          for (int u = 0; u < 8; u++) {
            const int j = j0 + u;
            if (a.ids)  // one token: slot j's row is row j
              rj[u] = j < a.ck && a.ids[j] >= 0 && a.ids[j] < a.nexp ? j : -1;
            else
              rj[u] = j < a.ck ? a.cpos[j] : -1;
            wj[u] = j0 + u < a.ck ? a.cw[j0 + u] : 0.f;
          }
#pragma unroll
          for (int u = 0; u < 8; u++)
            vj[u] = rj[u] >= 0 ? __hip_atomic_load(&a.C[(int64_t)rj[u] * a.ldc + n],
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                               : 0.f;
#pragma unroll
          for (int u = 0; u < 8; u++)
            if (rj[u] >= 0) sum = __fadd_rn(sum, __fmul_rn(wj[u], vj[u]));
        }
        a.cout[n] = sum;
      }
      if (lane == 0) __hip_atomic_store(&a.cnt[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
  }
  if (a.S == 1) return;
  gemv_splitk_tail(a, M, sidx, cg, t, tvalid, tid, lane, nthr, s_last);
}

template <int KIND, int CPW, int SPL, int GRP, int MR = 1>
void launch_wave4(const GemvArgs &a, int scf16, int stepm, size_t lds, dim3 grid,
                  unsigned nthr, hipStream_t st) {
  if constexpr (KIND == SGLQ_KIND_E2M1) {
    k_gemv_wave<KIND, CPW, SPL, true, false, GRP, MR><<<grid, nthr, lds, st>>>(a);
  } else {
    if (scf16) {
      if (stepm)
        k_gemv_wave<KIND, CPW, SPL, true, true, GRP, MR><<<grid, nthr, lds, st>>>(a);
      else
        k_gemv_wave<KIND, CPW, SPL, true, false, GRP, MR><<<grid, nthr, lds, st>>>(a);
    } else {
      if (stepm)
        k_gemv_wave<KIND, CPW, SPL, false, true, GRP, MR><<<grid, nthr, lds, st>>>(a);
      else
        k_gemv_wave<KIND, CPW, SPL, false, false, GRP, MR><<<grid, nthr, lds, st>>>(a);
    }
  }
}

template <int KIND>
void launch_wave(const GemvArgs &a, int cpw, bool split, int scf16, int stepm, size_t lds,
                 dim3 grid, unsigned nthr, hipStream_t st) {
  if (a.segs == nullptr && a.M == 2) {
    if (split)
      launch_wave4<KIND, 4, 2, 0, 2>(a, scf16, stepm, lds, grid, nthr, st);
    else
      launch_wave4<KIND, 4, 0, 0, 2>(a, scf16, stepm, lds, grid, nthr, st);
  } else if (a.segs == nullptr && cpw == 8) {
    if (split)
      launch_wave4<KIND, 8, 2, 0>(a, scf16, stepm, lds, grid, nthr, st);
    else
      launch_wave4<KIND, 8, 0, 0>(a, scf16, stepm, lds, grid, nthr, st);
  } else if (a.segs == nullptr && cpw == 12) {
    if constexpr (KIND != SGLQ_KIND_U8) {  // 8-bit codes never get 12-chunk slices
      if (split)
        launch_wave4<KIND, 12, 2, 0>(a, scf16, stepm, lds, grid, nthr, st);
      else
        launch_wave4<KIND, 12, 0, 0>(a, scf16, stepm, lds, grid, nthr, st);
    }
  } else if (a.segs == nullptr) {
    if (split)
      launch_wave4<KIND, 4, 2, 0>(a, scf16, stepm, lds, grid, nthr, st);
    else
      launch_wave4<KIND, 4, 0, 0>(a, scf16, stepm, lds, grid, nthr, st);
  } else if (a.M > 1) {  // segments of up to 4 rows (2-4 tokens)
    if (a.amode == 2)
      launch_wave4<KIND, 4, 2, 2, 4>(a, scf16, stepm, lds, grid, nthr, st);
    else if (split)
      launch_wave4<KIND, 4, 2, 1, 4>(a, scf16, stepm, lds, grid, nthr, st);
    else
      launch_wave4<KIND, 4, 0, 1, 4>(a, scf16, stepm, lds, grid, nthr, st);
  } else if (a.amode == 2) {
    launch_wave4<KIND, 4, 2, 2>(a, scf16, stepm, lds, grid, nthr, st);
  } else {
    if (split)
      launch_wave4<KIND, 4, 2, 1>(a, scf16, stepm, lds, grid, nthr, st);
    else
      launch_wave4<KIND, 4, 0, 1>(a, scf16, stepm, lds, grid, nthr, st);
  }
}

template <int KIND, int CPW, int SPL, int AM>
void launch4(const GemvArgs &a, int scf16, int stepm, size_t lds, dim3 grid, unsigned nthr,
             hipStream_t st) {
  if constexpr (KIND == SGLQ_KIND_E2M1) {
    k_gemv<KIND, CPW, SPL, true, false, AM><<<grid, nthr, lds, st>>>(a);
  } else {
    if (scf16) {
      if (stepm)
        k_gemv<KIND, CPW, SPL, true, true, AM><<<grid, nthr, lds, st>>>(a);
      else
        k_gemv<KIND, CPW, SPL, true, false, AM><<<grid, nthr, lds, st>>>(a);
    } else {
      if (stepm)
        k_gemv<KIND, CPW, SPL, false, true, AM><<<grid, nthr, lds, st>>>(a);
      else
        k_gemv<KIND, CPW, SPL, false, false, AM><<<grid, nthr, lds, st>>>(a);
    }
  }
}

template <int KIND, int CPW, int SPL>
void launch_am(const GemvArgs &a, int scf16, int stepm, int am, size_t lds, dim3 grid,
               unsigned nthr, hipStream_t st) {
  if (am == 2)
    launch4<KIND, CPW, SPL, 2>(a, scf16, stepm, lds, grid, nthr, st);
  else if (am == 1)
    launch4<KIND, CPW, SPL, 1>(a, scf16, stepm, lds, grid, nthr, st);
  else
    launch4<KIND, CPW, SPL, 0>(a, scf16, stepm, lds, grid, nthr, st);
}

template <int KIND, int CPW>
void launch_cpw(const GemvArgs &a, bool split, int scf16, int stepm, int am, size_t lds,
                dim3 grid, unsigned nthr, hipStream_t st) {
  // f32 activations of at most 8 rows: hi and lo parts share one MFMA
  if (split && a.M <= 8)
    launch_am<KIND, CPW, 2>(a, scf16, stepm, am, lds, grid, nthr, st);
  else if (split)
    launch_am<KIND, CPW, 1>(a, scf16, stepm, am, lds, grid, nthr, st);
  else
    launch_am<KIND, CPW, 0>(a, scf16, stepm, am, lds, grid, nthr, st);
}

template <int KIND>
void launch_kind(const GemvArgs &a, int cpw, bool split, int scf16, int stepm, int am,
                 size_t lds, dim3 grid, unsigned nthr, hipStream_t st) {
  switch (cpw) {
    case 4: launch_cpw<KIND, 4>(a, split, scf16, stepm, am, lds, grid, nthr, st); break;
    case 12: launch_cpw<KIND, 12>(a, split, scf16, stepm, am, lds, grid, nthr, st); break;
    default: launch_cpw<KIND, 8>(a, split, scf16, stepm, am, lds, grid, nthr, st); break;
  }
}

constexpr size_t kLdsBudget = 60 * 1024;
constexpr size_t kLdsBigBudget = 128 * 1024;  // staging of the several-row plan (1 workgroup/CU)
constexpr int kMaxWaves = 8;  // per workgroup (the kernel's launch bound is 512 threads)

struct Plan {
  int cpw, ks, tpg, S, ncg;
  size_t lds;
};

// Work split for one launch.  A workgroup stages one K range of the activations in LDS and
// its ks x tpg waves split that range (ks slices of cpw chunks) over tpg tiles; ranges beyond
// one workgroup (K longer than the staging budget allows) are added across workgroups.
Plan plan_gemv(const sglq_dev *d, int64_t M, bool split, bool grouped = false,
               bool wave = false) {
  const int64_t np = split ? 2 : 1;
  const int64_t max_chunks = ((int64_t)kLdsBudget / (np * M * 16) - 1) / (d->spc * 4);
  Plan best = {0, 0, 0, 1 << 30, 0, 0};
  const int cand[3] = {8, 12, 4};
  for (int cpw : cand) {
    int64_t ks = (d->nchunk + cpw - 1) / cpw;
    ks = ks < kMaxWaves ? ks : kMaxWaves;
    const int64_t kl = max_chunks / cpw;
    ks = ks < kl ? ks : kl;
    if (ks < 1) continue;
    const int S = (int)((d->nchunk + ks * cpw - 1) / (ks * cpw));
    if (S < best.S) best = {cpw, (int)ks, 0, S, 0, 0};
  }
  if (best.cpw == 0) best = {4, 1, 0, (int)((d->nchunk + 3) / 4), 0, 0};
  best.tpg = best.ks >= 4 ? 1 : 4 / best.ks;
  // Several rows over a long K: measured fastest with one K slice per wave, four tiles per
  // workgroup and the K range cut so that about 8-12 workgroups share a column group (many
  // short workgroups, each staging a short activation range, beat few long ones even with
  // the partial-sum pass).  One row, or short K, keeps the fewest splits above, and so does
  // the grouped launch (it needs a single K range).
  //
  // From 8 rows on, every workgroup's staging pass (a max and a conversion per element) is
  // repeated by each column group, so eight tiles per workgroup (half the column groups) with
  // the K range cut into at most 8 pieces measured faster, the staging allowed to use up to
  // 128 KiB (one workgroup per CU): M = 16 [11008, 4096] 22.3 -> 16.5 us (f32), 20.3 -> 15.4
  // (bf16); [4096, 11008] 30.8 -> 19.1, 21.7 -> 17.7; M = 8 [4096, 11008] 17.3 -> 15.7.  At
  // 2-4 rows it measured 0.5-1 us slower than four tiles.
  if (!grouped && M >= 2 && M < 8 && d->nchunk >= 24) {
    for (int cpw : {4, 8, 12}) {
      const int S = (int)((d->nchunk + cpw - 1) / cpw);
      if (cpw > max_chunks) break;
      best = {cpw, 1, 4, S, 0, 0};
      if (S <= 12) break;
    }
  } else if (!grouped && M >= 8 && d->nchunk >= 24) {
    const int64_t big = ((int64_t)kLdsBigBudget / (np * M * 16) - 1) / (d->spc * 4);
    for (int cpw : {4, 8, 12}) {
      const int S = (int)((d->nchunk + cpw - 1) / cpw);
      if (cpw > big) break;
      best = {cpw, 1, 8, S, 0, 0};
      // 16 rows: 4-chunk slices up to 16 K ranges.  [8192, 8192] M = 16 against 8-chunk
      // slices: MXFP4 bf16 23.6 -> 20.1 us, f32 25.1 -> 22.1, GPTQ4 f32 24.7 -> 20.8, bf16
      // 19.2 -> 19.8; at 22 ranges ([4096, 11008]) it measured 27% slower
      if (S <= 8 || (M >= 16 && cpw == 4 && S <= 16)) break;
    }
  }
  // A short K of 9-16 chunks in one range: 4-chunk slices (more loads in flight per tile than
  // two 8-chunk slices), two tiles per workgroup from two rows on.  W8 [4864, 896] (14
  // chunks): M = 1 4.75 -> 4.51 us, M = 8 6.83 -> 5.57 us; every split over K measured slower.
  if (!grouped && d->nchunk > 8 && d->nchunk <= 16 && 16 <= max_chunks)
    best = {4, (int)((d->nchunk + 3) / 4), M >= 2 ? 2 : 1, 1, 0, 0};
  // One row over more than 64 chunks (K > 8192 at 4 bits): two slices of 4 chunks on each of
  // two tiles per workgroup and the K range split 8 chunks at a time measured 7% faster than
  // one range of 12-chunk slices ([4096, 11008]: 11.7 vs 12.6 us, weights streamed from HBM).
  if (!grouped && M == 1 && d->nchunk > 64 && max_chunks >= 8)
    best = {4, 2, 2, (int)((d->nchunk + 7) / 8), 0, 0};
  // Grouped (MoE decode) launches keep one K range per workgroup; among those, the measured
  // best at the DeepSeek expert shapes covers K with the least padding: 4-chunk slices over
  // a whole multiple of 4 chunks (gate/up, 16 chunks: 9.8 vs 10.6 us), or one slice per wave
  // on four tiles up to 12 chunks (down, 11 chunks: 9.3 vs 10.6 us).
  if (grouped && M <= 4) {
    const int64_t nc = d->nchunk;
    if (nc >= 16 && nc <= 32 && nc % 4 == 0 && nc <= max_chunks)
      best = {4, (int)(nc / 4), 1, 1, 0, 0};
    else if (nc <= 12 && max_chunks >= 12)
      best = {nc <= 4 ? 4 : nc <= 8 ? 8 : 12, 1, 4, 1, 0, 0};
  }
  // One row through k_gemv_wave: 4-chunk slices on up to 8 waves of one tile, the rest of K
  // over workgroups.  Measured best of every (cpw 4/8, ks, tpg) with ks * tpg <= 8:
  // [11008, 4096] 8.3 us (next (8, 4, 1) 8.8), [4096, 11008] 10.0 us (next (4, 2, 1) 10.3).
  // One row over more chunks takes longer slices so that all of K stays in one workgroup (no
  // partial sums): 33-64 chunks 8-chunk slices (64 chunks, against 4-chunk slices and K split
  // in two: GPTQ4 [4096, 8192] 8.1 -> 6.8 us, GPTQ8 [4096, 4096] 7.7 -> 6.2, MXFP4 [8192, 8192]
  // 11.9 -> 10.4), 65-96 chunks of 4-bit codes 12-chunk slices ([4096, 11008] 10.4 -> 10.1;
  // a 12-chunk slice of 8-bit codes is not a whole number of 64-item passes).  Beyond that,
  // 4-chunk slices, four per tile on two tiles, with K split over workgroups: best or within
  // 0.2 us of the best in a sweep at GPTQ8 [4096, 11008], GPTQ4 [4096, 16384] and
  // [8192, 28672], W8 [4096, 8192] (8-chunk slices on 8 waves measured up to 20% slower).
  if (wave) {
    const int ks = (int)(d->nchunk < 32 ? (d->nchunk + 3) / 4 : 8);
    best = {4, ks, 1, (int)((d->nchunk + 4 * ks - 1) / (4 * ks)), 0, 0};
    if (M == 1 && !grouped && d->nchunk > 32) {
      if (d->nchunk <= 64)
        best = {8, (int)((d->nchunk + 7) / 8), 1, 1, 0, 0};
      else if (d->nchunk <= 96 && d->spc == 4)
        best = {12, (int)((d->nchunk + 11) / 12), 1, 1, 0, 0};
      else
        best = {4, 4, 2, (int)((d->nchunk + 15) / 16), 0, 0};
    }
  }
  best.ncg = (int)((d->ntile + best.tpg - 1) / best.tpg);
  const size_t stage = (size_t)np * M * (best.ks * best.cpw * d->spc * 4 + 1) * 16;
  const size_t red = (size_t)best.ks * best.tpg * 64 * 16;
  best.lds = stage > red ? stage : red;
  return best;
}

}  // namespace

int sglq_gemv_setup(sglq_dev *d) {
  // the most K ranges any launch splits over (cpw = 4, one slice per workgroup)
  d->gv_split = (int)((d->nchunk + 3) / 4);
  if (d->gv_split > 1) {
    SGLQ_HIP(hipMalloc(&d->gv_part, (size_t)d->gv_split * 16 * d->N * sizeof(float)));
    SGLQ_HIP(hipMalloc(&d->gv_cnt, (size_t)d->ntile * sizeof(int)));
    SGLQ_HIP(hipMemset(d->gv_cnt, 0, (size_t)d->ntile * sizeof(int)));
  }
  return 0;
fail:
  return -1;
}

namespace {

GemvArgs base_args(const sglq_dev *d, const Plan &pl, const void *A, int dt, int64_t lda,
                   int64_t M, const float *bias, float *C, int64_t ldc) {
  GemvArgs a;
  memset(&a, 0, sizeof(a));
  a.codes = d->codes;
  a.meta = d->meta;
  a.A = A;
  a.kmap = d->kident ? nullptr : d->kmap;
  a.bias = bias;
  a.C = C;
  a.part = d->gv_part;
  a.cnt = d->gv_cnt;
  a.lda = lda;
  a.ldc = ldc;
  a.N = (int)d->N;
  a.K = (int)d->K;
  a.M = (int)M;
  a.adt = dt;
  a.ntile = (int)d->ntile;
  a.nchunk = (int)d->nchunk;
  a.nmeta = (int)d->nmeta;
  a.cpg = d->cpg > 0 ? (int)d->cpg : 1;
  a.S = pl.S;
  a.ncg = pl.ncg;
  a.ks = pl.ks;
  a.tpg = pl.tpg;
  const uint64_t ipr = (uint64_t)pl.ks * pl.cpw * d->spc * 4;
  a.ipr_magic = (uint32_t)(((1ull << 32) + ipr - 1) / ipr);
  return a;
}

int stepm_of(const sglq_dev *d) { return d->meta_mode == SGLQ_META_STEP; }

int launch_gemv(const sglq_dev *d, const GemvArgs &a, const Plan &pl, bool split, bool fast,
                unsigned gy, hipStream_t st) {
  const dim3 grid((unsigned)(pl.ncg * pl.S), gy);
  const unsigned nthr = (unsigned)(pl.ks * pl.tpg * 64);
  // activation items per thread beyond the two held by default: hold up to eight
  const int64_t items = (int64_t)a.M * pl.ks * pl.cpw * d->spc * 4;
  const int am = !fast ? 0 : items > 2 * (int64_t)nthr ? 2 : 1;
  const int stepm = d->meta_mode == SGLQ_META_STEP;
  switch (d->kind) {
    case SGLQ_KIND_U4:
      launch_kind<SGLQ_KIND_U4>(a, pl.cpw, split, d->scf16, stepm, am, pl.lds, grid, nthr, st);
      break;
    case SGLQ_KIND_U8:
      launch_kind<SGLQ_KIND_U8>(a, pl.cpw, split, d->scf16, stepm, am, pl.lds, grid, nthr, st);
      break;
    default:
      launch_kind<SGLQ_KIND_E2M1>(a, pl.cpw, split, 1, 0, am, pl.lds, grid, nthr, st);
      break;
  }
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

}  // namespace

namespace {

// k_gemv_wave over plan pl (one row per launch or per segment), gy segments
int launch_gemv_wave(const sglq_dev *d, const GemvArgs &a, const Plan &pl, bool split,
                     unsigned gy, hipStream_t st) {
  // wave-private staging: [waves][rows][IPR + 1] operands, or the slice sums
  const int64_t waves = (int64_t)pl.ks * pl.tpg;
  const int64_t rows = (split ? 2 : 1) * a.M;  // a.M = most rows of a segment when grouped
  const size_t stage = (size_t)(waves * rows * (pl.cpw * d->spc * 4 + 1) * 16);
  const size_t red = (size_t)(waves * 64 * 16);
  const size_t lds = stage > red ? stage : red;
  const dim3 grid((unsigned)(pl.ncg * pl.S), gy);
  const unsigned nthr = (unsigned)(waves * 64);
  switch (d->kind) {
    case SGLQ_KIND_U4:
      launch_wave<SGLQ_KIND_U4>(a, pl.cpw, split, d->scf16, stepm_of(d), lds, grid, nthr, st);
      break;
    case SGLQ_KIND_U8:
      launch_wave<SGLQ_KIND_U8>(a, pl.cpw, split, d->scf16, stepm_of(d), lds, grid, nthr, st);
      break;
    default:
      launch_wave<SGLQ_KIND_E2M1>(a, pl.cpw, split, 1, 0, lds, grid, nthr, st);
      break;
  }
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

}  // namespace

// SGLQ_GEMV_ROW=0 in the environment keeps one-row launches on k_gemv_wave (A/B measurement)
static bool sglq_gemv_row_off() {
  static const int off = [] {
    const char *v = getenv("SGLQ_GEMV_ROW");
    return v && v[0] == '0' ? 1 : 0;
  }();
  return off != 0;
}

int sglq_gemv(sglq_dev *d, const void *A, int dt, int64_t lda, int64_t M, const float *bias,
              float *C, int64_t ldc, hipStream_t st) {
  const bool split = dt == SGLQ_DT_F32;
  const int64_t esz = dt == SGLQ_DT_F32 ? 4 : 2;
  const bool fast = d->kident && d->K % 8 == 0 && (uintptr_t)A % 16 == 0 &&
                    (lda * esz) % 16 == 0 && M * lda < (1ll << 31);
  // two rows only while K fits one workgroup range: [11008, 4096] 11.2 -> 9.8 us (f32), 10.2 ->
  // 9.7 (bf16); with K split over workgroups ([4096, 11008]) it measured equal or slower
  const bool wave = fast && (M == 1 || (M == 2 && d->nchunk > 16 && d->nchunk <= 32));
  if (M == 1 && fast && !sglq_gemv_row_off()) {
    const int r = sglq_gemv_row(d, A, dt, bias, C, st);
    if (r != 0) return r == 1 ? 0 : -1;
  }
  const Plan pl = plan_gemv(d, M, split, false, wave);
  if (pl.S > d->gv_split) {
    sglq_log_error("qlinear: GEMV split %d exceeds its state (%d)", pl.S, d->gv_split);
    return -1;
  }
  const GemvArgs a = base_args(d, pl, A, dt, lda, M, bias, C, ldc);
  if (wave) return launch_gemv_wave(d, a, pl, split, 1, st);
  return launch_gemv(d, a, pl, split, fast, 1, st);
}

int sglq_gemv_grouped_fits(const sglq_dev *d, int64_t max_rows, int split) {
  return max_rows <= 16 && plan_gemv(d, max_rows, split, true).S == 1;
}

// the grouped launch takes the wave-staged kernel: segments of at most 4 rows with K in one
// workgroup's 8 slices, aligned identity-order rows (SwiGLU rows: f32 gate and up halves, both
// 16-byte aligned)
static bool grouped_aligned(const sglq_dev *d, bool split, const void *A, int64_t a_rows,
                            int64_t lda) {
  const int64_t esz = split ? 4 : 2;
  return d->kident && d->K % 8 == 0 && (uintptr_t)A % 16 == 0 && (lda * esz) % 16 == 0 &&
         a_rows * lda < (1ll << 31);
}
static bool grouped_wave_ok(const sglq_dev *d, int64_t max_rows, bool split, int amode,
                            const void *A, int64_t a_rows, int64_t lda, int kcols) {
  return max_rows <= 4 && grouped_aligned(d, split, A, a_rows, lda) && d->nchunk <= 32 &&
         (amode != 2 || (split && kcols % 4 == 0 && a_rows * lda + kcols < (1ll << 31)));
}
// ... and the one-token down launch also does the combine (arrival counters per tile, one K
// range per workgroup)
static bool grouped_combine_ok(const sglq_dev *d, int64_t max_rows, bool split, int amode) {
  return max_rows == 1 && amode == 2 && d->gv_cnt && plan_gemv(d, 1, split, true, true).S == 1;
}

int sglq_moe_direct_ok(const sglq_dev *g0, const sglq_dev *d0, const void *h, int h_dtype,
                       int64_t E, const void *gu, int64_t k, int64_t mi) {
  const bool split1 = h_dtype == SGLQ_DT_F32;
  return sglq_gemv_grouped_fits(g0, 1, split1) && sglq_gemv_grouped_fits(d0, 1, 1) &&
         grouped_wave_ok(g0, 1, split1, 1, h, 1, E, 0) &&
         grouped_wave_ok(d0, 1, true, 2, gu, k, 2 * mi, (int)mi) &&
         grouped_combine_ok(d0, 1, true, 2);
}

int sglq_gemv_grouped(const sglq_dev *d, const sglq_group *grp, int64_t max_rows,
                      int64_t max_segs, const void *A, int dt, int64_t a_rows, int64_t lda,
                      int amode, const int32_t *rowmap, int kcols, float *C, int64_t ldc,
                      hipStream_t st, const sglq_combine *cmb) {
  const bool split = dt == SGLQ_DT_F32;
  const Plan pl = plan_gemv(d, max_rows, split, true);
  if (pl.S != 1 || max_rows > 16) {
    sglq_log_error("qlinear: grouped GEMV needs one K range per workgroup (rows %lld)",
                   (long long)max_rows);
    return -1;
  }
  GemvArgs a = base_args(d, pl, A, dt, lda, max_rows, nullptr, C, ldc);
  a.segs = (const int4 *)grp->segs;
  a.nseg = grp->nseg;
  a.codes_e = (const u32x4_t *const *)grp->codes;
  a.meta_e = grp->meta;
  a.rowmap = rowmap;
  a.amode = amode;
  a.kcols = kcols;
  // segments of at most 4 rows (decode of 1-4 tokens): the wave-staged kernel.  DeepSeek MoE
  // decode (64 experts, top-6): T = 1 23.2 -> 21.7 us, T = 4 51.4 -> 43.5
  if (grouped_wave_ok(d, max_rows, split, amode, A, a_rows, lda, kcols)) {
    const Plan pw = plan_gemv(d, 1, split, true, true);  // 4-chunk slices
    GemvArgs aw = a;
    aw.S = pw.S;
    aw.ncg = pw.ncg;
    aw.ks = pw.ks;
    aw.tpg = pw.tpg;
    if (grp->ids) {
      aw.ids = grp->ids;
      aw.nid = grp->nid;
      aw.nexp = grp->nexp;
    }
    if (cmb && grouped_combine_ok(d, max_rows, split, amode)) {
      aw.cpos = cmb->pos;
      aw.cw = cmb->wts;
      aw.cout = cmb->out;
      aw.ck = cmb->k;
      *cmb->done = 1;
    } else if (grp->ids && amode == 2) {
      sglq_log_error("qmoe: one-token segments without the fused combine");
      return -1;
    }
    return launch_gemv_wave(d, aw, pw, split, (unsigned)max_segs, st);
  }
  if (grp->ids) {
    sglq_log_error("qmoe: one-token segments need the wave-staged grouped GEMV");
    return -1;
  }
  return launch_gemv(d, a, pl, split, amode != 2 && grouped_aligned(d, split, A, a_rows, lda),
                     (unsigned)max_segs, st);
}

// C = A W^T (+ bias): decode GEMV up to 16 rows (and 17-32 rows as two GEMVs), prefill GEMM
// beyond.  ws == nullptr: the GEMM uses the handle's workspace (grown on first use at a size);
// otherwise ws (ws_bytes, 256-byte aligned) is the GEMM workspace and nothing is allocated.
int sglq_forward_ws(sglq_dev *d, const void *A, int dt, int64_t M, const float *bias, float *C,
                    void *stream, void *ws, size_t ws_bytes) {
  hipStream_t st = (hipStream_t)stream;
  const int64_t esz = dt == SGLQ_DT_F32 ? 4 : 2;
  SGLQ_HIP(hipSetDevice(d->dev));
  if (d->N > INT32_MAX || d->K > INT32_MAX / 2 || d->ntile * 16 * d->nmeta > INT32_MAX * 4LL) {
    sglq_log_error("qlinear: N=%lld K=%lld beyond the GEMV's 32-bit indexing", (long long)d->N,
                   (long long)d->K);
    return -1;
  }
  // 17-32 rows (f32) or 17-24 (16-bit activations): the decode GEMV on rows 0-15, then on the
  // rest, beats the prefill GEMM, whose smallest tiling costs about what M = 64 does
  // ([11008, 4096] f32 at M = 17: 48.6 us in the GEMM against about 27 us in two GEMVs)
  if (M > 16 && M <= (dt == SGLQ_DT_F32 ? 32 : 24)) {
    if (sglq_gemv(d, A, dt, d->K, 16, bias, C, d->N, st) != 0) return -1;
    return sglq_gemv(d, (const char *)A + 16 * d->K * esz, dt, d->K, M - 16, bias,
                     C + 16 * d->N, d->N, st);
  }
  if (M > 16) {
    if (!ws) return sglq_gemm(d, A, dt, d->K, M, bias, C, d->N, st);
    const size_t need = sglq_gemm_ws_bytes(d, dt, M);
    if (need > ws_bytes) {
      sglq_log_error("qlinear: %lld rows need %zu bytes of workspace, %zu available",
                     (long long)M, need, ws_bytes);
      return -1;
    }
    return sglq_gemm_ws(d, A, dt, d->K, M, bias, C, d->N, ws, st);
  }
  return sglq_gemv(d, A, dt, d->K, M, bias, C, d->N, st);
fail:
  return -1;
}

extern "C" int sglq_forward(sglq_dev *d, const void *A, int dt, int64_t M, const float *bias,
                            float *C, void *stream) {
  return sglq_forward_ws(d, A, dt, M, bias, C, stream, nullptr, 0);
}

