// moe.hip — routed-expert FFN over device-resident quantized experts (the expert loop and
// weighted combine of reference src/deepseek.c:655-677, gate/up fused as in its stacked
// branch :660-664; routing itself is an input).
//
// Launches, all on the caller's stream, no host synchronisation:
//   k_moe_route   one workgroup: counts (token, slot) pairs per expert, gives each pair a row
//                 among its expert's rows (experts in index order), and writes
//                 the row-block table of the grouped GEMMs (blocks of <= 64 rows of one expert)
//   prefill:  prep (gather) A operands of the expert-sorted rows of h
//             grouped GEMM  gu = h_rows * Wgu[e]^T, each row block with its expert's weights
//             prep (SwiGLU) A operands of silu(gu[:, :mi]) * gu[:, mi:]
//             grouped GEMM  o = a * Wdn[e]^T
//             (weights that take the LDS-dequant GEMM: the gate/up GEMM writes silu(g) * u
//             and its row maxima itself, and the down prep only converts)
//   decode (T <= 4): the same two products as grouped decode GEMVs that gather the token rows
//             and form the SwiGLU rows while staging their activations
//   k_moe_combine out[t] = sum_j w[t,j] * o[row of (t,j)], slots added in order j = 0..k-1
#include <string.h>

#include <algorithm>

#include "sglq_dev.hpp"

namespace {

constexpr int kMaxExperts = 256;

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}

// One workgroup.  Each pair p = t * k + j with a valid expert gets a row among that expert's
// rows (experts in index order); rowmap[row] = token, pos[p] = row.  Which of its expert's rows
// a pair gets depends on the order of the LDS atomics, but no result does: each row's product
// depends only on its token and its expert, and the combine reads rows through pos in slot
// order.  Row blocks hold at most bm rows of one expert: segs[b] = {expert, first row, rows, 0}.
__global__ __launch_bounds__(1024) void k_moe_route(const int32_t *__restrict__ ids, int P,
                                                    int k, int n_exp, int bm,
                                                    int32_t *__restrict__ rowmap,
                                                    int32_t *__restrict__ pos,
                                                    int *__restrict__ segs,
                                                    int *__restrict__ nseg,
                                                    int *__restrict__ rowmax) {
  __shared__ int run[kMaxExperts];  // rows of each expert, then its next free row
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int e = tid; e < kMaxExperts; e += 1024) run[e] = 0;
  for (int r = tid; r < P; r += 1024) {
    rowmap[r] = -1;  // rows past the routed pairs: zero rows
    if (rowmax) rowmax[r] = 0;  // for the fused SwiGLU's row maxima
  }
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int e = ids[p];
    if (e >= 0 && e < n_exp) atomicAdd(&run[e], 1);
  }
  __syncthreads();
  if (w == 0) {  // exclusive scans of rows and of row blocks over the experts, 4 per lane
    int c[4], rs = 0, bs = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      c[q] = run[lane * 4 + q];
      rs += c[q];
      bs += (c[q] + bm - 1) / bm;
    }
    const int ri = wave_incl_scan(rs, lane), bi = wave_incl_scan(bs, lane);
    int off = ri - rs, nb = bi - bs;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int e = lane * 4 + q;
      for (int r = 0; r < c[q]; r += bm) {
        segs[nb * 4 + 0] = e;
        segs[nb * 4 + 1] = off + r;
        segs[nb * 4 + 2] = min(bm, c[q] - r);
        segs[nb * 4 + 3] = 0;
        nb++;
      }
      run[e] = off;
      off += c[q];
    }
    if (lane == 63) *nseg = bi;
  }
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int e = ids[p];
    if (e >= 0 && e < n_exp) {
      const int dst = atomicAdd(&run[e], 1);
      rowmap[dst] = p / k;
      pos[p] = dst;
    } else {
      pos[p] = -1;
    }
  }
}

// out[t][c] = ((0 + w0 o0) + w1 o1) + ... in slot order, products and sums rounded separately
// as the reference's orow[i] += w * o[i] (reference src/deepseek.c:675-676)
// Up to 8 slots at a time: their rows and weights, then their products, are loaded before any
// is added, so a token's combine costs two dependent load latencies rather than two per slot
// (bench MoE lines: 4-token decode 45.4 -> 43.6 us, 512-token prefill 194.6 -> 191.1 us).
__global__ void k_moe_combine(const float *__restrict__ o, int64_t ldo,
                              const int32_t *__restrict__ pos, const float *__restrict__ wts,
                              int k, int E, float *__restrict__ out) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= E) return;
  float acc = 0.f;
  for (int j0 = 0; j0 < k; j0 += 8) {
    int r[8];
    float wv[8], v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      r[u] = j0 + u < k ? pos[t * k + j0 + u] : -1;
      wv[u] = j0 + u < k ? wts[t * k + j0 + u] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = r[u] >= 0 ? o[(int64_t)r[u] * ldo + c] : 0.f;
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (r[u] >= 0) acc = __fadd_rn(acc, __fmul_rn(wv[u], v[u]));
  }
  out[(int64_t)t * E + c] = acc;
}

bool same_format(const sglq_dev *a, const sglq_dev *b) {
  return a->N == b->N && a->K == b->K && a->kind == b->kind && a->scf16 == b->scf16 &&
         a->meta_mode == b->meta_mode && a->nchunk == b->nchunk && a->nmeta == b->nmeta &&
         a->cpg == b->cpg && a->kident == b->kident && a->dev == b->dev;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

extern "C" int sglq_moe_forward(sglq_dev *const *gate_up, sglq_dev *const *down, int n_exp,
                                const void *h, int h_dtype, int64_t T, const int32_t *topk_ids,
                                const float *topk_w, int k, float *out, void *stream) {
  hipStream_t st = (hipStream_t)stream;
  sglq_dev *g0 = gate_up[0], *d0 = down[0];
  if (n_exp > kMaxExperts) {
    sglq_log_error("qmoe: %d experts (at most %d)", n_exp, kMaxExperts);
    return -1;
  }
  if (g0->N % 2 != 0 || d0->N != g0->K || d0->K != g0->N / 2) {
    sglq_log_error("qmoe: gate_up [%lld,%lld] / down [%lld,%lld] do not form an expert FFN",
                   (long long)g0->N, (long long)g0->K, (long long)d0->N, (long long)d0->K);
    return -1;
  }
  for (int e = 0; e < n_exp; e++) {
    if (!same_format(gate_up[e], g0) || !same_format(down[e], d0)) {
      sglq_log_error("qmoe: expert %d differs in shape or format from expert 0", e);
      return -1;
    }
  }
  if (!g0->kident || !d0->kident) {
    sglq_log_error("qmoe: act-order (g_idx) experts are not supported");
    return -1;
  }
  if (T == 0) return 0;
  {
    const int64_t E = g0->K, mi = d0->K, P = T * k;
    // row blocks: at most 64 rows of one expert for the grouped GEMMs (at most gblk blocks,
    // the GEMMs' grid); at most T rows for the decode GEMVs, whose staging holds T rows (a token
    // that lists an expert twice gives it more rows than there are tokens), at most one block
    // per pair.  maxblk = the table's capacity.
    const int64_t gblk = (P + SGLQ_MOE_BM - 1) / SGLQ_MOE_BM + n_exp;
    const int64_t maxblk = std::max<int64_t>(gblk, P);
    const int64_t Mpad = (P + SGLQ_GEMM_BM - 1) / SGLQ_GEMM_BM * SGLQ_GEMM_BM + SGLQ_GEMM_BM;
    const int split1 = h_dtype == SGLQ_DT_F32;
    // workspace (kept in expert 0's gate_up handle)
    size_t off = 0;
    const size_t o_ptr = off; off = align256(off + (size_t)6 * n_exp * sizeof(void *));
    const size_t o_rowmap = off; off = align256(off + (size_t)Mpad * 4);
    const size_t o_pos = off; off = align256(off + (size_t)P * 4);
    const size_t o_segs = off; off = align256(off + (size_t)maxblk * 16);
    const size_t o_nseg = off; off = align256(off + 4);
    const size_t o_aop1 = off; off = align256(off + sglq_aop_bytes(g0, Mpad, split1));
    const size_t o_rexp1 = off; off = align256(off + (size_t)Mpad * 4);
    const size_t o_gu = off; off = align256(off + (size_t)Mpad * 2 * mi * 4);
    const size_t o_aop2 = off; off = align256(off + sglq_aop_bytes(d0, Mpad, 1));
    const size_t o_rexp2 = off; off = align256(off + (size_t)Mpad * 4);
    const size_t o_rmax = off; off = align256(off + (size_t)Mpad * 4);
    const size_t o_o = off; off = align256(off + (size_t)Mpad * E * 4);
    if (sglq_ws_reserve(g0, off) != 0) return -1;
    char *ws = (char *)g0->ws;
    // expert pointer tables: uploaded when they differ from the last upload
    const void **hp = (const void **)malloc((size_t)6 * n_exp * sizeof(void *));
    if (!hp) return -1;
    for (int e = 0; e < n_exp; e++) {
      hp[0 * n_exp + e] = gate_up[e]->codes;
      hp[1 * n_exp + e] = gate_up[e]->meta;
      hp[2 * n_exp + e] = gate_up[e]->colexp;
      hp[3 * n_exp + e] = down[e]->codes;
      hp[4 * n_exp + e] = down[e]->meta;
      hp[5 * n_exp + e] = down[e]->colexp;
    }
    const size_t tbl = (size_t)6 * n_exp * sizeof(void *);
    if (g0->moe_tbl_bytes != tbl || !g0->moe_tbl || memcmp(g0->moe_tbl, hp, tbl) != 0 ||
        g0->moe_tbl_ws != g0->ws) {
      if (hipMemcpy(ws + o_ptr, hp, tbl, hipMemcpyHostToDevice) != hipSuccess) {
        sglq_log_error("qmoe: uploading the expert table failed");
        free(hp);
        return -1;
      }
      free(g0->moe_tbl);
      g0->moe_tbl = hp;
      g0->moe_tbl_bytes = tbl;
      g0->moe_tbl_ws = g0->ws;
    } else {
      free(hp);
    }
    const void *const *dp = (const void *const *)(ws + o_ptr);
    int32_t *rowmap = (int32_t *)(ws + o_rowmap);
    int32_t *pos = (int32_t *)(ws + o_pos);
    int *segs = (int *)(ws + o_segs);
    int *nseg = (int *)(ws + o_nseg);
    float *gu = (float *)(ws + o_gu);
    float *o = (float *)(ws + o_o);
    // prefill of LDS-kernel experts: SwiGLU fused into the gate/up GEMM's epilogue
    const bool decode =
        T <= 4 && sglq_gemv_grouped_fits(g0, T, split1) && sglq_gemv_grouped_fits(d0, T, 1);
    const bool fuse = !decode && sglq_gemm_lds_direct(g0) && mi % 16 == 0;
    int *rowmax = fuse ? (int *)(ws + o_rmax) : nullptr;
    // one-token decode whose grouped GEMVs read the routing directly (slot j is its own
    // one-row segment): no routing kernel, on the one-row kernel where the weights allow, else
    // on the grouped wave-staged kernel.  DeepSeek MoE decode T = 1: 20.0 -> 15.5 us with the
    // fast silu.  Four tokens as 24 one-row pairs (experts two tokens share read twice)
    // measured slower than routed segments on the wave-staged kernel (46.7 against 39.8 us).
    const bool rowdirect = decode && T == 1 &&
                           sglq_gemv_row_grouped_ok(g0, 1, h, h_dtype, E, 0) &&
                           sglq_gemv_row_grouped_ok(d0, 2, gu, SGLQ_DT_F32, 2 * mi, (int)mi);
    const bool direct =
        rowdirect || (decode && T == 1 && sglq_moe_direct_ok(g0, d0, h, h_dtype, E, gu, k, mi));
    if (!direct) {
      k_moe_route<<<1, 1024, 0, st>>>(topk_ids, (int)P, k, n_exp, decode ? (int)T : SGLQ_MOE_BM,
                                      rowmap, pos, segs, nseg, rowmax);
      SGLQ_HIP(hipGetLastError());
    }
    sglq_group g1 = {dp, dp + n_exp, (const uint8_t *const *)(dp + 2 * n_exp), segs, nseg};
    sglq_group g2 = {dp + 3 * n_exp, dp + 4 * n_exp, (const uint8_t *const *)(dp + 5 * n_exp),
                     segs, nseg};
    if (direct) {
      g1.ids = g2.ids = topk_ids;
      g1.nid = g2.nid = (int)k;
      g1.nexp = g2.nexp = n_exp;
    }
    // decode-sized batches (every expert has at most T <= 4 rows): grouped GEMVs that read the
    // token rows and the SwiGLU rows directly; otherwise operand prep + grouped GEMMs
    int combined = 0;
    if (decode) {
      const int64_t max_segs = P;  // blocks of at most T rows, at least one row each
      // one token read straight from its routing: the one-row kernel where the weights allow
      // (f16 group scales, one group per chunk), else the grouped wave-staged kernel
      int r1 = 0, r2 = 0;
      if (rowdirect) {
        r1 = sglq_gemv_row_grouped(g0, g1.codes, g1.meta, topk_ids, (int)P, (int)k, n_exp, 1,
                                   h, h_dtype, E, 0, gu, 2 * mi, nullptr, nullptr, 0, st);
        // down: one workgroup per output tile holding every slot (combine through LDS), else
        // one per (slot, tile) with the combine done by the last slot of each tile
        r2 = r1 < 0 ? -1
                    : sglq_gemv_row_grouped(d0, g2.codes, g2.meta, topk_ids, (int)P, (int)k,
                                            n_exp, 3, gu, SGLQ_DT_F32, 2 * mi, (int)mi, o, E,
                                            topk_w, out, E, st);
        if (r2 == 0)
          r2 = sglq_gemv_row_grouped(d0, g2.codes, g2.meta, topk_ids, (int)P, (int)k, n_exp, 2,
                                     gu, SGLQ_DT_F32, 2 * mi, (int)mi, o, E, topk_w, out, E, st);
        if (r1 != 1 || r2 != 1) {
          sglq_log_error("qmoe: grouped one-row decode launch failed");
          return -1;
        }
        combined = 1;
      }
      if (!r1 && sglq_gemv_grouped(g0, &g1, T, max_segs, h, h_dtype, T, E, 1, rowmap, 0, gu,
                                   2 * mi, st) != 0)
        return -1;
      // one token: the down launch also does the combine when it can
      const sglq_combine cb = {pos, topk_w, k, out, &combined};
      if (!r2 && sglq_gemv_grouped(d0, &g2, T, max_segs, gu, SGLQ_DT_F32, P, 2 * mi, 2, nullptr,
                                   (int)mi, o, E, st, T == 1 ? &cb : nullptr) != 0)
        return -1;
    } else if (fuse) {
      // act[r] = silu(gate) * up of row r, [P, mi] f32, written by the gate/up GEMM together
      // with its row maxima; the down prep derives the row exponents from those
      g1.swiglu = (int)mi;
      g1.rowmax = rowmax;
      if (sglq_prep_a(g0, 1, h, h_dtype, E, P, Mpad, rowmap, 0, split1, ws + o_aop1,
                      (int *)(ws + o_rexp1), st) != 0)
        return -1;
      if (sglq_gemm_run(g0, &g1, ws + o_aop1, (const int *)(ws + o_rexp1), P, Mpad, gblk,
                        split1, nullptr, gu, mi, nullptr, st) != 0)
        return -1;
      // the down operands silu(g) * u (f32) as one f16 piece under the row's power of two (a
      // 2^-12 relative rounding, as the prescaled weights'): half the MFMAs and operand bytes
      // of the hi + lo split.  Config 5 prefill 199 -> 174 us; max rel error against the
      // reference 3.2e-4 -> 3.9e-4 (at most 5.2e-4 over the MoE tests; bar 1e-3).  Below 256
      // intermediate columns the down products are too few for that rounding to average out
      // (mi = 16, 8-bit experts: 1.06e-3 on one piece, 7.0e-4 on hi + lo), so they keep hi + lo.
      // SGLQ_MOE_DOWN_SPLIT=1 / 0 forces either.
      static int dsplit_env = -2;
      if (dsplit_env == -2) {
        const char *e = getenv("SGLQ_MOE_DOWN_SPLIT");
        dsplit_env = e ? atoi(e) : -1;
      }
      const int dsplit = dsplit_env >= 0 ? dsplit_env : mi < 256 ? 1 : 0;
      if (sglq_prep_a(d0, 0, gu, SGLQ_DT_F32, mi, P, Mpad, nullptr, 0, dsplit, ws + o_aop2,
                      (int *)(ws + o_rexp2), st, rowmax) != 0)
        return -1;
      if (sglq_gemm_run(d0, &g2, ws + o_aop2, (const int *)(ws + o_rexp2), P, Mpad, gblk,
                        dsplit, nullptr, o, E, nullptr, st) != 0)
        return -1;
    } else {
      // rows of Mpad beyond P: rowmap entries are never read (prep zeroes rows >= M)
      if (sglq_prep_a(g0, 1, h, h_dtype, E, P, Mpad, rowmap, 0, split1, ws + o_aop1,
                      (int *)(ws + o_rexp1), st) != 0)
        return -1;
      if (sglq_gemm_run(g0, &g1, ws + o_aop1, (const int *)(ws + o_rexp1), P, Mpad, gblk,
                        split1, nullptr, gu, 2 * mi, nullptr, st) != 0)
        return -1;
      if (sglq_prep_a(d0, 2, gu, SGLQ_DT_F32, 2 * mi, P, Mpad, nullptr, (int)mi, 1,
                      ws + o_aop2, (int *)(ws + o_rexp2), st) != 0)
        return -1;
      if (sglq_gemm_run(d0, &g2, ws + o_aop2, (const int *)(ws + o_rexp2), P, Mpad, gblk, 1,
                        nullptr, o, E, nullptr, st) != 0)
        return -1;
    }
    if (!combined) {
      dim3 grid((unsigned)((E + 255) / 256), (unsigned)T);
      k_moe_combine<<<grid, 256, 0, st>>>(o, E, pos, topk_w, k, (int)E, out);
      SGLQ_HIP(hipGetLastError());
    }
  }
  return 0;
fail:
  return -1;
}
