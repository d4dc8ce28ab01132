// route.hip — MoE routing and shared experts on the device, around the routed-expert FFN of
// moe.hip (reference src/deepseek.c:589-633 routing, :679-687 shared experts).
//
//   k_router_logits  logits[t][e] = h_t . router_w[e], one workgroup per token: the token row
//                    is staged once in LDS as f32 and each wave takes a quarter of the experts
//                    (128-bit loads of router_w, fp32 partial sums, wave reduction)
//   k_moe_gate       one wave per token: scores (sigmoid, or the softmax with its double sum
//                    taken in expert order), selection scores with the correction bias,
//                    group-limited greedy group choice, top-k as k wave argmaxes (strictly
//                    greater wins: ties go to the lower index, nothing at or below -1e30 is
//                    chosen), weights from the uncorrected scores, normalised in slot order
//   SwiGLU MLP       gate/up forward(s), k_swiglu, down forward: the shared experts (added
//                    after the routed sum, as the reference adds them) and the dense MLP block
//                    (reference src/llama.c:1162-1176)
#include <string.h>

#include "sglq_dev.hpp"

namespace {

constexpr int kMaxRouteExperts = 256;  // 4 per lane of the gate wave
constexpr int kMaxGroups = 64;

__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ w, int ne,
                                                       const void *__restrict__ h, int hdt,
                                                       int64_t E, float *__restrict__ logits) {
  extern __shared__ float s_h[];
  const int t = blockIdx.x, tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  const int64_t rb = (int64_t)t * E;
  for (int64_t i = tid; i < E; i += 256) {
    float x;
    if (hdt == SGLQ_DT_F32) {
      x = ((const float *)h)[rb + i];
    } else {
      const uint32_t b = ((const uint16_t *)h)[rb + i];
      x = hdt == SGLQ_DT_BF16 ? __uint_as_float(b << 16)
                              : (float)__builtin_bit_cast(_Float16, (uint16_t)b);
    }
    s_h[i] = x;
  }
  __syncthreads();
  const bool vec = E % 4 == 0 && ((uintptr_t)w & 15) == 0;
  for (int e = wv; e < ne; e += 4) {
    const float *wr = w + (int64_t)e * E;
    float acc = 0.f;
    if (vec) {
      for (int64_t i = (int64_t)lane * 4; i < E; i += 256) {
        const float4 x = *(const float4 *)(wr + i);
        acc = fmaf(x.x, s_h[i], acc);
        acc = fmaf(x.y, s_h[i + 1], acc);
        acc = fmaf(x.z, s_h[i + 2], acc);
        acc = fmaf(x.w, s_h[i + 3], acc);
      }
    } else {
      for (int64_t i = lane; i < E; i += 64) acc = fmaf(wr[i], s_h[i], acc);
    }
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) logits[(int64_t)t * ne + e] = acc;
  }
}

// e^x rounded once to float from a double-precision exp: the correctly rounded value except
// within about 2^-29 of a rounding midpoint.  The reference's host expf (glibc) is correctly
// rounded for all but a sliver of inputs, so the scores, and the experts chosen at near-ties,
// match it far more often than a single-precision device expf (1 ulp) does.
__device__ __forceinline__ float expf_cr(float x) { return (float)exp((double)x); }

__global__ __launch_bounds__(64) void k_moe_gate(const float *__restrict__ logits, int ne,
                                                 const float *__restrict__ bias, int sigmoid,
                                                 int ng, int tg, int k, int norm, float scale,
                                                 int32_t *__restrict__ ids,
                                                 float *__restrict__ wts) {
  __shared__ float s_s[kMaxRouteExperts], s_ch[kMaxRouteExperts], s_gs[kMaxGroups];
  __shared__ int s_keep[kMaxGroups];
  __shared__ float s_inv;
  const int t = blockIdx.x, lane = threadIdx.x;
  const float *lg = logits + (int64_t)t * ne;
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int i = lane + 64 * q;
    v[q] = i < ne ? lg[i] : 0.f;
  }
  if (sigmoid) {
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] = 1.0f / (1.0f + expf_cr(-v[q]));
  } else {
    // softmax as reference src/ops.c:220-231: max, expf(x - max), double sum in index order,
    // one float reciprocal
    float mx = lg[0];
#pragma unroll
    for (int q = 0; q < 4; q++)
      if (lane + 64 * q < ne) mx = fmaxf(mx, v[q]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
#pragma unroll
    for (int q = 0; q < 4; q++) {
      v[q] = expf_cr(v[q] - mx);
      if (lane + 64 * q < ne) s_s[lane + 64 * q] = v[q];
    }
    __syncthreads();
    if (lane == 0) {
      double sum = 0;
      for (int i = 0; i < ne; i++) sum += s_s[i];
      s_inv = (float)(1.0 / sum);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; q++) v[q] *= s_inv;
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int i = lane + 64 * q;
    if (i < ne) {
      s_s[i] = v[q];
      s_ch[i] = v[q] + (bias ? bias[i] : 0.0f);
    }
  }
  __syncthreads();
  if (ng > 1) {  // group-limited greedy (reference src/deepseek.c:601-628)
    const int epg = ne / ng;
    if (lane < ng) {
      float t1 = -1e30f, t2 = -1e30f;
      for (int i = 0; i < epg; i++) {
        const float x = s_ch[lane * epg + i];
        if (x > t1) {
          t2 = t1;
          t1 = x;
        } else if (x > t2) {
          t2 = x;
        }
      }
      s_gs[lane] = epg > 1 ? t1 + t2 : t1;
      s_keep[lane] = 0;
    }
    __syncthreads();
    if (lane == 0) {
      for (int g = 0; g < tg; g++) {
        int best = -1;
        float bv = -1e30f;
        for (int i = 0; i < ng; i++)
          if (!s_keep[i] && s_gs[i] > bv) {
            bv = s_gs[i];
            best = i;
          }
        if (best >= 0) s_keep[best] = 1;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int i = lane + 64 * q;
      if (i < ne && !s_keep[i / epg]) s_ch[i] = -1e30f;
    }
    __syncthreads();
  }
  float c[4];
  bool used[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int i = lane + 64 * q;
    c[q] = i < ne ? s_ch[i] : -1e30f;
    used[q] = i >= ne;
  }
  int32_t *sel = ids + (int64_t)t * k;
  float *sw = wts + (int64_t)t * k;
  for (int j = 0; j < k; j++) {
    float bv = -1e30f;
    int bi = -1;
#pragma unroll
    for (int q = 0; q < 4; q++)  // ascending index within the lane: the first maximum wins
      if (!used[q] && c[q] > bv) {
        bv = c[q];
        bi = lane + 64 * q;
      }
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const int oi = __shfl_xor(bi, o);
      if (ov > bv || (ov == bv && oi >= 0 && (bi < 0 || oi < bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi >= 0 && (bi & 63) == lane) used[bi >> 6] = true;
    if (lane == 0) {
      sel[j] = bi;
      sw[j] = bi >= 0 ? s_s[bi] : 0.0f;
    }
  }
  if (lane == 0) {
    if (k > 1 && norm) {
      double tot = 0;
      for (int j = 0; j < k; j++) tot += sw[j];
      tot += 1e-20;
      if (tot != 0)
        for (int j = 0; j < k; j++) sw[j] = (float)(sw[j] / tot);
    }
    for (int j = 0; j < k; j++) sw[j] *= scale;
  }
}

// act[t][c] = silu(g) * u with silu(g) = g / (1 + e^-g) (sglq_silu) rounded first, as the reference's
// sgl_silu_inplace followed by the product (reference src/ops.c:288-293, src/llama.c:1172-1173)
__global__ void k_swiglu(const float *__restrict__ g, int64_t ldg, const float *__restrict__ u,
                         int64_t ldu, int64_t T, int64_t I, float *__restrict__ act) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * I) return;
  const int64_t t = i / I, c = i - t * I;
  const float x = g[t * ldg + c];
  const float s = sglq_silu(x);
  act[i] = s * u[t * ldu + c];
}

__global__ void k_add_into(float *__restrict__ out, const float *__restrict__ o, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] += o[i];
}

}  // namespace

extern "C" int sglq_moe_router_logits(const float *router_w, int ne, const void *h, int h_dtype,
                                      int64_t T, int64_t E, float *logits, void *stream) {
  if (ne <= 0 || E <= 0 || E > 16384) {
    sglq_log_error("qmoe router: %d experts x %lld (hidden at most 16384)", ne, (long long)E);
    return -1;
  }
  if (T == 0) return 0;
  k_router_logits<<<(unsigned)T, 256, (size_t)E * sizeof(float), (hipStream_t)stream>>>(
      router_w, ne, h, h_dtype, E, logits);
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

extern "C" int sglq_moe_route(const float *logits, int64_t T, int ne, const float *bias,
                              int sigmoid, int n_group, int topk_group, int k, int norm,
                              float scale, int32_t *ids, float *wts, void *stream) {
  if (ne <= 0 || ne > kMaxRouteExperts || k <= 0 || k > ne) {
    sglq_log_error("qmoe route: %d experts, top-%d (at most %d experts)", ne, k,
                   kMaxRouteExperts);
    return -1;
  }
  if (n_group > 1 && (n_group > kMaxGroups || ne % n_group != 0 || topk_group <= 0 ||
                      topk_group > n_group)) {
    sglq_log_error("qmoe route: %d experts in %d groups, %d kept (groups must divide the "
                   "experts, at most %d)", ne, n_group, topk_group, kMaxGroups);
    return -1;
  }
  if (T == 0) return 0;
  k_moe_gate<<<(unsigned)T, 64, 0, (hipStream_t)stream>>>(logits, ne, bias, sigmoid, n_group,
                                                          topk_group, k, norm, scale, ids, wts);
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

// SwiGLU MLP of T rows: down(silu(h gate^T) * (h up^T)).  up == nullptr: gate is the fused
// [2 I, K] weight (gate rows, then up rows).  accumulate: out += MLP, else out = MLP.  The
// intermediate buffers live in gate's aux buffer.
static int swiglu_mlp(sglq_dev *gate, sglq_dev *up, sglq_dev *down, const void *h, int h_dtype,
                      int64_t T, float *out, bool accumulate, hipStream_t st) {
  const int64_t I = down->K, E = down->N;
  const bool fused = up == nullptr;
  if ((fused && gate->N != 2 * I) || (!fused && (gate->N != I || up->N != I || up->K != gate->K))
      || gate->K != E) {
    sglq_log_error("SwiGLU MLP: gate [%lld,%lld]%s / down [%lld,%lld] do not fit",
                   (long long)gate->N, (long long)gate->K, fused ? " (fused gate/up)" : "",
                   (long long)down->N, (long long)down->K);
    return -1;
  }
  if (T == 0) return 0;
  const size_t o_act = ((size_t)T * 2 * I * 4 + 255) / 256 * 256;
  const size_t o_o = o_act + ((size_t)T * I * 4 + 255) / 256 * 256;
  if (sglq_aux_reserve(gate, o_o + (accumulate ? (size_t)T * E * 4 : 0)) != 0) return -1;
  float *g = (float *)gate->aux;
  float *u = fused ? g + I : g + T * I;
  float *act = (float *)((char *)gate->aux + o_act);
  float *o = accumulate ? (float *)((char *)gate->aux + o_o) : out;
  if (sglq_forward(gate, h, h_dtype, T, nullptr, g, st) != 0) return -1;
  if (!fused && sglq_forward(up, h, h_dtype, T, nullptr, u, st) != 0) return -1;
  k_swiglu<<<sglq_blocks(T * I, 256), 256, 0, st>>>(g, fused ? 2 * I : I, u, fused ? 2 * I : I,
                                                    T, I, act);
  SGLQ_HIP(hipGetLastError());
  if (sglq_forward(down, act, SGLQ_DT_F32, T, nullptr, o, st) != 0) return -1;
  if (accumulate) {
    k_add_into<<<sglq_blocks(T * E, 256), 256, 0, st>>>(out, o, T * E);
    SGLQ_HIP(hipGetLastError());
  }
  return 0;
fail:
  return -1;
}

extern "C" int sglq_moe_shared(sglq_dev *gu, sglq_dev *dn, const void *h, int h_dtype,
                               int64_t T, float *out, void *stream) {
  return swiglu_mlp(gu, nullptr, dn, h, h_dtype, T, out, true, (hipStream_t)stream);
}

extern "C" int sglq_mlp_forward(sglq_dev *gate, sglq_dev *up, sglq_dev *down, const void *h,
                                int h_dtype, int64_t T, float *out, void *stream) {
  return swiglu_mlp(gate, up, down, h, h_dtype, T, out, false, (hipStream_t)stream);
}
