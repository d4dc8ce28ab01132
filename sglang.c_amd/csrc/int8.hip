// int8.hip — per-row symmetric int8 quantization, int8 row dequant and the f32 NT matmul
// behind the reference API entry points sgl_quant_rows_i8 / sgl_dequant_row_i8 /
// sgl_matmul_nt (reference src/quant.c:13-42, src/ops.c:243-279), computed on the GPU.
#include "sglq_dev.hpp"

// One workgroup per row.  Arithmetic is the reference's, step for step, without contraction:
// scale = maxabs / 127, inv = 1 / scale, v = trunc(x * inv +- 0.5) clamped to [-127, 127]
// (reference src/quant.c:13-32); an all-zero row gives scale 0 and zero codes.
__global__ __launch_bounds__(256) void k_quant_rows_i8(const float *__restrict__ x,
                                                       int8_t *__restrict__ q,
                                                       float *__restrict__ scales, int64_t dim) {
#pragma clang fp contract(off)
  const int64_t r = blockIdx.x;
  const float *row = x + r * dim;
  __shared__ float red[256];
  float m = 0.f;
  for (int64_t i = threadIdx.x; i < dim; i += 256) {
    const float a = row[i] < 0 ? -row[i] : row[i];
    if (a > m) m = a;
  }
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s && red[threadIdx.x + s] > red[threadIdx.x])
      red[threadIdx.x] = red[threadIdx.x + s];
    __syncthreads();
  }
  const float maxabs = red[0];
  int8_t *qr = q + r * dim;
  if (!(maxabs > 0)) {
    for (int64_t i = threadIdx.x; i < dim; i += 256) qr[i] = 0;
    if (threadIdx.x == 0) scales[r] = 0.f;
    return;
  }
  const float scale = maxabs / 127.0f;
  const float inv = 1.0f / scale;
  for (int64_t i = threadIdx.x; i < dim; i += 256) {
    const float xv = row[i];
    const float p = xv * inv;
    const float h = xv >= 0 ? 0.5f : -0.5f;
    const float r = p + h;
    // float -> int as the reference's x86 build converts (cvttss2si): out of range or NaN
    // gives INT_MIN, e.g. a denormal row whose 1/scale overflows to inf
    int v = (r >= -2147483648.0f && r < 2147483648.0f) ? (int)r : INT32_MIN;
    v = v > 127 ? 127 : (v < -127 ? -127 : v);
    qr[i] = (int8_t)v;
  }
  if (threadIdx.x == 0) scales[r] = scale;
}

__global__ void k_dequant_row_i8(const int8_t *__restrict__ q, float scale, float *__restrict__ o,
                                 int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) o[i] = (float)q[i] * scale;
}

// f32 C[M,N] = A[M,K] W[N,K]^T + bias: one wave per (n, 8-row block), lanes stride K with fp32
// fused multiply-add, combined across lanes in double.
__global__ __launch_bounds__(256) void k_matmul_nt(const float *__restrict__ A,
                                                   const float *__restrict__ W,
                                                   const float *__restrict__ bias,
                                                   float *__restrict__ C, int64_t M, int64_t N,
                                                   int64_t K) {
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t mblocks = (M + 7) / 8;
  if (wid >= N * mblocks) return;
  const int64_t n = wid / mblocks, m0 = (wid % mblocks) * 8;
  const float *wr = W + n * K;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int64_t k = lane; k < K; k += 64) {
    const float wv = wr[k];
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (m0 + i < M) acc[i] = fmaf(A[(m0 + i) * K + k], wv, acc[i]);
  }
#pragma unroll
  for (int i = 0; i < 8; i++) {
    double s = acc[i];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0 && m0 + i < M) C[(m0 + i) * N + n] = (float)s + (bias ? bias[n] : 0.f);
  }
}

// launches for the host-buffer entry points (hostio.hip)
int sglq_launch_quant_rows_i8(const float *x, int8_t *q, float *scales, int64_t rows,
                              int64_t dim, hipStream_t st) {
  k_quant_rows_i8<<<(unsigned)rows, 256, 0, st>>>(x, q, scales, dim);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
int sglq_launch_dequant_row_i8(const int8_t *q, float scale, float *o, int64_t n,
                               hipStream_t st) {
  k_dequant_row_i8<<<sglq_blocks(n, 256), 256, 0, st>>>(q, scale, o, n);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
int sglq_launch_matmul_nt(const float *A, const float *W, const float *bias, float *C,
                          int64_t M, int64_t N, int64_t K, hipStream_t st) {
  const int64_t waves = N * ((M + 7) / 8);
  k_matmul_nt<<<sglq_blocks(waves * 64, 256), 256, 0, st>>>(A, W, bias, C, M, N, K);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// out[r][i] = (float)q[r][i] * scales[r]: sgl_dequant_row_i8 over rows
__global__ void k_dequant_rows_i8(const int8_t *__restrict__ q, const float *__restrict__ sc,
                                  float *__restrict__ o, int64_t rows, int64_t dim) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows * dim) o[i] = (float)q[i] * sc[i / dim];
}

// device-pointer variants (stream-ordered): the int8 KV-cache rows quantized where they are
// produced (reference src/llama.c:1264-1267, 1485-1488 call sgl_quant_row_i8 on host rows)
extern "C" int sglq_quant_rows_i8_dev(const float *x, int8_t *out, float *scales, int64_t rows,
                                      int64_t dim, void *stream) {
  if (rows <= 0 || dim <= 0) return 0;
  k_quant_rows_i8<<<(unsigned)rows, 256, 0, (hipStream_t)stream>>>(x, out, scales, dim);
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}

extern "C" int sglq_dequant_rows_i8_dev(const int8_t *q, const float *scales, float *out,
                                        int64_t rows, int64_t dim, void *stream) {
  if (rows <= 0 || dim <= 0) return 0;
  k_dequant_rows_i8<<<sglq_blocks(rows * dim, 256), 256, 0, (hipStream_t)stream>>>(
      q, scales, out, rows, dim);
  SGLQ_HIP(hipGetLastError());
  return 0;
fail:
  return -1;
}
