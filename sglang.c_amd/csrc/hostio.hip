// hostio.hip — host-buffer entry points of the shim (the reference's C API takes host
// pointers: reference src/quant.c:13-89, src/ops.c:243-279).  Operands are copied through
// per-device staging buffers that grow to the largest call and are kept until the process ends,
// so a call allocates nothing once its sizes have been seen; weights the host layer caches
// (sglq_upload) stay resident between calls.  Calls are serialised per device (they share the
// staging buffers) and synchronous, as the reference's are.
#include <mutex>

#include "sglq_dev.hpp"

namespace {

constexpr int kMaxDev = 64;
constexpr int kBufs = 4;

struct Staging {
  std::mutex mu;
  void *buf[kBufs] = {nullptr, nullptr, nullptr, nullptr};
  size_t cap[kBufs] = {0, 0, 0, 0};
};
Staging g_stage[kMaxDev];

// device buffer i of the current device holding at least `bytes` (grown, never shrunk)
void *stage(Staging &s, int i, size_t bytes) {
  if (bytes == 0) bytes = 16;
  if (s.cap[i] >= bytes) return s.buf[i];
  (void)hipFree(s.buf[i]);
  s.buf[i] = nullptr;
  s.cap[i] = 0;
  const size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;  // at least 1 MiB
  if (hipMalloc(&s.buf[i], want) != hipSuccess) {
    sglq_log_error("host staging allocation of %zu bytes failed", want);
    return nullptr;
  }
  s.cap[i] = want;
  return s.buf[i];
}

Staging *staging_of(int dev) { return dev >= 0 && dev < kMaxDev ? &g_stage[dev] : nullptr; }

}  // namespace

extern "C" void *sglq_upload(const void *host, size_t bytes, int dev) {
  void *d = nullptr;
  SGLQ_HIP(hipSetDevice(dev));
  SGLQ_HIP(hipMalloc(&d, bytes ? bytes : 16));
  if (bytes) SGLQ_HIP(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  return d;
fail:
  (void)hipFree(d);
  return nullptr;
}

extern "C" void sglq_release(void *dptr, int dev) {
  if (!dptr) return;
  (void)hipSetDevice(dev);
  (void)hipFree(dptr);
}

extern "C" int sglq_forward_host(sglq_dev *d, const float *A, int64_t M, const float *bias,
                                 float *C) {
  Staging *s = staging_of(d->dev);
  if (!s) return -1;
  std::lock_guard<std::mutex> lk(s->mu);
  float *dA, *dC, *dB = nullptr;
  SGLQ_HIP(hipSetDevice(d->dev));
  dA = (float *)stage(*s, 0, (size_t)(M * d->K) * 4);
  dC = (float *)stage(*s, 1, (size_t)(M * d->N) * 4);
  if (!dA || !dC) return -1;
  SGLQ_HIP(hipMemcpy(dA, A, (size_t)(M * d->K) * 4, hipMemcpyHostToDevice));
  if (bias) {
    if (!(dB = (float *)stage(*s, 2, (size_t)d->N * 4))) return -1;
    SGLQ_HIP(hipMemcpy(dB, bias, (size_t)d->N * 4, hipMemcpyHostToDevice));
  }
  if (sglq_forward(d, dA, SGLQ_DT_F32, M, dB, dC, nullptr) != 0) return -1;
  SGLQ_HIP(hipMemcpy(C, dC, (size_t)(M * d->N) * 4, hipMemcpyDeviceToHost));
  return 0;
fail:
  return -1;
}

extern "C" int sglq_matmul_nt_dev_w(const float *A, const float *dW, const float *bias, float *C,
                                    int64_t M, int64_t N, int64_t K, int dev) {
  Staging *s = staging_of(dev);
  if (!s) return -1;
  std::lock_guard<std::mutex> lk(s->mu);
  float *dA, *dC, *dB = nullptr;
  SGLQ_HIP(hipSetDevice(dev));
  dA = (float *)stage(*s, 0, (size_t)(M * K) * 4);
  dC = (float *)stage(*s, 1, (size_t)(M * N) * 4);
  if (!dA || !dC) return -1;
  SGLQ_HIP(hipMemcpy(dA, A, (size_t)(M * K) * 4, hipMemcpyHostToDevice));
  if (bias) {
    if (!(dB = (float *)stage(*s, 2, (size_t)N * 4))) return -1;
    SGLQ_HIP(hipMemcpy(dB, bias, (size_t)N * 4, hipMemcpyHostToDevice));
  }
  if (sglq_launch_matmul_nt(dA, dW, dB, dC, M, N, K, nullptr) != 0) goto fail;
  SGLQ_HIP(hipMemcpy(C, dC, (size_t)(M * N) * 4, hipMemcpyDeviceToHost));
  return 0;
fail:
  sglq_log_error("matmul_nt: device failure");
  return -1;
}

extern "C" int sglq_quant_rows_i8_host(const float *x, int8_t *out, float *scales, int64_t rows,
                                       int64_t dim) {
  if (rows <= 0 || dim <= 0) return 0;
  Staging *s = staging_of(0);
  std::lock_guard<std::mutex> lk(s->mu);
  const size_t n = (size_t)(rows * dim);
  float *dx, *ds;
  int8_t *dq;
  SGLQ_HIP(hipSetDevice(0));
  dx = (float *)stage(*s, 0, n * 4);
  dq = (int8_t *)stage(*s, 1, n);
  ds = (float *)stage(*s, 2, (size_t)rows * 4);
  if (!dx || !dq || !ds) return -1;
  SGLQ_HIP(hipMemcpy(dx, x, n * 4, hipMemcpyHostToDevice));
  if (sglq_launch_quant_rows_i8(dx, dq, ds, rows, dim, nullptr) != 0) goto fail;
  SGLQ_HIP(hipMemcpy(out, dq, n, hipMemcpyDeviceToHost));
  SGLQ_HIP(hipMemcpy(scales, ds, (size_t)rows * 4, hipMemcpyDeviceToHost));
  return 0;
fail:
  return -1;
}

extern "C" int sglq_dequant_row_i8_host(const int8_t *q, float scale, float *out, int64_t n) {
  if (n <= 0) return 0;
  Staging *s = staging_of(0);
  std::lock_guard<std::mutex> lk(s->mu);
  int8_t *dq;
  float *dout;
  SGLQ_HIP(hipSetDevice(0));
  dq = (int8_t *)stage(*s, 0, (size_t)n);
  dout = (float *)stage(*s, 1, (size_t)n * 4);
  if (!dq || !dout) return -1;
  SGLQ_HIP(hipMemcpy(dq, q, (size_t)n, hipMemcpyHostToDevice));
  if (sglq_launch_dequant_row_i8(dq, scale, dout, n, nullptr) != 0) goto fail;
  SGLQ_HIP(hipMemcpy(out, dout, (size_t)n * 4, hipMemcpyDeviceToHost));
  return 0;
fail:
  return -1;
}
