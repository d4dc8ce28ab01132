// noalloc.hip — the forward for callers that cannot allocate device memory (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc): the prefill GEMM's
// workspace (A operands, row exponents, split-K partials) lives in one file-scope device array,
// `scratch`, instead of the handle's grow-on-demand workspace.  The decode GEMV needs no
// workspace beyond the per-handle state allocated when the handle was created.
//
// Every GPU holds its own copy of `scratch` until the process ends.  Every call on one GPU
// shares that copy and leaves its contents behind; nothing in it has to start at zero (each
// call writes every workspace byte it later reads).  Calls that can overlap on one GPU (two
// streams, two threads) race on it: order them.
#include <atomic>
#include <mutex>

#include "sglq_dev.hpp"

#define SGLQ_SCRATCH_BYTES (64u << 20)  // 64 MiB per GPU

static __device__ __align__(256) unsigned char scratch[SGLQ_SCRATCH_BYTES];

namespace {

constexpr int kMaxDev = 64;
std::atomic<void *> g_scratch[kMaxDev];
std::mutex g_scratch_mu;

// The device address of `scratch` on device dev, looked up once per device with that device
// current (host code must not use the array's name as an address).
void *scratch_ptr(int dev) {
  if (dev < 0 || dev >= kMaxDev) return nullptr;
  void *p = g_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  p = g_scratch[dev].load(std::memory_order_relaxed);
  if (p) return p;
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess || !p) {
    sglq_log_error("scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                   hipGetErrorName(e));
    return nullptr;
  }
  g_scratch[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" int sglq_forward_noalloc(sglq_dev *d, const void *A, int dt, int64_t M,
                                    const float *bias, float *C, void *stream) {
  void *ws = scratch_ptr(d->dev);
  if (!ws) return -1;
  return sglq_forward_ws(d, A, dt, M, bias, C, stream, ws, SGLQ_SCRATCH_BYTES);
}

extern "C" size_t sglq_scratch_bytes(void) { return SGLQ_SCRATCH_BYTES; }
