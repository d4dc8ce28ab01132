// ceiling.hip — microbenchmarks that measure the ceilings the product kernels are judged
// against on the box they run on (gfx950): a read-only HBM stream, an empty launch, and MFMA
// issue loops.  Built into its own library (libsgl_ceiling.so), never linked into the product.
// Each entry point enqueues one launch on `stream` and returns 0, or -1 on a launch error.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));

// Read-only stream: every thread issues U 128-bit loads (all in flight) per pass and XORs them.
// A workgroup covers 256 * U consecutive 16-byte items; the grid covers n16 items.  The fold is
// stored only when it equals a value no real input gives, so the loads cannot be dropped.
template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const u4_t *__restrict__ p, int64_t n16,
                                                     uint32_t *__restrict__ sink) {
  const int64_t base = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
  u4_t v[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int64_t i = base + (int64_t)u * 256;
    v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : u4_t{0, 0, 0, 0};
  }
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < U; u++) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  if (x == 0x9E3779B9u) sink[blockIdx.x & 1023] = x;
}

// L2-resident read stream: workgroup b reads its own slice of `slice16` 16-byte items `iters`
// times (plain loads, U per thread in flight per pass).  Slices small enough for the L2 of the
// workgroup's XCD measure how fast one CU takes in data that hits in L2.
template <int U>
__global__ __launch_bounds__(256) void k_l2_read(const u4_t *__restrict__ p, int slice16, int iters,
                                                 uint32_t *__restrict__ sink) {
  const u4_t *q = p + (int64_t)blockIdx.x * slice16;
  uint32_t x = 0;
  for (int it = 0; it < iters; it++) {
    for (int b = 0; b < slice16; b += 256 * U) {
      u4_t v[U];
#pragma unroll
      for (int u = 0; u < U; u++) v[u] = q[(b + u * 256 + threadIdx.x) % slice16];
#pragma unroll
      for (int u = 0; u < U; u++) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    x = x * 3u + (uint32_t)it;
  }
  if (x == 0x9E3779B9u) sink[blockIdx.x & 1023] = x;
}

// The same per-CU intake through global_load_lds_dwordx4 (data lands in LDS, no registers):
// U copies of 16 bytes per thread in flight into a ring of LDS buffers, then a wait.
template <int U>
__global__ __launch_bounds__(256) void k_l2_read_lds(const u4_t *__restrict__ p, int slice16,
                                                     int iters, uint32_t *__restrict__ sink) {
  __shared__ u4_t buf[U * 256];  // U x 4 KiB
  const u4_t *q = p + (int64_t)blockIdx.x * slice16;
  const int w = threadIdx.x >> 6;
  for (int it = 0; it < iters; it++) {
    for (int b = 0; b < slice16; b += 256 * U) {
#pragma unroll
      for (int u = 0; u < U; u++)
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void *)(q + (b + u * 256 + threadIdx.x) % slice16),
            (__attribute__((address_space(3))) void *)(buf + u * 256 + 64 * w), 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(0);
    }
  }
  __syncthreads();
  const uint32_t x = buf[threadIdx.x].x ^ buf[(threadIdx.x + 7) % (U * 256)].y;
  if (x == 0x9E3779B9u) sink[blockIdx.x & 1023] = x;
}

__global__ void k_empty() {}

// MFMA issue loops: every wave runs `iters` x 8 independent accumulation chains.  Operands come
// from the thread index so the compiler cannot fold them; the result is stored only when it
// equals a value the loop never produces.
__global__ __launch_bounds__(256) void k_mfma_16x16x32_f16(int iters, float *__restrict__ sink) {
  h8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (threadIdx.x + i));
    b[i] = (_Float16)(0.002f * (threadIdx.x - i));
  }
  // distinct starting values, and the 16x16 instructions as inline asm on VGPR accumulators:
  // with the builtin, hipcc (ROCm 7.2) rotates the eight accumulators through AGPR copies
  // every iteration, which measures the copies rather than the matrix unit
  const float z = (float)threadIdx.x;
  f4_t c0 = {z, 0, 0, 0}, c1 = {z + 1, 0, 0, 0}, c2 = {z + 2, 0, 0, 0}, c3 = {z + 3, 0, 0, 0};
  f4_t c4 = {z + 4, 0, 0, 0}, c5 = {z + 5, 0, 0, 0}, c6 = {z + 6, 0, 0, 0}, c7 = {z + 7, 0, 0, 0};
  for (int it = 0; it < iters; it++) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c4) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c5) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c6) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c7) : "v"(a), "v"(b));
  }
  const f4_t t = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
  const float s = (t[0] + t[1]) + (t[2] + t[3]);
  if (s == 1234.5678f) sink[threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_mfma_16x16x32_bf16(int iters, float *__restrict__ sink) {
  b8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (__bf16)(0.001f * (threadIdx.x + i));
    b[i] = (__bf16)(0.002f * (threadIdx.x - i));
  }
  // distinct starting values, and the 16x16 instructions as inline asm on VGPR accumulators:
  // with the builtin, hipcc (ROCm 7.2) rotates the eight accumulators through AGPR copies
  // every iteration, which measures the copies rather than the matrix unit
  const float z = (float)threadIdx.x;
  f4_t c0 = {z, 0, 0, 0}, c1 = {z + 1, 0, 0, 0}, c2 = {z + 2, 0, 0, 0}, c3 = {z + 3, 0, 0, 0};
  f4_t c4 = {z + 4, 0, 0, 0}, c5 = {z + 5, 0, 0, 0}, c6 = {z + 6, 0, 0, 0}, c7 = {z + 7, 0, 0, 0};
  for (int it = 0; it < iters; it++) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c4) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c5) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c6) : "v"(a), "v"(b));
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c7) : "v"(a), "v"(b));
  }
  const f4_t t = ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7));
  const float s = (t[0] + t[1]) + (t[2] + t[3]);
  if (s == 1234.5678f) sink[threadIdx.x] = s;
}

// The same loop through the compiler builtin (kept to show the cost of its accumulator copies).
__global__ __launch_bounds__(256) void k_mfma_16x16x32_f16_builtin(int iters,
                                                                   float *__restrict__ sink) {
  h8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (threadIdx.x + i));
    b[i] = (_Float16)(0.002f * (threadIdx.x - i));
  }
  f4_t c[8];
#pragma unroll
  for (int j = 0; j < 8; j++) c[j] = f4_t{(float)threadIdx.x + j, 0, 0, 0};
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
  }
  f4_t t = c[0];
#pragma unroll
  for (int j = 1; j < 8; j++) t += c[j];
  const float s = (t[0] + t[1]) + (t[2] + t[3]);
  if (s == 1234.5678f) sink[threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_mfma_32x32x16_f16(int iters, float *__restrict__ sink) {
  h8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (threadIdx.x + i));
    b[i] = (_Float16)(0.002f * (threadIdx.x - i));
  }
  const float z = (float)threadIdx.x;
  f16_t c0 = {}, c1 = {}, c2 = {}, c3 = {};
  c0[0] = z;
  c1[0] = z + 1;
  c2[0] = z + 2;
  c3[0] = z + 3;
  for (int it = 0; it < iters; it++) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
  }
  const f16_t t = (c0 + c1) + (c2 + c3);
  float s = 0;
#pragma unroll
  for (int i = 0; i < 16; i++) s += t[i];
  if (s == 1234.5678f) sink[threadIdx.x] = s;
}

// LDS read stream: every lane reads 16 B per ds_read_b128 from a 64 KiB LDS array, eight reads
// in flight, consecutive lanes on consecutive 16-byte slots (no bank conflicts).
// MFMA issue with independent VALU work: every wave runs `iters` x 8 independent accumulation
// chains of v_mfma_f32_16x16x32_f16, each instruction followed by NV v_pk_mul_f16 on registers
// no MFMA touches.  Run at one and two waves per SIMD, it shows whether the SIMD issues VALU
// work in the shadow of its own wave's MFMAs or only of another wave's.
template <int NV>
__global__ __launch_bounds__(256) void k_mfma_valu(int iters, float *__restrict__ sink) {
  h8_t a, b;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    a[i] = (_Float16)(0.001f * (threadIdx.x + i));
    b[i] = (_Float16)(0.002f * (threadIdx.x - i));
  }
  const float z = (float)threadIdx.x;
  f4_t c[8];
#pragma unroll
  for (int i = 0; i < 8; i++) c[i] = (f4_t){z + i, 0, 0, 0};
  uint32_t v[8];
#pragma unroll
  for (int i = 0; i < 8; i++) v[i] = 0x3c003c00u + threadIdx.x + i;
  const uint32_t m = 0x3c013c01u;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c[i]) : "v"(a), "v"(b));
#pragma unroll
      for (int u = 0; u < NV; u++)
        asm volatile("v_pk_mul_f16 %0, %0, %1" : "+v"(v[(i * NV + u) & 7]) : "v"(m));
    }
  }
  f4_t t = c[0];
#pragma unroll
  for (int i = 1; i < 8; i++) t += c[i];
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) x ^= v[i];
  const float s = (t[0] + t[1]) + (t[2] + t[3]) + (float)x;
  if (s == 1234.5678f) sink[threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void k_lds_read(int iters, int stride, uint32_t *__restrict__ sink) {
  __shared__ u4_t buf[4096];  // 64 KiB
  for (int i = threadIdx.x; i < 4096; i += 256) buf[i] = u4_t{(uint32_t)i, 1u, 2u, 3u};
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  u4_t x = {0, 0, 0, 0};
  for (int it = 0; it < iters; it++) {
    u4_t v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = buf[(it * stride + j * 256 + w * 64 + lane) & 4095];
#pragma unroll
    for (int j = 0; j < 8; j++) x += v[j];
  }
  if ((x.x ^ x.y ^ x.z ^ x.w) == 0x9E3779B9u) sink[threadIdx.x] = x.x;
}

extern "C" {

// bytes read = n16 * 16; u = loads in flight per thread (4 / 8 / 16)
__attribute__((visibility("default"))) int sglc_stream_read(const void *p, int64_t n16, int u, uint32_t *sink, void *stream) {
  hipStream_t st = (hipStream_t)stream;
  const int64_t per = 256LL * u;
  const unsigned grid = (unsigned)((n16 + per - 1) / per);
  if (u == 4)
    k_stream_read<4><<<grid, 256, 0, st>>>((const u4_t *)p, n16, sink);
  else if (u == 16)
    k_stream_read<16><<<grid, 256, 0, st>>>((const u4_t *)p, n16, sink);
  else
    k_stream_read<8><<<grid, 256, 0, st>>>((const u4_t *)p, n16, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

__attribute__((visibility("default"))) int sglc_empty(void *stream) {
  k_empty<<<1, 64, 0, (hipStream_t)stream>>>();
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// kind 0: 16x16x32 f16, 1: 16x16x32 bf16, 2: 32x32x16 f16, 3: 16x16x32 f16 via the builtin.  Flops per launch =
// grid * 4 waves * iters * chains * (2 * m * n * k) with 8 chains for 16x16, 4 for 32x32.
__attribute__((visibility("default"))) int sglc_mfma(int kind, int grid, int iters, float *sink, void *stream) {
  hipStream_t st = (hipStream_t)stream;
  if (kind == 0)
    k_mfma_16x16x32_f16<<<grid, 256, 0, st>>>(iters, sink);
  else if (kind == 1)
    k_mfma_16x16x32_bf16<<<grid, 256, 0, st>>>(iters, sink);
  else if (kind == 2)
    k_mfma_32x32x16_f16<<<grid, 256, 0, st>>>(iters, sink);
  else
    k_mfma_16x16x32_f16_builtin<<<grid, 256, 0, st>>>(iters, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// LDS read stream on `grid` workgroups of 256 threads: bytes read = grid * 256 * iters * 128.
__attribute__((visibility("default"))) int sglc_lds_read(int grid, int iters, uint32_t *sink,
                                                          void *stream) {
  // the stride (a multiple of 64 items, unknown to the compiler) keeps every read in the loop
  k_lds_read<<<grid, 256, 0, (hipStream_t)stream>>>(iters, 8 * 256 + 64, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// MFMA + VALU issue (k_mfma_valu): nv VALU per MFMA (0, 2, 4 or 6) on `grid` workgroups of 256.
__attribute__((visibility("default"))) int sglc_mfma_valu(int nv, int grid, int iters, float *sink,
                                                           void *stream) {
  hipStream_t st = (hipStream_t)stream;
  if (nv == 0) k_mfma_valu<0><<<grid, 256, 0, st>>>(iters, sink);
  else if (nv == 2) k_mfma_valu<2><<<grid, 256, 0, st>>>(iters, sink);
  else if (nv == 4) k_mfma_valu<4><<<grid, 256, 0, st>>>(iters, sink);
  else k_mfma_valu<6><<<grid, 256, 0, st>>>(iters, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// L2-resident read stream (k_l2_read; u = -8 / -16: k_l2_read_lds): bytes read =
// grid * slice16 * 16 * iters.
__attribute__((visibility("default"))) int sglc_l2_read(const void *p, int grid, int slice16,
                                                         int iters, int u, uint32_t *sink,
                                                         void *stream) {
  hipStream_t st = (hipStream_t)stream;
  if (u == 16)
    k_l2_read<16><<<grid, 256, 0, st>>>((const u4_t *)p, slice16, iters, sink);
  else if (u == 8)
    k_l2_read<8><<<grid, 256, 0, st>>>((const u4_t *)p, slice16, iters, sink);
  else if (u == -16)  // negative u: the global_load_lds form
    k_l2_read_lds<16><<<grid, 256, 0, st>>>((const u4_t *)p, slice16, iters, sink);
  else
    k_l2_read_lds<8><<<grid, 256, 0, st>>>((const u4_t *)p, slice16, iters, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
