// sglq_dev.hpp — device-side definitions shared by the HIP translation units: the resident
// weight layout, vector types and error plumbing.  gfx950 (CDNA4) only.
//
// Device layout of one quantized weight W [N, K] ("tile layout"):
//   * N is cut into tiles of 16 columns (t = n / 16); K is re-indexed through kmap into device
//     positions k' (act-order groups made contiguous, each group padded to a multiple of 32) and
//     cut into MFMA steps of 32 (s = k' / 32).
//   * codes: for every (tile t, chunk c) one 1 KiB block = 64 lanes x 16 B.  Lane l carries
//     column n = 16t + (l & 15) and k' = 32 s + 8 (l >> 4) + i, i.e. exactly the B operand of
//     v_mfma_f32_16x16x32_f16 for that step.  4-bit kinds: a chunk is 4 steps, word j of the
//     lane is step 4c+j, nibble i holds i.  8-bit kind: a chunk is 2 steps, words (2j, 2j+1)
//     are step 2c+j, byte b of the pair holds i = b.
//   * U4/U8 meta: scales [t][gpad][16] (f16 when every scale is f16-exact, else f32) and
//     zeros [t][gpad][16] u8 (the value subtracted from the code).
//   * E2M1 meta: e8m0 bytes [t][chunk][16] packed 4 steps per u32 (byte j = step 4c+j).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sglq_shim.h"

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct sglq_dev {
  int dev;
  int kind;    // SGLQ_KIND_*
  int scf16;   // U4/U8 scales stored as f16
  int src;     // SGLQ_SRC_* it was built from
  int64_t N, K;
  int64_t ntile;   // ceil(N / 16)
  int64_t nsteps;  // device K / 32
  int64_t spc;     // steps per chunk (4 for 4-bit kinds, 2 for 8-bit)
  int64_t nchunk;  // nsteps / spc
  int64_t spg;     // steps per group
  int64_t ngroups; // real groups
  int64_t gpad;    // groups stored per tile (>= nsteps / spg)
  u32x4_t *codes;
  void *scales;
  uint8_t *zeros;
  int32_t *kmap;  // [nsteps * 32]
  int32_t *kinv;  // [K]
  // forward workspace (grown on demand)
  void *ws;
  size_t ws_bytes;
};

#define SGLQ_HIP(expr)                                                                    \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess) {                                                               \
      sglq_log_error("HIP error %s at %s:%d: %s", hipGetErrorName(e_), __FILE__, __LINE__, \
                     #expr);                                                              \
      goto fail;                                                                          \
    }                                                                                     \
  } while (0)

static inline unsigned sglq_blocks(int64_t n, int threads) {
  return (unsigned)((n + threads - 1) / threads);
}

// Grows d->ws to at least `bytes` (device memory, kept for the handle's lifetime).
int sglq_ws_reserve(sglq_dev *d, size_t bytes);
