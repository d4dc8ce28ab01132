// gemv_ops.hpp — operand helpers shared by the decode GEMV kernels (gemv.hip, gemv_row.hip):
// activation element decoding, 4/8-bit code and e2m1 unpacking into the f16 B operand of
// v_mfma_f32_16x16x32_f16, and the meta entry (scale, zero) decoding.
#pragma once
#include <type_traits>

#include "sglq_dev.hpp"

namespace sglq {

__device__ __forceinline__ float bf16_bits(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ float f16_bits(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// (x & m) | o as one v_and_or_b32 (the compiler otherwise emits an AND and an OR)
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(o));
  return r;
}

union H8 {
  half8_t v;
  uint32_t u[4];
  half2_t h[4];
};

// Codes of step j of a chunk -> B operand.  U4 element order is nibbles {0,4,1,5,2,6,3,7}:
// (x & 0x000F000F) | 0x6400 gives 1024 + q, (x & 0x00F000F0) | 0x5400 gives 64 + q, and the
// matching exact offsets zA = -(1024 + z), zB = -(64 + z) leave q - z.
template <int KIND>
__device__ __forceinline__ half8_t unpack(const u32x4_t &w, int j, half2_t zA, half2_t zB) {
  H8 r;
  if constexpr (KIND == SGLQ_KIND_U4) {
    const uint32_t x = w[j], y = x >> 8;
    r.u[0] = and_or(x, 0x000F000Fu, 0x64006400u);
    r.u[1] = and_or(x, 0x00F000F0u, 0x54005400u);
    r.u[2] = and_or(y, 0x000F000Fu, 0x64006400u);
    r.u[3] = and_or(y, 0x00F000F0u, 0x54005400u);
    r.h[0] = r.h[0] + zA;
    r.h[1] = r.h[1] + zB;
    r.h[2] = r.h[2] + zA;
    r.h[3] = r.h[3] + zB;
  } else if constexpr (KIND == SGLQ_KIND_U8) {
    const uint32_t x0 = w[2 * j], x1 = w[2 * j + 1];
    r.u[0] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u);  // 1024 + b0, 1024 + b1
    r.u[1] = __builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u);
    r.u[2] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u);
    r.u[3] = __builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u);
#pragma unroll
    for (int i = 0; i < 4; i++) r.h[i] = r.h[i] + zA;
  } else {
    const uint32_t x = w[j];
    r.h[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 0);
    r.h[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 1);
    r.h[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 2);
    r.h[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(x, 1.0f, 3);
  }
  return r.v;
}

template <bool SCF16>
using meta_t = typename std::conditional<SCF16, uint32_t, uint64_t>::type;

template <bool SCF16>
__device__ __forceinline__ void decode_meta(meta_t<SCF16> m, float &sc, half2_t &zA,
                                            half2_t &zB) {
  uint32_t zb;
  if constexpr (SCF16) {
    sc = f16_bits(m & 0xFFFFu);
    zb = m >> 16;
  } else {
    sc = __uint_as_float((uint32_t)m);
    zb = (uint32_t)(m >> 32) & 0xFFFFu;
  }
  const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)zb);
  zA = (half2_t){z, z};
  const _Float16 z2 = z + (_Float16)960.0f;  // -(64 + zero), exact
  zB = (half2_t){z2, z2};
}

// element i of a U4 operand holds k-offset {0,4,1,5,2,6,3,7}[i]
__device__ __forceinline__ constexpr int kofs4(int i) { return (i >> 1) + 4 * (i & 1); }

}  // namespace sglq
