// bf16 MFMA building blocks shared by the attention kernels (gfx950, wave64).
//
// v_mfma_f32_16x16x32_bf16 operand layout (lane l, c = l % 16, g = l / 16):
//   A (16 x 32, M x K): lane l holds row c, k = 8 g .. 8 g + 7 (8 bf16, 16 bytes);
//   B (32 x 16, K x N): lane l holds column c, k = 8 g .. 8 g + 7;
//   C/D (16 x 16):      lane l holds column c, rows 4 g .. 4 g + 3 (4 fp32).
// An MFMA pairs element e of lane group g in A with element e of group g in B whatever k that
// is inside the instruction, so any key order common to both operands gives the same product.
#pragma once

#include "common.h"

namespace mdl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2eF = 1.4426950408889634f;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// 8 bf16 ones: the A operand that turns an MFMA into a column sum of B
__device__ __forceinline__ bf16x8_t bf16_ones8() {
  return as_bf16x8(make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i & 3 of the 8-byte
// rows addressed by lanes 4 k + (i >> 2), k = 0..3 (lane mapping pinned on the GPU).
__device__ __forceinline__ s16x4_t lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(p));
}

// The V^T A operand of key step kk (keys 32 kk .. 32 kk + 31) and dims 16 db .. 16 db + 15 from
// a row-major [key][dim] bf16 tile with row stride `ld`: two transposing reads.  Lane c of group
// g addresses key rows 32 kk + 4 g + c / 4 (and + 16) at dims 16 db + 4 (c % 4) .. + 3, which
// yields V^T[dim 16 db + c] over keys 32 kk + (e < 4 ? 4 g + e : 16 + 4 g + e - 4) -- the key
// order of the P^T operand built from the S^T accumulators (score block 2 kk and 2 kk + 1).
__device__ __forceinline__ bf16x8_t vt_operand(const uint16_t* tile, int ld, int kk, int db,
                                               int c16, int g) {
  const int r0 = 32 * kk + 4 * g + (c16 >> 2);
  const int cc = 16 * db + 4 * (c16 & 3);
  const s16x4_t lo4 = lds_read_tr16(tile + r0 * ld + cc);
  const s16x4_t hi4 = lds_read_tr16(tile + (r0 + 16) * ld + cc);
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
}

// The P^T B operand of key step kk from the S^T score blocks 2 kk and 2 kk + 1 (bf16, round to
// nearest even).
__device__ __forceinline__ bf16x8_t pt_operand(const f32x4_t& s0, const f32x4_t& s1) {
  return bf16x8_t{(__bf16)s0[0], (__bf16)s0[1], (__bf16)s0[2], (__bf16)s0[3],
                  (__bf16)s1[0], (__bf16)s1[1], (__bf16)s1[2], (__bf16)s1[3]};
}

// Maximum over lanes l, l^16, l^32, l^48 (one column's four lane groups) with gfx950's VALU
// lane swaps: v_permlane16_swap / v_permlane32_swap of a value with itself return
// {x[l], x[l^16]} / {x[l], x[l^32]} (checked on the GPU).  Replaces two ds_bpermute round trips
// through the LDS unit on the softmax's critical path (measured 3% on the prefill kernel,
// bit-identical).
__device__ __forceinline__ float max_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

}  // namespace mdl
