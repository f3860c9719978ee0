// Shared device helpers for the mdlarc HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mdlarc_hip.h"

namespace mdl {

constexpr int kWave = 64;
constexpr int kHeadDim = 64;

// ---- bf16 <-> f32 (bf16 stored as raw 16-bit words) ------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t h16) { return __uint_as_float(h16 << 16); }

// f32 -> bf16 with v_cvt_pk_bf16_f32: round to nearest even (the rounding torch uses for
// .to(bfloat16)), NaN stays NaN.  One VALU op per pair; a bit-twiddling rounding with a NaN test
// compiles to exec-masked branches around every value.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{static_cast<__bf16>(lo), static_cast<__bf16>(hi)});
}

// 8 bf16 held in a uint4 -> 8 floats
__device__ __forceinline__ void unpack8(const uint4 v, float* f) {
  f[0] = bf2f(v.x & 0xffffu); f[1] = bf2f(v.x >> 16);
  f[2] = bf2f(v.y & 0xffffu); f[3] = bf2f(v.y >> 16);
  f[4] = bf2f(v.z & 0xffffu); f[5] = bf2f(v.z >> 16);
  f[6] = bf2f(v.w & 0xffffu); f[7] = bf2f(v.w >> 16);
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf2(f[0], f[1]); v.y = pack_bf2(f[2], f[3]);
  v.z = pack_bf2(f[4], f[5]); v.w = pack_bf2(f[6], f[7]);
  return v;
}

// silu(a) * b, the SwiGLU gate, in the one form every kernel that computes it uses (K3 and the
// fused epilogues of K5 and K6 then agree bit for bit).  a * rcp(1 + e^-a): the hardware
// reciprocal (1 ulp) in place of an IEEE division, which is ten instructions per value and made
// the SwiGLU epilogue a fifth of the gate / up GEMM's time at prompt sizes.  1 + e^-a >= 1, so
// the reciprocal never meets a denormal; e^-a = inf gives a * 0.
__device__ __forceinline__ float silu_mul(float a, float b) {
  return a * __builtin_amdgcn_rcpf(1.f + __expf(-a)) * b;
}

// ---- split activations -----------------------------------------------------------------------
// A GEMM input row of width K is stored as 2K bf16: hi = bf16(v) in columns [0, K) and
// lo = bf16(v - hi) in [K, 2K) (v - hi is exact in fp32).  Against a weight packed as [W | W]
// the bf16 GEMM then returns (hi + lo) . w, i.e. v to about 2^-17 relative instead of the 2^-9
// of a single bf16 rounding; the same buffer read as [2M, K] gives hi.w and lo.w as row pairs.
// v is the rounded fp32 value: contraction is off here, so a product feeding v is never fused
// into v - hi (the compiler otherwise fuses it in some instantiations of a kernel and not in
// others, and the same activation then splits differently in different kernels).
__device__ __forceinline__ void split_bf2(float a, float b, uint32_t& hi, uint32_t& lo) {
#pragma clang fp contract(off)
  const bf16x2_t h = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  hi = __builtin_bit_cast(uint32_t, h);
  // the two rounded halves widened from the packed pair itself (a bf16 is the top half of its
  // fp32): the low one by a byte permute (bytes 1, 0 of hi to bytes 3, 2, zeros below), which
  // the compiler cannot turn back into a second rounding of a plus a shift, as it does `hi << 16`
  const float h0 = __builtin_bit_cast(float, __builtin_amdgcn_perm(0u, hi, 0x01000c0cu));
  const float h1 = __builtin_bit_cast(float, hi & 0xffff0000u);
  lo = pack_bf2(a - h0, b - h1);
}

// 4 floats -> hi (uint2) and lo (uint2)
__device__ __forceinline__ void split4(const float* f, uint2& hi, uint2& lo) {
  split_bf2(f[0], f[1], hi.x, lo.x);
  split_bf2(f[2], f[3], hi.y, lo.y);
}

// 8 floats -> hi (uint4) and lo (uint4)
__device__ __forceinline__ void split8(const float* f, uint4& hi, uint4& lo) {
  split_bf2(f[0], f[1], hi.x, lo.x);
  split_bf2(f[2], f[3], hi.y, lo.y);
  split_bf2(f[4], f[5], hi.z, lo.z);
  split_bf2(f[6], f[7], hi.w, lo.w);
}

// 16-byte streaming load with the non-temporal hint.  Data read once per kernel (the KV cache
// in decode attention) then does not displace what later kernels reuse from the caches (the
// projection weights), and on MI355X the stream itself runs faster: decode attention measured
// 6.75 TB/s with it against 5.9 TB/s with plain loads.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load_nt16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- streaming activations -------------------------------------------------------------------
// A whole prompt batch's activations (hundreds of MB) cannot stay in L2 / the 256 MB MALL until
// their consumer reads them, so the memory-bound kernels read and write them with the
// non-temporal hint when the host asks for it (NT = true; measured on MI355X: K2 5.5 -> 6.2 TB/s,
// both hints together).  Outputs below kStreamBytes (the decode step's) keep the default policy,
// so the next GEMM still finds them in cache.
constexpr int64_t kStreamBytes = int64_t{64} << 20;

typedef float f32x4_vt __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

template <bool NT>
__device__ __forceinline__ float4 ld_f4(const float* p) {
  if constexpr (NT) {
    const f32x4_vt v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_vt*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const float4*>(p);
  }
}

template <bool NT>
__device__ __forceinline__ void st_f4(float* p, float4 v) {
  if constexpr (NT)
    __builtin_nontemporal_store(f32x4_vt{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4_vt*>(p));
  else
    *reinterpret_cast<float4*>(p) = v;
}

template <bool NT>
__device__ __forceinline__ void st_u2(void* p, uint2 v) {
  if constexpr (NT)
    __builtin_nontemporal_store(u32x2_t{v.x, v.y}, reinterpret_cast<u32x2_t*>(p));
  else
    *reinterpret_cast<uint2*>(p) = v;
}

template <bool NT>
__device__ __forceinline__ void st_u4(void* p, uint4 v) {
  if constexpr (NT)
    __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(p));
  else
    *reinterpret_cast<uint4*>(p) = v;
}

__device__ __forceinline__ void load8f(const float* p, float* f) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
  f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// ---- wave64 reductions -----------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Element offset of (row m, column j) of a [rows, cols] bf16 matrix in the MFMA tile layout
// (MDL_LAYOUT_TILES; cols a multiple of 32).  Columns j .. j + 7 with j % 8 == 0 are contiguous.
__device__ __forceinline__ int64_t tile_off(int64_t m, int j, int cols) {
  return 512 * ((m >> 4) * (cols >> 5) + (j >> 5)) + 8 * (16 * ((j >> 3) & 3) + (m & 15)) +
         (j & 7);
}

// Element offset of (row m, column j) of a [rows, cols] fp32 matrix in the fp32 tile layout
// (MDL_LAYOUT_TILES for fp32; cols a multiple of 32): 16 x 32 blocks of 512 floats in the order
// of the bf16 layout; inside a block, row m % 16, columns 8 q .. 8 q + 7 (q = (j / 8) % 4) belong
// to lane l = 16 q + m % 16, whose elements 0..3 sit at 4 l and 4..7 at 256 + 4 l, so a wave
// reads a block as two contiguous kilobytes.  Columns j .. j + 3 with j % 4 == 0 are contiguous.
__device__ __forceinline__ int64_t tile_off32(int64_t m, int j, int cols) {
  return 512 * ((m >> 4) * (cols >> 5) + (j >> 5)) + 256 * ((j >> 2) & 1) +
         4 * (16 * ((j >> 3) & 3) + (m & 15)) + (j & 3);
}

// ---- host-side launch checking ---------------------------------------------------------------
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MDL_OK : static_cast<int>(e);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace mdl
