// 3D RoPE lookup shared by K2 (mdl_qkv_rope_cache) and the fused decode attention.
//
// Pair j of a 64-dim head rotates with axis x for j < px, y for px <= j < px+py and z otherwise
// (RotaryEmbedding3D.apply_rotary, src/transformer.py:132-187); positions clamp to [0, max-1]
// per axis (:152-154).  The fp32 table is [cos_x | sin_x | cos_y | sin_y | cos_z | sin_z], each
// axis block [n_pos, pairs] (RotaryEmbedding3D._build_cache, :95-126).  A pair (a, b) rotates to
// (a c - b s, b c + a s), the interleaved-pair form of _rotate_half (:51-58).
#pragma once

#include <stdint.h>

namespace mdl {

struct RopeArgs {
  int max_x, max_y, max_z, px, py, pz;
};

// cos / sin of pair j for the token at position (p0, p1, p2) = (x, y, z).
__device__ __forceinline__ void rope_cos_sin3(int j, int64_t p0, int64_t p1, int64_t p2,
                                              const float* __restrict__ tab, const RopeArgs& ra,
                                              float& cs, float& sn) {
  int n_pos, pairs, jj, off;
  int64_t p;
  if (j < ra.px) {
    n_pos = ra.max_x; pairs = ra.px; jj = j; off = 0; p = p0;
  } else if (j < ra.px + ra.py) {
    n_pos = ra.max_y; pairs = ra.py; jj = j - ra.px; off = 2 * ra.max_x * ra.px; p = p1;
  } else {
    n_pos = ra.max_z; pairs = ra.pz; jj = j - ra.px - ra.py;
    off = 2 * ra.max_x * ra.px + 2 * ra.max_y * ra.py; p = p2;
  }
  p = p < 0 ? 0 : (p >= n_pos ? n_pos - 1 : p);
  const int ti = off + static_cast<int>(p) * pairs + jj;
  cs = tab[ti];
  sn = tab[ti + n_pos * pairs];
}

// cos / sin of pair j for the token at pos3 (x, y, z).
__device__ __forceinline__ void rope_cos_sin(int j, const int64_t* __restrict__ pos3,
                                             const float* __restrict__ tab, const RopeArgs& ra,
                                             float& cs, float& sn) {
  // all three positions, unconditionally (one 24-byte line): a load per axis behind a lane-
  // dependent branch serialises the table reads that follow it
  rope_cos_sin3(j, pos3[0], pos3[1], pos3[2], tab, ra, cs, sn);
}

// A pair (a, b) rotated by (cs, sn): (a cs - b sn, b cs + a sn), each a fused multiply-add onto
// a rounded product.  Written out so that every kernel rotating a pair (K2, the fused prefill
// projection) produces the same bits whatever the compiler contracts elsewhere.
__device__ __forceinline__ void rope_rot(float a, float b, float cs, float sn, float& o0,
                                         float& o1) {
#pragma clang fp contract(off)
  const float bs = b * sn, as = a * sn;
  o0 = fmaf(a, cs, -bs);
  o1 = fmaf(b, cs, as);
}

}  // namespace mdl
