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

// cos / sin of pair j for the token at pos3 (x, y, z).
__device__ __forceinline__ void rope_cos_sin(int j, const int64_t* __restrict__ pos3,
                                             const float* __restrict__ tab, const RopeArgs& ra,
                                             float& cs, float& sn) {
  int axis, n_pos, pairs, jj, off;
  if (j < ra.px) {
    axis = 0; n_pos = ra.max_x; pairs = ra.px; jj = j; off = 0;
  } else if (j < ra.px + ra.py) {
    axis = 1; n_pos = ra.max_y; pairs = ra.py; jj = j - ra.px; off = 2 * ra.max_x * ra.px;
  } else {
    axis = 2; n_pos = ra.max_z; pairs = ra.pz; jj = j - ra.px - ra.py;
    off = 2 * ra.max_x * ra.px + 2 * ra.max_y * ra.py;
  }
  int64_t p = pos3[axis];
  p = p < 0 ? 0 : (p >= n_pos ? n_pos - 1 : p);
  const int ti = off + static_cast<int>(p) * pairs + jj;
  cs = tab[ti];
  sn = tab[ti + n_pos * pairs];
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
