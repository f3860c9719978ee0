// K2 -- RMSNorm scale + Q/K/V split + 3D RoPE + static-cache write, one pass over the qkv GEMM
// output.
//
// qkv is the fp32 output of the projection GEMM (the GEMM accumulates in fp32 and returns it
// unrounded).  Work item = 8 consecutive values of one token's qkv row (two 16-byte loads).
// Items are numbered token-major, so a wavefront reads 2 KiB of contiguous qkv and writes q
// (contiguous) or a 128-byte head row of the K/V cache per 8 lanes.  The 8 values are 4
// interleaved RoPE pairs of
// one head, rotated in fp32 with the per-axis cos/sin tables of the reference
// (RotaryEmbedding3D._build_cache); pair j of a head uses axis x for j < px, y for
// px <= j < px+py and z otherwise, exactly the split of RotaryEmbedding3D.apply_rotary.
#include "common.h"

namespace mdl {

struct RopeArgs {
  int max_x, max_y, max_z, px, py, pz;
};

__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ rstd,
    const int64_t* __restrict__ pos, const float* __restrict__ tab, RopeArgs ra, int64_t rows,
    int seq, int n_heads, float q_scale, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int slots, int slot0,
    const int32_t* __restrict__ slot_dev) {
  const int d = n_heads * kHeadDim;
  const int per_region = d / 8;
  const int per_tok = 3 * per_region;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * per_tok) return;
  const int64_t m = idx / per_tok;
  const int c = static_cast<int>(idx - m * per_tok);
  const int region = c / per_region;            // 0 q, 1 k, 2 v
  const int cc = c - region * per_region;
  const int h = cc >> 3;
  const int dim0 = (cc & 7) * 8;

  float f[8];
  load8f(qkv + m * ld + c * 8, f);
  const float r = rstd ? rstd[m] : 1.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] *= r;

  if (region < 2) {
    const int64_t* p = pos + m * 3;
    int64_t cx = p[0], cy = p[1], cz = p[2];
    cx = cx < 0 ? 0 : (cx >= ra.max_x ? ra.max_x - 1 : cx);
    cy = cy < 0 ? 0 : (cy >= ra.max_y ? ra.max_y - 1 : cy);
    cz = cz < 0 ? 0 : (cz >= ra.max_z ? ra.max_z - 1 : cz);
    const int off_y = 2 * ra.max_x * ra.px;
    const int off_z = off_y + 2 * ra.max_y * ra.py;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int j = (dim0 >> 1) + k;
      int base, half, jj;
      if (j < ra.px) {
        half = ra.max_x * ra.px; base = static_cast<int>(cx) * ra.px; jj = j;
      } else if (j < ra.px + ra.py) {
        half = ra.max_y * ra.py; base = off_y + static_cast<int>(cy) * ra.py; jj = j - ra.px;
      } else {
        half = ra.max_z * ra.pz; base = off_z + static_cast<int>(cz) * ra.pz;
        jj = j - ra.px - ra.py;
      }
      const float cs = tab[base + jj];
      const float sn = tab[base + half + jj];
      const float a = f[2 * k], b = f[2 * k + 1];
      f[2 * k] = a * cs - b * sn;
      f[2 * k + 1] = b * cs + a * sn;
    }
  }
  if (region == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] *= q_scale;
    *reinterpret_cast<uint4*>(q_out + m * d + h * kHeadDim + dim0) = pack8(f);
  } else {
    const int64_t b = m / seq;
    const int s = static_cast<int>(m - b * seq);
    const int slot = (slot_dev ? *slot_dev : slot0) + s;
    if (slot < 0 || slot >= slots) return;       // host guarantees range; never write outside
    uint16_t* dst = (region == 1 ? kc : vc) +
                    ((b * n_heads + h) * static_cast<int64_t>(slots) + slot) * kHeadDim + dim0;
    *reinterpret_cast<uint4*>(dst) = pack8(f);
  }
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_qkv_rope_cache(const float* qkv, int64_t qkv_ld, const float* rstd,
                                  const int64_t* pos, const float* rope_tab, int batch, int seq,
                                  int n_heads, int head_dim, int max_x, int max_y, int max_z,
                                  int px, int py, int pz, float q_scale, uint16_t* q_out,
                                  uint16_t* k_cache, uint16_t* v_cache, int cache_slots,
                                  int slot0, const int32_t* slot_dev, void* stream) {
  if (!qkv || !pos || !rope_tab || !q_out || !k_cache || !v_cache) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || seq <= 0 || n_heads <= 0 || max_x <= 0 || max_y <= 0 || max_z <= 0 ||
      px < 0 || py < 0 || pz < 0 || px + py + pz != kHeadDim / 2 || qkv_ld < 3 * n_heads * 64)
    return MDL_ERR_SHAPE;
  if (cache_slots <= 0 || (!slot_dev && (slot0 < 0 || slot0 + seq > cache_slots)))
    return MDL_ERR_CACHE;
  if (!aligned16(qkv) || qkv_ld % 4 != 0 || !aligned16(q_out) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned4(rope_tab))
    return MDL_ERR_ALIGN;
  const int64_t rows = static_cast<int64_t>(batch) * seq;
  if (rows == 0) return MDL_OK;
  const int64_t items = rows * 3 * n_heads * 8;
  const RopeArgs ra{max_x, max_y, max_z, px, py, pz};
  qkv_rope_cache_kernel<<<dim3(static_cast<unsigned>((items + 255) / 256)), 256, 0,
                          static_cast<hipStream_t>(stream)>>>(
      qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, n_heads, q_scale, q_out, k_cache,
      v_cache, cache_slots, slot0, slot_dev);
  return launch_status();
}
