// K2 -- RMSNorm scale + Q/K/V split + 3D RoPE + static-cache write, one pass over the qkv GEMM
// output.
//
// qkv is the fp32 output of the projection GEMM (unrounded fp32 accumulators).  One wavefront
// owns one token (a 256-thread block holds 4 tokens).  Lane l owns RoPE pair j = l % 32 of the
// heads h = l / 32, l / 32 + 2, ...: it looks its cos/sin up once (pair j rotates with axis x
// for j < px, y for px <= j < px+py and z otherwise, the split of RotaryEmbedding3D.apply_rotary)
// and applies it to that pair of q and of k of each of its heads.  A half-wave therefore reads
// 256 contiguous bytes of one head and writes 128 contiguous bytes of q or of one cache row;
// v (no rotation) is streamed as float4 per lane.  Rotation (a, b) -> (a c - b s, b c + a s) is
// the interleaved-pair form of _rotate_half.
#include "common.h"
#include "rope.h"

namespace mdl {

__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ rstd,
    const int64_t* __restrict__ pos, const float* __restrict__ tab, RopeArgs ra, int64_t rows,
    int seq, int n_heads, float q_scale, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int slots, int slot0,
    const int32_t* __restrict__ slot_dev) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  const int j = lane & 31, first_head = lane >> 5;
  const int d = n_heads * kHeadDim;

  float cs, sn;
  rope_cos_sin(j, pos + m * 3, tab, ra, cs, sn);
  const float r = rstd ? rstd[m] : 1.f;

  const float* row = qkv + m * ld;
  const int64_t b = m / seq;
  const int slot = (slot_dev ? *slot_dev : slot0) + static_cast<int>(m - b * seq);
  const bool in_cache = slot >= 0 && slot < slots;   // host guarantees range; never write outside
  uint16_t* qrow = q_out + m * d;
  const int64_t head_stride = static_cast<int64_t>(slots) * kHeadDim;
  const int64_t cache_row = (b * n_heads * static_cast<int64_t>(slots) + slot) * kHeadDim;

  for (int h = first_head; h < n_heads; h += 2) {
    const int c = h * kHeadDim + 2 * j;
    const float2 qa = *reinterpret_cast<const float2*>(row + c);
    const float2 ka = *reinterpret_cast<const float2*>(row + d + c);
    const float q0 = qa.x * r, q1 = qa.y * r, k0 = ka.x * r, k1 = ka.y * r;
    *reinterpret_cast<uint32_t*>(qrow + c) =
        pack_bf2((q0 * cs - q1 * sn) * q_scale, (q1 * cs + q0 * sn) * q_scale);
    if (in_cache)
      *reinterpret_cast<uint32_t*>(kc + cache_row + h * head_stride + 2 * j) =
          pack_bf2(k0 * cs - k1 * sn, k1 * cs + k0 * sn);
  }
  if (!in_cache) return;
  for (int idx = lane; idx < d / 4; idx += 64) {
    const float4 v = *reinterpret_cast<const float4*>(row + 2 * d + 4 * idx);
    const int hv = (4 * idx) / kHeadDim, dm = (4 * idx) % kHeadDim;
    uint2 o;
    o.x = pack_bf2(v.x * r, v.y * r);
    o.y = pack_bf2(v.z * r, v.w * r);
    *reinterpret_cast<uint2*>(vc + cache_row + hv * head_stride + dm) = o;
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
  const RopeArgs ra{max_x, max_y, max_z, px, py, pz};
  qkv_rope_cache_kernel<<<dim3(static_cast<unsigned>((rows + 3) / 4)), 256, 0,
                          static_cast<hipStream_t>(stream)>>>(
      qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, n_heads, q_scale, q_out, k_cache,
      v_cache, cache_slots, slot0, slot_dev);
  return launch_status();
}
