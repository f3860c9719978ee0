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

// Cache row (batch row b) and slot of token m: token m of a [batch, seq] prompt goes to slot
// (slot_dev ? *slot_dev : slot0) + m % seq of row m / seq; a packed token list names both per
// token (tok_row / tok_slot; a negative slot writes nothing).
__device__ __forceinline__ void token_slot(int64_t m, int seq, int slot0,
                                           const int32_t* __restrict__ slot_dev,
                                           const int32_t* __restrict__ tok_row,
                                           const int32_t* __restrict__ tok_slot, int64_t& b,
                                           int& slot) {
  if (tok_slot) {
    b = tok_row[m];
    slot = tok_slot[m];
  } else {
    b = m / seq;
    slot = (slot_dev ? *slot_dev : slot0) + static_cast<int>(m - b * seq);
  }
}

// Stores of the K2 outputs in the cache dtype: bf16 (the attention kernels' MFMA operands) or
// fp32 (the fp32 form: a model with fp32 parameters keeps an fp32 cache, src/inference.py:522).
__device__ __forceinline__ void store2(uint16_t* p, float a, float b) {
  *reinterpret_cast<uint32_t*>(p) = pack_bf2(a, b);
}
__device__ __forceinline__ void store2(float* p, float a, float b) {
  *reinterpret_cast<float2*>(p) = make_float2(a, b);
}
__device__ __forceinline__ void store4(uint16_t* p, float4 v) {
  *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
}
__device__ __forceinline__ void store4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }

template <typename TO>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ rstd,
    const int64_t* __restrict__ pos, const float* __restrict__ tab, RopeArgs ra, int64_t rows,
    int seq, int n_heads, float q_scale, TO* __restrict__ q_out, TO* __restrict__ kc,
    TO* __restrict__ vc, int slots, int slot0, const int32_t* __restrict__ slot_dev,
    const int32_t* __restrict__ tok_row, const int32_t* __restrict__ tok_slot, int64_t batch) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  const int j = lane & 31, first_head = lane >> 5;
  const int d = n_heads * kHeadDim;

  float cs, sn;
  rope_cos_sin(j, pos + m * 3, tab, ra, cs, sn);
  const float r = rstd ? rstd[m] : 1.f;

  const float* row = qkv + m * ld;
  int64_t b;
  int slot;
  token_slot(m, seq, slot0, slot_dev, tok_row, tok_slot, b, slot);
  // host guarantees the range; never write outside
  const bool in_cache = slot >= 0 && slot < slots && b >= 0 && b < batch;
  TO* qrow = q_out + m * d;
  const int64_t head_stride = static_cast<int64_t>(slots) * kHeadDim;
  const int64_t cache_row = (b * n_heads * static_cast<int64_t>(slots) + slot) * kHeadDim;

  for (int h = first_head; h < n_heads; h += 2) {
    const int c = h * kHeadDim + 2 * j;
    const float2 qa = *reinterpret_cast<const float2*>(row + c);
    const float2 ka = *reinterpret_cast<const float2*>(row + d + c);
    const float q0 = qa.x * r, q1 = qa.y * r, k0 = ka.x * r, k1 = ka.y * r;
    float y0, y1, z0, z1;
    rope_rot(q0, q1, cs, sn, y0, y1);
    rope_rot(k0, k1, cs, sn, z0, z1);
    store2(qrow + c, y0 * q_scale, y1 * q_scale);
    if (in_cache) store2(kc + cache_row + h * head_stride + 2 * j, z0, z1);
  }
  if (!in_cache) return;
  for (int idx = lane; idx < d / 4; idx += 64) {
    const float4 v = *reinterpret_cast<const float4*>(row + 2 * d + 4 * idx);
    const int hv = (4 * idx) / kHeadDim, dm = (4 * idx) % kHeadDim;
    store4(vc + cache_row + hv * head_stride + dm,
           make_float4(v.x * r, v.y * r, v.z * r, v.w * r));
  }
}

// Same work with the whole qkv row in flight at once, for H % 4 == 0 (every configured model):
// lane l owns the NCH = 3H/4 float4 chunks c = l + 64 i of the row.  A chunk's four channels sit
// at dims 4 (l % 16) .. +3 of their head, i.e. RoPE pairs 2 (l % 16) and 2 (l % 16) + 1 for every
// chunk of the lane, so one cos/sin lookup pair per token serves all of them, and chunk i belongs
// to q, k or v for i / (H/4) = 0, 1, 2.  All NCH loads are issued before the first store;
// prompt-sized batches stream with the non-temporal hint (common.h, kStreamBytes).
// 4 consecutive qkv channels as floats: an fp32 row (the GEMM output) or a bf16 one (the
// config-1 format, 8 bytes per lane)
template <bool NT>
__device__ __forceinline__ float4 ld_qkv4(const float* p) {
  return ld_f4<NT>(p);
}
template <bool NT>
__device__ __forceinline__ float4 ld_qkv4(const uint16_t* p) {
  uint2 u;
  if constexpr (NT) {
    const u32x2_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    u = make_uint2(t.x, t.y);
  } else {
    u = *reinterpret_cast<const uint2*>(p);
  }
  return make_float4(bf2f(u.x & 0xffffu), bf2f(u.x >> 16), bf2f(u.y & 0xffffu), bf2f(u.y >> 16));
}

template <int NCH, bool NT, typename TI = float>
__global__ __launch_bounds__(256) void qkv_rope_cache_vec_kernel(
    const TI* __restrict__ qkv, int64_t ld, const float* __restrict__ rstd,
    const int64_t* __restrict__ pos, const float* __restrict__ tab, RopeArgs ra, int64_t rows,
    int seq, float q_scale, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, int slots, int slot0, const int32_t* __restrict__ slot_dev,
    const int32_t* __restrict__ tok_row, const int32_t* __restrict__ tok_slot, int64_t batch) {
  constexpr int kH = 4 * NCH / 3, kD = kH * kHeadDim, kPart = NCH / 3;
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  const TI* row = qkv + m * ld;
  float4 v[NCH];
#pragma unroll
  for (int i = 0; i < NCH; ++i)
    v[i] = ld_qkv4<NT>(row + 4 * (lane + 64 * i));

  float cs0, sn0, cs1, sn1;
  rope_cos_sin(2 * (lane & 15), pos + m * 3, tab, ra, cs0, sn0);
  rope_cos_sin(2 * (lane & 15) + 1, pos + m * 3, tab, ra, cs1, sn1);
  const float r = rstd ? rstd[m] : 1.f;
  int64_t b;
  int slot;
  token_slot(m, seq, slot0, slot_dev, tok_row, tok_slot, b, slot);
  // host guarantees the range; never write outside
  const bool in_cache = slot >= 0 && slot < slots && b >= 0 && b < batch;
  const int64_t head_stride = static_cast<int64_t>(slots) * kHeadDim;
  const int64_t cache_row = (b * kH * static_cast<int64_t>(slots) + slot) * kHeadDim;

#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int e = 4 * (lane + 64 * i) - (i / kPart) * kD;   // channel inside the q/k/v part
    const float a0 = v[i].x * r, a1 = v[i].y * r, a2 = v[i].z * r, a3 = v[i].w * r;
    float y0, y1, y2, y3;
    rope_rot(a0, a1, cs0, sn0, y0, y1);
    rope_rot(a2, a3, cs1, sn1, y2, y3);
    if (i < kPart) {
      uint2 o;
      o.x = pack_bf2(y0 * q_scale, y1 * q_scale);
      o.y = pack_bf2(y2 * q_scale, y3 * q_scale);
      st_u2<NT>(q_out + m * kD + e, o);
    } else if (in_cache) {
      uint2 o;
      uint16_t* dst;
      if (i < 2 * kPart) {
        o.x = pack_bf2(y0, y1);
        o.y = pack_bf2(y2, y3);
        dst = kc;
      } else {
        o.x = pack_bf2(a0, a1);
        o.y = pack_bf2(a2, a3);
        dst = vc;
      }
      st_u2<NT>(dst + cache_row + (e / kHeadDim) * head_stride + e % kHeadDim, o);
    }
  }
}

}  // namespace mdl

using namespace mdl;

namespace mdl {

int launch_k2(const float* qkv, int64_t qkv_ld, const float* rstd, const int64_t* pos,
              const float* rope_tab, int64_t rows, int seq, int n_heads, const RopeArgs& ra,
              float q_scale, void* q_out_v, void* k_cache_v, void* v_cache_v, int out_dtype,
              int cache_slots, int slot0, const int32_t* slot_dev, const int32_t* tok_row,
              const int32_t* tok_slot, int64_t batch, hipStream_t st) {
  if (rows == 0) return MDL_OK;
  if ((rows + 3) / 4 > 0x7fffffff) return MDL_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  if (out_dtype == MDL_DTYPE_F32) {
    qkv_rope_cache_kernel<float><<<grid, 256, 0, st>>>(
        qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, n_heads, q_scale,
        static_cast<float*>(q_out_v), static_cast<float*>(k_cache_v),
        static_cast<float*>(v_cache_v), cache_slots, slot0, slot_dev, tok_row, tok_slot, batch);
    return launch_status();
  }
  uint16_t* q_out = static_cast<uint16_t*>(q_out_v);
  uint16_t* k_cache = static_cast<uint16_t*>(k_cache_v);
  uint16_t* v_cache = static_cast<uint16_t*>(v_cache_v);
  const bool nt = rows * n_heads * kHeadDim * 18 >= kStreamBytes;
#define MDL_K2_VEC(NCH)                                                                        \
  if (nt)                                                                                     \
    qkv_rope_cache_vec_kernel<NCH, true><<<grid, 256, 0, st>>>(                               \
        qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, q_scale, q_out, k_cache, v_cache,    \
        cache_slots, slot0, slot_dev, tok_row, tok_slot, batch);                              \
  else                                                                                        \
    qkv_rope_cache_vec_kernel<NCH, false><<<grid, 256, 0, st>>>(                              \
        qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, q_scale, q_out, k_cache, v_cache,    \
        cache_slots, slot0, slot_dev, tok_row, tok_slot, batch)
  switch (n_heads) {
    case 4: MDL_K2_VEC(3); break;
    case 12: MDL_K2_VEC(9); break;
    case 16: MDL_K2_VEC(12); break;
    case 20: MDL_K2_VEC(15); break;
    default:
      qkv_rope_cache_kernel<uint16_t><<<grid, 256, 0, st>>>(
          qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, n_heads, q_scale, q_out, k_cache,
          v_cache, cache_slots, slot0, slot_dev, tok_row, tok_slot, batch);
  }
#undef MDL_K2_VEC
  return launch_status();
}

int check_k2(const float* qkv, int64_t qkv_ld, const int64_t* pos, const float* rope_tab,
             int n_heads, int head_dim, int max_x, int max_y, int max_z, int px, int py, int pz,
             const void* q_out, const void* k_cache, const void* v_cache, int out_dtype) {
  if (!qkv || !pos || !rope_tab || !q_out || !k_cache || !v_cache) return MDL_ERR_NULL;
  if (out_dtype != MDL_DTYPE_F32 && out_dtype != MDL_DTYPE_BF16) return MDL_ERR_DTYPE;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (n_heads <= 0 || max_x <= 0 || max_y <= 0 || max_z <= 0 || px < 0 || py < 0 || pz < 0 ||
      px + py + pz != kHeadDim / 2 || qkv_ld < 3 * n_heads * 64)
    return MDL_ERR_SHAPE;
  if (!aligned16(qkv) || qkv_ld % 4 != 0 || !aligned16(q_out) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned4(rope_tab))
    return MDL_ERR_ALIGN;
  return MDL_OK;
}

}  // namespace mdl

extern "C" int mdl_qkv_rope_cache(const float* qkv, int64_t qkv_ld, const float* rstd,
                                  const int64_t* pos, const float* rope_tab, int batch, int seq,
                                  int n_heads, int head_dim, int max_x, int max_y, int max_z,
                                  int px, int py, int pz, float q_scale, void* q_out,
                                  void* k_cache, void* v_cache, int out_dtype, int cache_slots,
                                  int slot0, const int32_t* slot_dev, void* stream) {
  const int c = check_k2(qkv, qkv_ld, pos, rope_tab, n_heads, head_dim, max_x, max_y, max_z, px,
                         py, pz, q_out, k_cache, v_cache, out_dtype);
  if (c != MDL_OK) return c;
  if (batch < 0 || seq <= 0) return MDL_ERR_SHAPE;
  if (cache_slots <= 0 || (!slot_dev && (slot0 < 0 || slot0 + seq > cache_slots)))
    return MDL_ERR_CACHE;
  const RopeArgs ra{max_x, max_y, max_z, px, py, pz};
  return launch_k2(qkv, qkv_ld, rstd, pos, rope_tab, static_cast<int64_t>(batch) * seq, seq,
                   n_heads, ra, q_scale, q_out, k_cache, v_cache, out_dtype, cache_slots, slot0,
                   slot_dev, nullptr, nullptr, batch, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_qkv_rope_cache_bf16(const uint16_t* qkv, int64_t qkv_ld, const float* rstd,
                                       const int64_t* pos, const float* rope_tab, int batch,
                                       int seq, int n_heads, int head_dim, int max_x, int max_y,
                                       int max_z, int px, int py, int pz, float q_scale,
                                       uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                       int cache_slots, int slot0, void* stream) {
  if (!qkv || !pos || !rope_tab || !q_out || !k_cache || !v_cache) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (n_heads != 4 && n_heads != 12 && n_heads != 16 && n_heads != 20) return MDL_ERR_SHAPE;
  if (max_x <= 0 || max_y <= 0 || max_z <= 0 || px < 0 || py < 0 || pz < 0 ||
      px + py + pz != kHeadDim / 2 || qkv_ld < 3 * n_heads * 64 || batch < 0 || seq <= 0)
    return MDL_ERR_SHAPE;
  if (cache_slots <= 0 || slot0 < 0 || slot0 + seq > cache_slots) return MDL_ERR_CACHE;
  if (!aligned8(qkv) || qkv_ld % 4 != 0 || !aligned16(q_out) || !aligned16(k_cache) ||
      !aligned16(v_cache) || !aligned4(rope_tab))
    return MDL_ERR_ALIGN;
  const int64_t rows = static_cast<int64_t>(batch) * seq;
  if (rows == 0) return MDL_OK;
  if ((rows + 3) / 4 > 0x7fffffff) return MDL_ERR_SHAPE;
  const RopeArgs ra{max_x, max_y, max_z, px, py, pz};
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool nt = rows * n_heads * kHeadDim * 12 >= kStreamBytes;
#define MDL_K2_BF(NCH)                                                                         \
  if (nt)                                                                                     \
    qkv_rope_cache_vec_kernel<NCH, true, uint16_t><<<grid, 256, 0, st>>>(                     \
        qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, q_scale, q_out, k_cache, v_cache,    \
        cache_slots, slot0, nullptr, nullptr, nullptr, batch);                                \
  else                                                                                        \
    qkv_rope_cache_vec_kernel<NCH, false, uint16_t><<<grid, 256, 0, st>>>(                    \
        qkv, qkv_ld, rstd, pos, rope_tab, ra, rows, seq, q_scale, q_out, k_cache, v_cache,    \
        cache_slots, slot0, nullptr, nullptr, nullptr, batch)
  switch (n_heads) {
    case 4: MDL_K2_BF(3); break;
    case 12: MDL_K2_BF(9); break;
    case 16: MDL_K2_BF(12); break;
    default: MDL_K2_BF(15); break;
  }
#undef MDL_K2_BF
  return launch_status();
}

extern "C" int mdl_qkv_rope_cache_packed(const float* qkv, int64_t qkv_ld, const float* rstd,
                                         const int64_t* pos, const float* rope_tab,
                                         int64_t n_tokens, const int32_t* token_row,
                                         const int32_t* token_slot, int batch, int n_heads,
                                         int head_dim, int max_x, int max_y, int max_z, int px,
                                         int py, int pz, float q_scale, void* q_out,
                                         void* k_cache, void* v_cache, int out_dtype,
                                         int cache_slots, void* stream) {
  const int c = check_k2(qkv, qkv_ld, pos, rope_tab, n_heads, head_dim, max_x, max_y, max_z, px,
                         py, pz, q_out, k_cache, v_cache, out_dtype);
  if (c != MDL_OK) return c;
  if (!token_row || !token_slot) return MDL_ERR_NULL;
  if (n_tokens < 0 || batch < 0 || cache_slots <= 0) return MDL_ERR_SHAPE;
  const RopeArgs ra{max_x, max_y, max_z, px, py, pz};
  return launch_k2(qkv, qkv_ld, rstd, pos, rope_tab, n_tokens, 1, n_heads, ra, q_scale, q_out,
                   k_cache, v_cache, out_dtype, cache_slots, 0, nullptr, token_row, token_slot,
                   batch, static_cast<hipStream_t>(stream));
}
