// K4a -- prefill / full-sequence attention on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
// Block = 4 wavefronts = 64 queries of one (b, h); wave w owns queries q0+16w .. q0+16w+15.
// Key tiles of 64 are staged in LDS: K row-major (A operand of S^T = K Q^T), V transposed
// (A operand of O^T = V^T P^T).  Working with S^T instead of S makes the MFMA accumulator of the
// scores (lane = one query, 4 keys per 16-key block) exactly the B-operand layout P^T needs for
// the second product, so probabilities never leave registers:
//   score block nb (keys 16nb..16nb+15), lane (c = lane%16, g = lane/16) holds keys 16nb+4g+i,
//   i = 0..3, of query c.  The P^T operand of k-step kk takes blocks 2kk and 2kk+1, element j of
//   group g = key 32kk + (j<4 ? 4g+j : 16+4g+j-4).  V^T is stored in LDS with its keys permuted
//   into that same order, so the A operand of each k-step is one 16-byte LDS read.
// An MFMA pairs element j of lane group g in A with element j of group g in B, whatever k that
// is inside the instruction, so any common key order of the two operands is exact.
//
// Online softmax in the log2 domain, fp32 throughout; the per-lane partial row sums are merged
// across the 4 lane groups once at the end.  Queries with no visible key produce 0.  The output
// (the out-projection GEMM input) is written as a hi|lo bf16 pair per row, see common.h.
#include "common.h"

namespace mdl {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 64;          // queries per block
constexpr int kBN = 64;          // keys per tile
constexpr int kLds = 72;         // LDS row stride (bf16 elements): 144 B rows, 16 B aligned
constexpr float kLog2eP = 1.4426950408889634f;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// LDS position of key `k` (0..63) inside a transposed V row (see file comment).
__device__ __forceinline__ int vt_pos(int k) {
  const int nb = k >> 4, w = k & 15;
  return 32 * (nb >> 1) + 8 * (w >> 2) + 4 * (nb & 1) + (w & 3);
}

__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int S, int H, int slots, const uint8_t* __restrict__ kmask,
    const int32_t* __restrict__ kv_start, int causal, uint16_t* __restrict__ out) {
  const int qt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int q0 = qt * kBM;

  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * kLds];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kHeadDim * kLds];
  __shared__ uint8_t Ms[kBN];

  const int qi = q0 + 16 * wave + c16;
  bf16x8_t qf[2];
  if (qi < S) {
    const uint16_t* qp = q + ((static_cast<int64_t>(b) * S + qi) * H + h) * kHeadDim;
    qf[0] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 8 * g));
    qf[1] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 32 + 8 * g));
  } else {
    qf[0] = as_bf16x8(make_uint4(0, 0, 0, 0));
    qf[1] = qf[0];
  }

  const int64_t head_off = (static_cast<int64_t>(b) * H + h) * slots * kHeadDim;
  const uint16_t* Kg = kc + head_off;
  const uint16_t* Vg = vc + head_off;
  const int kstart = kv_start ? kv_start[b] : 0;
  const int kt0 = (kstart / kBN) * kBN;
  const int kend = causal ? min(S, q0 + kBM) : S;

  float m_run = -INFINITY, l_run = 0.f;
  f32x4_t o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int kt = kt0; kt < kend; kt += kBN) {
    __syncthreads();   // the previous tile's LDS readers are done
#pragma unroll
    for (int rep = 0; rep < 2; ++rep) {
      const int ch = tid + rep * 256;
      const int key = ch >> 3, d0 = (ch & 7) * 8;
      const int kj = kt + key;
      uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
      if (kj < S) {
        kv = *reinterpret_cast<const uint4*>(Kg + static_cast<int64_t>(kj) * kHeadDim + d0);
        vv = *reinterpret_cast<const uint4*>(Vg + static_cast<int64_t>(kj) * kHeadDim + d0);
      }
      *reinterpret_cast<uint4*>(&Ks[key * kLds + d0]) = kv;
      const int p = vt_pos(key);
      const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        Vt[(d0 + 2 * i) * kLds + p] = static_cast<uint16_t>(w4[i] & 0xffffu);
        Vt[(d0 + 2 * i + 1) * kLds + p] = static_cast<uint16_t>(w4[i] >> 16);
      }
    }
    if (tid < kBN) {
      const int kj = kt + tid;
      Ms[tid] = (kj < S && kj >= kstart &&
                 (!kmask || kmask[static_cast<int64_t>(b) * S + kj] != 0)) ? 1 : 0;
    }
    __syncthreads();

    // S^T = K Q^T for 4 blocks of 16 keys
    f32x4_t sc[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      sc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8_t a = as_bf16x8(
            *reinterpret_cast<const uint4*>(&Ks[(nb * 16 + c16) * kLds + 32 * kk + 8 * g]));
        sc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[kk], sc[nb], 0, 0, 0);
      }
    }

    float s[4][4];
    float tmax = -INFINITY;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kl = nb * 16 + 4 * g + i;
        const bool ok = Ms[kl] && (!causal || kt + kl <= qi);
        s[nb][i] = ok ? sc[nb][i] * kLog2eP : -INFINITY;
        tmax = fmaxf(tmax, s[nb][i]);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float mnew = fmaxf(m_run, tmax);
    const float alpha = (mnew == -INFINITY) ? 1.f : exp2f(m_run - mnew);
    float psum = 0.f;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = (mnew == -INFINITY) ? 0.f : exp2f(s[nb][i] - mnew);
        s[nb][i] = p;
        psum += p;
      }
    }
    l_run = l_run * alpha + psum;
    m_run = mnew;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= alpha;

    // O^T += V^T P^T, two k-steps of 32 keys
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      uint4 pw;
      pw.x = pack_bf2(s[2 * kk][0], s[2 * kk][1]);
      pw.y = pack_bf2(s[2 * kk][2], s[2 * kk][3]);
      pw.z = pack_bf2(s[2 * kk + 1][0], s[2 * kk + 1][1]);
      pw.w = pack_bf2(s[2 * kk + 1][2], s[2 * kk + 1][3]);
      const bf16x8_t pb = as_bf16x8(pw);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8_t a = as_bf16x8(
            *reinterpret_cast<const uint4*>(&Vt[(16 * db + c16) * kLds + 32 * kk + 8 * g]));
        o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[db], 0, 0, 0);
      }
    }
  }

  float l = l_run + __shfl_xor(l_run, 16, kWave);
  l += __shfl_xor(l, 32, kWave);
  if (qi < S) {
    // output row (b, qi) holds 2*H*64 bf16: hi of every head, then lo of every head
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t d = static_cast<int64_t>(H) * kHeadDim;
    uint16_t* op = out + (static_cast<int64_t>(b) * S + qi) * 2 * d + h * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const float t[4] = {o[db][0] * inv, o[db][1] * inv, o[db][2] * inv, o[db][3] * inv};
      uint2 hi, lo;
      split4(t, hi, lo);
      *reinterpret_cast<uint2*>(op + 16 * db + 4 * g) = hi;
      *reinterpret_cast<uint2*>(op + d + 16 * db + 4 * g) = lo;
    }
  }
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_attn_prefill(const uint16_t* q, const uint16_t* k_cache,
                                const uint16_t* v_cache, int batch, int seq, int n_heads,
                                int head_dim, int cache_slots, const uint8_t* key_mask,
                                const int32_t* kv_start, int causal, uint16_t* out,
                                void* stream) {
  if (!q || !k_cache || !v_cache || !out) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || seq < 0 || n_heads <= 0 || n_heads > 65535 || batch > 65535)
    return MDL_ERR_SHAPE;
  if (seq > cache_slots) return MDL_ERR_CACHE;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned8(out))
    return MDL_ERR_ALIGN;
  if (batch == 0 || seq == 0) return MDL_OK;
  const dim3 grid((seq + kBM - 1) / kBM, n_heads, batch);
  attn_prefill_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      q, k_cache, v_cache, seq, n_heads, cache_slots, key_mask, kv_start, causal ? 1 : 0, out);
  return launch_status();
}
