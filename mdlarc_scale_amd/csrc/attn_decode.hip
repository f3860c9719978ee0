// K4b -- decode attention: one query per (row, head) against the static KV cache.
//
// Split-K flash decoding.  Work item = (b*h, split): a 256-thread block streams `split_len`
// cache slots of one head.  Inside a wavefront, lane = 8*grp + sub: the 8 lanes of a group own
// one slot at a time and `sub` selects 8 of the 64 channels, so one 16-byte load per lane covers
// 8 consecutive slots = 1 KiB of contiguous K (then V).  U slots per group are loaded before any
// arithmetic, so each lane keeps 2*U 16-byte loads in flight.  Scores are reduced over the 8
// lanes of a group with 3 xor-shuffles; every group keeps its own online-softmax state (max, sum,
// 8 accumulators) in the log2 domain.  At the end the 8 groups, then the 4 waves (LDS), then the
// splits (second kernel) are merged with the usual max-rescaled sums.  K and V are streamed with
// non-temporal loads (read once per launch; keeps the projection weights cached between layers).
//
// Slot j of row b is visible iff kv_start[b] <= j <= t and (j >= prompt_len or
// prompt_mask[b, j]), the decode mask of the reference (prompt mask, then every generated slot).
// row_holes[b] == 0 (from mdl_grid_init) says the prompt mask of row b is one contiguous run
// starting at kv_start[b]; such rows skip the per-slot mask reads.
#include "common.h"
#include "rope.h"

namespace mdl {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kPart = 2 + kHeadDim;   // m, l, acc[64] per split

// Channel `lane` of head h = bh % n_heads of batch row b = bh / n_heads into the out-projection
// GEMM input: row b holds 2*n_heads*64 bf16, hi of every head then lo of every head.
__device__ __forceinline__ void store_split(uint16_t* out, int bh, int n_heads, int lane,
                                            float o) {
  const int b = bh / n_heads, h = bh - b * n_heads;
  const int64_t d = static_cast<int64_t>(n_heads) * kHeadDim;
  uint16_t* p = out + static_cast<int64_t>(b) * 2 * d + h * kHeadDim + lane;
  const uint32_t hi = f2bf(o);
  p[0] = static_cast<uint16_t>(hi);
  p[d] = static_cast<uint16_t>(f2bf(o - bf2f(hi)));
}

// K2 inputs for the fused variant: the fp32 qkv GEMM output of the decode token of each row.
struct RopeIn {
  const float* qkv;
  int64_t ld;
  const float* rstd;
  const int64_t* pos;
  const float* tab;
  RopeArgs ra;
  float q_scale;
};

// FUSED: the block first does K2's work for its own (row, head) -- wave 0 rotates q (lanes
// 0-31, one pair each) and k (lanes 32-63) of the decode token, rounds q to bf16 exactly as K2
// does and hands it to the other waves through LDS, and the block whose slot range holds t
// writes the token's K/V into cache slot t -- then attends as the unfused kernel.  The cache
// row is stored before the barrier and read after it, so the block sees its own write.
template <int U, bool FUSED>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const uint16_t* __restrict__ q, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    int n_heads, int slots, const uint8_t* __restrict__ pmask, int plen,
    const uint8_t* __restrict__ row_holes, const int32_t* __restrict__ kv_start,
    const int32_t* __restrict__ row_order, int seq_pos, const int32_t* __restrict__ seq_dev,
    int n_split, int split_len, float* __restrict__ ws, uint16_t* __restrict__ out,
    RopeIn rin) {
  // blocks are dispatched in blockIdx order; row_order lists the rows longest-first so the
  // short rows fill the tail of the launch
  const int ri = blockIdx.x / n_heads;
  const int n_rows = gridDim.x / n_heads;
  // a caller's bad permutation entry is clamped into range: wrong rows, never a wild address
  const int b = row_order ? min(max(row_order[ri], 0), n_rows - 1) : ri;
  const int bh = b * n_heads + (blockIdx.x - ri * n_heads);
  const int split = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int grp = lane >> 3;
  const int sub = lane & 7;
  const int t = seq_dev ? *seq_dev : seq_pos;
  const int start = kv_start ? kv_start[b] : 0;
  const int lo = start + split * split_len;
  const int hi = min(lo + split_len, min(t + 1, slots));

  __shared__ float red[4][kPart];
  __shared__ float q_lds[FUSED ? kHeadDim : 1];

  if (FUSED) {
    if (wave == 0) {
      const int h = bh - b * n_heads;
      const int d = n_heads * kHeadDim;
      const float* row = rin.qkv + static_cast<int64_t>(b) * rin.ld;
      const bool is_k = lane >= 32;
      const int j = lane & 31;
      float cs, sn;
      rope_cos_sin(j, rin.pos + static_cast<int64_t>(b) * 3, rin.tab, rin.ra, cs, sn);
      const float r = rin.rstd[b];
      const float2 a = *reinterpret_cast<const float2*>(row + (is_k ? d : 0) + h * kHeadDim +
                                                        2 * j);
      const float x0 = a.x * r, x1 = a.y * r;
      const float y0 = x0 * cs - x1 * sn, y1 = x1 * cs + x0 * sn;
      const bool writes = t >= lo && t < lo + split_len && t < slots;
      const int64_t slot_row = (static_cast<int64_t>(bh) * slots + t) * kHeadDim;
      if (!is_k) {
        const uint32_t qb = pack_bf2(y0 * rin.q_scale, y1 * rin.q_scale);
        q_lds[2 * j] = bf2f(qb & 0xffffu);
        q_lds[2 * j + 1] = bf2f(qb >> 16);
      } else if (writes) {
        *reinterpret_cast<uint32_t*>(kc + slot_row + 2 * j) = pack_bf2(y0, y1);
      }
      if (writes && lane < kHeadDim / 4) {
        const float4 v = *reinterpret_cast<const float4*>(row + 2 * d + h * kHeadDim + 4 * lane);
        uint2 o;
        o.x = pack_bf2(v.x * r, v.y * r);
        o.y = pack_bf2(v.z * r, v.w * r);
        *reinterpret_cast<uint2*>(vc + slot_row + 4 * lane) = o;
      }
      __threadfence_block();
    }
    __syncthreads();
  }

  float m = -INFINITY, l = 0.f, acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;

  if (lo < hi) {
    float qf[8];
    if (FUSED) {
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[i] = q_lds[sub * 8 + i];
    } else {
      unpack8(*reinterpret_cast<const uint4*>(q + static_cast<int64_t>(bh) * kHeadDim + sub * 8),
              qf);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[i] *= kLog2e;
    const uint16_t* K = kc + static_cast<int64_t>(bh) * slots * kHeadDim + sub * 8;
    const uint16_t* V = vc + static_cast<int64_t>(bh) * slots * kHeadDim + sub * 8;
    // rows whose prompt mask is one contiguous run from kv_start need no per-slot mask reads
    const bool dense = row_holes && row_holes[b] == 0;
    const uint8_t* pm = (pmask && !dense) ? pmask + static_cast<int64_t>(b) * plen : nullptr;

    for (int base = lo + wave * 8 * U; base < hi; base += 4 * 8 * U) {
      uint4 kr[U], vr[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * 8 + grp;
        ok[u] = j < hi;
        if (ok[u]) {
          kr[u] = load_nt16(K + static_cast<int64_t>(j) * kHeadDim);
          vr[u] = load_nt16(V + static_cast<int64_t>(j) * kHeadDim);
          if (pm && j < plen) ok[u] = pm[j] != 0;
        } else {
          kr[u] = make_uint4(0, 0, 0, 0);
          vr[u] = make_uint4(0, 0, 0, 0);
        }
      }
      float s[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float kf[8];
        unpack8(kr[u], kf);
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) a += qf[i] * kf[i];
        a += __shfl_xor(a, 1, kWave);
        a += __shfl_xor(a, 2, kWave);
        a += __shfl_xor(a, 4, kWave);
        s[u] = ok[u] ? a : -INFINITY;
      }
      float mx = m;
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u]);
      if (mx == -INFINITY) continue;
      const float alpha = exp2f(m - mx);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2f(s[u] - mx);
        l += p;
        float vf[8];
        unpack8(vr[u], vf);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += p * vf[i];
      }
      m = mx;
    }
  }

  // merge the 8 slot groups of this wave
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
    const float mo = __shfl_xor(m, off, kWave);
    const float lo2 = __shfl_xor(l, off, kWave);
    const float mn = fmaxf(m, mo);
    const float a = (m == -INFINITY) ? 0.f : exp2f(m - mn);
    const float c = (mo == -INFINITY) ? 0.f : exp2f(mo - mn);
    l = l * a + lo2 * c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ao = __shfl_xor(acc[i], off, kWave);
      acc[i] = acc[i] * a + ao * c;
    }
    m = mn;
  }
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) red[wave][2 + sub * 8 + i] = acc[i];
    if (sub == 0) {
      red[wave][0] = m;
      red[wave][1] = l;
    }
  }
  __syncthreads();
  if (wave == 0) {
    float M = red[0][0];
#pragma unroll
    for (int w = 1; w < 4; ++w) M = fmaxf(M, red[w][0]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float mw = red[w][0];
      const float sc = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
      L += red[w][1] * sc;
      O += red[w][2 + lane] * sc;
    }
    if (n_split == 1) {
      store_split(out, bh, n_heads, lane, L > 0.f ? O / L : 0.f);
    } else {
      float* p = ws + (static_cast<int64_t>(bh) * n_split + split) * kPart;
      if (lane == 0) {
        p[0] = M;
        p[1] = L;
      }
      p[2 + lane] = O;
    }
  }
}

// Merge the per-split partial states of one (b, h): lane = channel.
__global__ __launch_bounds__(256) void attn_decode_combine_kernel(const float* __restrict__ ws,
                                                                  int n_bh, int n_heads,
                                                                  int n_split,
                                                                  uint16_t* __restrict__ out) {
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (bh >= n_bh) return;
  const float* p = ws + static_cast<int64_t>(bh) * n_split * kPart;
  float M = -INFINITY;
  for (int s = 0; s < n_split; ++s) M = fmaxf(M, p[s * kPart]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < n_split; ++s) {
    const float ms = p[s * kPart];
    const float sc = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
    L += p[s * kPart + 1] * sc;
    O += p[s * kPart + 2 + lane] * sc;
  }
  store_split(out, bh, n_heads, lane, L > 0.f ? O / L : 0.f);
}

constexpr int kUnroll = 4;
constexpr int kSlotsPerIter = 4 * 8 * kUnroll;   // slots a block consumes per loop trip

static int n_splits(int cache_slots, int split_len) {
  return (cache_slots + split_len - 1) / split_len;
}

}  // namespace mdl

using namespace mdl;

extern "C" int64_t mdl_attn_decode_workspace_bytes(int batch, int n_heads, int cache_slots,
                                                   int split_len) {
  if (batch <= 0 || n_heads <= 0 || cache_slots <= 0 || split_len <= 0) return 0;
  const int ns = n_splits(cache_slots, split_len);
  if (ns <= 1) return 0;
  return static_cast<int64_t>(batch) * n_heads * ns * kPart * static_cast<int64_t>(sizeof(float));
}

namespace mdl {

static int decode_impl(bool fused, const RopeIn& rin, const uint16_t* q, uint16_t* k_cache,
                       uint16_t* v_cache, int batch, int n_heads, int head_dim, int cache_slots,
                       const uint8_t* prompt_mask, int prompt_len, const uint8_t* row_holes,
                       const int32_t* kv_start, const int32_t* row_order, int seq_pos,
                       const int32_t* seq_dev, float* workspace, int64_t workspace_bytes,
                       int split_len, uint16_t* out, void* stream) {
  if ((!fused && !q) || !k_cache || !v_cache || !out) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || n_heads <= 0 || cache_slots <= 0 || prompt_len < 0 ||
      (prompt_mask && prompt_len == 0) || split_len < kSlotsPerIter ||
      split_len % kSlotsPerIter != 0)
    return MDL_ERR_SHAPE;
  if (!seq_dev && (seq_pos < 0 || seq_pos >= cache_slots)) return MDL_ERR_CACHE;
  if ((!fused && !aligned16(q)) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned4(out))
    return MDL_ERR_ALIGN;
  if (batch == 0) return MDL_OK;
  const int ns = n_splits(cache_slots, split_len);
  const int64_t need = mdl_attn_decode_workspace_bytes(batch, n_heads, cache_slots, split_len);
  if (need > 0 && (!workspace || workspace_bytes < need)) return MDL_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int n_bh = batch * n_heads;
  const dim3 grid(n_bh, ns);
  if (fused)
    attn_decode_kernel<kUnroll, true><<<grid, 256, 0, s>>>(
        q, k_cache, v_cache, n_heads, cache_slots, prompt_mask, prompt_len, row_holes,
        kv_start, row_order, seq_pos, seq_dev, ns, split_len, workspace, out, rin);
  else
    attn_decode_kernel<kUnroll, false><<<grid, 256, 0, s>>>(
        q, k_cache, v_cache, n_heads, cache_slots, prompt_mask, prompt_len, row_holes,
        kv_start, row_order, seq_pos, seq_dev, ns, split_len, workspace, out, rin);
  if (ns > 1)
    attn_decode_combine_kernel<<<dim3((n_bh + 3) / 4), 256, 0, s>>>(workspace, n_bh, n_heads,
                                                                     ns, out);
  return launch_status();
}

}  // namespace mdl

extern "C" int mdl_attn_decode(const uint16_t* q, const uint16_t* k_cache,
                               const uint16_t* v_cache, int batch, int n_heads, int head_dim,
                               int cache_slots, const uint8_t* prompt_mask, int prompt_len,
                               const uint8_t* row_holes, const int32_t* kv_start,
                               const int32_t* row_order, int seq_pos,
                               const int32_t* seq_dev, float* workspace,
                               int64_t workspace_bytes, int split_len, uint16_t* out,
                               void* stream) {
  const RopeIn none{};
  return decode_impl(false, none, q, const_cast<uint16_t*>(k_cache),
                     const_cast<uint16_t*>(v_cache), batch, n_heads, head_dim, cache_slots,
                     prompt_mask, prompt_len, row_holes, kv_start, row_order, seq_pos, seq_dev,
                     workspace, workspace_bytes, split_len, out, stream);
}

extern "C" int mdl_attn_decode_rope(const float* qkv, int64_t qkv_ld, const float* rstd,
                                    const int64_t* pos, const float* rope_tab, int max_x,
                                    int max_y, int max_z, int px, int py, int pz, float q_scale,
                                    uint16_t* k_cache, uint16_t* v_cache, int batch,
                                    int n_heads, int head_dim, int cache_slots,
                                    const uint8_t* prompt_mask, int prompt_len,
                                    const uint8_t* row_holes, const int32_t* kv_start,
                                    const int32_t* row_order, int seq_pos,
                                    const int32_t* seq_dev, float* workspace,
                                    int64_t workspace_bytes, int split_len, uint16_t* out,
                                    void* stream) {
  if (!qkv || !rstd || !pos || !rope_tab) return MDL_ERR_NULL;
  if (max_x <= 0 || max_y <= 0 || max_z <= 0 || px < 0 || py < 0 || pz < 0 ||
      px + py + pz != kHeadDim / 2 || n_heads <= 0 || qkv_ld < 3 * int64_t(n_heads) * kHeadDim)
    return MDL_ERR_SHAPE;
  if (!aligned16(qkv) || qkv_ld % 4 != 0 || !aligned4(rope_tab)) return MDL_ERR_ALIGN;
  const RopeIn rin{qkv, qkv_ld, rstd, pos, rope_tab, RopeArgs{max_x, max_y, max_z, px, py, pz},
                   q_scale};
  return decode_impl(true, rin, nullptr, k_cache, v_cache, batch, n_heads, head_dim,
                     cache_slots, prompt_mask, prompt_len, row_holes, kv_start, row_order,
                     seq_pos, seq_dev, workspace, workspace_bytes, split_len, out, stream);
}
