// K4b -- decode attention: one query per (row, head) against the static KV cache, on bf16 MFMA.
//
// Split-K flash decoding.  Work item = (b*h, split): a 256-thread block attends over `split_len`
// cache slots of one head; its 4 wavefronts take tiles of kT = 16 NB consecutive slots in turn
// (NB = 2 or 4).  Per tile, on v_mfma_f32_16x16x32_bf16 (operand layouts in mfma.h):
//   S^T = K q^T: the A operand is K -- each wave loads its K tile with coalesced 16-byte loads
//     (eight lanes per 128-byte slot row), stages it in its own LDS region and reads lane
//     (c, g)'s 16 bytes of slot row 16 nb + c at dims 32 kk + 8 g back in the MFMA layout
//     (loading that layout straight from HBM makes every load instruction touch 16 rows and
//     measured 1-3% slower); the B operand is q replicated over the 16 columns, so every lane
//     ends up holding real scores (slots 16 nb + 4 g + i) and the softmax needs no cross-lane
//     gather beyond the 4-group max;
//   O^T = V^T P^T: V is staged through the wave's own LDS tile (row-major, 144-byte rows) and read
//     back transposed (ds_read_b64_tr_b16); P^T comes from the score accumulators, in the key
//     order the transposing reads produce; the row sum is one more MFMA against ones, so it sums
//     the same bf16-rounded probabilities the PV product uses.
// q comes multiplied by the softmax scale and log2(e), so the scores are the exponents of a base-2
// softmax (v_exp_f32).  The single query costs 15/16 of every MFMA, which is free: the kernel
// streams 256 bytes of K/V per slot from HBM and does 2 x 128 useful flops per slot, so MFMA and
// VALU stay far below their rates.  K and V use non-temporal loads (read once per launch; keeps
// the projection weights cached between layers).  The 4 waves, then the splits (second kernel)
// merge with the usual max-rescaled sums.
//
// Slot j of row b is visible iff kv_start[b] <= j <= t and (j >= prompt_len or
// prompt_mask[b, j]), the decode mask of the reference (prompt mask, then every generated slot).
// row_holes[b] == 0 (from mdl_grid_init) says the prompt mask of row b is one contiguous run
// starting at kv_start[b]; such rows skip the per-slot mask reads.
#include <mutex>

#include "mfma.h"
#include "rope.h"


namespace mdl {

constexpr int kPart = 2 + kHeadDim;   // m, l, acc[64] per split

// Channel `lane` of head h = bh % n_heads of batch row b = bh / n_heads into the out-projection
// GEMM input: row b holds 2*n_heads*64 bf16, hi of every head then lo of every head (row-major,
// or MFMA tiles when `tiled`).
__device__ __forceinline__ void store_split(uint16_t* out, int bh, int n_heads, int lane,
                                            float o, int tiled) {
  const int b = bh / n_heads, h = bh - b * n_heads;
  const int d = n_heads * kHeadDim;
  const int j = h * kHeadDim + lane;
  const uint32_t hi = f2bf(o);
  const uint16_t lo = static_cast<uint16_t>(f2bf(o - bf2f(hi)));
  if (tiled) {
    out[tile_off(b, j, 2 * d)] = static_cast<uint16_t>(hi);
    out[tile_off(b, d + j, 2 * d)] = lo;
  } else {
    uint16_t* p = out + static_cast<int64_t>(b) * 2 * d + j;
    p[0] = static_cast<uint16_t>(hi);
    p[d] = lo;
  }
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

constexpr int kVld = 72;      // LDS row stride of a staged V tile (bf16): 144-byte rows

// FUSED: the block first does K2's work for its own (row, head) -- wave 0 rotates q (lanes
// 0-31, one pair each) and k (lanes 32-63) of the decode token, rounds q to bf16 exactly as K2
// does and hands it to the other waves through LDS, and the block whose slot range holds t
// writes the token's K/V into cache slot t -- then attends as the unfused kernel.  The cache
// row is stored before the barrier and read after it, so the block sees its own write.
// NB: 16-slot score blocks per wave tile.
template <bool FUSED, int NB>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const uint16_t* __restrict__ q, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    int n_heads, int slots, const uint8_t* __restrict__ pmask, int plen,
    const uint8_t* __restrict__ row_holes, const int32_t* __restrict__ kv_start,
    const int32_t* __restrict__ row_order, int seq_pos, const int32_t* __restrict__ seq_dev,
    int n_split, int split_len, float* __restrict__ ws, uint16_t* __restrict__ out,
    int out_tiled, RopeIn rin) {
  const int ri = blockIdx.x / n_heads;
  const int n_rows = gridDim.x / n_heads;
  const int b = row_order ? min(max(row_order[ri], 0), n_rows - 1) : ri;
  const int bh = b * n_heads + (blockIdx.x - ri * n_heads);
  const int split = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, g = lane >> 4;
  const int t = seq_dev ? *seq_dev : seq_pos;
  const int start = kv_start ? kv_start[b] : 0;
  const int lo = start + split * split_len;
  const int hi = min(lo + split_len, min(t + 1, slots));

  __shared__ float red[4][kPart];
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[kHeadDim];
  constexpr int kT = 16 * NB;   // slots per wave tile
  __shared__ __attribute__((aligned(16))) uint16_t Vs[4][kT * kVld];
  __shared__ __attribute__((aligned(16))) uint16_t Ks[4][kT * kVld];

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
      float y0, y1;
      rope_rot(x0, x1, cs, sn, y0, y1);
      const bool writes = t >= lo && t < lo + split_len && t < slots;
      const int64_t slot_row = (static_cast<int64_t>(bh) * slots + t) * kHeadDim;
      if (!is_k) {
        *reinterpret_cast<uint32_t*>(q_lds + 2 * j) = pack_bf2(y0 * rin.q_scale,
                                                               y1 * rin.q_scale);
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

  float m = -INFINITY;
  f32x4_t lsum = {0.f, 0.f, 0.f, 0.f}, o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (lo < hi) {
    bf16x8_t qf[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      qf[kk] = as_bf16x8(
          FUSED ? *reinterpret_cast<const uint4*>(q_lds + 32 * kk + 8 * g)
                : *reinterpret_cast<const uint4*>(q + static_cast<int64_t>(bh) * kHeadDim +
                                                  32 * kk + 8 * g));
    const bf16x8_t ones = bf16_ones8();
    const uint16_t* K = kc + static_cast<int64_t>(bh) * slots * kHeadDim;
    const uint16_t* V = vc + static_cast<int64_t>(bh) * slots * kHeadDim;
    const bool dense = row_holes && row_holes[b] == 0;
    const uint8_t* pm = (pmask && !dense) ? pmask + static_cast<int64_t>(b) * plen : nullptr;
    uint16_t* Vw = Vs[wave];
    uint16_t* Kw = Ks[wave];

    for (int base = lo + wave * kT; base < hi; base += 4 * kT) {
      uint4 kf[NB][2], kr[2 * NB], vr[2 * NB];
#pragma unroll
      for (int r = 0; r < 2 * NB; ++r) {
        const int key = base + 8 * r + (lane >> 3);
        kr[r] = key < hi ? load_nt16(K + static_cast<int64_t>(key) * kHeadDim + 8 * (lane & 7))
                         : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 2 * NB; ++r) {
        const int key = base + 8 * r + (lane >> 3);
        vr[r] = key < hi ? load_nt16(V + static_cast<int64_t>(key) * kHeadDim + 8 * (lane & 7))
                         : make_uint4(0, 0, 0, 0);
      }
      // the K tile through this wave's LDS region, read back in the MFMA A layout (same
      // program-order hand-over as the V tile below; 144-byte rows keep the 16-byte reads of a
      // lane group on distinct banks)
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = 0; r < 2 * NB; ++r)
        *reinterpret_cast<uint4*>(Kw + (8 * r + (lane >> 3)) * kVld + 8 * (lane & 7)) = kr[r];
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          kf[nb][kk] = *reinterpret_cast<const uint4*>(Kw + (16 * nb + c16) * kVld + 32 * kk +
                                                       8 * g);
      f32x4_t sc[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        sc[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          sc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[nb][kk]), qf[kk],
                                                           sc[nb], 0, 0, 0);
      }
      // Vw is this wave's alone, and LDS operations of one wavefront execute in issue order, so
      // program order is all that the tile hand-over needs: the wavefront-scope fences keep the
      // compiler from moving the stores above the previous tile's transposing reads (here) or
      // below this tile's (further down)
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int r = 0; r < 2 * NB; ++r)
        *reinterpret_cast<uint4*>(Vw + (8 * r + (lane >> 3)) * kVld + 8 * (lane & 7)) = vr[r];
      // score block nb, element i of lane group g is slot base + 16 nb + 4 g + i
      if (base + kT > hi || pm) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = base + 16 * nb + 4 * g + i;
            const bool vis = key < hi && (!pm || key >= plen || pm[key] != 0);
            if (!vis) sc[nb][i] = -INFINITY;
          }
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, sc[nb][i]);
      tmax = max_over_groups(tmax);
      const float mnew = fmaxf(m, tmax);   // q carries log2(e): scores are log2-domain
      const float mb = (mnew == -INFINITY) ? 0.f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(m - mb);
      m = mnew;
      lsum *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          sc[nb][i] = __builtin_amdgcn_exp2f(sc[nb][i] - mb);
      bf16x8_t pb[NB / 2];
#pragma unroll
      for (int kk = 0; kk < NB / 2; ++kk) pb[kk] = pt_operand(sc[2 * kk], sc[2 * kk + 1]);
      // the staged V tile is visible to the whole wave (program order, as above)
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int kk = 0; kk < NB / 2; ++kk) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt_operand(Vw, kVld, kk, db, c16, g),
                                                          pb[kk], o[db], 0, 0, 0);
        lsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[kk], lsum, 0, 0, 0);
      }
    }
  }

  // every column of the replicated products holds the same values: lanes 0, 16, 32, 48 publish
  if (c16 == 0) {
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[wave][2 + 16 * db + 4 * g + i] = o[db][i];
    if (g == 0) {
      red[wave][0] = m;
      red[wave][1] = lsum[0];
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
      store_split(out, bh, n_heads, lane, L > 0.f ? O / L : 0.f, out_tiled);
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
                                                                  uint16_t* __restrict__ out,
                                                                  int out_tiled) {
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
  store_split(out, bh, n_heads, lane, L > 0.f ? O / L : 0.f, out_tiled);
}

constexpr int kSlotsPerIter = 128;   // split_len granularity
// Work items that can exceed this many slots take 64-slot wave tiles, shorter ones 32-slot
// tiles (measured: 32 is 1-3% faster at config 2's items of at most 2,048 slots, 64 faster at
// configs 3 and 4, whose items run to 3,300-4,100 slots).
constexpr int kLongItem = 2048;

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
                       int split_len, uint16_t* out, int out_layout, void* stream) {
  if ((!fused && !q) || !k_cache || !v_cache || !out) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || n_heads <= 0 || cache_slots <= 0 || prompt_len < 0 ||
      (prompt_mask && prompt_len == 0) || split_len < kSlotsPerIter ||
      split_len % kSlotsPerIter != 0 ||
      (out_layout != MDL_LAYOUT_ROWS && out_layout != MDL_LAYOUT_TILES))
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
  const bool long_items = std::min(split_len, cache_slots) > kLongItem;
#define MDL_DECODE(FUSED, NB)                                                                  \
  attn_decode_kernel<FUSED, NB><<<grid, 256, 0, s>>>(                                          \
      q, k_cache, v_cache, n_heads, cache_slots, prompt_mask, prompt_len, row_holes, kv_start, \
      row_order, seq_pos, seq_dev, ns, split_len, workspace, out, out_layout, rin)
  if (fused) {
    if (long_items) MDL_DECODE(true, 4);
    else MDL_DECODE(true, 2);
  } else {
    if (long_items) MDL_DECODE(false, 4);
    else MDL_DECODE(false, 2);
  }
#undef MDL_DECODE
  if (ns > 1)
    attn_decode_combine_kernel<<<dim3((n_bh + 3) / 4), 256, 0, s>>>(workspace, n_bh, n_heads,
                                                                     ns, out, out_layout);
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
                               int out_layout, void* stream) {
  const RopeIn none{};
  return decode_impl(false, none, q, const_cast<uint16_t*>(k_cache),
                     const_cast<uint16_t*>(v_cache), batch, n_heads, head_dim, cache_slots,
                     prompt_mask, prompt_len, row_holes, kv_start, row_order, seq_pos, seq_dev,
                     workspace, workspace_bytes, split_len, out, out_layout, stream);
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
                                    int out_layout, void* stream) {
  if (!qkv || !rstd || !pos || !rope_tab) return MDL_ERR_NULL;
  if (max_x <= 0 || max_y <= 0 || max_z <= 0 || px < 0 || py < 0 || pz < 0 ||
      px + py + pz != kHeadDim / 2 || n_heads <= 0 || qkv_ld < 3 * int64_t(n_heads) * kHeadDim)
    return MDL_ERR_SHAPE;
  if (!aligned16(qkv) || qkv_ld % 4 != 0 || !aligned4(rope_tab)) return MDL_ERR_ALIGN;
  const RopeIn rin{qkv, qkv_ld, rstd, pos, rope_tab, RopeArgs{max_x, max_y, max_z, px, py, pz},
                   q_scale};
  return decode_impl(true, rin, nullptr, k_cache, v_cache, batch, n_heads, head_dim,
                     cache_slots, prompt_mask, prompt_len, row_holes, kv_start, row_order,
                     seq_pos, seq_dev, workspace, workspace_bytes, split_len, out, out_layout,
                     stream);
}

// ------------------------------------------------------------ no-allocation variant
//
// The split partials of mdl_attn_decode_rope_noalloc live in `scratch`, one fixed array per
// device (the code object's own copy on each GPU it is loaded on, held until the process ends).
// Every split block writes all kPart floats of its partial before the combine kernel reads them,
// so nothing in it has to start at zero.  Host code never passes `scratch` itself (in host code
// the name is only a stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, once per device, with that device current.

static __device__ __align__(256) float scratch[MDL_DECODE_SCRATCH_BYTES / sizeof(float)];

namespace mdl {

constexpr int kMaxDevices = 256;

// Device address of `scratch` on the current device, looked up on the first call per device.
static int scratch_for_current_device(float** ptr) {
  static std::mutex mu;
  static float* addr[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return MDL_ERR_SHAPE;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    addr[dev] = static_cast<float*>(p);
  }
  *ptr = addr[dev];
  return MDL_OK;
}

}  // namespace mdl

extern "C" int mdl_attn_decode_rope_noalloc(
    const float* qkv, int64_t qkv_ld, const float* rstd, const int64_t* pos,
    const float* rope_tab, int max_x, int max_y, int max_z, int px, int py, int pz,
    float q_scale, uint16_t* k_cache, uint16_t* v_cache, int batch, int n_heads, int head_dim,
    int cache_slots, const uint8_t* prompt_mask, int prompt_len, const uint8_t* row_holes,
    const int32_t* kv_start, const int32_t* row_order, int seq_pos, const int32_t* seq_dev,
    int split_len, uint16_t* out, int out_layout, void* stream) {
  const int64_t need = mdl_attn_decode_workspace_bytes(batch, n_heads, cache_slots, split_len);
  if (need > MDL_DECODE_SCRATCH_BYTES) return MDL_ERR_SCRATCH;
  float* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_for_current_device(&ws);
    if (rc != MDL_OK) return rc;
  }
  return mdl_attn_decode_rope(qkv, qkv_ld, rstd, pos, rope_tab, max_x, max_y, max_z, px, py, pz,
                              q_scale, k_cache, v_cache, batch, n_heads, head_dim, cache_slots,
                              prompt_mask, prompt_len, row_holes, kv_start, row_order, seq_pos,
                              seq_dev, ws, need, split_len, out, out_layout, stream);
}
