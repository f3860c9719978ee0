// K4f -- attention over an fp32 static cache on fp32 MFMA (gfx950 v_mfma_f32_16x16x4_f32).
//
// A model whose parameters are fp32 keeps its cache in fp32 (the reference allocates the cache in
// the parameter dtype, src/inference.py:522, :544) and computes its attention in fp32
// (F.scaled_dot_product_attention at src/inference.py:409 and :452).  This kernel is that
// attention for the fp32 form of the inference path: q, K and V enter the products unrounded, the
// scores and probabilities stay fp32, and only the output is stored as the split (hi|lo bf16)
// input of the out projection, which carries it to ~2^-17.
//
// Work item: 16 consecutive query positions of one (batch row, head).  One wave per item, four
// independent waves per block; no LDS and no barrier.  Lane l = (c, g), c = l % 16, g = l / 16.
//
//   S^T = K . Q^T   16 keys x 16 queries, 16 MFMAs of k = 4.  MFMA kb pairs lane group g's
//                   A element K[key c][16 g + kb] with its B element q[query c][16 g + kb], so a
//                   lane loads dims 16 g .. 16 g + 15 of one key row and of one query row: four
//                   float4 each.  The accumulator of lane (c, g) holds S^T[keys 4 g .. 4 g + 3]
//                   [query c].
//   softmax         per query column c over the four lane groups (base 2: q carries the softmax
//                   scale times log2(e)), online across key tiles.
//   O^T = V^T . P^T 64 dims x 16 queries as 4 dim blocks x 4 key steps.  Key step r pairs lane
//                   group g's B element P^T[key 4 g + r][query c] -- accumulator element r of
//                   the score MFMA, no data movement -- with A element V[key 4 g + r][4 c + db] of
//                   dim block db, so a lane loads one float4 (dims 4 c .. 4 c + 3) per key step.
//                   Row i of dim block db's accumulator is dim 4 i + db, so lane (c, g) ends
//                   with dims 16 g .. 16 g + 15 of query c (element r of block db = dim
//                   16 g + 4 r + db).
//
// Modes: prefill over [batch, seq] query rows (row b * seq + i), prefill over a packed token
// list (row q_offset[b] + i - kv_start[b], queries i >= kv_start[b] only), and decode (one query
// per batch row at cache slot t).  Key j is visible to the query at position i iff
// kv_start[b] <= j < n_keys, (causal) j <= i, and (j >= mask_len or mask[b * mask_len + j] != 0);
// a query with no visible key outputs 0 (what torch's CPU SDPA returns for an all -inf row).
// At decode a work item is one split_len-slot chunk of one (row, head): one wave streaming its
// keys a 16-key tile at a time is latency-bound, so the chunks are what fills the GPU.  With
// several chunks each writes its running state (m, l, unnormalised o) to the workspace, and
// attn_f32_combine_kernel merges them.
#include "common.h"
#include "mfma.h"

namespace mdl {

namespace {

constexpr int kQT = 16;          // queries per work item
constexpr int kWavesF = 4;       // independent waves per block

enum Mode { M_PADDED = 0, M_PACKED = 1, M_DECODE = 2 };

struct F32Args {
  const float* q;                // [rows, H, 64], pre-scaled (softmax scale * log2(e))
  const float* kc;               // [batch, H, slots, 64]
  const float* vc;
  const uint8_t* mask;           // [batch, mask_len] or NULL
  int mask_len;
  const int32_t* kv_start;       // [batch] or NULL (0)
  const int32_t* q_offset;       // M_PACKED: [batch]
  const int32_t* seq_dev;        // M_DECODE: slot of the query (NULL: seq_pos)
  int seq_pos;
  int batch, heads, slots, seq;  // seq: prefill query / key count
  int causal;
  int q_tiles;                   // work items per (row, head) (M_DECODE: the chunks)
  int64_t items;
  uint16_t* out;                 // split bf16 [rows, 2 d]
  int out_layout;
  int split_len;                 // M_DECODE: slots per chunk
  float* ws;                     // M_DECODE with more than one chunk: kPartF floats per chunk
};

constexpr int kPartF = 2 + kHeadDim;   // m, l, o[64] of one decode chunk

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int MODE>
__global__ __launch_bounds__(64 * kWavesF) void attn_f32_kernel(const F32Args p) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kWavesF + (threadIdx.x >> 6);
  if (item >= p.items) return;   // whole wave; the kernel has no barrier
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int64_t bh = item / p.q_tiles;
  // the longest query tiles of a row first (causal prefill: the last tiles see the most keys);
  // at decode, the chunk index
  const int qt = p.q_tiles - 1 - static_cast<int>(item - bh * p.q_tiles);
  const int b = static_cast<int>(bh / p.heads), h = static_cast<int>(bh - b * p.heads);
  const int d = p.heads * kHeadDim;

  // key range [klo, n_keys) and this lane's query position / output row
  int n_keys, klo = 0;
  if constexpr (MODE == M_DECODE) {
    const int t = p.seq_dev ? *p.seq_dev : p.seq_pos;
    n_keys = min(t + 1, p.slots);
  } else {
    n_keys = p.seq;
  }
  if (p.kv_start) klo = min(max(p.kv_start[b], 0), n_keys);
  int khi = n_keys;   // keys this item visits: [klo, khi)
  if constexpr (MODE == M_DECODE) {
    klo = min(klo + qt * p.split_len, n_keys);
    khi = min(klo + p.split_len, n_keys);
  }
  int qpos, qfirst;   // this lane's query position; the tile's first position
  int64_t qrow;
  bool qvalid;
  if constexpr (MODE == M_DECODE) {
    qfirst = qpos = n_keys - 1;
    qvalid = c == 0;
    qrow = b;
  } else if constexpr (MODE == M_PACKED) {
    qfirst = klo + kQT * qt;
    qpos = qfirst + c;
    qvalid = qpos < p.seq;
    qrow = static_cast<int64_t>(p.q_offset[b]) + (qvalid ? qpos : qfirst) - klo;
  } else {
    qfirst = kQT * qt;
    qpos = qfirst + c;
    qvalid = qpos < p.seq;
    qrow = static_cast<int64_t>(b) * p.seq + (qvalid ? qpos : qfirst);
  }
  if (qfirst >= p.seq && MODE != M_DECODE) return;   // the whole tile lies past the row
  // keys the tile's last query can see
  if (p.causal && MODE != M_DECODE) khi = min(n_keys, min(qfirst + kQT, p.seq));

  // q: dims 16 g .. 16 g + 15 of query c
  float qv[16];
  {
    const float* qp = p.q + (qrow * p.heads + h) * kHeadDim + 16 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = *reinterpret_cast<const float4*>(qp + 4 * i);
      qv[4 * i] = v.x; qv[4 * i + 1] = v.y; qv[4 * i + 2] = v.z; qv[4 * i + 3] = v.w;
    }
  }
  const int64_t head_base = (static_cast<int64_t>(b) * p.heads + h) * p.slots * kHeadDim;
  const float* K = p.kc + head_base;
  const float* V = p.vc + head_base;
  const uint8_t* mrow = p.mask ? p.mask + static_cast<int64_t>(b) * p.mask_len : nullptr;
  const int qlim = (p.causal || MODE == M_DECODE) ? qpos : n_keys - 1;   // last key for query c

  float m_run = -INFINITY, l_run = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = klo; k0 < khi; k0 += kQT) {
    // S^T: K rows k0 + c (clamped into [0, n_keys); the clamped rows are masked below)
    const float* kp = K + static_cast<int64_t>(min(k0 + c, n_keys - 1)) * kHeadDim + 16 * g;
    float kv[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = *reinterpret_cast<const float4*>(kp + 4 * i);
      kv[4 * i] = v.x; kv[4 * i + 1] = v.y; kv[4 * i + 2] = v.z; kv[4 * i + 3] = v.w;
    }
    float4 vv[4];   // V rows k0 + 4 g + r, dims 4 c .. 4 c + 3
#pragma unroll
    for (int r = 0; r < 4; ++r)
      vv[r] = *reinterpret_cast<const float4*>(
          V + static_cast<int64_t>(min(k0 + 4 * g + r, n_keys - 1)) * kHeadDim + 4 * c);
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 16; ++kb)
      s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[kb], qv[kb], s, 0, 0, 0);

    // visibility of keys k0 + 4 g + r to query c
    float sv[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = k0 + 4 * g + r;
      bool ok = qvalid && j < khi && j <= qlim;
      if (ok && mrow && j < p.mask_len) ok = mrow[j] != 0;
      sv[r] = ok ? s[r] : -INFINITY;
      tmax = fmaxf(tmax, sv[r]);
    }
    tmax = max_over_groups(tmax);
    const float m_new = fmaxf(m_run, tmax);
    float pr[4], psum = 0.f, alpha = 1.f;
    if (m_new == -INFINITY) {
#pragma unroll
      for (int r = 0; r < 4; ++r) pr[r] = 0.f;
    } else {
      alpha = exp2f(m_run - m_new);    // m_run = -inf: 0 (o and l are 0 then)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[r] = exp2f(sv[r] - m_new);  // -inf: 0
        psum += pr[r];
      }
    }
    psum += __shfl_xor(psum, 16, kWave);
    psum += __shfl_xor(psum, 32, kWave);
    l_run = fmaf(l_run, alpha, psum);
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] *= alpha;
    // O^T += V^T . P^T, key step r: lane group g contributes key 4 g + r
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ve[4] = {vv[r].x, vv[r].y, vv[r].z, vv[r].w};
#pragma unroll
      for (int db = 0; db < 4; ++db)
        o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(ve[db], pr[r], o[db], 0, 0, 0);
    }
  }

  if (!qvalid) return;
  if (MODE == M_DECODE && p.ws) {
    // this chunk's state: m and l (the same in every lane of query column 0), o unnormalised;
    // lane (0, g) holds dims 16 g + 4 r + db as element r of block db
    float* part = p.ws + item * kPartF;
    if (g == 0) {
      part[0] = m_run;
      part[1] = l_run;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int db = 0; db < 4; ++db) part[2 + 16 * g + 4 * r + db] = o[db][r];
    return;
  }
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  float res[16];   // dims 16 g + e of query c: element r of block db is dim 16 g + 4 r + db
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int db = 0; db < 4; ++db) res[4 * r + db] = o[db][r] * inv;
  uint4 hi0, lo0, hi1, lo1;
  split8(res, hi0, lo0);
  split8(res + 8, hi1, lo1);
  const int col = h * kHeadDim + 16 * g;
  if (p.out_layout == MDL_LAYOUT_TILES) {
    *reinterpret_cast<uint4*>(p.out + tile_off(qrow, col, 2 * d)) = hi0;
    *reinterpret_cast<uint4*>(p.out + tile_off(qrow, col + 8, 2 * d)) = hi1;
    *reinterpret_cast<uint4*>(p.out + tile_off(qrow, d + col, 2 * d)) = lo0;
    *reinterpret_cast<uint4*>(p.out + tile_off(qrow, d + col + 8, 2 * d)) = lo1;
  } else {
    uint16_t* orow = p.out + qrow * 2 * d;
    *reinterpret_cast<uint4*>(orow + col) = hi0;
    *reinterpret_cast<uint4*>(orow + col + 8) = hi1;
    *reinterpret_cast<uint4*>(orow + d + col) = lo0;
    *reinterpret_cast<uint4*>(orow + d + col + 8) = lo1;
  }
}

// The decode chunks of one (row, head) merged, lane = channel: the states rescaled to their
// largest m (base 2), o / l, stored as the split output of mdl_attn_decode_f32.
__global__ __launch_bounds__(256) void attn_f32_combine_kernel(const float* __restrict__ ws,
                                                               int n_bh, int n_heads,
                                                               int n_split,
                                                               uint16_t* __restrict__ out,
                                                               int out_layout) {
  const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (bh >= n_bh) return;
  const float* part = ws + static_cast<int64_t>(bh) * n_split * kPartF;
  float M = -INFINITY;
  for (int s = 0; s < n_split; ++s) M = fmaxf(M, part[s * kPartF]);
  float L = 0.f, O = 0.f;
  for (int s = 0; s < n_split; ++s) {
    const float ms = part[s * kPartF];
    const float sc = ms == -INFINITY ? 0.f : exp2f(ms - M);
    L = fmaf(part[s * kPartF + 1], sc, L);
    O = fmaf(part[s * kPartF + 2 + lane], sc, O);
  }
  const float v = L > 0.f ? O / L : 0.f;
  const int b = bh / n_heads, h = bh - b * n_heads;
  const int d = n_heads * kHeadDim, col = h * kHeadDim + lane;
  const uint16_t hi = static_cast<uint16_t>(f2bf(v));
  const uint16_t lo = static_cast<uint16_t>(f2bf(v - bf2f(hi)));
  if (out_layout == MDL_LAYOUT_TILES) {
    out[tile_off(b, col, 2 * d)] = hi;
    out[tile_off(b, d + col, 2 * d)] = lo;
  } else {
    out[static_cast<int64_t>(b) * 2 * d + col] = hi;
    out[static_cast<int64_t>(b) * 2 * d + d + col] = lo;
  }
}

template <int MODE>
int launch_f32(F32Args p, hipStream_t st) {
  if (p.items == 0) return MDL_OK;
  const int64_t blocks = (p.items + kWavesF - 1) / kWavesF;
  if (blocks > 0x7fffffff) return MDL_ERR_SHAPE;
  hipLaunchKernelGGL(attn_f32_kernel<MODE>, dim3(static_cast<unsigned>(blocks)),
                     dim3(64 * kWavesF), 0, st, p);
  return launch_status();
}

int check_f32(const float* q, const float* k_cache, const float* v_cache, int batch,
              int n_heads, int head_dim, int cache_slots, const uint16_t* out, int out_layout) {
  if (!q || !k_cache || !v_cache || !out) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || n_heads <= 0 || n_heads > (1 << 16) || cache_slots <= 0 ||
      (out_layout != MDL_LAYOUT_ROWS && out_layout != MDL_LAYOUT_TILES))
    return MDL_ERR_SHAPE;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
    return MDL_ERR_ALIGN;
  return MDL_OK;
}

}  // namespace

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_attn_prefill_f32(const float* q, const float* k_cache, const float* v_cache,
                                    int batch, int seq, int n_heads, int head_dim,
                                    int cache_slots, const uint8_t* key_mask,
                                    const int32_t* kv_start, const int32_t* q_offset, int causal,
                                    uint16_t* out, int out_layout, void* stream) {
  const int rc = check_f32(q, k_cache, v_cache, batch, n_heads, head_dim, cache_slots, out,
                           out_layout);
  if (rc != MDL_OK) return rc;
  if (seq <= 0) return MDL_ERR_SHAPE;
  if (seq > cache_slots) return MDL_ERR_CACHE;
  if (q_offset && !kv_start) return MDL_ERR_NULL;
  F32Args p{};
  p.q = q; p.kc = k_cache; p.vc = v_cache;
  p.mask = key_mask; p.mask_len = seq;
  p.kv_start = kv_start; p.q_offset = q_offset;
  p.batch = batch; p.heads = n_heads; p.slots = cache_slots; p.seq = seq;
  p.causal = causal != 0;
  p.q_tiles = (seq + kQT - 1) / kQT;
  p.items = static_cast<int64_t>(batch) * n_heads * p.q_tiles;
  p.out = out; p.out_layout = out_layout;
  auto st = static_cast<hipStream_t>(stream);
  return q_offset ? launch_f32<M_PACKED>(p, st) : launch_f32<M_PADDED>(p, st);
}

extern "C" int mdl_attn_decode_f32(const float* q, const float* k_cache, const float* v_cache,
                                   int batch, int n_heads, int head_dim, int cache_slots,
                                   const uint8_t* prompt_mask, int prompt_len,
                                   const int32_t* kv_start, int seq_pos, const int32_t* seq_dev,
                                   float* workspace, int64_t workspace_bytes, int split_len,
                                   uint16_t* out, int out_layout, void* stream) {
  const int rc = check_f32(q, k_cache, v_cache, batch, n_heads, head_dim, cache_slots, out,
                           out_layout);
  if (rc != MDL_OK) return rc;
  if (prompt_len < 0 || (prompt_mask && prompt_len == 0) || split_len < kQT ||
      split_len % kQT != 0)
    return MDL_ERR_SHAPE;
  if (!seq_dev && (seq_pos < 0 || seq_pos >= cache_slots)) return MDL_ERR_CACHE;
  const int n_split = (cache_slots + split_len - 1) / split_len;
  const int64_t n_bh = static_cast<int64_t>(batch) * n_heads;
  if (n_split > 1) {
    if (!workspace) return MDL_ERR_WORKSPACE;
    if (workspace_bytes < n_bh * n_split * kPartF * static_cast<int64_t>(sizeof(float)))
      return MDL_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MDL_ERR_ALIGN;
  }
  F32Args p{};
  p.q = q; p.kc = k_cache; p.vc = v_cache;
  p.mask = prompt_mask; p.mask_len = prompt_len;
  p.kv_start = kv_start;
  p.seq_dev = seq_dev; p.seq_pos = seq_pos;
  p.batch = batch; p.heads = n_heads; p.slots = cache_slots; p.seq = cache_slots;
  p.causal = 1;
  p.q_tiles = n_split;
  p.split_len = split_len;
  p.ws = n_split > 1 ? workspace : nullptr;
  p.items = n_bh * n_split;
  p.out = out; p.out_layout = out_layout;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int rc2 = launch_f32<M_DECODE>(p, st);
  if (rc2 != MDL_OK || n_split == 1 || n_bh == 0) return rc2;
  if ((n_bh + 3) / 4 > 0x7fffffff) return MDL_ERR_SHAPE;
  hipLaunchKernelGGL(attn_f32_combine_kernel, dim3(static_cast<unsigned>((n_bh + 3) / 4)),
                     dim3(256), 0, st, workspace, static_cast<int>(n_bh), n_heads, n_split, out,
                     out_layout);
  return launch_status();
}
