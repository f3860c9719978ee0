// Final RMSNorm + LM head + greedy argmax (+ token commit), grid-state initialisation and
// stepping, token commit.
//
// These are the per-step bookkeeping kernels of batched greedy decode: everything the reference
// does between two decode steps on tiny [B] / [B, 14] tensors (about 40 eager launches) becomes
// a couple of launches that keep state on the device, so a decode step needs no host round trip.
#include "common.h"
#include "grid.h"

namespace mdl {

constexpr int kVmax = 32;

// mdl_logit_constraints by value in the kernel arguments (a captured graph keeps them).
struct HeadCons {
  uint32_t disallow;
  const uint8_t* palette;
  float palette_penalty;
  const int32_t* shape;
  const int32_t* gx;
  const int32_t* gy;
  float shape_penalty;
};

// Row r's logit of vocab slot `slot` after the constraints, in the reference's order of
// operations (one fp32 subtraction per penalty).
__device__ __forceinline__ float constrain(float v, int slot, int r, const HeadCons& c) {
  if ((c.disallow >> slot) & 1u) v = -INFINITY;
  const bool colour = slot < 10, newline = slot == kNewline;
  if (c.palette && colour && c.palette[static_cast<int64_t>(r) * 10 + slot] == 0)
    v = v - c.palette_penalty;
  if (c.shape) {
    const int th = c.shape[2 * static_cast<int64_t>(r)];
    const int tw = c.shape[2 * static_cast<int64_t>(r) + 1];
    if (th >= 0 && tw >= 0) {
      const int x = c.gx[r], y = c.gy[r];
      if (x >= tw && colour) v = v - c.shape_penalty;
      if (x < tw && newline) v = v - c.shape_penalty;
      if (y >= th && colour) v = v - c.shape_penalty;
      if (y >= th && newline) v = v - c.shape_penalty;
    }
  }
  return v;
}

// One 256-thread block per output row; wave w owns vocab slots KW*w .. KW*w + KW-1 (KW = NV/4),
// so a launch of B rows fills B blocks across the chip and each lane carries KW rows' worth of
// weight loads (all in flight at once) rather than NV.  Every wave holds the row's NC 4-channel
// chunks of x * gamma and its sum of squares; the lane's partial dot products with the wave's
// KW vocab rows are reduced with a reduce-scatter butterfly (log2(KW) halving levels, then
// 6 - log2(KW) plain levels) that leaves the logit of slot KW*w + (lane >> (6 - log2 KW)) in
// every lane.  The logits, after the constraints, meet in LDS; wave 0 takes the argmax with the
// first index winning ties (torch argmax) and commits the token.
// Weight slots t >= vocab re-read the last vocab row (an L1 hit) instead of branching around
// their loads, which would serialise them; those slots never reach the logits or the argmax.
template <int NC, int NV>
__global__ __launch_bounds__(256) void head_kernel(
    const float* __restrict__ x, const int32_t* __restrict__ row_index, int rows, int d,
    const float* __restrict__ gamma, float eps, const float* __restrict__ w, int vocab,
    float* __restrict__ logits, int64_t* __restrict__ token, int64_t* __restrict__ out_ids,
    int64_t ld, int col, const int32_t* __restrict__ counters, int32_t* __restrict__ finish,
    int gen_base, int64_t end_id, HeadCons cons, int x_tiled) {
  constexpr int KW = NV / 4;                       // vocab slots per wave
  constexpr int LOG_KW = KW == 4 ? 2 : 3;
  __shared__ float lg[NV];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = blockIdx.x;
  if (r >= rows) return;
  const int64_t m = row_index ? row_index[r] : r;
  const float* xr = x + m * d;   // row-major; x_tiled: the fp32 tile layout (tile_off32)
  float v[NC][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (i < NC - 1 || e < d) {
      const float4 a = *reinterpret_cast<const float4*>(x_tiled ? x + tile_off32(m, e, d)
                                                                 : xr + e);
      const float4 gm = *reinterpret_cast<const float4*>(gamma + e);
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      v[i][0] = a.x * gm.x; v[i][1] = a.y * gm.y; v[i][2] = a.z * gm.z; v[i][3] = a.w * gm.w;
    } else {
      v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0.f;
    }
  }
  float acc[KW];
#pragma unroll
  for (int k = 0; k < KW; ++k) {
    const int t = KW * wave + k;
    const float* wr = w + static_cast<int64_t>(t < vocab ? t : vocab - 1) * d;
    acc[k] = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      const int e = 4 * (lane + 64 * i);
      if (i < NC - 1 || e < d) {
        const float4 wv = *reinterpret_cast<const float4*>(wr + e);
        acc[k] += v[i][0] * wv.x + v[i][1] * wv.y + v[i][2] * wv.z + v[i][3] * wv.w;
      }
    }
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / static_cast<float>(d) + eps);
#pragma unroll
  for (int lvl = 0; lvl < LOG_KW; ++lvl) {
    const int half = KW >> (lvl + 1);
    const int mask = 32 >> lvl;
    const bool up = (lane & mask) != 0;
#pragma unroll
    for (int k = 0; k < KW / 2; ++k) {
      if (k < half) {
        const float keep = up ? acc[half + k] : acc[k];
        const float send = up ? acc[k] : acc[half + k];
        acc[k] = keep + __shfl_xor(send, mask, kWave);
      }
    }
  }
  float tot = acc[0];
#pragma unroll
  for (int mask = 32 >> LOG_KW; mask > 0; mask >>= 1) tot += __shfl_xor(tot, mask, kWave);
  const int slot = KW * wave + (lane >> (6 - LOG_KW));
  if ((lane & ((64 >> LOG_KW) - 1)) == 0) {
    float logit = tot * rs;
    if (slot < vocab) {
      logit = constrain(logit, slot, r, cons);
      if (logits) logits[static_cast<int64_t>(r) * vocab + slot] = logit;
    }
    lg[slot] = slot < vocab ? logit : -INFINITY;
  }
  __syncthreads();
  if (wave != 0) return;
  float bv = lane < NV ? lg[lane] : -INFINITY;
  int bi = lane;
#pragma unroll
  for (int mask = NV / 2; mask > 0; mask >>= 1) {
    const float ov = __shfl_xor(bv, mask, kWave);
    const int oi = __shfl_xor(bi, mask, kWave);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane != 0) return;
  if (token) token[r] = bi;
  if (out_ids) {
    const int c = counters ? counters[1] : col;
    if (c < 0 || c >= ld) return;   // more steps than output columns: never write outside
    out_ids[static_cast<int64_t>(r) * ld + c] = bi;
    if (finish && bi == end_id && finish[r] < 0) finish[r] = c - gen_base;
  }
}

__global__ __launch_bounds__(256) void grid_init_kernel(
    const int64_t* __restrict__ ids, const int64_t* __restrict__ pos,
    const uint8_t* __restrict__ mask, const int32_t* __restrict__ row_shift, int batch, int seq,
    int max_x, int max_y, int32_t* gx,
    int32_t* gy, uint8_t* io, int32_t* kv_start, int32_t* last_row, uint8_t* row_holes) {
  // one wavefront per batch row: the lanes scan the mask row together
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= batch) return;
  int n = 0, first = seq;
  if (mask) {
    const uint8_t* mr = mask + static_cast<int64_t>(b) * seq;
    for (int j = lane; j < seq; j += kWave) {
      if (mr[j]) {
        ++n;
        first = min(first, j);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      n += __shfl_xor(n, o, kWave);
      first = min(first, __shfl_xor(first, o, kWave));
    }
  } else {
    n = seq;
    first = 0;
  }
  if (lane != 0) return;
  // the reference reads the token at index len-1 of each row, a right-padding index, in the
  // batch it padded the row in; row_shift maps that index into this (wider) batch
  const int shift = row_shift ? row_shift[b] : 0;
  const int last = clampi(shift + (n > 0 ? n - 1 : 0), 0, seq - 1);
  const int64_t row = static_cast<int64_t>(b) * seq + last;
  const int64_t t = ids[row];
  int64_t x = pos[row * 3], y = pos[row * 3 + 1];
  const int64_t z = pos[row * 3 + 2];
  bool out = z >= 3;
  if (t == kStart) out = false;
  if (t == kSep) out = true;
  if (t == kStart || t == kSep) x = y = 0;
  if (t == kNewline) {
    x = 0;
    y = y + 1 < max_y ? y + 1 : max_y;
  }
  if (t < 10) x = x + 1 < max_x ? x + 1 : max_x;
  x = clampi(x, 0, max_x);
  y = clampi(y, 0, max_y);
  if (n == 0) {
    x = y = 0;
    out = true;
  }
  gx[b] = static_cast<int32_t>(x);
  gy[b] = static_cast<int32_t>(y);
  io[b] = out ? 1 : 0;
  if (kv_start) kv_start[b] = first;
  if (last_row) last_row[b] = static_cast<int32_t>(row);
  // valid positions form one run [first, seq) iff there are seq - first of them
  if (row_holes) row_holes[b] = (n == seq - first) ? 0 : 1;
}

__global__ void grid_step_kernel(const int64_t* __restrict__ token, int batch, int max_x,
                                 int max_y, int32_t* gx, int32_t* gy, uint8_t* io,
                                 int64_t* __restrict__ pos_out, int32_t* counters) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b == 0 && counters) {
    counters[0] = counters[0] + 1;
    counters[1] = counters[1] + 1;
  }
  if (b >= batch) return;
  int32_t x = gx[b], y = gy[b];
  uint8_t o = io[b];
  grid_position_step(token[b], max_x, max_y, x, y, o, pos_out + static_cast<int64_t>(b) * 3);
  gx[b] = x;
  gy[b] = y;
  io[b] = o;
}

__global__ void decode_commit_kernel(const int64_t* __restrict__ token, int batch,
                                     int64_t* __restrict__ out_ids, int64_t ld, int col,
                                     const int32_t* __restrict__ counters,
                                     int32_t* __restrict__ finish, int gen_base, int64_t end_id) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int c = counters ? counters[1] : col;
  if (c < 0 || c >= ld) return;   // more steps than output columns: never write outside
  const int64_t t = token[b];
  out_ids[static_cast<int64_t>(b) * ld + c] = t;
  if (finish && t == end_id && finish[b] < 0) finish[b] = c - gen_base;
}

template <int NC>
struct LaunchHead {
  static void run(int nv, dim3 grid, hipStream_t s, const float* x, const int32_t* row_index,
                  int rows, int d, const float* gamma, float eps, const float* w, int vocab,
                  float* logits, int64_t* token, int64_t* out_ids, int64_t ld, int col,
                  const int32_t* counters, int32_t* finish, int gen_base, int64_t end_id,
                  const HeadCons& cons, int x_tiled) {
    if (nv == 16)
      head_kernel<NC, 16><<<grid, 256, 0, s>>>(x, row_index, rows, d, gamma, eps, w, vocab,
                                               logits, token, out_ids, ld, col, counters, finish,
                                               gen_base, end_id, cons, x_tiled);
    else
      head_kernel<NC, 32><<<grid, 256, 0, s>>>(x, row_index, rows, d, gamma, eps, w, vocab,
                                               logits, token, out_ids, ld, col, counters, finish,
                                               gen_base, end_id, cons, x_tiled);
  }
};

// x in `layout`: the fp32 tile layout needs whole 32-column blocks
inline bool x_layout_ok(int layout, int d) {
  return layout == MDL_LAYOUT_ROWS || (layout == MDL_LAYOUT_TILES && d % 32 == 0);
}

int launch_head(const float* x, const int32_t* row_index, int rows, int d, const float* gamma,
                float eps, const float* w, int vocab, float* logits, int64_t* token,
                int64_t* out_ids, int64_t ld, int col, const int32_t* counters, int32_t* finish,
                int gen_base, int64_t end_id, const mdl_logit_constraints* c, int x_tiled,
                hipStream_t s) {
  HeadCons cons{0u, nullptr, 0.f, nullptr, nullptr, nullptr, 0.f};
  if (c) {
    if (c->target_shape && (!c->grid_x || !c->grid_y)) return MDL_ERR_NULL;
    cons = HeadCons{c->disallow_mask, c->palette_mask, c->palette_penalty, c->target_shape,
                    c->grid_x, c->grid_y, c->shape_penalty};
  }
  const dim3 grid(rows);
  const int nv = vocab <= 16 ? 16 : 32;
#define MDL_HEAD(N)                                                                            \
  case N:                                                                                      \
    LaunchHead<N>::run(nv, grid, s, x, row_index, rows, d, gamma, eps, w, vocab, logits, token, \
                       out_ids, ld, col, counters, finish, gen_base, end_id, cons, x_tiled);   \
    break;
  switch ((d + 255) / 256) { MDL_HEAD(1) MDL_HEAD(2) MDL_HEAD(3) MDL_HEAD(4) MDL_HEAD(5)
                             MDL_HEAD(6) MDL_HEAD(7) MDL_HEAD(8) }
#undef MDL_HEAD
  return launch_status();
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_version(void) { return 200; }

extern "C" const char* mdl_error_string(int code) {
  switch (code) {
    case MDL_OK: return "ok";
    case MDL_ERR_NULL: return "required pointer is NULL";
    case MDL_ERR_ALIGN: return "pointer or leading dimension is misaligned";
    case MDL_ERR_SHAPE: return "dimension out of the supported range";
    case MDL_ERR_HEAD_DIM: return "head_dim must be 64";
    case MDL_ERR_CACHE: return "slot range outside the KV cache";
    case MDL_ERR_WORKSPACE: return "workspace too small";
    case MDL_ERR_DTYPE: return "unsupported dtype code";
    case MDL_ERR_SCRATCH:
      return "work exceeds the static scratch buffer (MDL_DECODE_SCRATCH_BYTES)";
    default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown";
  }
}

extern "C" int mdl_lm_head(const float* x, const int32_t* row_index, int rows, int d,
                           const float* gamma, float eps, const float* w_head, int vocab,
                           float* logits_out, int64_t* token_out,
                           const mdl_logit_constraints* constraints, int x_layout,
                           void* stream) {
  if (!x || !gamma || !w_head) return MDL_ERR_NULL;
  if (rows < 0 || d <= 0 || d % 4 != 0 || d > 2048 || vocab <= 0 || vocab > kVmax ||
      !x_layout_ok(x_layout, d))
    return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(w_head)) return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  return launch_head(x, row_index, rows, d, gamma, eps, w_head, vocab, logits_out, token_out,
                     nullptr, 0, 0, nullptr, nullptr, 0, 0, constraints, x_layout,
                     static_cast<hipStream_t>(stream));
}

extern "C" int mdl_decode_head(const float* x, int batch, int d, const float* gamma, float eps,
                               const float* w_head, int vocab, float* logits_out,
                               int64_t* token_out, int64_t* out_ids, int64_t out_ld, int col,
                               const int32_t* counters, int32_t* finish_step, int gen_base,
                               int end_id, const mdl_logit_constraints* constraints,
                               int x_layout, void* stream) {
  if (!x || !gamma || !w_head || !token_out || !out_ids) return MDL_ERR_NULL;
  if (batch < 0 || d <= 0 || d % 4 != 0 || d > 2048 || vocab <= 0 || vocab > kVmax ||
      out_ld <= 0 || (!counters && (col < 0 || col >= out_ld)) || !x_layout_ok(x_layout, d))
    return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(w_head)) return MDL_ERR_ALIGN;
  if (batch == 0) return MDL_OK;
  return launch_head(x, nullptr, batch, d, gamma, eps, w_head, vocab, logits_out, token_out,
                     out_ids, out_ld, col, counters, finish_step, gen_base, end_id, constraints,
                     x_layout, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_grid_init(const int64_t* ids, const int64_t* pos, const uint8_t* mask,
                             const int32_t* row_shift, int batch, int seq, int max_x, int max_y,
                             int32_t* gx, int32_t* gy, uint8_t* in_out, int32_t* kv_start,
                             int32_t* last_row, uint8_t* row_holes, void* stream) {
  if (!ids || !pos || !gx || !gy || !in_out) return MDL_ERR_NULL;
  if (batch < 0 || seq <= 0 || max_x < 0 || max_y < 0 ||
      static_cast<int64_t>(batch) * seq > INT32_MAX)
    return MDL_ERR_SHAPE;
  if (batch == 0) return MDL_OK;
  grid_init_kernel<<<dim3((batch + 3) / 4), 256, 0, static_cast<hipStream_t>(stream)>>>(
      ids, pos, mask, row_shift, batch, seq, max_x, max_y, gx, gy, in_out, kv_start, last_row,
      row_holes);
  return launch_status();
}

extern "C" int mdl_grid_step(const int64_t* token, int batch, int max_x, int max_y, int32_t* gx,
                             int32_t* gy, uint8_t* in_out, int64_t* pos_out, int32_t* counters,
                             void* stream) {
  if (!token || !gx || !gy || !in_out || !pos_out) return MDL_ERR_NULL;
  if (batch < 0 || max_x < 0 || max_y < 0) return MDL_ERR_SHAPE;
  const int blocks = batch > 0 ? (batch + 255) / 256 : 1;
  grid_step_kernel<<<dim3(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
      token, batch, max_x, max_y, gx, gy, in_out, pos_out, counters);
  return launch_status();
}

extern "C" int mdl_decode_commit(const int64_t* token, int batch, int64_t* out_ids,
                                 int64_t out_ld, int col, const int32_t* counters,
                                 int32_t* finish_step, int gen_base, int end_id, void* stream) {
  if (!token || !out_ids) return MDL_ERR_NULL;
  if (batch < 0 || out_ld <= 0 || (!counters && (col < 0 || col >= out_ld))) return MDL_ERR_SHAPE;
  if (batch == 0) return MDL_OK;
  decode_commit_kernel<<<dim3((batch + 255) / 256), 256, 0, static_cast<hipStream_t>(stream)>>>(
      token, batch, out_ids, out_ld, col, counters, finish_step, gen_base, end_id);
  return launch_status();
}
