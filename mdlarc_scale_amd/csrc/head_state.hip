// Final RMSNorm + LM head + greedy argmax, grid-state position tracking and token commit.
//
// These are the per-step bookkeeping kernels of batched greedy decode: everything the reference
// does between two decode steps on tiny [B] / [B, 14] tensors (about 40 eager launches) becomes
// three launches that keep state on the device, so a decode step needs no host round trip.
#include "common.h"

namespace mdl {

constexpr int kVmax = 32;

// One wavefront per output row.  The lane keeps 4-channel chunks of x in registers, reduces the
// sum of squares, then accumulates all vocab dot products at once and reduces them together.
template <int NC>
__global__ __launch_bounds__(256) void lm_head_kernel(const float* __restrict__ x,
                                                      const int32_t* __restrict__ row_index,
                                                      int rows, int d,
                                                      const float* __restrict__ gamma, float eps,
                                                      const float* __restrict__ w, int vocab,
                                                      float* __restrict__ logits,
                                                      int64_t* __restrict__ token) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int64_t m = row_index ? row_index[r] : r;
  const float* xr = x + m * d;
  float v[NC][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (e < d) {
      const float4 a = *reinterpret_cast<const float4*>(xr + e);
      const float4 gm = *reinterpret_cast<const float4*>(gamma + e);
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      v[i][0] = a.x * gm.x; v[i][1] = a.y * gm.y; v[i][2] = a.z * gm.z; v[i][3] = a.w * gm.w;
    } else {
      v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0.f;
    }
  }
  ss = wave_sum(ss);
  const float rs = rsqrtf(ss / static_cast<float>(d) + eps);
  float acc[kVmax];
#pragma unroll
  for (int t = 0; t < kVmax; ++t) {
    acc[t] = 0.f;
    if (t < vocab) {
#pragma unroll
      for (int i = 0; i < NC; ++i) {
        const int e = 4 * (lane + 64 * i);
        if (e < d) {
          const float4 wv = *reinterpret_cast<const float4*>(w + static_cast<int64_t>(t) * d + e);
          acc[t] += v[i][0] * wv.x + v[i][1] * wv.y + v[i][2] * wv.z + v[i][3] * wv.w;
        }
      }
      acc[t] = wave_sum(acc[t]) * rs;
    }
  }
  if (lane == 0) {
    int best = 0;
    float bv = acc[0];
#pragma unroll
    for (int t = 1; t < kVmax; ++t) {
      if (t < vocab && acc[t] > bv) {   // strict: first index wins ties
        bv = acc[t];
        best = t;
      }
    }
    if (token) token[r] = best;
  }
  if (logits && lane < vocab) {
    float val = 0.f;
#pragma unroll
    for (int t = 0; t < kVmax; ++t)
      if (t == lane) val = acc[t];
    logits[static_cast<int64_t>(r) * vocab + lane] = val;
  }
}

constexpr int64_t kStart = 10, kNewline = 11, kSep = 12, kEnd = 13;

__device__ __forceinline__ int64_t clampi(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

__global__ void grid_init_kernel(const int64_t* __restrict__ ids, const int64_t* __restrict__ pos,
                                 const uint8_t* __restrict__ mask, int batch, int seq, int max_x,
                                 int max_y, int32_t* gx, int32_t* gy, uint8_t* io,
                                 int32_t* kv_start, int32_t* last_row) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  int n = 0, first = seq;
  for (int j = 0; j < seq; ++j) {
    if (!mask || mask[static_cast<int64_t>(b) * seq + j]) {
      if (n == 0) first = j;
      ++n;
    }
  }
  const int last = n > 0 ? n - 1 : 0;
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
  const int64_t t = token[b];
  const bool st = t == kStart, sp = t == kSep, en = t == kEnd, nl = t == kNewline;
  int64_t x = gx[b], y = gy[b];
  bool out = io[b] != 0;
  int64_t z = out ? 3 : 1;
  if (st) z = 0;
  if (sp) z = 2;
  if (en) z = 4;
  pos_out[b * 3 + 0] = (st || sp || en || nl) ? 0 : clampi(x, 0, max_x);
  pos_out[b * 3 + 1] = (st || sp || en) ? 0 : clampi(y, 0, max_y);
  pos_out[b * 3 + 2] = z;
  if (st || sp) x = y = 0;
  if (st) out = false;
  if (sp) out = true;
  if (nl) {
    x = 0;
    y = y + 1 < max_y ? y + 1 : max_y;
  }
  if (t < 10) x = x + 1 < max_x ? x + 1 : max_x;
  gx[b] = static_cast<int32_t>(clampi(x, 0, max_x));
  gy[b] = static_cast<int32_t>(clampi(y, 0, max_y));
  io[b] = out ? 1 : 0;
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

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_version(void) { return 100; }

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
    default: return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown";
  }
}

extern "C" int mdl_lm_head(const float* x, const int32_t* row_index, int rows, int d,
                           const float* gamma, float eps, const float* w_head, int vocab,
                           float* logits_out, int64_t* token_out, void* stream) {
  if (!x || !gamma || !w_head) return MDL_ERR_NULL;
  if (rows < 0 || d <= 0 || d % 4 != 0 || d > 2048 || vocab <= 0 || vocab > kVmax)
    return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(w_head)) return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const dim3 grid((rows + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define MDL_HEAD(N)                                                                      \
  case N:                                                                                \
    lm_head_kernel<N><<<grid, 256, 0, s>>>(x, row_index, rows, d, gamma, eps, w_head, vocab, \
                                           logits_out, token_out);                       \
    break;
  switch ((d + 255) / 256) { MDL_HEAD(1) MDL_HEAD(2) MDL_HEAD(3) MDL_HEAD(4) MDL_HEAD(5)
                             MDL_HEAD(6) MDL_HEAD(7) MDL_HEAD(8) }
#undef MDL_HEAD
  return launch_status();
}

extern "C" int mdl_grid_init(const int64_t* ids, const int64_t* pos, const uint8_t* mask,
                             int batch, int seq, int max_x, int max_y, int32_t* gx, int32_t* gy,
                             uint8_t* in_out, int32_t* kv_start, int32_t* last_row,
                             void* stream) {
  if (!ids || !pos || !gx || !gy || !in_out) return MDL_ERR_NULL;
  if (batch < 0 || seq <= 0 || max_x < 0 || max_y < 0 ||
      static_cast<int64_t>(batch) * seq > INT32_MAX)
    return MDL_ERR_SHAPE;
  if (batch == 0) return MDL_OK;
  grid_init_kernel<<<dim3((batch + 63) / 64), 64, 0, static_cast<hipStream_t>(stream)>>>(
      ids, pos, mask, batch, seq, max_x, max_y, gx, gy, in_out, kv_start, last_row);
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
