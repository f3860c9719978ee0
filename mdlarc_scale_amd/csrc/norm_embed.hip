// K1 (token/example embedding gather + RMSNorm), the residual-add + RMSNorm kernel and the fused
// decode-step embedding (grid position + K1).
//
// One wavefront owns one token row; a 256-thread block holds 4 rows.  A lane owns NC chunks of
// 4 consecutive channels (chunk c = lane + 64*i), so every global access is a fully coalesced
// 16-byte (fp32) or 8-byte (bf16) vector per lane and the row's sum of squares is one wave64
// shuffle reduction.  Everything stays in registers between the reduction and the stores, so a
// row is read once and written once.  gamma is loaded before the row so its latency overlaps the
// row loads; optional inputs / outputs are template flags, so no runtime branch sits between the
// loads and the stores.
//
// Outputs per row: the fp32 residual x, rstd = 1/sqrt(mean(x^2)+eps) and xs = split(x * gamma),
// the GEMM input of the next projection as a hi|lo bf16 pair (2d values, see common.h).  The
// RMSNorm multiply by rstd is deferred to the consumer of that GEMM (K2 for q/k/v, K3 for
// gate/up), which is exact algebra: (x * rstd * gamma) @ W^T == rstd * ((x * gamma) @ W^T).
//
// Prompt-sized add+RMSNorm passes read and write with the non-temporal hint (common.h,
// kStreamBytes; measured 5.75 -> 6.26 TB/s).  K1 keeps the default policy: the hint on its
// stores measured 5.9 -> 5.6 TB/s.
#include "common.h"
#include "grid.h"

namespace mdl {

template <typename T>
__device__ __forceinline__ void load4(const T* p, float* f);

template <>
__device__ __forceinline__ void load4<float>(const float* p, float* f) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
}

template <>
__device__ __forceinline__ void load4<uint16_t>(const uint16_t* p, float* f) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  f[0] = bf2f(v.x & 0xffffu); f[1] = bf2f(v.x >> 16);
  f[2] = bf2f(v.y & 0xffffu); f[3] = bf2f(v.y >> 16);
}

// Chunk i (channels e..e+3) lies inside the row.  Only the last chunk can stick out, and only
// when d is not a multiple of 256 (TAIL): per-chunk runtime guards on every chunk cost about a
// fifth of the bandwidth of these kernels, so full rows carry none.
template <int NC, bool TAIL>
__device__ __forceinline__ bool in_row(int i, int e, int d) {
  return !TAIL || i < NC - 1 || e < d;
}

template <int NC, bool TAIL>
__device__ __forceinline__ void load_gamma(const float* gamma, int lane, int d, float (*g)[4]) {
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (in_row<NC, TAIL>(i, e, d)) load4<float>(gamma + e, g[i]);
  }
}

// x (fp32) and split(x * gamma) stores (non-temporal if NT) of the row held in v into row m of
// x ([rows, d]: row-major, or the fp32 tile layout when `x_tiled`) and xs ([rows, 2d]:
// row-major, or MFMA tiles when `tiled`), then the row's rstd (stored when rstd_out is not
// NULL).
template <int NC, bool TAIL, bool HAS_XS, bool NT>
__device__ __forceinline__ void finish_row(int lane, int d, float eps, const float (*v)[4],
                                           const float (*g)[4], float ss, float* x, int x_tiled,
                                           uint16_t* xs, int64_t m, int tiled,
                                           float* rstd_out) {
  // Chunk i of the lane covers columns 4 lane + 256 i: 8 whole 32-column blocks further on, so
  // in either layout its offsets are chunk 0's plus i times one stride (row-major 256 elements,
  // tiles 8 blocks of 512); the layout is chosen once per row, not per store.
  const int e0 = 4 * lane;
  float* xr = x + (x_tiled ? tile_off32(m, e0, d) : m * d + e0);
  const int x_step = x_tiled ? 4096 : 256;
  uint16_t* hr = nullptr;
  int64_t lo_off = 0;
  int xs_step = 0;
  if (HAS_XS) {
    hr = xs + (tiled ? tile_off(m, e0, 2 * d) : m * 2 * d + e0);
    lo_off = tiled ? tile_off(m, d + e0, 2 * d) - tile_off(m, e0, 2 * d) : d;
    xs_step = tiled ? 4096 : 256;
  }
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = e0 + 256 * i;
    if (in_row<NC, TAIL>(i, e, d)) {
      st_f4<NT>(xr + x_step * i, make_float4(v[i][0], v[i][1], v[i][2], v[i][3]));
      if (HAS_XS) {
        const float t[4] = {v[i][0] * g[i][0], v[i][1] * g[i][1], v[i][2] * g[i][2],
                            v[i][3] * g[i][3]};
        uint2 hi, lo;
        split4(t, hi, lo);
        st_u2<NT>(hr + xs_step * i, hi);
        st_u2<NT>(hr + xs_step * i + lo_off, lo);
      }
    }
  }
  // the row's reduction comes after the stores in program order: the layout choice above
  // splits the code into blocks, and stores issued first overlap the reduction's latency
  ss = wave_sum(ss);
  if (lane == 0 && rstd_out) *rstd_out = rsqrtf(ss / static_cast<float>(d) + eps);
}

// x = tok[t] (+ ex[e]) for one row into v; returns the row's partial sum of squares.
template <int NC, bool TAIL, typename TT, bool HAS_EX>
__device__ __forceinline__ float gather_row(const TT* trow, const TT* erow, int lane, int d,
                                            float (*v)[4]) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (in_row<NC, TAIL>(i, e, d)) {
      load4<TT>(trow + e, v[i]);
      if (HAS_EX) {
        float w[4];
        load4<TT>(erow + e, w);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] += w[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += v[i][j] * v[i][j];
    }
  }
  return ss;
}

__device__ __forceinline__ int64_t clamp_id(int64_t t, int n) {
  return t < 0 ? 0 : (t >= n ? n - 1 : t);
}

template <int NC, bool TAIL, typename TT, bool HAS_EX, bool HAS_XS>
__global__ __launch_bounds__(256) void embed_rmsnorm_kernel(
    const int64_t* __restrict__ ids, const int64_t* __restrict__ ex_ids,
    const TT* __restrict__ tok, const TT* __restrict__ ex, int vocab, int n_ex, int rows,
    int row_len, int d, const float* __restrict__ gamma, float eps, float* __restrict__ x_out,
    uint16_t* __restrict__ xs_out, float* __restrict__ rstd_out, int tiled) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  float g[NC][4], v[NC][4];
  if (HAS_XS) load_gamma<NC, TAIL>(gamma, lane, d, g);
  const TT* trow = tok + clamp_id(ids[m], vocab) * d;
  const TT* erow = HAS_EX ? ex + clamp_id(ex_ids[m / row_len], n_ex) * d : nullptr;
  const float ss = gather_row<NC, TAIL, TT, HAS_EX>(trow, erow, lane, d, v);
  finish_row<NC, TAIL, HAS_XS, false>(lane, d, eps, v, g, ss, x_out, tiled, xs_out, m, tiled,
                                      rstd_out ? rstd_out + m : nullptr);
}

// Decode step entry: lane 0 of each row's wave turns the token the row just emitted into its 3D
// position (grid.h) and advances the row's grid state, then the wave embeds the token as K1.
template <int NC, bool TAIL, typename TT, bool HAS_EX, bool HAS_XS>
__global__ __launch_bounds__(256) void decode_embed_kernel(
    const int64_t* __restrict__ token, const int64_t* __restrict__ ex_ids,
    const TT* __restrict__ tok, const TT* __restrict__ ex, int vocab, int n_ex, int batch, int d,
    const float* __restrict__ gamma, float eps, int32_t* __restrict__ gx,
    int32_t* __restrict__ gy, uint8_t* __restrict__ gio, int max_x, int max_y,
    int64_t* __restrict__ pos_out, int32_t* __restrict__ counters, float* __restrict__ x_out,
    uint16_t* __restrict__ xs_out, float* __restrict__ rstd_out, int tiled) {
  const int lane = threadIdx.x & 63;
  if (counters && blockIdx.x == 0 && threadIdx.x == 0) {
    counters[0] = counters[0] + 1;
    counters[1] = counters[1] + 1;
  }
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= batch) return;
  float g[NC][4], v[NC][4];
  if (HAS_XS) load_gamma<NC, TAIL>(gamma, lane, d, g);
  const int64_t t = token[m];
  if (lane == 0) {
    int32_t x = gx[m], y = gy[m];
    uint8_t io = gio[m];
    grid_position_step(t, max_x, max_y, x, y, io, pos_out + m * 3);
    gx[m] = x;
    gy[m] = y;
    gio[m] = io;
  }
  const TT* trow = tok + clamp_id(t, vocab) * d;
  const TT* erow = HAS_EX ? ex + clamp_id(ex_ids[m], n_ex) * d : nullptr;
  const float ss = gather_row<NC, TAIL, TT, HAS_EX>(trow, erow, lane, d, v);
  finish_row<NC, TAIL, HAS_XS, false>(lane, d, eps, v, g, ss, x_out, tiled, xs_out, m, tiled,
                                      rstd_out ? rstd_out + m : nullptr);
}

template <int NC, bool TAIL, bool HAS_DELTA, bool HAS_BIAS, bool HAS_XS, bool NT>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    float* __restrict__ x, const float* __restrict__ delta, const float* __restrict__ bias,
    int rows, int d, const float* __restrict__ gamma, float eps, uint16_t* __restrict__ xs_out,
    float* __restrict__ rstd_out, int xs_tiled) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  float g[NC][4], v[NC][4];
  if (HAS_XS) load_gamma<NC, TAIL>(gamma, lane, d, g);
  float* xr = x + m * d;
  const float* dr = HAS_DELTA ? delta + m * d : nullptr;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (in_row<NC, TAIL>(i, e, d)) {
      const float4 xv = ld_f4<NT>(xr + e);
      v[i][0] = xv.x; v[i][1] = xv.y; v[i][2] = xv.z; v[i][3] = xv.w;
      if (HAS_DELTA) {
        const float4 w = ld_f4<NT>(dr + e);
        v[i][0] += w.x; v[i][1] += w.y; v[i][2] += w.z; v[i][3] += w.w;
      }
      if (HAS_BIAS) {
        float w[4];
        load4<float>(bias + e, w);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] += w[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += v[i][j] * v[i][j];
    }
  }
  finish_row<NC, TAIL, HAS_XS, NT>(lane, d, eps, v, g, ss, x, 0, xs_out, m, xs_tiled,
                                   rstd_out + m);
}

// Config-1 format of K1: bf16 activations in and out.  x = bf16(tok[t] + ex[e]) (the residual
// a bf16 model holds) and xn = bf16(x * rstd * gamma) with rstd from the rounded x, both
// [rows, d] row-major.  A half-wave owns a row and a lane 8 consecutive channels per pass of 256
// (NP passes), so every load and store is 16 bytes and a half-wave instruction covers 512
// contiguous bytes; the row's sum of squares is a 32-lane shuffle reduction.  The stores of x go
// first; xn needs the row's rstd and follows the reduction.  Prompt-sized outputs are stored
// with the non-temporal hint (NT; measured at config 1: 4.6 -> 5.6 TB/s).
template <int NP, bool TAIL, bool HAS_EX, bool NT>
__global__ __launch_bounds__(256) void embed_rmsnorm_bf16_kernel(
    const int64_t* __restrict__ ids, const int64_t* __restrict__ ex_ids,
    const uint16_t* __restrict__ tok, const uint16_t* __restrict__ ex, int vocab, int n_ex,
    int rows, int row_len, int d, const float* __restrict__ gamma, float eps,
    uint16_t* __restrict__ x_out, uint16_t* __restrict__ xn_out) {
  const int hl = threadIdx.x & 31;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  const bool live = m < rows;            // dead half-waves still take part in the shuffles
  const int64_t mm = live ? m : 0;
  float v[NP][8];
  const uint16_t* trow = tok + clamp_id(ids[mm], vocab) * d;
  const uint16_t* erow = HAS_EX ? ex + clamp_id(ex_ids[mm / row_len], n_ex) * d : nullptr;
  float ss = 0.f;
  uint16_t* xr = x_out + mm * d;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int e = 8 * (hl + 32 * i);
    if (!TAIL || e < d) {
      unpack8(*reinterpret_cast<const uint4*>(trow + e), v[i]);
      if (HAS_EX) {
        float w[8];
        unpack8(*reinterpret_cast<const uint4*>(erow + e), w);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[i][j] += w[j];
      }
      const uint4 o = pack8(v[i]);
      if (live) st_u4<NT>(xr + e, o);
      unpack8(o, v[i]);                  // the norm sees the rounded residual
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += v[i][j] * v[i][j];
    }
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 32);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  uint16_t* nr = xn_out + mm * d;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int e = 8 * (hl + 32 * i);
    if ((!TAIL || e < d) && live) {
      float g[8], t[8];
      load8f(gamma + e, g);
#pragma unroll
      for (int j = 0; j < 8; ++j) t[j] = v[i][j] * r * g[j];
      st_u4<NT>(nr + e, pack8(t));
    }
  }
}

constexpr int kMaxChunks = 8;  // d <= 2048

// Instantiate F<NC, TAIL>::run for a row of d channels: NC = ceil(d / 256) chunks per lane,
// TAIL = the last chunk is partial.
template <template <int, bool> class F, typename... A>
void dispatch_nc(int d, A&&... a) {
  const bool tail = d % 256 != 0;
#define MDL_NC(N)                     \
  case N:                             \
    if (tail) F<N, true>::run(a...);  \
    else F<N, false>::run(a...);      \
    break;
  switch ((d + 255) / 256) {
    MDL_NC(1) MDL_NC(2) MDL_NC(3) MDL_NC(4) MDL_NC(5) MDL_NC(6) MDL_NC(7)
    default: if (tail) F<8, true>::run(a...); else F<8, false>::run(a...); break;
  }
#undef MDL_NC
}

template <int NC, bool TAIL>
struct LaunchEmbed {
  template <typename TT>
  static void run(dim3 grid, hipStream_t s, bool has_ex, bool has_xs, const int64_t* ids,
                  const int64_t* ex_ids, const TT* tok, const TT* ex, int vocab, int n_ex,
                  int rows, int row_len, int d, const float* gamma, float eps, float* x,
                  uint16_t* xs, float* r, int tiled) {
#define MDL_EMB(E, X)                                                                         \
  embed_rmsnorm_kernel<NC, TAIL, TT, E, X><<<grid, 256, 0, s>>>(                              \
      ids, ex_ids, tok, ex, vocab, n_ex, rows, row_len, d, gamma, eps, x, xs, r, tiled)
    if (has_ex && has_xs) MDL_EMB(true, true);
    else if (has_ex) MDL_EMB(true, false);
    else if (has_xs) MDL_EMB(false, true);
    else MDL_EMB(false, false);
#undef MDL_EMB
  }
};

// NP = ceil(d / 256) passes of 32 lanes x 8 channels (the same count as dispatch_nc's chunks)
template <int NP, bool TAIL>
struct LaunchEmbedBf16 {
  static void run(dim3 grid, hipStream_t s, bool has_ex, const int64_t* ids,
                  const int64_t* ex_ids, const uint16_t* tok, const uint16_t* ex, int vocab,
                  int n_ex, int rows, int row_len, int d, const float* gamma, float eps,
                  uint16_t* x, uint16_t* xn) {
    if (static_cast<int64_t>(rows) * d * 4 >= kStreamBytes) go<true>(grid, s, has_ex, ids,
        ex_ids, tok, ex, vocab, n_ex, rows, row_len, d, gamma, eps, x, xn);
    else go<false>(grid, s, has_ex, ids, ex_ids, tok, ex, vocab, n_ex, rows, row_len, d, gamma,
                   eps, x, xn);
  }
  template <bool NT>
  static void go(dim3 grid, hipStream_t s, bool has_ex, const int64_t* ids,
                 const int64_t* ex_ids, const uint16_t* tok, const uint16_t* ex, int vocab,
                 int n_ex, int rows, int row_len, int d, const float* gamma, float eps,
                 uint16_t* x, uint16_t* xn) {
    if (has_ex)
      embed_rmsnorm_bf16_kernel<NP, TAIL, true, NT><<<grid, 256, 0, s>>>(
          ids, ex_ids, tok, ex, vocab, n_ex, rows, row_len, d, gamma, eps, x, xn);
    else
      embed_rmsnorm_bf16_kernel<NP, TAIL, false, NT><<<grid, 256, 0, s>>>(
          ids, ex_ids, tok, ex, vocab, n_ex, rows, row_len, d, gamma, eps, x, xn);
  }
};

template <int NC, bool TAIL>
struct LaunchDecodeEmbed {
  template <typename TT>
  static void run(dim3 grid, hipStream_t s, bool has_ex, const int64_t* token,
                  const int64_t* ex_ids, const TT* tok, const TT* ex, int vocab, int n_ex,
                  int batch, int d, const float* gamma, float eps, int32_t* gx, int32_t* gy,
                  uint8_t* gio, int max_x, int max_y, int64_t* pos, int32_t* counters, float* x,
                  uint16_t* xs, float* r, int tiled) {
#define MDL_DEC(E, X)                                                                        \
  decode_embed_kernel<NC, TAIL, TT, E, X><<<grid, 256, 0, s>>>(                              \
      token, ex_ids, tok, ex, vocab, n_ex, batch, d, gamma, eps, gx, gy, gio, max_x, max_y,  \
      pos, counters, x, xs, r, tiled)
    if (has_ex && xs) MDL_DEC(true, true);
    else if (has_ex) MDL_DEC(true, false);
    else if (xs) MDL_DEC(false, true);
    else MDL_DEC(false, false);
#undef MDL_DEC
  }
};

template <int NC, bool TAIL>
struct LaunchAdd {
  static void run(dim3 grid, hipStream_t s, bool nt, float* x, const float* delta,
                  const float* bias, int rows, int d, const float* gamma, float eps, uint16_t* xs,
                  float* r, int tiled) {
    if (nt) go<true>(grid, s, x, delta, bias, rows, d, gamma, eps, xs, r, tiled);
    else go<false>(grid, s, x, delta, bias, rows, d, gamma, eps, xs, r, tiled);
  }

  template <bool NT>
  static void go(dim3 grid, hipStream_t s, float* x, const float* delta, const float* bias,
                 int rows, int d, const float* gamma, float eps, uint16_t* xs, float* r,
                 int tiled) {
    const int key = (delta ? 4 : 0) | (bias ? 2 : 0) | (xs ? 1 : 0);
#define MDL_ADD(D, B, X)                                                                     \
  add_rmsnorm_kernel<NC, TAIL, D, B, X, NT><<<grid, 256, 0, s>>>(x, delta, bias, rows, d, gamma, \
                                                                 eps, xs, r, tiled)
    switch (key) {
      case 7: MDL_ADD(true, true, true); break;
      case 6: MDL_ADD(true, true, false); break;
      case 5: MDL_ADD(true, false, true); break;
      case 4: MDL_ADD(true, false, false); break;
      case 3: MDL_ADD(false, true, true); break;
      case 2: MDL_ADD(false, true, false); break;
      case 1: MDL_ADD(false, false, true); break;
      default: MDL_ADD(false, false, false); break;
    }
#undef MDL_ADD
  }
};

// a split output of 2d columns in `layout` (MDL_LAYOUT_TILES needs 2d % 32 == 0), and with
// `with_x` the fp32 x of d columns as well (d % 32 == 0)
inline bool layout_ok(int layout, int d, bool with_x = false) {
  return layout == MDL_LAYOUT_ROWS ||
         (layout == MDL_LAYOUT_TILES && d % (with_x ? 32 : 16) == 0);
}

// host-side checks shared by the two embedding entry points
inline int check_tables(const void* tok_table, const void* ex_table, bool use_ex, int table_dtype,
                        int vocab, int n_examples, int d) {
  if (!tok_table || (use_ex && !ex_table)) return MDL_ERR_NULL;
  if (d <= 0 || d % 4 != 0 || d > 4 * 64 * kMaxChunks || vocab <= 0 ||
      (use_ex && n_examples <= 0))
    return MDL_ERR_SHAPE;
  if (table_dtype != MDL_DTYPE_F32 && table_dtype != MDL_DTYPE_BF16) return MDL_ERR_DTYPE;
  const bool f32 = table_dtype == MDL_DTYPE_F32;
  if (!(f32 ? aligned16(tok_table) : aligned8(tok_table)) ||
      (use_ex && !(f32 ? aligned16(ex_table) : aligned8(ex_table))))
    return MDL_ERR_ALIGN;
  return MDL_OK;
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_embed_rmsnorm(const int64_t* ids, const int64_t* example_ids,
                                 const void* tok_table, const void* ex_table, int table_dtype,
                                 int vocab, int n_examples, int rows, int row_len, int d,
                                 const float* gamma, float eps, float* x_out, uint16_t* xs_out,
                                 float* rstd_out, int layout, void* stream) {
  if (!ids || !gamma || !x_out) return MDL_ERR_NULL;
  const bool use_ex = example_ids != nullptr;
  const int tc = check_tables(tok_table, ex_table, use_ex, table_dtype, vocab, n_examples, d);
  if (tc != MDL_OK) return tc;
  if (rows < 0 || row_len <= 0 || !layout_ok(layout, d, true)) return MDL_ERR_SHAPE;
  if (!aligned16(x_out) || !aligned16(gamma) || (xs_out && !aligned8(xs_out)))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const dim3 grid((rows + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (table_dtype == MDL_DTYPE_F32)
    dispatch_nc<LaunchEmbed>(d, grid, s, use_ex, xs_out != nullptr, ids, example_ids,
                             static_cast<const float*>(tok_table),
                             static_cast<const float*>(ex_table), vocab, n_examples, rows,
                             row_len, d, gamma, eps, x_out, xs_out, rstd_out, layout);
  else
    dispatch_nc<LaunchEmbed>(d, grid, s, use_ex, xs_out != nullptr, ids, example_ids,
                             static_cast<const uint16_t*>(tok_table),
                             static_cast<const uint16_t*>(ex_table), vocab, n_examples, rows,
                             row_len, d, gamma, eps, x_out, xs_out, rstd_out, layout);
  return launch_status();
}

extern "C" int mdl_embed_rmsnorm_bf16(const int64_t* ids, const int64_t* example_ids,
                                      const uint16_t* tok_table, const uint16_t* ex_table,
                                      int vocab, int n_examples, int rows, int row_len, int d,
                                      const float* gamma, float eps, uint16_t* x_out,
                                      uint16_t* xn_out, void* stream) {
  if (!ids || !gamma || !x_out || !xn_out) return MDL_ERR_NULL;
  const bool use_ex = example_ids != nullptr;
  const int tc = check_tables(tok_table, ex_table, use_ex, MDL_DTYPE_BF16, vocab, n_examples, d);
  if (tc != MDL_OK) return tc;
  if (rows < 0 || row_len <= 0 || d % 8 != 0) return MDL_ERR_SHAPE;
  if (!aligned16(tok_table) || (use_ex && !aligned16(ex_table)) || !aligned16(x_out) ||
      !aligned16(xn_out) || !aligned16(gamma))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  dispatch_nc<LaunchEmbedBf16>(d, dim3((rows + 7) / 8), static_cast<hipStream_t>(stream), use_ex,
                               ids, example_ids, tok_table, ex_table, vocab, n_examples, rows,
                               row_len, d, gamma, eps, x_out, xn_out);
  return launch_status();
}

extern "C" int mdl_decode_embed(const int64_t* token, const int64_t* example_ids,
                                const void* tok_table, const void* ex_table, int table_dtype,
                                int vocab, int n_examples, int batch, int d, const float* gamma,
                                float eps, int32_t* gx, int32_t* gy, uint8_t* in_out, int max_x,
                                int max_y, int64_t* pos_out, int32_t* counters, float* x_out,
                                uint16_t* xs_out, float* rstd_out, int layout,
                                void* stream) {
  if (!token || !gamma || !gx || !gy || !in_out || !pos_out || !x_out) return MDL_ERR_NULL;
  const bool use_ex = example_ids != nullptr;
  const int tc = check_tables(tok_table, ex_table, use_ex, table_dtype, vocab, n_examples, d);
  if (tc != MDL_OK) return tc;
  if (batch < 0 || max_x < 0 || max_y < 0 || !layout_ok(layout, d, true)) return MDL_ERR_SHAPE;
  if (!aligned16(x_out) || !aligned16(gamma) || (xs_out && !aligned8(xs_out)))
    return MDL_ERR_ALIGN;
  if (batch == 0) return MDL_OK;
  const dim3 grid((batch + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (table_dtype == MDL_DTYPE_F32)
    dispatch_nc<LaunchDecodeEmbed>(d, grid, s, use_ex, token, example_ids,
                                   static_cast<const float*>(tok_table),
                                   static_cast<const float*>(ex_table), vocab, n_examples, batch,
                                   d, gamma, eps, gx, gy, in_out, max_x, max_y, pos_out, counters,
                                   x_out, xs_out, rstd_out, layout);
  else
    dispatch_nc<LaunchDecodeEmbed>(d, grid, s, use_ex, token, example_ids,
                                   static_cast<const uint16_t*>(tok_table),
                                   static_cast<const uint16_t*>(ex_table), vocab, n_examples,
                                   batch, d, gamma, eps, gx, gy, in_out, max_x, max_y, pos_out,
                                   counters, x_out, xs_out, rstd_out, layout);
  return launch_status();
}

extern "C" int mdl_add_rmsnorm(float* x, const float* delta, const float* bias, int rows,
                               int d, const float* gamma, float eps, uint16_t* xs_out,
                               float* rstd_out, int xs_layout, void* stream) {
  if (!x || !gamma || !rstd_out) return MDL_ERR_NULL;
  if (rows < 0 || d <= 0 || d % 4 != 0 || d > 4 * 64 * kMaxChunks || !layout_ok(xs_layout, d))
    return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || (delta && !aligned16(delta)) ||
      (bias && !aligned16(bias)) || (xs_out && !aligned8(xs_out)))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const bool nt = static_cast<int64_t>(rows) * d * (8 + (delta ? 4 : 0) + (xs_out ? 4 : 0)) >=
                  kStreamBytes;
  dispatch_nc<LaunchAdd>(d, dim3((rows + 3) / 4), static_cast<hipStream_t>(stream), nt,
                         x, delta, bias, rows, d, gamma, eps, xs_out, rstd_out, xs_layout);
  return launch_status();
}
