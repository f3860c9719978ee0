// K1 (token/example embedding gather + RMSNorm) and the residual-add + RMSNorm kernel.
//
// One wavefront owns one token row; a 256-thread block holds 4 rows.  A lane owns NC chunks of
// 4 consecutive channels (chunk c = lane + 64*i), so every global access is a fully coalesced
// 16-byte (fp32) or 8-byte (bf16) vector per lane and the row's sum of squares is one wave64
// shuffle reduction.  Everything stays in registers between the reduction and the stores, so a
// row is read once and written once.
//
// Outputs per row: the fp32 residual x, rstd = 1/sqrt(mean(x^2)+eps) and xs = split(x * gamma),
// the GEMM input of the next projection as a hi|lo bf16 pair (2d values, see common.h).  The
// RMSNorm multiply by rstd is deferred to the consumer of that GEMM (K2 for q/k/v, K3 for
// gate/up), which is exact algebra: (x * rstd * gamma) @ W^T == rstd * ((x * gamma) @ W^T).
#include "common.h"

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

// x row (fp32) at xo, split(x * gamma) at xs (hi) and xs + d (lo); xs may be NULL.
__device__ __forceinline__ void store_row(float* xo, uint16_t* xs, int d, const float* gamma,
                                          int e, const float* v) {
  *reinterpret_cast<float4*>(xo + e) = make_float4(v[0], v[1], v[2], v[3]);
  if (xs) {
    const float4 g = *reinterpret_cast<const float4*>(gamma + e);
    const float t[4] = {v[0] * g.x, v[1] * g.y, v[2] * g.z, v[3] * g.w};
    uint2 hi, lo;
    split4(t, hi, lo);
    *reinterpret_cast<uint2*>(xs + e) = hi;
    *reinterpret_cast<uint2*>(xs + d + e) = lo;
  }
}

template <int NC, typename TT>
__global__ __launch_bounds__(256) void embed_rmsnorm_kernel(
    const int64_t* __restrict__ ids, const int64_t* __restrict__ ex_ids,
    const TT* __restrict__ tok, const TT* __restrict__ ex, int vocab, int n_ex, int rows,
    int row_len, int d, const float* __restrict__ gamma, float eps, float* __restrict__ x_out,
    uint16_t* __restrict__ xs_out, float* __restrict__ rstd_out) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  int64_t t = ids[m];
  t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
  const TT* trow = tok + t * d;
  const TT* erow = nullptr;
  if (ex_ids) {
    int64_t e = ex_ids[m / row_len];
    e = e < 0 ? 0 : (e >= n_ex ? n_ex - 1 : e);
    erow = ex + e * d;
  }
  float v[NC][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (e < d) {
      load4<TT>(trow + e, v[i]);
      if (erow) {
        float w[4];
        load4<TT>(erow + e, w);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] += w[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += v[i][j] * v[i][j];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  float* xo = x_out + m * d;
  uint16_t* xs = xs_out ? xs_out + m * 2 * d : nullptr;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (e < d) store_row(xo, xs, d, gamma, e, v[i]);
  }
  if (lane == 0) rstd_out[m] = r;
}

template <int NC>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    float* __restrict__ x, const float* __restrict__ delta, const float* __restrict__ bias,
    int rows, int d, const float* __restrict__ gamma, float eps, uint16_t* __restrict__ xs_out,
    float* __restrict__ rstd_out) {
  const int lane = threadIdx.x & 63;
  const int64_t m = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (m >= rows) return;
  float* xr = x + m * d;
  const float* dr = delta ? delta + m * d : nullptr;
  float v[NC][4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (e < d) {
      load4<float>(xr + e, v[i]);
      if (dr) {
        float w[4];
        load4<float>(dr + e, w);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] += w[j];
      }
      if (bias) {
        float w[4];
        load4<float>(bias + e, w);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] += w[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) ss += v[i][j] * v[i][j];
    }
  }
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / static_cast<float>(d) + eps);
  uint16_t* xs = xs_out ? xs_out + m * 2 * d : nullptr;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int e = 4 * (lane + 64 * i);
    if (e < d) store_row(xr, xs, d, gamma, e, v[i]);
  }
  if (lane == 0) rstd_out[m] = r;
}

constexpr int kMaxChunks = 8;  // d <= 2048

template <typename TT>
static void launch_embed(int nc, dim3 grid, hipStream_t s, const int64_t* ids, const int64_t* ex_ids,
                         const TT* tok, const TT* ex, int vocab, int n_ex, int rows, int row_len,
                         int d, const float* gamma, float eps, float* x, uint16_t* xs, float* r) {
#define MDL_EMB(N)                                                                          \
  case N:                                                                                   \
    embed_rmsnorm_kernel<N, TT><<<grid, 256, 0, s>>>(ids, ex_ids, tok, ex, vocab, n_ex, rows, \
                                                     row_len, d, gamma, eps, x, xs, r);      \
    break;
  switch (nc) { MDL_EMB(1) MDL_EMB(2) MDL_EMB(3) MDL_EMB(4) MDL_EMB(5) MDL_EMB(6) MDL_EMB(7)
                MDL_EMB(8) }
#undef MDL_EMB
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_embed_rmsnorm(const int64_t* ids, const int64_t* example_ids,
                                 const void* tok_table, const void* ex_table, int table_dtype,
                                 int vocab, int n_examples, int rows, int row_len, int d,
                                 const float* gamma, float eps, float* x_out, uint16_t* xs_out,
                                 float* rstd_out, void* stream) {
  if (!ids || !tok_table || !gamma || !x_out || !rstd_out) return MDL_ERR_NULL;
  if (example_ids && !ex_table) return MDL_ERR_NULL;
  if (rows < 0 || row_len <= 0 || d <= 0 || d % 4 != 0 || d > 4 * 64 * kMaxChunks ||
      vocab <= 0 || (example_ids && n_examples <= 0))
    return MDL_ERR_SHAPE;
  if (table_dtype != MDL_DTYPE_F32 && table_dtype != MDL_DTYPE_BF16) return MDL_ERR_DTYPE;
  const bool f32 = table_dtype == MDL_DTYPE_F32;
  if (!aligned16(x_out) || !aligned16(gamma) || (xs_out && !aligned8(xs_out)) ||
      !(f32 ? aligned16(tok_table) : aligned8(tok_table)) ||
      (ex_table && !(f32 ? aligned16(ex_table) : aligned8(ex_table))))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const int nc = (d + 255) / 256;
  const dim3 grid((rows + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (f32)
    launch_embed<float>(nc, grid, s, ids, example_ids, static_cast<const float*>(tok_table),
                        static_cast<const float*>(ex_table), vocab, n_examples, rows, row_len, d,
                        gamma, eps, x_out, xs_out, rstd_out);
  else
    launch_embed<uint16_t>(nc, grid, s, ids, example_ids,
                           static_cast<const uint16_t*>(tok_table),
                           static_cast<const uint16_t*>(ex_table), vocab, n_examples, rows,
                           row_len, d, gamma, eps, x_out, xs_out, rstd_out);
  return launch_status();
}

extern "C" int mdl_add_rmsnorm(float* x, const float* delta, const float* bias, int rows,
                               int d, const float* gamma, float eps, uint16_t* xs_out,
                               float* rstd_out, void* stream) {
  if (!x || !gamma || !rstd_out) return MDL_ERR_NULL;
  if (rows < 0 || d <= 0 || d % 4 != 0 || d > 4 * 64 * kMaxChunks) return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || (delta && !aligned16(delta)) ||
      (bias && !aligned16(bias)) || (xs_out && !aligned8(xs_out)))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const dim3 grid((rows + 3) / 4);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define MDL_ADD(N)                                                                         \
  case N:                                                                                  \
    add_rmsnorm_kernel<N><<<grid, 256, 0, s>>>(x, delta, bias, rows, d, gamma, eps, xs_out, \
                                               rstd_out);                                  \
    break;
  switch ((d + 255) / 256) { MDL_ADD(1) MDL_ADD(2) MDL_ADD(3) MDL_ADD(4) MDL_ADD(5) MDL_ADD(6)
                             MDL_ADD(7) MDL_ADD(8) }
#undef MDL_ADD
  return launch_status();
}
