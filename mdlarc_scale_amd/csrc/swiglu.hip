// K3 -- SwiGLU gate: h = silu(rstd*g + b_g) * (rstd*u + b_u), the down-projection input.
//
// gate|up come from ONE concatenated GEMM, [rows, 2*d_ff] fp32 (the GEMM's unrounded fp32
// accumulators).  A work item is 8 channels: two 16-byte loads from the gate half, two from the
// up half, 2x32 bytes of fp32 bias (L2 resident) and two 16-byte stores of h as a hi|lo bf16
// pair ([rows, 2*d_ff], hi in [0, d_ff), lo in [d_ff, 2*d_ff)), so each wavefront streams 2 KiB
// per input operand with no reuse -- a pure HBM-bound pass.  rstd applies ln2's RMSNorm
// multiply deferred past the GEMM.  Prompt-sized batches store h with the non-temporal hint
// (common.h, kStreamBytes; measured 5.83 -> 5.97 TB/s); the same hint on the loads costs 10%.
#include "common.h"

namespace mdl {

template <bool NT>
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gu, int64_t ld,
                                                     const float* __restrict__ rstd,
                                                     const float* __restrict__ bg,
                                                     const float* __restrict__ bu, int64_t rows,
                                                     int d_ff, uint16_t* __restrict__ h,
                                                     int tiled) {
  const int per_row = d_ff >> 3;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int64_t m = idx / per_row;
  const int c = static_cast<int>(idx - m * per_row) * 8;
  const float* row = gu + m * ld;
  float g[8], u[8], b1[8], b2[8];
  load8f(row + c, g);
  load8f(row + d_ff + c, u);
  // biases as two 16-byte loads each (scalar per-channel loads double the load count and
  // halve the achieved bandwidth)
  if (bg) {
    load8f(bg + c, b1);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) b1[i] = 0.f;
  }
  if (bu) {
    load8f(bu + c, b2);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) b2[i] = 0.f;
  }
  const float r = rstd ? rstd[m] : 1.f;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = fmaf(r, g[i], b1[i]);   // explicit: the fused K5 epilogue computes the same
    const float b = fmaf(r, u[i], b2[i]);
    o[i] = silu_mul(a, b);
  }
  uint4 hi, lo;
  split8(o, hi, lo);
  if (tiled) {
    st_u4<NT>(h + tile_off(m, c, 2 * d_ff), hi);
    st_u4<NT>(h + tile_off(m, d_ff + c, 2 * d_ff), lo);
  } else {
    uint16_t* hr = h + m * 2 * d_ff + c;
    st_u4<NT>(hr, hi);
    st_u4<NT>(hr + d_ff, lo);
  }
}

// Config-1 format of K3: gate|up [rows, 2 d_ff] bf16 in, h [rows, d_ff] bf16 out (one rounding).
// Block (y, x) covers channels 2048 y .. 2048 y + 2047 of rows kBf16Rows x .. kBf16Rows x + 3, a
// thread 8 channels of each: the rows' 16-byte loads from both halves are all issued before the
// first store (8 loads in flight per thread), no index division.  Prompt-sized batches take the
// non-temporal hint on loads and stores.  Measured at config 1 (65,536 rows, d_ff 2,048):
// one row per block 151 us; four rows, plain loads 131 us; four rows, both hints 126 us (6.38
// TB/s), against 123 us for a copy kernel that moves the same bytes with both hints.
constexpr int kBf16Rows = 4;

template <bool NT>
__global__ __launch_bounds__(256) void swiglu_bf16_kernel(const uint16_t* __restrict__ gu,
                                                          int64_t ld,
                                                          const float* __restrict__ rstd,
                                                          const float* __restrict__ bg,
                                                          const float* __restrict__ bu, int rows,
                                                          int d_ff, uint16_t* __restrict__ h) {
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * kBf16Rows;
  const int c = 8 * (static_cast<int>(blockIdx.y) * 256 + static_cast<int>(threadIdx.x));
  if (c >= d_ff) return;
  uint4 G[kBf16Rows], U[kBf16Rows];
  float rs[kBf16Rows];
#pragma unroll
  for (int r = 0; r < kBf16Rows; ++r) {
    const int64_t m = min(m0 + r, static_cast<int64_t>(rows) - 1);   // tail rows: loads only
    const uint16_t* row = gu + m * ld;
    if constexpr (NT) {
      G[r] = load_nt16(row + c);
      U[r] = load_nt16(row + d_ff + c);
    } else {
      G[r] = *reinterpret_cast<const uint4*>(row + c);
      U[r] = *reinterpret_cast<const uint4*>(row + d_ff + c);
    }
    rs[r] = rstd ? rstd[m] : 1.f;
  }
  float b1[8], b2[8];
  if (bg) {
    load8f(bg + c, b1);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) b1[i] = 0.f;
  }
  if (bu) {
    load8f(bu + c, b2);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) b2[i] = 0.f;
  }
#pragma unroll
  for (int r = 0; r < kBf16Rows; ++r) {
    if (m0 + r >= rows) break;
    float g[8], u[8], o[8];
    unpack8(G[r], g);
    unpack8(U[r], u);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = silu_mul(fmaf(rs[r], g[i], b1[i]), fmaf(rs[r], u[i], b2[i]));
    st_u4<NT>(h + (m0 + r) * d_ff + c, pack8(o));
  }
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_swiglu_bf16(const uint16_t* gate_up, int64_t ld, const float* rstd,
                               const float* bias_gate, const float* bias_up, int rows, int d_ff,
                               uint16_t* h_out, void* stream) {
  if (!gate_up || !h_out) return MDL_ERR_NULL;
  // grid (rows, d_ff / 2048): at most 65535 column blocks
  if (rows < 0 || d_ff <= 0 || d_ff % 8 != 0 || d_ff > 65535 * 2048 ||
      ld < 2 * static_cast<int64_t>(d_ff))
    return MDL_ERR_SHAPE;
  if (!aligned16(gate_up) || ld % 8 != 0 || !aligned16(h_out) ||
      (bias_gate && !aligned16(bias_gate)) || (bias_up && !aligned16(bias_up)))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const dim3 grid(static_cast<unsigned>((rows + kBf16Rows - 1) / kBf16Rows),
                  static_cast<unsigned>((d_ff + 2047) / 2048));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (static_cast<int64_t>(rows) * d_ff * 6 >= kStreamBytes)
    swiglu_bf16_kernel<true><<<grid, 256, 0, st>>>(gate_up, ld, rstd, bias_gate, bias_up, rows,
                                                   d_ff, h_out);
  else
    swiglu_bf16_kernel<false><<<grid, 256, 0, st>>>(gate_up, ld, rstd, bias_gate, bias_up, rows,
                                                    d_ff, h_out);
  return launch_status();
}

extern "C" int mdl_swiglu(const float* gate_up, int64_t ld, const float* rstd,
                          const float* bias_gate, const float* bias_up, int rows, int d_ff,
                          uint16_t* h_out, int h_layout, void* stream) {
  if (!gate_up || !h_out) return MDL_ERR_NULL;
  // the tiled store computes 2 * d_ff and d_ff + c in int: d_ff stays below 2^29
  if (rows < 0 || d_ff <= 0 || d_ff % 8 != 0 || d_ff > (1 << 29) ||
      ld < 2 * static_cast<int64_t>(d_ff))
    return MDL_ERR_SHAPE;
  if (h_layout != MDL_LAYOUT_ROWS && !(h_layout == MDL_LAYOUT_TILES && d_ff % 16 == 0))
    return MDL_ERR_SHAPE;
  if (!aligned16(gate_up) || ld % 4 != 0 || !aligned16(h_out) ||
      (bias_gate && !aligned16(bias_gate)) || (bias_up && !aligned16(bias_up)))
    return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const int64_t items = static_cast<int64_t>(rows) * (d_ff / 8);
  if ((items + 255) / 256 > 0x7fffffff) return MDL_ERR_SHAPE;
  const dim3 grid(static_cast<unsigned>((items + 255) / 256));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (static_cast<int64_t>(rows) * d_ff * 12 >= kStreamBytes)
    swiglu_kernel<true><<<grid, 256, 0, st>>>(gate_up, ld, rstd, bias_gate, bias_up, rows, d_ff,
                                              h_out, h_layout);
  else
    swiglu_kernel<false><<<grid, 256, 0, st>>>(gate_up, ld, rstd, bias_gate, bias_up, rows, d_ff,
                                               h_out, h_layout);
  return launch_status();
}
