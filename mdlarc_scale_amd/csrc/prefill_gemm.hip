// K6: split-activation GEMM for prompt-sized row counts (prefill) on bf16 MFMA (gfx950), with
// the RMSNorm of its input in the prologue and the SwiGLU gate or the residual add in the
// epilogue, so a prefill layer needs no fp32 gate / up round trip and no add+RMSNorm pass.
//
//   acc[m, n] (fp32) = sum_k (a_hi[m, k] + a_lo[m, k]) * w[n, k],   k < K
//
// w: bf16 [N, K] in the MFMA tile layout (MDL_LAYOUT_TILES, the decode copies of the weights).
// a (AMODE): A_ROWS  split [M, 2K] row-major (hi in [0, K), lo in [K, 2K)), row stride lda;
//            A_TILES the same matrix in the tile layout;
//            A_NORM  split(x * gamma) of the fp32 residual stream x [M, K] in the fp32 tile
//                    layout, formed after the LDS read; the block sees whole rows, so it sums
//                    x^2 and has rstd.
// AP (activation parts) 1 drops the lo term: A_ROWS / A_TILES then hold hi alone ([M, K]),
// A_NORM uses bf16(x * gamma); half the MFMAs and, for the split forms, a third fewer loads.
// epilogue (EPI): E_STORE     out = acc (fp32 row-major; with A_NORM also rstd[m]);
//                 E_SWIGLU    h = split(silu(rstd g + b_g) * (rstd u + b_u)) from the gate / up
//                             accumulator pairs (weights with 16-row gate / up blocks
//                             interleaved), h [M, 2F] in the tile layout (h_parts 1: hi alone,
//                             [M, F], for a consumer with AP 1);
//                 E_RESIDUAL  x[m, n] += acc (+ bias[n]) in place, x [M, N] in the fp32 tile
//                             layout;
//                 E_QKV       K2 on the qkv accumulators (A_NORM): rstd, 3D RoPE of q and k, the
//                             softmax scale on q; q bf16 [M, d], K / V bf16 into their cache
//                             slots, and fp32 acc only for the lead rows (the first `lead` tokens
//                             of each row, which the exact lead-attention pass reads).
//
// Block: a 256 x 256 output tile (activation rows x weight rows) on 8 waves, each owning 32 MFMA
// tiles (128 fp32 accumulators per lane): 64 rows x 128 weight rows in a 4 x 2 wave grid for the
// split forms, 32 rows x 256 weight rows (8 x 1) for A_NORM.  K advances 32 at a time through a
// ring of three LDS stages of 48 KB.  A stage holds 16 weight fragments and 32 activation
// fragments of 1 KB in MFMA lane order (bf16 {hi, lo} of 16 row blocks; for A_NORM the fp32 x of
// 16 row blocks in the fp32 tile layout, split after the read), so every fragment read is one
// conflict-free 16-byte LDS read per lane.  Global data goes straight to LDS
// (global_load_lds_dwordx4, 16 bytes per lane, one kilobyte per wave instruction), issued two
// k-steps ahead; nothing is staged in registers, and a step ends with one barrier after an exact
// vmcnt wait for the next stage's loads.  Blocks are persistent (one per CU, each walking its
// tiles), and the load ring runs on across tile boundaries, so a tile's epilogue overlaps the
// next tile's first loads. Every weight fragment feeds two MFMAs (hi and lo rows), as in K5.
// Blocks are numbered so that an XCD (block i runs on XCD i mod 8) takes a contiguous run of
// tiles, row tile major: the N tiles of one row tile share its activation rows in one L2.
// Summation order is fixed (k-steps in order, hi before lo), so results are reproducible.
#include <algorithm>

#include "common.h"
#include "lds_dma.h"
#include "mfma.h"
#include "rope.h"

namespace mdl {

namespace {

constexpr int kBM = 256, kBN = 256;
constexpr int kWaves = 8, kThreads = 64 * kWaves;
constexpr int kAFrags = (kBM / 16) * 2;   // {hi, lo} fragments of 16 row blocks
constexpr int kWFrags = kBN / 16;
constexpr int kStage = (kAFrags + kWFrags) * 1024;   // bytes of one LDS stage
constexpr int kRing = 3;                             // LDS stages (loads run 2 k-steps ahead)
// DMA instructions per thread per stage: two weight fragments and four activation fragments
// (two for the split forms with the hi part alone)
template <int AMODE, int AP>
constexpr int loads_per_stage() { return AMODE != 2 && AP == 1 ? 4 : 6; }
constexpr int kMaxNormK = 2048;                      // A_NORM: gamma lives in LDS

enum AMode { A_ROWS = 0, A_TILES = 1, A_NORM = 2 };
enum Epi { E_STORE = 0, E_SWIGLU = 1, E_RESIDUAL = 2, E_QKV = 3 };

struct Args {
  const uint16_t* a;   // A_ROWS / A_TILES
  int64_t lda;
  const float* x;      // A_NORM: [M, K] in the fp32 tile layout
  const float* gamma;
  float eps;
  const uint16_t* w;   // tiled [N, K]
  float* out;          // E_STORE
  int64_t ldo;
  float* rstd_out;     // E_STORE with A_NORM (may be NULL)
  const float* bias_a; // E_SWIGLU gate bias / E_RESIDUAL bias (may be NULL)
  const float* bias_b; // E_SWIGLU up bias (may be NULL)
  uint16_t* h;         // E_SWIGLU: tiled [M, h_parts d_ff] (hi, then lo when h_parts is 2)
  int d_ff, h_parts;
  float* x_res;        // E_RESIDUAL: [M, N] in the fp32 tile layout
  // E_QKV: row m is token slot tok_slot[m] of batch row tok_row[m] (packed), or slot m % seq of
  // row m / seq; out (may be NULL) receives the lead rows' fp32 acc
  const int64_t* pos;
  const float* rope_tab;
  RopeArgs ra;
  float q_scale;
  uint16_t* q_out;
  uint16_t* kc;
  uint16_t* vc;
  const int32_t* tok_row;
  const int32_t* tok_slot;
  const int32_t* kv_start;
  int slots, seq, batch, lead;
  int M, N, K, tiles_n, tiles, per_xcd;
};

// Wait until at most N of this wave's global memory operations are in flight, then a block
// barrier that also waits for this wave's LDS traffic; the memory clobbers keep the compiler from
// moving LDS accesses across either.  N counts the copies issued for later stages; any other
// load or store the wave issued after this stage's copies (epilogue traffic of the previous
// tile) only makes the wait stricter.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" :: "n"(N) : "memory");
}

template <int AMODE, int EPI, int AP>
__global__ __launch_bounds__(kThreads, 1) void prefill_gemm_kernel(const Args p) {
  static_assert(AP == 1 || AP == 2, "activation parts: hi, or hi and lo");
  constexpr int kLoads = loads_per_stage<AMODE, AP>();
  constexpr int kGammaBytes = AMODE == A_NORM ? kMaxNormK * 4 : 0;
  __shared__ __align__(16) uint8_t lds[kRing * kStage + kGammaBytes];
  __shared__ float rstd_s[kBM];
  // Persistent blocks: XCD x = blockIdx % 8 owns logical tiles [x per_xcd, (x + 1) per_xcd), row
  // tile major; its bpx blocks take every bpx-th of them, so the XCD's CUs work on consecutive
  // tiles at any time.
  const int bpx = gridDim.x >> 3;
  const int t_lo = (blockIdx.x & 7) * p.per_xcd;
  const int t_hi = min(t_lo + p.per_xcd, p.tiles);
  const int first = t_lo + (blockIdx.x >> 3);
  if (first >= t_hi) return;   // whole block, before any barrier
  const int M = p.M, N = p.N, K = p.K, nk = K >> 5;
  const int total = (t_hi - first + bpx - 1) / bpx * nk;   // k-steps over this block's tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // wave grid WMW x WNW over the tile: wave (wm, wn) owns FM row blocks and FN weight fragments.
  // The A_NORM forms split x * gamma in registers after the LDS read, so there every row block
  // belongs to one wave (8 x 1) and is converted once; the split forms use 4 x 2 (8 activation
  // and 8 weight fragment reads per wave and k-step).
  constexpr int WMW = AMODE == A_NORM ? 8 : 4, WNW = kWaves / WMW;
  constexpr int FM = kBM / 16 / WMW, FN = kBN / 16 / WNW;
  const int wm = wave % WMW, wn = wave / WMW;
  const int c = lane & 15, g = lane >> 4;
  const int last_nb = (N + 15) / 16 - 1, last_mb = (M + 15) / 16 - 1;
  const uint32_t lds0 = lds_addr(lds);

  // The loads of k-step s of the tile at (m0, n0) into ring stage b.  Wave w copies weight
  // fragments 8 j + w (j = 0, 1: row block n0 / 16 + 8 j + w) and activation fragments f = 8 j +
  // w (j = 0..3): row block f / 2, part f % 2 (hi / lo; for A_NORM the first or second kilobyte of
  // the fp32 16 x 32 block, lane l's columns 0..3 or 4..7); with the hi part alone (AP 1, split
  // forms) f = 2 (8 j + w), j = 0, 1.  Fragment f lands in stage slot f either way.  Every copy is
  // one contiguous kilobyte per wave, except row-major A.  Row blocks past M or N load valid
  // memory (clamped to the last; tile-layout buffers hold its padding rows); their results are
  // never stored.
  auto issue = [&](int m0, int n0, int s, int b) {
    const uint32_t base = lds0 + b * kStage;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int nb = min(n0 / 16 + 8 * j + wave, last_nb);
      dma16(p.w + (static_cast<int64_t>(nb) * nk + s) * 512 + 8 * lane,
            __builtin_amdgcn_readfirstlane(base + (kAFrags + 8 * j + wave) * 1024));
    }
    constexpr bool kHiOnly = AMODE != A_NORM && AP == 1;
#pragma unroll
    for (int j = 0; j < (kHiOnly ? 2 : 4); ++j) {
      const int f = kHiOnly ? 2 * (8 * j + wave) : 8 * j + wave, rb = f >> 1, part = f & 1;
      const void* src;
      if constexpr (AMODE == A_NORM) {
        const int64_t blk = static_cast<int64_t>(min(m0 / 16 + rb, last_mb)) * nk + s;
        src = p.x + blk * 512 + 256 * part + 4 * lane;
      } else if constexpr (AMODE == A_TILES) {
        const int64_t blk = static_cast<int64_t>(min(m0 / 16 + rb, last_mb)) * AP * nk;
        src = p.a + (blk + part * nk + s) * 512 + 8 * lane;
      } else {
        const int row = min(m0 + 16 * rb + c, M - 1);
        src = p.a + static_cast<int64_t>(row) * p.lda + part * K + 32 * s + 8 * g;
      }
      dma16(src, __builtin_amdgcn_readfirstlane(base + f * 1024));
    }
  };

  const float* gam_s = reinterpret_cast<const float*>(lds + kRing * kStage);
  if constexpr (AMODE == A_NORM) {
    float* gw = reinterpret_cast<float*>(lds + kRing * kStage);
    for (int i = tid; i < K; i += kThreads) gw[i] = p.gamma[i];
    __syncthreads();   // before any stage load is in flight (it waits for every load)
  }

  f32x4_t acc[FN][FM];
  float ss[FM];   // A_NORM: this lane's part of sum(x^2) of row 16 (FM wm + j) + c
  auto reset = [&]() {
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
      for (int j = 0; j < FM; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < FM; ++j) ss[j] = 0.f;
  };

  auto compute = [&](int s, int b) {
    const uint8_t* base = lds + b * kStage;
    bf16x8_t ah[FM], al[FM];
    if constexpr (AMODE == A_NORM) {
      // x of row 16 (FM wm + j) + c, columns 8 g .. 8 g + 7: the split of x * gamma, as the
      // norm kernels write it (t rounded, then split)
      const float4 g0 = *reinterpret_cast<const float4*>(gam_s + 32 * s + 8 * g);
      const float4 g1 = *reinterpret_cast<const float4*>(gam_s + 32 * s + 8 * g + 4);
      const float ge[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const float4 x0 =
            *reinterpret_cast<const float4*>(base + (2 * (FM * wm + j)) * 1024 + 16 * lane);
        const float4 x1 =
            *reinterpret_cast<const float4*>(base + (2 * (FM * wm + j) + 1) * 1024 + 16 * lane);
        const float xe[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float t[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          t[e] = xe[e] * ge[e];
          ss[j] = fmaf(xe[e], xe[e], ss[j]);
        }
        if constexpr (AP == 2) {
          uint4 hi, lo;
          split8(t, hi, lo);
          ah[j] = as_bf16x8(hi);
          al[j] = as_bf16x8(lo);
        } else {
          ah[j] = as_bf16x8(pack8(t));
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        ah[j] =
            *reinterpret_cast<const bf16x8_t*>(base + (2 * (FM * wm + j)) * 1024 + 16 * lane);
        if constexpr (AP == 2)
          al[j] = *reinterpret_cast<const bf16x8_t*>(base + (2 * (FM * wm + j) + 1) * 1024 +
                                                     16 * lane);
      }
    }
    // The hi products before the lo products, so that consecutive MFMAs write different
    // accumulators (each accumulator still adds hi before lo).  The split forms (8 weight
    // fragments) hold all their weight fragments and run two passes; the norm forms (16, whose
    // registers that would exhaust) take four fragments at a time: hi for the four fragments
    // and both row blocks, then lo, so an accumulator's lo product issues eight MFMAs after its
    // hi product (measured at config 2 against one fragment at a time: qkv 7%, gate/up 6%
    // faster; two at a time sits between; eight is within 1% of four and takes the E_QKV form
    // to the 256-register limit).
    if constexpr (AMODE == A_NORM) {
      constexpr int kGroup = 4;
      static_assert(FN % kGroup == 0, "the norm forms group their weight fragments");
#pragma unroll
      for (int i = 0; i < FN; i += kGroup) {
        bf16x8_t wf[kGroup];
#pragma unroll
        for (int u = 0; u < kGroup; ++u)
          wf[u] = *reinterpret_cast<const bf16x8_t*>(base + (kAFrags + FN * wn + i + u) * 1024 +
                                                     16 * lane);
#pragma unroll
        for (int u = 0; u < kGroup; ++u)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i + u][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[u], ah[j], acc[i + u][j],
                                                                    0, 0, 0);
        if constexpr (AP == 2) {
#pragma unroll
          for (int u = 0; u < kGroup; ++u)
#pragma unroll
            for (int j = 0; j < FM; ++j)
              acc[i + u][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[u], al[j],
                                                                      acc[i + u][j], 0, 0, 0);
        }
      }
    } else {
      bf16x8_t wf[FN];
#pragma unroll
      for (int i = 0; i < FN; ++i)
        wf[i] = *reinterpret_cast<const bf16x8_t*>(base + (kAFrags + FN * wn + i) * 1024 +
                                                   16 * lane);
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[i], ah[j], acc[i][j], 0, 0, 0);
      if constexpr (AP == 2) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[i], al[j], acc[i][j], 0, 0, 0);
      }
    }
  };

  // the finished tile at (m0, n0): lane (c, g) of accumulator tile (i, j) holds
  // acc[row 16 (FM wm + j) + c][weight rows 16 (FN wn + i) + 4 g ..]
  auto epilogue = [&](int m0, int n0) {
    if constexpr (AMODE == A_NORM) {
      // the four lane groups of a row in a fixed order (one wave per row block: WNW = 1); the
      // barrier waits for LDS only, so the next tile's loads stay in flight (rstd_s was last read
      // in the previous tile's epilogue, nk >= 1 stage barriers ago)
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        float v = ss[j];
        v += __shfl_xor(v, 16, kWave);
        v += __shfl_xor(v, 32, kWave);
        if (g == 0) rstd_s[16 * (FM * wm + j) + c] = rsqrtf(v / static_cast<float>(K) + p.eps);
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if constexpr (EPI == E_STORE || EPI == E_QKV) {
        if (p.rstd_out && n0 == 0 && tid < kBM && m0 + tid < M) p.rstd_out[m0 + tid] = rstd_s[tid];
      }
    }
    if constexpr (EPI == E_QKV) {
      static_assert(AMODE == A_NORM && WNW == 1, "E_QKV follows the norm prologue");
      // the arithmetic of K2 (rope_cache.hip); n0 and d are multiples of 64, so lane (c, g) of
      // weight fragment i holds dims 16 (i % 4) + 4 g .. + 3 of its head: RoPE pairs
      // 8 (i % 4) + 2 g and + 1
      const int d = N / 3;
      const int64_t head_stride = static_cast<int64_t>(p.slots) * kHeadDim;
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const int r = 16 * (FM * wm + j) + c;
        const int m = m0 + r;
        if (m >= M) continue;
        int64_t b;
        int slot;
        if (p.tok_slot) {
          b = p.tok_row[m];
          slot = p.tok_slot[m];
        } else {
          b = m / p.seq;
          slot = static_cast<int>(m - b * p.seq);
        }
        const bool in_cache = slot >= 0 && slot < p.slots && b >= 0 && b < p.batch;
        // clamped below at 0 as the lead-attention pass (K4c) clamps it, so the rows written
        // here are exactly the rows it reads
        const int ks = (p.kv_start && b >= 0 && b < p.batch) ? max(p.kv_start[b], 0) : 0;
        const bool lead_row = p.out != nullptr && slot >= ks && slot - ks < p.lead;
        const float rs = rstd_s[r];
        const int64_t* pos3 = p.pos + static_cast<int64_t>(m) * 3;
        float cs[8], sn[8];
#pragma unroll
        for (int t = 0; t < 8; ++t)
          rope_cos_sin(8 * (t >> 1) + 2 * g + (t & 1), pos3, p.rope_tab, p.ra, cs[t], sn[t]);
        const int64_t cache_row = (b * (d / kHeadDim) * static_cast<int64_t>(p.slots) + slot) *
                                  kHeadDim;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
          const int n = n0 + 16 * i + 4 * g;
          if (n >= N) continue;
          const f32x4_t v = acc[i][j];
          if (lead_row)
            *reinterpret_cast<float4*>(p.out + static_cast<int64_t>(m) * p.ldo + n) =
                make_float4(v[0], v[1], v[2], v[3]);
          const int part = n / d, e = n - part * d;
          const int head = e / kHeadDim, dim = e - head * kHeadDim;
          const int q4 = i & 3;
          const float a0 = v[0] * rs, a1 = v[1] * rs, a2 = v[2] * rs, a3 = v[3] * rs;
          uint2 o;
          if (part == 2) {
            if (!in_cache) continue;
            o.x = pack_bf2(a0, a1);
            o.y = pack_bf2(a2, a3);
            *reinterpret_cast<uint2*>(p.vc + cache_row + head * head_stride + dim) = o;
            continue;
          }
          float y0, y1, y2, y3;
          rope_rot(a0, a1, cs[2 * q4], sn[2 * q4], y0, y1);
          rope_rot(a2, a3, cs[2 * q4 + 1], sn[2 * q4 + 1], y2, y3);
          if (part == 0) {
            o.x = pack_bf2(y0 * p.q_scale, y1 * p.q_scale);
            o.y = pack_bf2(y2 * p.q_scale, y3 * p.q_scale);
            *reinterpret_cast<uint2*>(p.q_out + static_cast<int64_t>(m) * d + e) = o;
          } else if (in_cache) {
            o.x = pack_bf2(y0, y1);
            o.y = pack_bf2(y2, y3);
            *reinterpret_cast<uint2*>(p.kc + cache_row + head * head_stride + dim) = o;
          }
        }
      }
    } else if constexpr (EPI == E_SWIGLU) {
      // Gate fragment 2 pb, up fragment 2 pb + 1: channels 16 (n0 / 32 + FN wn / 2 + pb) + 4 g.
      // The bias loads of kG pairs are issued together, and those of the next kG pairs before
      // this group's stores: the compiler's wait for a load also waits for every older memory
      // operation (the stores before it, the next tile's copies), so loads issued one pair at a
      // time after the previous pair's stores took a full round trip per pair.
      const int F = p.d_ff;
      constexpr int kG = 2, NP = FN / 2;
      static_assert(NP % (2 * kG) == 0, "bias groups");
      auto chan = [&](int pb) { return 16 * (n0 / 32 + NP * wn + pb) + 4 * g; };
      auto load_bias = [&](int pb0, float4 (&bg)[kG], float4 (&bu)[kG]) {
#pragma unroll
        for (int q = 0; q < kG; ++q) {
          const int ch = min(chan(pb0 + q), F - 4);   // in bounds; unused past F
          bg[q] = p.bias_a ? *reinterpret_cast<const float4*>(p.bias_a + ch)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
          bu[q] = p.bias_b ? *reinterpret_cast<const float4*>(p.bias_b + ch)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      };
      auto store_h = [&](int pb0, const float4 (&bg)[kG], const float4 (&bu)[kG]) {
#pragma unroll
        for (int q = 0; q < kG; ++q) {
          const int pb = pb0 + q, ch = chan(pb);
          if (2 * ch >= N) continue;
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const int r = 16 * (FM * wm + j) + c;
            const int m = m0 + r;
            if (m >= M) continue;
            const float rs = AMODE == A_NORM ? rstd_s[r] : 1.f;
            const f32x4_t gs = acc[2 * pb][j], us = acc[2 * pb + 1][j];
            // the arithmetic of K3 (swiglu.hip)
            const float o[4] = {silu_mul(fmaf(rs, gs[0], bg[q].x), fmaf(rs, us[0], bu[q].x)),
                                silu_mul(fmaf(rs, gs[1], bg[q].y), fmaf(rs, us[1], bu[q].y)),
                                silu_mul(fmaf(rs, gs[2], bg[q].z), fmaf(rs, us[2], bu[q].z)),
                                silu_mul(fmaf(rs, gs[3], bg[q].w), fmaf(rs, us[3], bu[q].w))};
            uint2 hi, lo;
            split4(o, hi, lo);
            *reinterpret_cast<uint2*>(p.h + tile_off(m, ch, p.h_parts * F)) = hi;
            if (p.h_parts == 2) *reinterpret_cast<uint2*>(p.h + tile_off(m, F + ch, 2 * F)) = lo;
          }
        }
      };
      float4 ga[kG], ua[kG], gb[kG], ub[kG];
      load_bias(0, ga, ua);
#pragma unroll
      for (int pb0 = 0; pb0 < NP; pb0 += 2 * kG) {
        load_bias(pb0 + kG, gb, ub);
        store_h(pb0, ga, ua);
        if (pb0 + 2 * kG < NP) load_bias(pb0 + 2 * kG, ga, ua);
        store_h(pb0 + kG, gb, ub);
      }
    } else {
      // The residual's loads of kG weight fragments are issued together, and those of the next
      // kG before this group's stores (see E_SWIGLU: one load and its wait per fragment, after
      // the previous fragment's store, took a full round trip each).
      constexpr int kG = 2;
      static_assert(FN % (2 * kG) == 0, "residual groups");
      auto col = [&](int i) { return n0 + 16 * (FN * wn + i) + 4 * g; };
      auto row = [&](int j) { return m0 + 16 * (FM * wm + j) + c; };
      auto load_x = [&](int i0, float4 (&xv)[kG][FM], float4 (&bv)[kG]) {
        if constexpr (EPI == E_RESIDUAL) {
#pragma unroll
          for (int u = 0; u < kG; ++u) {
            const int n = min(col(i0 + u), N - 4);   // in bounds; unused past N or M
            bv[u] = p.bias_a ? *reinterpret_cast<const float4*>(p.bias_a + n)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int j = 0; j < FM; ++j)
              xv[u][j] = *reinterpret_cast<const float4*>(
                  p.x_res + tile_off32(min(row(j), M - 1), n, N));
          }
        }
      };
      auto store_x = [&](int i0, const float4 (&xv)[kG][FM], const float4 (&bv)[kG]) {
#pragma unroll
        for (int u = 0; u < kG; ++u) {
          const int n = col(i0 + u);
          if (n >= N) continue;
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const int m = row(j);
            if (m >= M) continue;
            const f32x4_t v = acc[i0 + u][j];
            if constexpr (EPI == E_RESIDUAL) {
              // x + delta, then + bias: the order of the add+RMSNorm kernel it replaces
              float4 x = xv[u][j];
              x.x += v[0]; x.y += v[1]; x.z += v[2]; x.w += v[3];
              if (p.bias_a) {
                x.x += bv[u].x; x.y += bv[u].y; x.z += bv[u].z; x.w += bv[u].w;
              }
              *reinterpret_cast<float4*>(p.x_res + tile_off32(m, n, N)) = x;
            } else {
              *reinterpret_cast<float4*>(p.out + static_cast<int64_t>(m) * p.ldo + n) =
                  make_float4(v[0], v[1], v[2], v[3]);
            }
          }
        }
      };
      float4 xa[kG][FM], ba[kG], xb[kG][FM], bb[kG];
      load_x(0, xa, ba);
#pragma unroll
      for (int i0 = 0; i0 < FN; i0 += 2 * kG) {
        load_x(i0 + kG, xb, bb);
        store_x(i0, xa, ba);
        if (i0 + 2 * kG < FN) load_x(i0 + 2 * kG, xa, ba);
        store_x(i0 + kG, xb, bb);
      }
    }
  };

  // Step u (over all k-steps of this block's tiles, tile after tile) computes ring stage u % 3
  // while steps u + 1 and u + 2 load -- across a tile boundary too, so the next tile's first
  // stages are in flight during this tile's epilogue.  The stage step u overwrites,
  // (u + 2) % 3, was last read in step u - 1, before that step's barrier.  Every wave runs the
  // same steps (all counters are block-uniform), so every barrier is reached by all.
  auto tile_origin = [&](int t, int& m0, int& n0) {
    const int mt = t / p.tiles_n;
    m0 = mt * kBM;
    n0 = (t - mt * p.tiles_n) * kBN;
  };
  int it = first, is = 0, im0, in0;   // issue cursor: tile, k-step, tile origin
  tile_origin(it, im0, in0);
  auto advance_issue = [&]() {
    if (++is == nk) {
      is = 0;
      it += bpx;
      tile_origin(it, im0, in0);
    }
  };
  issue(im0, in0, is, 0);
  advance_issue();
  if (total > 1) {
    issue(im0, in0, is, 1);
    advance_issue();
    stage_barrier<kLoads>();
  } else {
    stage_barrier<0>();
  }
  int ct = first, cs = 0, cm0, cn0;   // compute cursor
  tile_origin(ct, cm0, cn0);
  reset();
  int b = 0;
  for (int u = 0; u < total; ++u) {
    const int b2 = b == 0 ? 2 : b - 1;   // (u + 2) % 3
    if (u + 2 < total) {
      issue(im0, in0, is, b2);
      advance_issue();
    }
    compute(cs, b);
    if (u + 2 < total) stage_barrier<kLoads>();
    else stage_barrier<0>();
    b = b == 2 ? 0 : b + 1;
    if (++cs == nk) {
      epilogue(cm0, cn0);
      reset();
      cs = 0;
      ct += bpx;
      tile_origin(ct, cm0, cn0);
    }
  }
}

// CUs of the current device (hipDeviceAttributeMultiprocessorCount), cached per device
int device_cus() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <int AMODE, int EPI, int AP = 2>
int launch(Args p, hipStream_t st) {
  const int64_t tm = (static_cast<int64_t>(p.M) + kBM - 1) / kBM;
  const int64_t tn = (static_cast<int64_t>(p.N) + kBN - 1) / kBN;
  const int64_t tiles = tm * tn;
  if (tiles > 0x7fffffff - 8) return MDL_ERR_SHAPE;
  const int64_t per_xcd = (tiles + 7) / 8;
  // one block per CU (the LDS ring allows no second); blocks per XCD capped by its tiles
  const int64_t bpx = std::min<int64_t>((device_cus() + 7) / 8, per_xcd);
  p.tiles_n = static_cast<int>(tn);
  p.tiles = static_cast<int>(tiles);
  p.per_xcd = static_cast<int>(per_xcd);
  prefill_gemm_kernel<AMODE, EPI, AP>
      <<<dim3(static_cast<unsigned>(8 * bpx)), kThreads, 0, st>>>(p);
  return launch_status();
}

// shared argument checks: k a positive multiple of 32, n of 16, 16-byte aligned operands
int check_common(const uint16_t* w, int m, int n, int k) {
  if (!w) return MDL_ERR_NULL;
  if (m < 0 || n <= 0 || k <= 0 || k % 32 != 0 || n % 16 != 0) return MDL_ERR_SHAPE;
  if (!aligned16(w)) return MDL_ERR_ALIGN;
  return MDL_OK;
}

int check_a(const uint16_t* a, int64_t lda, int a_layout, int a_parts, int k) {
  if (!a) return MDL_ERR_NULL;
  if (a_layout != MDL_LAYOUT_ROWS && a_layout != MDL_LAYOUT_TILES) return MDL_ERR_SHAPE;
  if (a_parts != 1 && a_parts != 2) return MDL_ERR_SHAPE;
  if (a_layout == MDL_LAYOUT_ROWS && lda < a_parts * static_cast<int64_t>(k))
    return MDL_ERR_SHAPE;
  if (!aligned16(a) || (a_layout == MDL_LAYOUT_ROWS && lda % 8 != 0)) return MDL_ERR_ALIGN;
  return MDL_OK;
}

// the split forms by A layout and parts
template <int EPI>
int launch_split(const Args& p, int a_layout, int a_parts, hipStream_t st) {
  if (a_layout == MDL_LAYOUT_TILES)
    return a_parts == 1 ? launch<A_TILES, EPI, 1>(p, st) : launch<A_TILES, EPI, 2>(p, st);
  return a_parts == 1 ? launch<A_ROWS, EPI, 1>(p, st) : launch<A_ROWS, EPI, 2>(p, st);
}

}  // namespace
}  // namespace mdl

using namespace mdl;

extern "C" int mdl_prefill_gemm_split(const uint16_t* a, int64_t lda, int a_layout, int a_parts,
                                      const uint16_t* w, float* out, int64_t ldo, int m, int n,
                                      int k, void* stream) {
  int rc = check_common(w, m, n, k);
  if (rc == MDL_OK) rc = check_a(a, lda, a_layout, a_parts, k);
  if (rc != MDL_OK) return rc;
  if (!out) return MDL_ERR_NULL;
  if (ldo < n) return MDL_ERR_SHAPE;
  if (!aligned16(out) || ldo % 4 != 0) return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  Args p{};
  p.a = a; p.lda = lda; p.w = w; p.out = out; p.ldo = ldo; p.M = m; p.N = n; p.K = k;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return launch_split<E_STORE>(p, a_layout, a_parts, st);
}

extern "C" int mdl_prefill_gemm_norm(const float* x, const float* gamma, float eps,
                                     const uint16_t* w, float* out, int64_t ldo, float* rstd_out,
                                     int m, int n, int k, void* stream) {
  int rc = check_common(w, m, n, k);
  if (rc != MDL_OK) return rc;
  if (!x || !gamma || !out) return MDL_ERR_NULL;
  if (ldo < n || k > kMaxNormK) return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(out) || ldo % 4 != 0)
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  Args p{};
  p.x = x; p.gamma = gamma; p.eps = eps; p.w = w; p.out = out; p.ldo = ldo;
  p.rstd_out = rstd_out; p.M = m; p.N = n; p.K = k;
  return launch<A_NORM, E_STORE>(p, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_prefill_gemm_norm_swiglu(const float* x, const float* gamma, float eps,
                                            int a_parts, const uint16_t* w_gu,
                                            const float* bias_gate, const float* bias_up,
                                            uint16_t* h_out, int h_parts, int m, int d_ff, int k,
                                            void* stream) {
  if (d_ff <= 0 || d_ff % 16 != 0 || d_ff > (1 << 28)) return MDL_ERR_SHAPE;
  if ((a_parts != 1 && a_parts != 2) || (h_parts != 1 && h_parts != 2)) return MDL_ERR_SHAPE;
  int rc = check_common(w_gu, m, 2 * d_ff, k);
  if (rc != MDL_OK) return rc;
  if (!x || !gamma || !h_out) return MDL_ERR_NULL;
  if (k > kMaxNormK) return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned8(h_out) ||
      (bias_gate && !aligned16(bias_gate)) || (bias_up && !aligned16(bias_up)))
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  Args p{};
  p.x = x; p.gamma = gamma; p.eps = eps; p.w = w_gu; p.bias_a = bias_gate; p.bias_b = bias_up;
  p.h = h_out; p.d_ff = d_ff; p.h_parts = h_parts; p.M = m; p.N = 2 * d_ff; p.K = k;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return a_parts == 1 ? launch<A_NORM, E_SWIGLU, 1>(p, st) : launch<A_NORM, E_SWIGLU, 2>(p, st);
}

extern "C" int mdl_prefill_gemm_split_residual(const uint16_t* a, int64_t lda, int a_layout,
                                               int a_parts, const uint16_t* w, float* x,
                                               const float* bias, int m, int n, int k,
                                               void* stream) {
  int rc = check_common(w, m, n, k);
  if (rc == MDL_OK) rc = check_a(a, lda, a_layout, a_parts, k);
  if (rc != MDL_OK) return rc;
  if (!x) return MDL_ERR_NULL;
  if (n % 32 != 0) return MDL_ERR_SHAPE;   // x in the fp32 tile layout: whole 32-column blocks
  if (!aligned16(x) || (bias && !aligned16(bias))) return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  Args p{};
  p.a = a; p.lda = lda; p.w = w; p.x_res = x; p.bias_a = bias; p.M = m; p.N = n; p.K = k;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return launch_split<E_RESIDUAL>(p, a_layout, a_parts, st);
}

extern "C" int mdl_prefill_gemm_norm_qkv(
    const float* x, const float* gamma, float eps, const uint16_t* w, int m, int n_heads,
    float* rstd_out, float* qkv_lead, int64_t ldq, int lead, const int32_t* kv_start,
    const int64_t* pos, const float* rope_tab, int max_x, int max_y, int max_z, int px, int py,
    int pz, float q_scale, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
    int cache_slots, int batch, int seq, const int32_t* token_row, const int32_t* token_slot,
    void* stream) {
  if (n_heads <= 0 || n_heads * kHeadDim > kMaxNormK) return MDL_ERR_SHAPE;
  const int d = n_heads * kHeadDim;
  int rc = check_common(w, m, 3 * d, d);
  if (rc != MDL_OK) return rc;
  if (!x || !gamma || !pos || !rope_tab || !q_out || !k_cache || !v_cache) return MDL_ERR_NULL;
  if ((token_row == nullptr) != (token_slot == nullptr)) return MDL_ERR_NULL;
  if (max_x <= 0 || max_y <= 0 || max_z <= 0 || px < 0 || py < 0 || pz < 0 ||
      px + py + pz != kHeadDim / 2 || batch < 0 || cache_slots <= 0 || lead < 0)
    return MDL_ERR_SHAPE;
  if (!token_slot) {   // [batch, seq] rows: token i of row b is slot i
    if (seq <= 0 || static_cast<int64_t>(batch) * seq != m) return MDL_ERR_SHAPE;
    if (seq > cache_slots) return MDL_ERR_CACHE;
  }
  if (qkv_lead && (ldq < 3 * static_cast<int64_t>(d) || ldq % 4 != 0 || !aligned16(qkv_lead)))
    return qkv_lead && ldq < 3 * static_cast<int64_t>(d) ? MDL_ERR_SHAPE : MDL_ERR_ALIGN;
  if (!aligned16(x) || !aligned16(gamma) || !aligned8(q_out) || !aligned8(k_cache) ||
      !aligned8(v_cache) || !aligned4(rope_tab))
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  Args p{};
  p.x = x; p.gamma = gamma; p.eps = eps; p.w = w; p.out = qkv_lead; p.ldo = ldq;
  p.rstd_out = rstd_out; p.pos = pos; p.rope_tab = rope_tab;
  p.ra = RopeArgs{max_x, max_y, max_z, px, py, pz};
  p.q_scale = q_scale; p.q_out = q_out; p.kc = k_cache; p.vc = v_cache;
  p.tok_row = token_row; p.tok_slot = token_slot; p.kv_start = kv_start;
  p.slots = cache_slots; p.seq = seq; p.batch = batch; p.lead = lead;
  p.M = m; p.N = 3 * d; p.K = d;
  return launch<A_NORM, E_QKV>(p, static_cast<hipStream_t>(stream));
}
