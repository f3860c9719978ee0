// K5: split-activation GEMM for decode-sized row counts on bf16 MFMA (gfx950).
//
//   out[m, n] (fp32) = sum_k (a[m, k] + a[m, K + k]) * w[n, k],   k < K
//
// a is a split activation (hi in columns [0, K), lo in [K, 2K)), w a bf16 weight in nn.Linear
// orientation ([N, K]); either may be row-major or in the MFMA tile layout of mdl_tile_matrix
// (MDL_LAYOUT_TILES).  A row-major w may be the left half of the [W | W] operand the prefill
// GEMMs take (ldw = 2K).
//
// Why not the library GEMM at decode: at M <= 256 rows hipBLASLt runs 64x64 or 32x32 tiles over
// the doubled K of [W | W] (each weight byte read twice) on at most 144 workgroups for the small
// model's projections, each waiting on a K loop of dependent loads.  Here:
//   - every weight fragment is loaded once and feeds two MFMAs (the hi and the lo rows);
//   - the 8 waves of a block split K and meet once, in LDS, at the end: a wave has 1-14 k-steps
//     of 32 and issues the loads of 4 of them before its first MFMA;
//   - the row tiles sharing one weight tile run on one XCD (block i runs on XCD i mod 8), so the
//     weight tile comes from HBM once and from that XCD's L2 after that;
//   - with both operands tiled, each wave load is one contiguous kilobyte.  A row-major operand
//     fragment spans 16 rows of 64 bytes and four consecutive lanes touch four cache lines; at
//     these sizes that costs 1.5x (weight) and 2x (both) in time (measured at the model shapes).
//
// MFMA formulation: D^T = W . A^T with v_mfma_f32_16x16x32_bf16 (layouts in mfma.h).  The A
// operand is 16 weight rows, the B operand 16 activation rows; lane (c, g) holds row c at
// k = 32 s + 8 g .. + 7 (the tile layout stores exactly these 16 bytes at lane order).  The
// accumulator of lane (c, g) holds out[m0 + c][n0 + 4 g .. + 3]: one float4 per lane.
// Summation order is fixed (each wave's k-steps in order, hi before lo, waves summed 0..7 in the
// reduction), so a given tile shape is bit-reproducible; layouts do not change the result.
#include "common.h"
#include "mfma.h"

namespace mdl {

namespace {

constexpr int kGemmWaves = 8;
constexpr int kU = 4;   // k-steps whose loads are in flight together

// Pointer to lane (c, g)'s 16 bytes of row block `rb` (rows 16 rb + c) at k-step 0 of an
// operand with `cols` columns: row-major (row stride ld, rows clamped to n_rows - 1) or tiled
// (row blocks clamped to the last one; its padding rows exist in a tiled buffer).
template <bool TILED>
__device__ __forceinline__ const uint16_t* frag_base(const uint16_t* p, int64_t ld, int rb,
                                                     int n_rows, int cols, int lane) {
  if constexpr (TILED) {
    const int last = (n_rows + 15) / 16 - 1;
    return p + static_cast<int64_t>(min(rb, last)) * (cols / 32) * 512 + 8 * lane;
  } else {
    return p + static_cast<int64_t>(min(16 * rb + (lane & 15), n_rows - 1)) * ld +
           8 * (lane >> 4);
  }
}
// element step from k-step 0 to k-step s (k = 32 s)
template <bool TILED>
__device__ __forceinline__ int64_t frag_step(int s) {
  return TILED ? static_cast<int64_t>(512) * s : static_cast<int64_t>(32) * s;
}

// SwiGLU epilogue (the gate / up projection with the MLP gate fused): w holds [W_gate; W_up]
// with their 16-row blocks interleaved (block 2 b = gate rows 16 b .., block 2 b + 1 = up rows
// 16 b ..), so output fragments 2 p and 2 p + 1 of a block are the gate and the up value of the
// same 16 channels.
struct SwigluEpi {
  const float* rstd;       // [M] or NULL (1)
  const float* bias_gate;  // [F] or NULL (0)
  const float* bias_up;    // [F] or NULL (0)
  uint16_t* h;             // split bf16 [M, 2F] in the tile layout
  int d_ff;
};

template <int TN, int TM, bool WT, bool AT, bool SWIGLU = false>
__global__ __launch_bounds__(64 * kGemmWaves) void split_gemm_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ w, int64_t ldw,
    float* __restrict__ out, int64_t ldo, int M, int N, int K, int n_tiles, int m_tiles,
    int per_xcd, SwigluEpi epi = {}) {
  constexpr int FN = TN / 16, FM = TM / 16, NW = kGemmWaves;
  static_assert(TN % 16 == 0 && TM % 16 == 0, "tile must be a multiple of 16");
  // logical tile of this block: tiles per_xcd * x .. per_xcd * (x + 1) - 1 run on XCD x
  const int L = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (L >= n_tiles * m_tiles) return;   // whole block, before any barrier
  const int nt = L / m_tiles, mt = L - nt * m_tiles;
  const int n0 = nt * TN, m0 = mt * TM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // rows past M / N load a valid row (in bounds; their results are never stored)
  const uint16_t* wp[FN];
  const uint16_t* ap[FM];
#pragma unroll
  for (int i = 0; i < FN; ++i) wp[i] = frag_base<WT>(w, ldw, n0 / 16 + i, N, K, lane);
#pragma unroll
  for (int j = 0; j < FM; ++j) ap[j] = frag_base<AT>(a, lda, m0 / 16 + j, M, 2 * K, lane);
  const int64_t lo_off = frag_step<AT>(K / 32);   // hi k-step s -> lo k-step s + K / 32

  f32x4_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // k-steps of 32: wave w takes [nk w / NW, nk (w + 1) / NW), contiguous
  const int nk = K >> 5;
  const int s0 = (nk * wave) / NW, s1 = (nk * (wave + 1)) / NW;
  for (int s = s0; s < s1; s += kU) {
    uint4 wf[kU][FN], ah[kU][FM], al[kU][FM];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      // steps past s1 reload step s1 - 1 (same lines, in bounds) and are not multiplied
      const int su = min(s + u, s1 - 1);
#pragma unroll
      for (int i = 0; i < FN; ++i)
        wf[u][i] = *reinterpret_cast<const uint4*>(wp[i] + frag_step<WT>(su));
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        ah[u][j] = *reinterpret_cast<const uint4*>(ap[j] + frag_step<AT>(su));
        al[u][j] = *reinterpret_cast<const uint4*>(ap[j] + frag_step<AT>(su) + lo_off);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (s + u < s1) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wf[u][i]),
                                                                as_bf16x8(ah[u][j]), acc[i][j],
                                                                0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wf[u][i]),
                                                                as_bf16x8(al[u][j]), acc[i][j],
                                                                0, 0, 0);
          }
      }
    }
  }

  // cross-wave reduction: every wave parks its accumulators (16 bytes per lane, lane-major,
  // conflict-free), then each thread sums one float4 over the waves in wave order and stores it
  __shared__ f32x4_t red[NW][FN * FM][64];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) red[wave][i * FM + j][lane] = acc[i][j];
  __syncthreads();
  if constexpr (SWIGLU) {
    static_assert(FN % 2 == 0, "the SwiGLU epilogue pairs gate and up fragments");
    // q = (channel block p, row block j, lane): gate fragment 2 p, up fragment 2 p + 1
    for (int q = threadIdx.x; q < (FN / 2) * FM * 64; q += 64 * NW) {
      const int pj = q >> 6, ln = q & 63;
      const int p = pj / FM, j = pj - p * FM;
      const int tg = (2 * p) * FM + j, tu = (2 * p + 1) * FM + j;
      f32x4_t gv = red[0][tg][ln], uv = red[0][tu][ln];
#pragma unroll
      for (int wv = 1; wv < NW; ++wv) {
        gv += red[wv][tg][ln];
        uv += red[wv][tu][ln];
      }
      const int m = m0 + 16 * j + (ln & 15);
      const int ch = 16 * (n0 / 32 + p) + 4 * (ln >> 4);   // gate / up channel of element 0
      if (m < M && 2 * ch < N) {
        const float r = epi.rstd ? epi.rstd[m] : 1.f;
        const float4 bg = epi.bias_gate ? *reinterpret_cast<const float4*>(epi.bias_gate + ch)
                                        : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 bu = epi.bias_up ? *reinterpret_cast<const float4*>(epi.bias_up + ch)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
        // the arithmetic of K3 (swiglu.hip), so fused and unfused agree bit for bit
        const float o[4] = {silu_mul(fmaf(r, gv[0], bg.x), fmaf(r, uv[0], bu.x)),
                            silu_mul(fmaf(r, gv[1], bg.y), fmaf(r, uv[1], bu.y)),
                            silu_mul(fmaf(r, gv[2], bg.z), fmaf(r, uv[2], bu.z)),
                            silu_mul(fmaf(r, gv[3], bg.w), fmaf(r, uv[3], bu.w))};
        uint2 hi, lo;
        split4(o, hi, lo);
        *reinterpret_cast<uint2*>(epi.h + tile_off(m, ch, 2 * epi.d_ff)) = hi;
        *reinterpret_cast<uint2*>(epi.h + tile_off(m, epi.d_ff + ch, 2 * epi.d_ff)) = lo;
      }
    }
  } else {
    for (int q = threadIdx.x; q < FN * FM * 64; q += 64 * NW) {
      const int t = q >> 6, ln = q & 63;
      f32x4_t v = red[0][t][ln];
#pragma unroll
      for (int wv = 1; wv < NW; ++wv) v += red[wv][t][ln];
      const int i = t / FM, j = t - i * FM;
      const int m = m0 + 16 * j + (ln & 15);
      const int n = n0 + 16 * i + 4 * (ln >> 4);
      if (m < M && n < N)
        *reinterpret_cast<float4*>(out + static_cast<int64_t>(m) * ldo + n) =
            make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

// The compiled block shapes (TN weight rows x TM activation rows), numbered from 1 by the
// `tile` argument.  Shapes with 4 or 16 waves, 16 x 64 and 32 x 64 were measured and never won.
struct GemmTile {
  int tn, tm;
};
constexpr GemmTile kTiles[] = {{64, 64}, {128, 32}, {64, 32}, {32, 32}, {64, 16}, {32, 16}};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

// The automatic choice: the tile minimising the bytes one block moves into its CU times the
// number of 256-block rounds, ties to the lower total traffic.  A block holds a CU's load path
// for about a memory latency, so the critical path is one block's operand bytes per round.  At
// the 12 decode shapes of the reference presets (M = 256 / 128 / 64) it picks the measured
// fastest shape or one within 3% of it.
int pick_tile(int M, int N, int K) {
  int best = 0;
  double best_key = 1e300, best_total = 1e300;
  for (int t = 0; t < kNumTiles; ++t) {
    const double blocks = static_cast<double>((N + kTiles[t].tn - 1) / kTiles[t].tn) *
                          ((M + kTiles[t].tm - 1) / kTiles[t].tm);
    const double per_block = (2.0 * kTiles[t].tn + 4.0 * kTiles[t].tm) * K;
    const double rounds = static_cast<double>((static_cast<int64_t>(blocks) + 255) / 256);
    const double key = per_block * rounds, total = per_block * blocks;
    if (key < best_key * 0.999 || (key < best_key * 1.001 && total < best_total)) {
      best = t;
      best_key = key;
      best_total = total;
    }
  }
  return best + 1;
}

template <int TN, int TM, bool WT, bool AT, bool SWIGLU = false>
int launch_tile(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, float* out,
                int64_t ldo, int M, int N, int K, hipStream_t st, SwigluEpi epi = {}) {
  const int n_tiles = (N + TN - 1) / TN, m_tiles = (M + TM - 1) / TM;
  const int64_t tiles = static_cast<int64_t>(n_tiles) * m_tiles;
  const int64_t per_xcd = (tiles + 7) / 8;
  if (8 * per_xcd > 0x7fffffff) return MDL_ERR_SHAPE;
  hipLaunchKernelGGL((split_gemm_kernel<TN, TM, WT, AT, SWIGLU>),
                     dim3(static_cast<unsigned>(8 * per_xcd)), dim3(64 * kGemmWaves), 0, st, a,
                     lda, w, ldw, out, ldo, M, N, K, n_tiles, m_tiles,
                     static_cast<int>(per_xcd), epi);
  return launch_status();
}

template <bool WT, bool AT>
int launch_layouts(int tile, const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw,
                   float* out, int64_t ldo, int M, int N, int K, hipStream_t st) {
  switch (tile) {
    case 1: return launch_tile<64, 64, WT, AT>(a, lda, w, ldw, out, ldo, M, N, K, st);
    case 2: return launch_tile<128, 32, WT, AT>(a, lda, w, ldw, out, ldo, M, N, K, st);
    case 3: return launch_tile<64, 32, WT, AT>(a, lda, w, ldw, out, ldo, M, N, K, st);
    case 4: return launch_tile<32, 32, WT, AT>(a, lda, w, ldw, out, ldo, M, N, K, st);
    case 5: return launch_tile<64, 16, WT, AT>(a, lda, w, ldw, out, ldo, M, N, K, st);
    case 6: return launch_tile<32, 16, WT, AT>(a, lda, w, ldw, out, ldo, M, N, K, st);
    default: return MDL_ERR_SHAPE;
  }
}

int launch_swiglu(int tile, const uint16_t* a, const uint16_t* w, int M, int N, int K,
                  hipStream_t st, const SwigluEpi& epi) {
  switch (tile) {
    case 1: return launch_tile<64, 64, true, true, true>(a, 0, w, 0, nullptr, 0, M, N, K, st, epi);
    case 2: return launch_tile<128, 32, true, true, true>(a, 0, w, 0, nullptr, 0, M, N, K, st, epi);
    case 3: return launch_tile<64, 32, true, true, true>(a, 0, w, 0, nullptr, 0, M, N, K, st, epi);
    case 4: return launch_tile<32, 32, true, true, true>(a, 0, w, 0, nullptr, 0, M, N, K, st, epi);
    case 5: return launch_tile<64, 16, true, true, true>(a, 0, w, 0, nullptr, 0, M, N, K, st, epi);
    case 6: return launch_tile<32, 16, true, true, true>(a, 0, w, 0, nullptr, 0, M, N, K, st, epi);
    default: return MDL_ERR_SHAPE;
  }
}

// dst = src in the tile layout, rows padded to a multiple of 16 with zeros.  One thread per
// 16-byte lane chunk of dst.
__global__ void tile_matrix_kernel(const uint16_t* __restrict__ src, int64_t ld, int rows,
                                   int cols, int64_t chunks, uint16_t* __restrict__ dst) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= chunks) return;
  const int64_t blk = q >> 6;
  const int l = static_cast<int>(q & 63), c = l & 15, g = l >> 4;
  const int64_t rb = blk / (cols / 32), cb = blk - rb * (cols / 32);
  const int64_t r = 16 * rb + c;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (r < rows) v = *reinterpret_cast<const uint4*>(src + r * ld + 32 * cb + 8 * g);
  *reinterpret_cast<uint4*>(dst + 8 * q) = v;
}

}  // namespace

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_gemm_split(const uint16_t* a, int64_t lda, int a_layout, const uint16_t* w,
                              int64_t ldw, int w_layout, float* out, int64_t ldo, int m, int n,
                              int k, int tile, void* stream) {
  if (!a || !w || !out) return MDL_ERR_NULL;
  const bool at = a_layout == MDL_LAYOUT_TILES, wt = w_layout == MDL_LAYOUT_TILES;
  if ((!at && a_layout != MDL_LAYOUT_ROWS) || (!wt && w_layout != MDL_LAYOUT_ROWS))
    return MDL_ERR_SHAPE;
  if (m < 0 || n < 0 || k <= 0 || k % 32 != 0 || n % 4 != 0 || tile < 0 || tile > kNumTiles ||
      ldo < n || (!at && lda < 2 * static_cast<int64_t>(k)) || (!wt && ldw < k))
    return MDL_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(w) || !aligned16(out) || (!at && lda % 8 != 0) ||
      (!wt && ldw % 8 != 0) || ldo % 4 != 0)
    return MDL_ERR_ALIGN;
  if (m == 0 || n == 0) return MDL_OK;
  auto st = static_cast<hipStream_t>(stream);
  const int t = tile ? tile : pick_tile(m, n, k);
  if (wt && at) return launch_layouts<true, true>(t, a, lda, w, ldw, out, ldo, m, n, k, st);
  if (wt) return launch_layouts<true, false>(t, a, lda, w, ldw, out, ldo, m, n, k, st);
  if (at) return launch_layouts<false, true>(t, a, lda, w, ldw, out, ldo, m, n, k, st);
  return launch_layouts<false, false>(t, a, lda, w, ldw, out, ldo, m, n, k, st);
}

extern "C" int mdl_gemm_split_tiles(void) { return kNumTiles; }

extern "C" int mdl_gemm_split_pick(int m, int n, int k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return pick_tile(m, n, k);
}

extern "C" int mdl_tile_matrix(const uint16_t* src, int64_t ld, int rows, int cols,
                               uint16_t* dst, void* stream) {
  if (!src || !dst) return MDL_ERR_NULL;
  if (rows < 0 || cols <= 0 || cols % 32 != 0 || ld < cols) return MDL_ERR_SHAPE;
  if (!aligned16(src) || !aligned16(dst) || ld % 8 != 0) return MDL_ERR_ALIGN;
  if (rows == 0) return MDL_OK;
  const int64_t chunks = static_cast<int64_t>((rows + 15) / 16) * 16 * (cols / 8);
  const int64_t blocks = (chunks + 255) / 256;
  if (blocks > 0x7fffffff) return MDL_ERR_SHAPE;
  hipLaunchKernelGGL(tile_matrix_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, ld, rows, cols, chunks, dst);
  return launch_status();
}

extern "C" int mdl_gemm_split_swiglu(const uint16_t* a, const uint16_t* w_gu, const float* rstd,
                                     const float* bias_gate, const float* bias_up,
                                     uint16_t* h_out, int m, int d_ff, int k, int tile,
                                     void* stream) {
  if (!a || !w_gu || !h_out) return MDL_ERR_NULL;
  if (m < 0 || d_ff <= 0 || d_ff % 16 != 0 || k <= 0 || k % 32 != 0 || tile < 0 ||
      tile > kNumTiles)
    return MDL_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(w_gu) || !aligned8(h_out) ||
      (bias_gate && !aligned16(bias_gate)) || (bias_up && !aligned16(bias_up)))
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  const int n = 2 * d_ff;
  const SwigluEpi epi{rstd, bias_gate, bias_up, h_out, d_ff};
  return launch_swiglu(tile ? tile : pick_tile(m, n, k), a, w_gu, m, n, k,
                       static_cast<hipStream_t>(stream), epi);
}
