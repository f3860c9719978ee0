// K5: split-activation GEMM for decode-sized row counts on bf16 MFMA (gfx950).
//
//   acc[m, n] (fp32) = sum_k (a_hi[m, k] + a_lo[m, k]) * w[n, k],   k < K
//
// w is a bf16 weight in nn.Linear orientation ([N, K]); a is the split activation (hi = bf16(v),
// lo = bf16(v - hi)) of v[m, k], taken from one of three sources (AMODE):
//   A_ROWS   a split [M, 2K] row-major (hi in columns [0, K), lo in [K, 2K));
//   A_TILES  the same matrix in the MFMA tile layout (MDL_LAYOUT_TILES);
//   A_NORM   v = x * gamma from the fp32 residual stream x [M, K] in the fp32 tile layout: the
//            RMSNorm of the next projection done in the GEMM's prologue.  A block sees whole
//            rows (its waves cover all of K), so it also sums x^2 and has rstd of its rows.
// and acc goes to one of three epilogues (EPI):
//   E_STORE     out[m, n] = acc (fp32, row-major); with A_NORM the n-tile-0 blocks also store
//               rstd[m] (the decode attention applies it to q / k / v);
//   E_SWIGLU    h = split(silu(rstd g + b_g) * (rstd u + b_u)) from the gate / up pair of
//               fragments (weights with 16-row gate / up blocks interleaved), tiled;
//   E_RESIDUAL  x[m, n] += acc (+ bias[n]) in place on the fp32 tile-layout residual stream
//               (each element has one owner block, so the update needs no synchronisation);
//   E_QKV       K2 for the decode token of each row on the qkv accumulators (A_NORM): rstd,
//               3D RoPE of q and k, the softmax scale on q; q bf16 [M, d] and K / V into cache
//               slot t (*slot_dev) of row m, so the attention launch needs no prologue.
//
// Why not the library GEMM at decode: at M <= 256 rows hipBLASLt runs 64x64 or 32x32 tiles over
// the doubled K of [W | W] (each weight byte read twice) on at most 144 workgroups for the small
// model's projections, each waiting on a K loop of dependent loads.  Here:
//   - every weight fragment is loaded once and feeds two MFMAs (the hi and the lo rows);
//   - the 8 waves of a block split K and meet once, in LDS, at the end: a wave has 1-14 k-steps
//     of 32 and issues the loads of 4 of them (3 in the two largest A_NORM tiles) before its
//     first MFMA;
//   - the row tiles sharing one weight tile run on one XCD (block i runs on XCD i mod 8), so the
//     weight tile comes from HBM once and from that XCD's L2 after that;
//   - with tiled operands each wave load is one contiguous kilobyte.  A row-major operand
//     fragment spans 16 rows of 64 bytes and four consecutive lanes touch four cache lines; at
//     these sizes that costs 1.5x (weight) and 2x (both) in time (measured at the model shapes).
//
// MFMA formulation: D^T = W . A^T with v_mfma_f32_16x16x32_bf16 (layouts in mfma.h).  The A
// operand is 16 weight rows, the B operand 16 activation rows; lane (c, g) holds row c at
// k = 32 s + 8 g .. + 7 (the tile layouts store exactly these elements at lane order).  The
// accumulator of lane (c, g) holds acc[m0 + c][n0 + 4 g .. + 3]: one float4 per lane.
// Summation order is fixed (each wave's k-steps in order, hi before lo, waves summed 0..7 in the
// reduction), so a given tile shape is bit-reproducible; the A source and the layouts do not
// change the result.
//
// fp32 weights (WL forms): a model whose parameters are fp32 passes its weight as two bf16
// matrices in the same tile layout, w = bf16(W) and w_lo = bf16(W - w).  Every k-step then adds
// a third product, a_hi . w_lo, after the hi and lo products, so the GEMM sees W to ~2^-17 like
// the activation (the dropped a_lo . w_lo term is ~2^-18 of the product).
#include "common.h"
#include "mfma.h"
#include "rope.h"

namespace mdl {

namespace {

constexpr int kGemmWaves = 8;
constexpr int kU = 4;   // k-steps whose loads are in flight together (A_NORM, large tiles: 2)

enum AMode { A_ROWS = 0, A_TILES = 1, A_NORM = 2 };
enum Epi { E_STORE = 0, E_SWIGLU = 1, E_RESIDUAL = 2, E_QKV = 3 };

struct GemmArgs {
  const uint16_t* a;       // A_ROWS / A_TILES: split activation
  int64_t lda;             // A_ROWS row stride (elements)
  const float* x;          // A_NORM: fp32 residual stream, tile layout, [M, K]
  const float* gamma;      // A_NORM: RMSNorm gain [K]
  float eps;
  const uint16_t* w;
  const uint16_t* wl;      // WL forms: low bf16 part of an fp32 weight, tiled like w
  int64_t ldw;             // row-major w row stride (elements)
  float* out;              // E_STORE: [M, N] fp32, row stride ldo
  int64_t ldo;
  float* rstd_out;         // E_STORE with A_NORM: [M] (may be NULL)
  const float* rstd_in;    // E_SWIGLU with a split A: [M] or NULL (1)
  const float* bias_a;     // E_SWIGLU: gate bias [F]; E_RESIDUAL: bias [N] (may be NULL)
  const float* bias_b;     // E_SWIGLU: up bias [F] (may be NULL)
  uint16_t* h;             // E_SWIGLU: split [M, 2F], tile layout
  float* x_res;            // E_RESIDUAL: fp32 residual stream [M, N], tile layout
  int d_ff;
  // E_QKV: row m's token at pos[m], its K / V to slot *slot_dev (or slot0) of cache row m
  const int64_t* pos;
  const float* rope_tab;
  RopeArgs ra;
  float q_scale;
  uint16_t* q_out;
  uint16_t* kc;
  uint16_t* vc;
  const int32_t* slot_dev;
  int slot0, slots;
  int M, N, K, n_tiles, m_tiles, per_xcd;
};

// Pointer to lane (c, g)'s 16 bytes of row block `rb` (rows 16 rb + c) at k-step 0 of a bf16
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
// element step from k-step 0 to k-step s (k = 32 s) of a bf16 operand
template <bool TILED>
__device__ __forceinline__ int64_t frag_step(int s) {
  return TILED ? static_cast<int64_t>(512) * s : static_cast<int64_t>(32) * s;
}

template <int TN, int TM, bool WT, int AMODE, int EPI, bool WL>
__global__ __launch_bounds__(64 * kGemmWaves) void split_gemm_kernel(const GemmArgs p) {
  constexpr int FN = TN / 16, FM = TM / 16, NW = kGemmWaves;
  static_assert(!WL || WT, "the low weight part is tiled");
  // k-steps in flight: the fp32 x and gamma fragments of A_NORM take twice the registers of a
  // split operand, and 4 steps of the two largest tiles would spill; the WL forms hold a second
  // weight fragment per step
  constexpr int U = WL ? 2 : ((AMODE == A_NORM && FN * FM >= 16) ? 3 : kU);
  static_assert(TN % 16 == 0 && TM % 16 == 0, "tile must be a multiple of 16");
  const int M = p.M, N = p.N, K = p.K;
  // logical tile of this block: tiles per_xcd * x .. per_xcd * (x + 1) - 1 run on XCD x
  const int L = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
  if (L >= p.n_tiles * p.m_tiles) return;   // whole block, before any barrier
  const int nt = L / p.m_tiles, mt = L - nt * p.m_tiles;
  const int n0 = nt * TN, m0 = mt * TM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4;

  // rows past M / N load a valid row (in bounds; their results are never stored)
  const uint16_t* wp[FN];
#pragma unroll
  for (int i = 0; i < FN; ++i) wp[i] = frag_base<WT>(p.w, p.ldw, n0 / 16 + i, N, K, lane);
  const uint16_t* wlp[WL ? FN : 1];
  if constexpr (WL) {
#pragma unroll
    for (int i = 0; i < FN; ++i) wlp[i] = frag_base<true>(p.wl, 0, n0 / 16 + i, N, K, lane);
  }
  const uint16_t* ap[FM];
  const float* xp[FM];
  int64_t lo_off = 0;
  if constexpr (AMODE == A_NORM) {
    // fp32 tile layout: 16 x 32 blocks of 512 floats, lane l's elements 0..3 at 4 l and 4..7 at
    // 256 + 4 l; padding rows of the last row block exist
    const int last = (M + 15) / 16 - 1;
#pragma unroll
    for (int j = 0; j < FM; ++j)
      xp[j] = p.x + static_cast<int64_t>(min(m0 / 16 + j, last)) * (K / 32) * 512 + 4 * lane;
  } else {
#pragma unroll
    for (int j = 0; j < FM; ++j)
      ap[j] = frag_base<AMODE == A_TILES>(p.a, p.lda, m0 / 16 + j, M, 2 * K, lane);
    lo_off = frag_step<AMODE == A_TILES>(K / 32);   // hi k-step s -> lo k-step s + K / 32
  }

  f32x4_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[FM];   // A_NORM: this lane's part of sum(x^2) of row m0 + 16 j + c
#pragma unroll
  for (int j = 0; j < FM; ++j) ss[j] = 0.f;

  // E_QKV: the epilogue's RoPE inputs are fetched ahead -- the positions of its rows here, the
  // table entries right after the k-loop (their latency under the cross-wave reduction) -- so
  // no chain of dependent loads follows the GEMM.  Thread's element group gi is q = tid + gi *
  // 64 NW of the epilogue loop below.
  constexpr int G = (FN * FM + NW - 1) / NW;   // epilogue element groups per thread
  int64_t rpos[EPI == E_QKV ? G : 1][3];
  if constexpr (EPI == E_QKV) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int q = threadIdx.x + gi * 64 * NW;
      const int t = q >> 6, ln = q & 63;
      const int m = min(m0 + 16 * (t % FM) + (ln & 15), M - 1);
      const int64_t* pos3 = p.pos + static_cast<int64_t>(m) * 3;
      rpos[gi][0] = pos3[0];
      rpos[gi][1] = pos3[1];
      rpos[gi][2] = pos3[2];
    }
  }

  // E_RESIDUAL: the epilogue's x elements (and bias) are loaded here, before the k-loop: this
  // block is their only writer, so the values are those the epilogue would read, and the load
  // latency is spent under the GEMM instead of after the reduction
  float4 xpre[EPI == E_RESIDUAL ? G : 1], bpre[EPI == E_RESIDUAL ? G : 1];
  if constexpr (EPI == E_RESIDUAL) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int q = threadIdx.x + gi * 64 * NW;
      const int t = q >> 6, ln = q & 63;
      const int i = t / FM, j = t - i * FM;
      const int m = m0 + 16 * j + (ln & 15);
      const int n = n0 + 16 * i + 4 * (ln >> 4);
      xpre[gi] = bpre[gi] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (q < FN * FM * 64 && m < M && n < N) {
        xpre[gi] = *reinterpret_cast<const float4*>(p.x_res + tile_off32(m, n, N));
        if (p.bias_a) bpre[gi] = *reinterpret_cast<const float4*>(p.bias_a + n);
      }
    }
  }

  // k-steps of 32: wave w takes [nk w / NW, nk (w + 1) / NW), contiguous
  const int nk = K >> 5;
  const int s0 = (nk * wave) / NW, s1 = (nk * (wave + 1)) / NW;
  for (int s = s0; s < s1; s += U) {
    uint4 wf[U][FN], ah[U][FM], al[U][FM], wlf[U][WL ? FN : 1];
    float4 xv[U][FM][2], gv[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // steps past s1 reload step s1 - 1 (same lines, in bounds) and are not multiplied
      const int su = min(s + u, s1 - 1);
#pragma unroll
      for (int i = 0; i < FN; ++i)
        wf[u][i] = *reinterpret_cast<const uint4*>(wp[i] + frag_step<WT>(su));
      if constexpr (WL) {
#pragma unroll
        for (int i = 0; i < FN; ++i)
          wlf[u][i] = *reinterpret_cast<const uint4*>(wlp[i] + frag_step<true>(su));
      }
      if constexpr (AMODE == A_NORM) {
        gv[u][0] = *reinterpret_cast<const float4*>(p.gamma + 32 * su + 8 * g);
        gv[u][1] = *reinterpret_cast<const float4*>(p.gamma + 32 * su + 8 * g + 4);
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          xv[u][j][0] = *reinterpret_cast<const float4*>(xp[j] + 512 * static_cast<int64_t>(su));
          xv[u][j][1] =
              *reinterpret_cast<const float4*>(xp[j] + 512 * static_cast<int64_t>(su) + 256);
        }
      } else {
#pragma unroll
        for (int j = 0; j < FM; ++j) {
          ah[u][j] = *reinterpret_cast<const uint4*>(ap[j] + frag_step<AMODE == A_TILES>(su));
          al[u][j] =
              *reinterpret_cast<const uint4*>(ap[j] + frag_step<AMODE == A_TILES>(su) + lo_off);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s + u < s1) {
        if constexpr (AMODE == A_NORM) {
          // the split of x * gamma, as the norm kernels write it (t rounded, then split)
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const float xe[8] = {xv[u][j][0].x, xv[u][j][0].y, xv[u][j][0].z, xv[u][j][0].w,
                                 xv[u][j][1].x, xv[u][j][1].y, xv[u][j][1].z, xv[u][j][1].w};
            const float ge[8] = {gv[u][0].x, gv[u][0].y, gv[u][0].z, gv[u][0].w,
                                 gv[u][1].x, gv[u][1].y, gv[u][1].z, gv[u][1].w};
            float t[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              t[e] = xe[e] * ge[e];
              ss[j] = fmaf(xe[e], xe[e], ss[j]);
            }
            split8(t, ah[u][j], al[u][j]);
          }
        }
        // every hi product before the lo products: consecutive MFMAs write different
        // accumulators, and each accumulator still adds hi before lo
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wf[u][i]),
                                                                as_bf16x8(ah[u][j]), acc[i][j],
                                                                0, 0, 0);
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int j = 0; j < FM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wf[u][i]),
                                                                as_bf16x8(al[u][j]), acc[i][j],
                                                                0, 0, 0);
        if constexpr (WL) {
#pragma unroll
          for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int j = 0; j < FM; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  as_bf16x8(wlf[u][i]), as_bf16x8(ah[u][j]), acc[i][j], 0, 0, 0);
        }
      }
    }
  }

  // E_QKV: cos / sin of RoPE pairs dim / 2 and dim / 2 + 1 of each element group (q, k parts)
  float rcs[EPI == E_QKV ? G : 1][4];
  if constexpr (EPI == E_QKV) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int q = threadIdx.x + gi * 64 * NW;
      const int t = q >> 6, ln = q & 63;
      const int n = min(n0 + 16 * (t / FM) + 4 * (ln >> 4), N - 1);
      const int d = N / 3;
      const int e = n - (n / d) * d;
      const int dim = e - (e / kHeadDim) * kHeadDim;
      rope_cos_sin3(dim / 2, rpos[gi][0], rpos[gi][1], rpos[gi][2], p.rope_tab, p.ra,
                    rcs[gi][0], rcs[gi][1]);
      rope_cos_sin3(dim / 2 + 1, rpos[gi][0], rpos[gi][1], rpos[gi][2], p.rope_tab, p.ra,
                    rcs[gi][2], rcs[gi][3]);
    }
  }

  // cross-wave reduction: every wave parks its accumulators (16 bytes per lane, lane-major,
  // conflict-free), then each thread sums one float4 over the waves in wave order
  __shared__ f32x4_t red[NW][FN * FM][64];
  __shared__ float ss_red[NW][TM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j) red[wave][i * FM + j][lane] = acc[i][j];
  if constexpr (AMODE == A_NORM) {
    // the four lane groups of a row, then the waves (below): a fixed order
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      float v = ss[j];
      v += __shfl_xor(v, 16, kWave);
      v += __shfl_xor(v, 32, kWave);
      if (g == 0) ss_red[wave][16 * j + (lane & 15)] = v;
    }
  }
  __syncthreads();
  // rstd of local row r (A_NORM), as the norm kernels compute it from the sum of squares
  auto row_rstd = [&](int r) {
    float tot = ss_red[0][r];
#pragma unroll
    for (int wv = 1; wv < NW; ++wv) tot += ss_red[wv][r];
    return rsqrtf(tot / static_cast<float>(K) + p.eps);
  };
  if constexpr (AMODE == A_NORM && (EPI == E_STORE || EPI == E_QKV)) {
    if (p.rstd_out && nt == 0 && threadIdx.x < TM && m0 + static_cast<int>(threadIdx.x) < M)
      p.rstd_out[m0 + threadIdx.x] = row_rstd(threadIdx.x);
  }
  if constexpr (EPI == E_SWIGLU) {
    static_assert(FN % 2 == 0, "the SwiGLU epilogue pairs gate and up fragments");
    // q = (channel block pb, row block j, lane): gate fragment 2 pb, up fragment 2 pb + 1
    for (int q = threadIdx.x; q < (FN / 2) * FM * 64; q += 64 * NW) {
      const int pj = q >> 6, ln = q & 63;
      const int pb = pj / FM, j = pj - pb * FM;
      const int tg = (2 * pb) * FM + j, tu = (2 * pb + 1) * FM + j;
      f32x4_t gsum = red[0][tg][ln], usum = red[0][tu][ln];
#pragma unroll
      for (int wv = 1; wv < NW; ++wv) {
        gsum += red[wv][tg][ln];
        usum += red[wv][tu][ln];
      }
      const int m = m0 + 16 * j + (ln & 15);
      const int ch = 16 * (n0 / 32 + pb) + 4 * (ln >> 4);   // gate / up channel of element 0
      if (m < M && 2 * ch < N) {
        float r = 1.f;
        if constexpr (AMODE == A_NORM) r = row_rstd(16 * j + (ln & 15));
        else if (p.rstd_in) r = p.rstd_in[m];
        const float4 bg = p.bias_a ? *reinterpret_cast<const float4*>(p.bias_a + ch)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 bu = p.bias_b ? *reinterpret_cast<const float4*>(p.bias_b + ch)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        // the arithmetic of K3 (swiglu.hip), so fused and unfused agree bit for bit
        const float o[4] = {silu_mul(fmaf(r, gsum[0], bg.x), fmaf(r, usum[0], bu.x)),
                            silu_mul(fmaf(r, gsum[1], bg.y), fmaf(r, usum[1], bu.y)),
                            silu_mul(fmaf(r, gsum[2], bg.z), fmaf(r, usum[2], bu.z)),
                            silu_mul(fmaf(r, gsum[3], bg.w), fmaf(r, usum[3], bu.w))};
        uint2 hi, lo;
        split4(o, hi, lo);
        *reinterpret_cast<uint2*>(p.h + tile_off(m, ch, 2 * p.d_ff)) = hi;
        *reinterpret_cast<uint2*>(p.h + tile_off(m, p.d_ff + ch, 2 * p.d_ff)) = lo;
      }
    }
  } else {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int q = threadIdx.x + gi * 64 * NW;
      if (q >= FN * FM * 64) break;
      const int t = q >> 6, ln = q & 63;
      f32x4_t v = red[0][t][ln];
#pragma unroll
      for (int wv = 1; wv < NW; ++wv) v += red[wv][t][ln];
      const int i = t / FM, j = t - i * FM;
      const int m = m0 + 16 * j + (ln & 15);
      const int n = n0 + 16 * i + 4 * (ln >> 4);
      if (m < M && n < N) {
        if constexpr (EPI == E_QKV) {
          static_assert(AMODE == A_NORM, "E_QKV follows the norm prologue");
          // the arithmetic of K2 (rope_cache.hip): channels n .. n + 3 of row m are dims
          // dim .. dim + 3 of one head of q, k or v (d is a multiple of 64), RoPE pairs dim / 2
          // and dim / 2 + 1
          const int d = N / 3;
          const int part = n / d, e = n - part * d;
          const int head = e / kHeadDim, dim = e - head * kHeadDim;
          const float r = row_rstd(16 * j + (ln & 15));
          const float a0 = v[0] * r, a1 = v[1] * r, a2 = v[2] * r, a3 = v[3] * r;
          const int t = p.slot_dev ? *p.slot_dev : p.slot0;
          const bool in_cache = t >= 0 && t < p.slots;
          // K / V go out with the non-temporal hint: 8 bytes per (row, head, slot t) of cache
          // rows megabytes apart, read next by the attention's non-temporal loads
          const int64_t crow =
              ((static_cast<int64_t>(m) * (d / kHeadDim) + head) * p.slots + t) * kHeadDim + dim;
          uint2 o;
          if (part == 2) {
            if (in_cache) {
              o.x = pack_bf2(a0, a1);
              o.y = pack_bf2(a2, a3);
              st_u2<true>(p.vc + crow, o);
            }
          } else {
            float y0, y1, y2, y3;
            rope_rot(a0, a1, rcs[gi][0], rcs[gi][1], y0, y1);
            rope_rot(a2, a3, rcs[gi][2], rcs[gi][3], y2, y3);
            if (part == 0) {
              o.x = pack_bf2(y0 * p.q_scale, y1 * p.q_scale);
              o.y = pack_bf2(y2 * p.q_scale, y3 * p.q_scale);
              *reinterpret_cast<uint2*>(p.q_out + static_cast<int64_t>(m) * d + e) = o;
            } else if (in_cache) {
              o.x = pack_bf2(y0, y1);
              o.y = pack_bf2(y2, y3);
              st_u2<true>(p.kc + crow, o);
            }
          }
        } else if constexpr (EPI == E_RESIDUAL) {
          // x + delta, then + bias: the order of the add+RMSNorm kernel it replaces
          float4 xv = xpre[gi];
          xv.x += v[0]; xv.y += v[1]; xv.z += v[2]; xv.w += v[3];
          if (p.bias_a) {
            const float4 b = bpre[gi];
            xv.x += b.x; xv.y += b.y; xv.z += b.z; xv.w += b.w;
          }
          *reinterpret_cast<float4*>(p.x_res + tile_off32(m, n, N)) = xv;
        } else {
          *reinterpret_cast<float4*>(p.out + static_cast<int64_t>(m) * p.ldo + n) =
              make_float4(v[0], v[1], v[2], v[3]);
        }
      }
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
// fastest shape or one within 3% of it.  `a_bytes` is what one activation element costs a
// block: 4 for a split operand (hi + lo), 8 for A_NORM, whose fp32 x also goes through the
// norm and split arithmetic in every block sharing its rows (with 8 it picks the measured
// fastest shape at the 6 norm-fused decode shapes).
int pick_tile(int M, int N, int K, double a_bytes = 4.0, double w_bytes = 2.0) {
  int best = 0;
  double best_key = 1e300, best_total = 1e300;
  for (int t = 0; t < kNumTiles; ++t) {
    const double blocks = static_cast<double>((N + kTiles[t].tn - 1) / kTiles[t].tn) *
                          ((M + kTiles[t].tm - 1) / kTiles[t].tm);
    const double per_block = (w_bytes * kTiles[t].tn + a_bytes * kTiles[t].tm) * K;
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

template <int TN, int TM, bool WT, int AMODE, int EPI, bool WL>
int launch_tile(GemmArgs p, hipStream_t st) {
  p.n_tiles = (p.N + TN - 1) / TN;
  p.m_tiles = (p.M + TM - 1) / TM;
  const int64_t tiles = static_cast<int64_t>(p.n_tiles) * p.m_tiles;
  const int64_t per_xcd = (tiles + 7) / 8;
  if (8 * per_xcd > 0x7fffffff) return MDL_ERR_SHAPE;
  p.per_xcd = static_cast<int>(per_xcd);
  hipLaunchKernelGGL((split_gemm_kernel<TN, TM, WT, AMODE, EPI, WL>),
                     dim3(static_cast<unsigned>(8 * per_xcd)), dim3(64 * kGemmWaves), 0, st, p);
  return launch_status();
}

template <bool WT, int AMODE, int EPI, bool WL = false>
int launch(int tile, const GemmArgs& p, hipStream_t st) {
  switch (tile ? tile : pick_tile(p.M, p.N, p.K, AMODE == A_NORM ? 8.0 : 4.0, WL ? 4.0 : 2.0)) {
    case 1: return launch_tile<64, 64, WT, AMODE, EPI, WL>(p, st);
    case 2: return launch_tile<128, 32, WT, AMODE, EPI, WL>(p, st);
    case 3: return launch_tile<64, 32, WT, AMODE, EPI, WL>(p, st);
    case 4: return launch_tile<32, 32, WT, AMODE, EPI, WL>(p, st);
    case 5: return launch_tile<64, 16, WT, AMODE, EPI, WL>(p, st);
    case 6: return launch_tile<32, 16, WT, AMODE, EPI, WL>(p, st);
    default: return MDL_ERR_SHAPE;
  }
}

// the plain form, or the WL form when the caller passes the low weight part
template <int AMODE, int EPI>
int launch_w(int tile, const GemmArgs& p, hipStream_t st) {
  return p.wl ? launch<true, AMODE, EPI, true>(tile, p, st)
              : launch<true, AMODE, EPI, false>(tile, p, st);
}

// dst = src in the bf16 tile layout, rows padded to a multiple of 16 with zeros.  One thread per
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

// common host checks of the tiled decode entries: k a positive multiple of 32, n of 16
inline bool decode_shape_ok(int m, int n, int k, int tile) {
  return m >= 0 && n >= 0 && k > 0 && k % 32 == 0 && n % 16 == 0 && tile >= 0 &&
         tile <= kNumTiles;
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
  GemmArgs p{};
  p.a = a;
  p.lda = lda;
  p.w = w;
  p.ldw = ldw;
  p.out = out;
  p.ldo = ldo;
  p.M = m;
  p.N = n;
  p.K = k;
  auto st = static_cast<hipStream_t>(stream);
  if (wt && at) return launch<true, A_TILES, E_STORE>(tile, p, st);
  if (wt) return launch<true, A_ROWS, E_STORE>(tile, p, st);
  if (at) return launch<false, A_TILES, E_STORE>(tile, p, st);
  return launch<false, A_ROWS, E_STORE>(tile, p, st);
}

extern "C" int mdl_gemm_split_swiglu(const uint16_t* a, const uint16_t* w_gu, const float* rstd,
                                     const float* bias_gate, const float* bias_up,
                                     uint16_t* h_out, int m, int d_ff, int k, int tile,
                                     void* stream) {
  if (!a || !w_gu || !h_out) return MDL_ERR_NULL;
  if (d_ff <= 0 || d_ff % 16 != 0 || d_ff > (1 << 29) || !decode_shape_ok(m, 2 * d_ff, k, tile))
    return MDL_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(w_gu) || !aligned8(h_out) ||
      (bias_gate && !aligned16(bias_gate)) || (bias_up && !aligned16(bias_up)))
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  GemmArgs p{};
  p.a = a;
  p.w = w_gu;
  p.rstd_in = rstd;
  p.bias_a = bias_gate;
  p.bias_b = bias_up;
  p.h = h_out;
  p.d_ff = d_ff;
  p.M = m;
  p.N = 2 * d_ff;
  p.K = k;
  return launch<true, A_TILES, E_SWIGLU>(tile, p, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_gemm_norm(const float* x, const float* gamma, float eps, const uint16_t* w,
                             const uint16_t* w_lo, float* out, int64_t ldo, float* rstd_out,
                             int m, int n, int k, int tile, void* stream) {
  if (!x || !gamma || !w || !out) return MDL_ERR_NULL;
  if (!decode_shape_ok(m, n, k, tile) || ldo < n) return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(w) || !aligned16(out) || ldo % 4 != 0 ||
      (w_lo && !aligned16(w_lo)))
    return MDL_ERR_ALIGN;
  if (m == 0 || n == 0) return MDL_OK;
  GemmArgs p{};
  p.x = x;
  p.gamma = gamma;
  p.eps = eps;
  p.w = w;
  p.wl = w_lo;
  p.out = out;
  p.ldo = ldo;
  p.rstd_out = rstd_out;
  p.M = m;
  p.N = n;
  p.K = k;
  return launch_w<A_NORM, E_STORE>(tile, p, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_gemm_norm_qkv(const float* x, const float* gamma, float eps,
                                 const uint16_t* w, int m, int n_heads, float* rstd_out,
                                 const int64_t* pos, const float* rope_tab, int max_x, int max_y,
                                 int max_z, int px, int py, int pz, float q_scale,
                                 uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                 int cache_slots, int slot0, const int32_t* slot_dev, int tile,
                                 void* stream) {
  if (!x || !gamma || !w || !pos || !rope_tab || !q_out || !k_cache || !v_cache)
    return MDL_ERR_NULL;
  if (n_heads <= 0 || n_heads > (1 << 16)) return MDL_ERR_SHAPE;
  const int d = n_heads * kHeadDim;
  if (!decode_shape_ok(m, 3 * d, d, tile) || max_x <= 0 || max_y <= 0 || max_z <= 0 ||
      px < 0 || py < 0 || pz < 0 || px + py + pz != kHeadDim / 2)
    return MDL_ERR_SHAPE;
  if (cache_slots <= 0 || (!slot_dev && (slot0 < 0 || slot0 >= cache_slots))) return MDL_ERR_CACHE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(w) || !aligned8(q_out) ||
      !aligned8(k_cache) || !aligned8(v_cache) || !aligned4(rope_tab))
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  GemmArgs p{};
  p.x = x;
  p.gamma = gamma;
  p.eps = eps;
  p.w = w;
  p.rstd_out = rstd_out;
  p.pos = pos;
  p.rope_tab = rope_tab;
  p.ra = RopeArgs{max_x, max_y, max_z, px, py, pz};
  p.q_scale = q_scale;
  p.q_out = q_out;
  p.kc = k_cache;
  p.vc = v_cache;
  p.slot_dev = slot_dev;
  p.slot0 = slot0;
  p.slots = cache_slots;
  p.M = m;
  p.N = 3 * d;
  p.K = d;
  return launch<true, A_NORM, E_QKV>(tile, p, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_gemm_norm_swiglu(const float* x, const float* gamma, float eps,
                                    const uint16_t* w_gu, const uint16_t* w_gu_lo,
                                    const float* bias_gate, const float* bias_up, uint16_t* h_out,
                                    int m, int d_ff, int k, int tile, void* stream) {
  if (!x || !gamma || !w_gu || !h_out) return MDL_ERR_NULL;
  if (d_ff <= 0 || d_ff % 16 != 0 || d_ff > (1 << 29) || !decode_shape_ok(m, 2 * d_ff, k, tile))
    return MDL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(gamma) || !aligned16(w_gu) || !aligned8(h_out) ||
      (bias_gate && !aligned16(bias_gate)) || (bias_up && !aligned16(bias_up)) ||
      (w_gu_lo && !aligned16(w_gu_lo)))
    return MDL_ERR_ALIGN;
  if (m == 0) return MDL_OK;
  GemmArgs p{};
  p.x = x;
  p.gamma = gamma;
  p.eps = eps;
  p.w = w_gu;
  p.wl = w_gu_lo;
  p.bias_a = bias_gate;
  p.bias_b = bias_up;
  p.h = h_out;
  p.d_ff = d_ff;
  p.M = m;
  p.N = 2 * d_ff;
  p.K = k;
  return launch_w<A_NORM, E_SWIGLU>(tile, p, static_cast<hipStream_t>(stream));
}

extern "C" int mdl_gemm_split_residual(const uint16_t* a, const uint16_t* w,
                                       const uint16_t* w_lo, float* x, const float* bias, int m,
                                       int n, int k, int tile, void* stream) {
  if (!a || !w || !x) return MDL_ERR_NULL;
  if (!decode_shape_ok(m, n, k, tile) || n % 32 != 0) return MDL_ERR_SHAPE;
  if (!aligned16(a) || !aligned16(w) || !aligned16(x) || (bias && !aligned16(bias)) ||
      (w_lo && !aligned16(w_lo)))
    return MDL_ERR_ALIGN;
  if (m == 0 || n == 0) return MDL_OK;
  GemmArgs p{};
  p.a = a;
  p.w = w;
  p.wl = w_lo;
  p.x_res = x;
  p.bias_a = bias;
  p.M = m;
  p.N = n;
  p.K = k;
  return launch_w<A_TILES, E_RESIDUAL>(tile, p, static_cast<hipStream_t>(stream));
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
