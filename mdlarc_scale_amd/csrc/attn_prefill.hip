// K4a -- prefill / full-sequence attention on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
// Block = 4 wavefronts = 128 queries of one (b, h); wave w owns queries q0+32w .. q0+32w+31 as
// two groups of 16 (j = 0, 1).  Working with S^T = K Q^T instead of S makes the MFMA accumulator
// of the scores (lane = one query, 4 keys per 16-key block) exactly the B-operand layout P^T
// needs in O^T = V^T P^T, so the probabilities never leave registers:
//   score block nb (keys 16nb..16nb+15), lane (c = lane%16, g = lane/16) holds keys 16nb+4g+i,
//   i = 0..3, of query c.  The P^T operand of k-step kk takes blocks 2kk and 2kk+1: element e of
//   lane group g is key 32kk + (e<4 ? 4g+e : 16+4g+e-4).
// The matching V^T operand comes straight from the row-major V tile through two transposing LDS
// reads (ds_read_b64_tr_b16): within each 16-lane group, lane i receives element i&3 of the 8-byte
// rows addressed by lanes 4k + (i>>2), k = 0..3.  Lane c of group g addresses key row
// 32kk + 4g + c/4 (and +16), dims 16db + 4(c%4) .. +3, which yields exactly V^T[dim 16db + c] over
// the key order above.  An MFMA pairs element e of lane group g in A with element e of group g in
// B whatever k that is inside the instruction, so any common key order of the operands is exact.
// Each A operand read from LDS (K rows, V^T rows) feeds both query groups' MFMAs.
//
// Staging: key tiles of 64 go through a ring of two LDS stages (K and V, 8 KB each, 128-byte
// rows) filled by direct global -> LDS copies (global_load_lds_dwordx4: each wave instruction
// writes one contiguous kilobyte, 8 key rows).  The copy of tile t+1 is issued right after the
// barrier that publishes tile t, so it runs under tile t's MFMA and softmax work; one barrier per
// tile.  Rows cannot be padded within a kilobyte, so the 16-byte chunks of a row are XOR-swizzled
// instead (chunk c of row r at chunk c ^ swz(r)): the column reads of the K operand (16 rows, one
// chunk) and the transposing V reads then hit distinct banks.  Key tiles start at the row's first
// valid key (kv_start) and packed query tiles at its first query, so no tile straddles the row
// start; keys past S in a row's last tile load the nearest valid key (finite data; their
// probabilities are 0, so they add exact zeros).
//
// Masking: each wave folds key validity (inside [kv_start, S) and the key mask) of a tile into a
// 64-bit ballot: from a mask byte it loaded one tile ahead, or, for a row without a key mask (or
// whose mask row_holes marks as the run [kv_start, S)), from the range alone, all ones for tiles
// inside it.  Tiles that are fully valid and entirely in the past of the wave's queries skip all
// per-element work; the others AND the ballot with the causal prefix of each query.
//
// Online softmax in the log2 domain, fp32 (v_exp_f32 directly: results below 2^-126 flush to 0,
// which no softmax weight of a visible key can reach relative to the running maximum).  q comes
// multiplied by log2(e) with the softmax scale, and each QK^T accumulator starts at -m, so the
// MFMA yields the exponent s - m itself.  A query's reference maximum m moves only when a score
// exceeds it by more than a factor 2^8 (its first visible key always sets it), so
// p = 2^(s - m) <= 256 and the o / row-sum rescale runs only in the tiles where some query's
// maximum jumps.  That decision is per query (the other queries are left untouched), so results
// do not depend on which queries share a wave; wave-wide ballots only skip the code (the
// cross-lane maximum, the rescale) when no lane needs it.  The row sums come from one more MFMA
// per k-step against a ones operand, so they sum the same bf16-rounded probabilities the PV
// product uses.  Queries with no visible key produce 0.  The output (the out-projection GEMM
// input) is written as a hi|lo bf16 pair per row, see common.h.
//
// Block order: block i runs on XCD i % 8; each (b, h) is pinned to one XCD, whose L2 then serves
// all of that head's query tiles, and heads are dealt round-robin over the XCDs so that rows of
// different lengths spread evenly.  Within a head the latest (most expensive) query tile runs
// first.
#include <type_traits>

#include "lds_dma.h"
#include "mfma.h"
#include "rope.h"

namespace mdl {

constexpr int kQW = 32;          // queries per wave
constexpr int kBM = 4 * kQW;     // queries per block
constexpr int kBN = 64;          // keys per tile
constexpr int kXcds = 8;
constexpr int kTileBytes = kBN * kHeadDim * 2;   // one K or V tile: 64 rows of 128 bytes
constexpr float kRescaleGap = 8.f;               // log2 of the largest p between rescales

// Chunk swizzle of the K / V tiles, a function of the row's low 4 bits (bit 0 = r0^r3,
// bit 1 = r0^r2, bit 2 = r1).  Chosen by exhaustive search over the linear swizzles so that both
// operand reads are free of bank conflicts whether the LDS serves 16-byte reads 8 lanes and
// 8-byte reads 16 lanes a cycle (32 banks) or 16 and 32 lanes (64 banks).
__device__ __forceinline__ int tile_swz(int r) {
  return ((r ^ (r >> 3)) & 1) | (((r ^ (r >> 2)) & 1) << 1) | (((r >> 1) & 1) << 2);
}

__global__ __launch_bounds__(256, 3) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, int S, int H, int slots, const uint8_t* __restrict__ kmask,
    const uint8_t* __restrict__ row_holes, const int32_t* __restrict__ kv_start,
    const int32_t* __restrict__ q_offset, int causal, uint16_t* __restrict__ out, int out_tiled,
    int nqt, int n_bh) {
  const int slot = blockIdx.x / kXcds;
  const int kq = slot / nqt;
  const int bh = blockIdx.x % kXcds + kXcds * kq;
  if (bh >= n_bh) return;                       // heads padded to a multiple of 8: extras exit
  const int qt = nqt - 1 - (slot - kq * nqt);
  const int b = bh / H, h = bh - b * H;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63, c16 = lane & 15, g = lane >> 4;
  const int kstart = kv_start ? min(max(kv_start[b], 0), S) : 0;
  // packed rows: query qi >= kstart of row b is row q_offset[b] + qi - kstart of q and out;
  // queries before kstart are not part of the packed list and are neither read nor written
  const int qlo = q_offset ? kstart : 0;
  // query tiles start at the row's first query (packed rows; 0 otherwise), key tiles at its
  // first valid key: no tile straddles the row start
  const int q0 = qlo + qt * kBM;
  if (q0 >= S) return;                          // the whole query tile is past the row end
  const int64_t qbase = q_offset ? static_cast<int64_t>(q_offset[b]) - kstart
                                 : static_cast<int64_t>(b) * S;

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kBN * kHeadDim];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][kBN * kHeadDim];

  const int wq0 = q0 + kQW * wave;
  int qi[2];
  bf16x8_t qf[2][2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    qi[j] = wq0 + 16 * j + c16;
    if (qi[j] < S && qi[j] >= qlo) {
      const uint16_t* qp = q + ((qbase + qi[j]) * H + h) * kHeadDim;
      qf[j][0] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 8 * g));
      qf[j][1] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 32 + 8 * g));
    } else {
      qf[j][0] = as_bf16x8(make_uint4(0, 0, 0, 0));
      qf[j][1] = qf[j][0];
    }
  }

  const int64_t head_off = (static_cast<int64_t>(b) * H + h) * slots * kHeadDim;
  const uint16_t* Kg = kc + head_off;
  const uint16_t* Vg = vc + head_off;
  const int kt0 = kstart;
  // a row with no valid key attends to nothing: its tiles are skipped (o and the sum stay 0)
  const int kend = kstart >= S ? kt0 : (causal ? min(S, q0 + kBM) : S);
  // row_holes[b] == 0: the key mask of row b is exactly [kstart, S), which kstart already says
  const bool dense = row_holes && row_holes[b] == 0;
  const uint8_t* mrow = kmask && !dense ? kmask + static_cast<int64_t>(b) * S : nullptr;
  const bf16x8_t ones = bf16_ones8();

  // Tile kt -> stage st: wave w copies key rows 8 (4 r + w) .. + 7 (r = 0, 1), one kilobyte of K
  // and one of V per r; lane l takes physical chunk l % 8 of row l / 8, i.e. logical chunk
  // (l % 8) ^ swz(row).  A tile inside [kstart, S) is copied from the scalar tile address plus a
  // fixed lane offset; in the first and last tiles of a row, rows outside [kstart, S) copy the
  // nearest valid key instead.
  const uint32_t ks0 = lds_addr(&Ks[0][0]), vs0 = lds_addr(&Vs[0][0]);
  uint32_t loff[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int row = 8 * (4 * r + wave) + (lane >> 3);
    loff[r] = row * 128 + 16 * ((lane & 7) ^ tile_swz(row));
  }
  auto issue = [&](int kt, int st) {
    if (kt >= kstart && kt + kBN <= S) {
      const uint16_t* kb = Kg + static_cast<int64_t>(kt) * kHeadDim;
      const uint16_t* vb = Vg + static_cast<int64_t>(kt) * kHeadDim;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint32_t run = st * kTileBytes + (4 * r + wave) * 1024;
        dma16_sbase(kb, loff[r], __builtin_amdgcn_readfirstlane(ks0 + run));
        dma16_sbase(vb, loff[r], __builtin_amdgcn_readfirstlane(vs0 + run));
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int row = 8 * (4 * r + wave) + (lane >> 3);
      const int kj = min(max(kt + row, kstart), S - 1);
      const int64_t off =
          static_cast<int64_t>(kj) * kHeadDim + 8 * ((lane & 7) ^ tile_swz(row));
      const uint32_t run = st * kTileBytes + (4 * r + wave) * 1024;
      dma16(Kg + off, __builtin_amdgcn_readfirstlane(ks0 + run));
      dma16(Vg + off, __builtin_amdgcn_readfirstlane(vs0 + run));
    }
  };
  // this lane's key of tile kt is valid: inside [kstart, S) and not masked
  auto mask_byte = [&](int kt) -> int {
    const int kj = kt + lane;
    if (kj >= S || kj < kstart) return 0;
    return mrow ? mrow[kj] : 1;
  };

  // Lane parts of the swizzled LDS read addresses (bytes).  The swizzle of a row depends on its
  // low 4 bits only, so it is the same for rows 16 apart.  K operand (score block nb, k-step
  // kk): row 16 nb + c16, logical chunk 4 kk + g, physical chunk (g ^ swz(c16)) ^ 4 kk.  V^T
  // operand (k-step kk, dim block db, rows r0 and r0 + 16, r0 = 32 kk + rl, rl = 4 g + c16 / 4,
  // dims 16 db + 4 (c16 % 4) ..): physical chunk (c16 / 2 % 2 ^ swz(rl)) ^ 2 db.  The row and
  // stage parts are immediate offsets.
  uint32_t kofs[2], vofs[4];
  {
    const int L = g ^ tile_swz(c16);
    const int rl = 4 * g + (c16 >> 2);
    const int Mv = ((c16 >> 1) & 1) ^ tile_swz(rl);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) kofs[kk] = c16 * 128 + 16 * (L ^ (4 * kk));
#pragma unroll
    for (int db = 0; db < 4; ++db) vofs[db] = rl * 128 + 16 * (Mv ^ (2 * db)) + 8 * (c16 & 1);
  }
  const char* Kb = reinterpret_cast<const char*>(&Ks[0][0]);
  const char* Vb = reinterpret_cast<const char*>(&Vs[0][0]);

  // Per query: negm = -m, the negated reference maximum (0 before the first visible key), and
  // thr, the tile maximum (relative to m) that moves the reference: -inf before the first
  // visible key, then the gap.  Both change only when the reference moves.
  float negm[2] = {0.f, 0.f}, thr[2] = {-INFINITY, -INFINITY};
  f32x4_t lsum[2], o[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    lsum[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int db = 0; db < 4; ++db) o[j][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](const char* Kt, const char* Vt, int kt, uint64_t mw) {
    // S^T = K Q^T: 4 blocks of 16 keys for both query groups.  Every accumulator starts at -m,
    // its query's reference maximum (0 before the query's first visible key); q carries log2(e),
    // so the MFMA yields the exponents s - m of the log2-domain softmax directly.
    f32x4_t sc[2][4];
    f32x4_t minit[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      minit[j] = f32x4_t{negm[j], negm[j], negm[j], negm[j]};
    }
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16x8_t a =
            as_bf16x8(*reinterpret_cast<const uint4*>(Kt + kofs[kk] + 2048 * nb));
#pragma unroll
        for (int j = 0; j < 2; ++j)
          sc[j][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[j][kk],
                                                              kk == 0 ? minit[j] : sc[j][nb],
                                                              0, 0, 0);
      }
    }

    const bool full = (mw == ~0ull) && (!causal || kt + kBN - 1 <= wq0);
    if (!full) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        uint64_t vis = mw;
        if (causal) {
          const int x = qi[j] - kt;    // offset of the last key query qi[j] may see
          vis &= x >= 63 ? ~0ull : (x < 0 ? 0ull : (2ull << x) - 1ull);
        }
        vis >>= 4 * g;
        const uint32_t lo = static_cast<uint32_t>(vis), hi = static_cast<uint32_t>(vis >> 32);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t word = nb < 2 ? lo : hi;
            if (!((word >> (16 * (nb & 1) + i)) & 1u)) sc[j][nb][i] = -INFINITY;
          }
      }
    }

    bf16x8_t pb[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float lmax = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) lmax = fmaxf(lmax, sc[j][nb][i]);
      // Move a query's reference when its maximum over the tile passes it by more than the gap
      // (or on its first visible key, while m = -inf and the scores are absolute; alpha = 0);
      // other queries are left untouched.  That maximum can pass only if one of its four lanes'
      // maxima does (same test), so the cross-lane maximum is formed only in those tiles.
      if (__ballot(lmax > thr[j]) != 0) {
        const float tmax = max_over_groups(lmax);
        if (tmax > thr[j]) {
          const bool fresh = thr[j] == -INFINITY;
          const float alpha = fresh ? 0.f : __builtin_amdgcn_exp2f(-tmax);
          // -(m + tmax), as (-m) - tmax: the same value bit for bit
          negm[j] = fresh ? -tmax : negm[j] - tmax;
          thr[j] = kRescaleGap;
#pragma unroll
          for (int nb = 0; nb < 4; ++nb) sc[j][nb] -= tmax;
          lsum[j] *= alpha;
#pragma unroll
          for (int db = 0; db < 4; ++db) o[j][db] *= alpha;
        }
      }
      // p = 2^(s - m): 0 for masked keys (and for a query with no visible key yet)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[j][nb][i] = __builtin_amdgcn_exp2f(sc[j][nb][i]);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) pb[j][kk] = pt_operand(sc[j][2 * kk], sc[j][2 * kk + 1]);
    }

    // O^T += V^T P^T and the row sums, two k-steps of 32 keys.  A k-step's 8 transposing reads
    // are issued together (the scheduling barrier keeps them ahead of the MFMAs): one LDS round
    // trip per k-step instead of one per dim block, in the same 122 registers (1-2% faster at
    // configs 2-4; both k-steps' 16 reads at once need 134, occupancy 3, and ran 3-7% slower)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8_t va[4];
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const s16x4_t lo4 = lds_read_tr16(
            reinterpret_cast<const uint16_t*>(Vt + vofs[db] + 4096 * kk));
        const s16x4_t hi4 = lds_read_tr16(
            reinterpret_cast<const uint16_t*>(Vt + vofs[db] + 4096 * kk + 2048));
        va[db] = __builtin_bit_cast(
            bf16x8_t, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        o[0][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db], pb[0][kk], o[0][db], 0, 0, 0);
        o[1][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[db], pb[1][kk], o[1][db], 0, 0, 0);
      }
      lsum[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[0][kk], lsum[0], 0, 0, 0);
      lsum[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[1][kk], lsum[1], 0, 0, 0);
    }
  };

  // with a key mask, this lane's key validity for the next tile's ballot (loaded a tile ahead)
  int mb_next = 0;
  if (kt0 < kend) {
    if (mrow) mb_next = mask_byte(kt0);
    issue(kt0, 0);
  }
  // One tile in stage ST (a compile-time constant, so the stage offset folds into the LDS reads).
  // Every wave of the block runs the same tiles, so the barriers match.
  auto tile = [&](int kt, auto stc) {
    constexpr int ST = decltype(stc)::value;
    // tile kt has landed in stage ST for every wave, and every wave is done with stage ST ^ 1.
    // The wait is the builtin, not assembly, so that the compiler sees every load it knows of
    // (q, the mask bytes) completed here: otherwise it waits for the q fragments again at their
    // first use inside the loop, and that vmcnt wait also covers the copies of tile kt + 64
    // issued just before, which then no longer run under this tile's work (5% at config 2).
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    asm volatile("s_barrier" ::: "memory");
    uint64_t mw;
    if (mrow)
      mw = __ballot(mb_next != 0);
    else if (kt >= kstart && kt + kBN <= S)
      mw = ~0ull;
    else
      mw = __ballot(kt + lane >= kstart && kt + lane < S);
    if (kt + kBN < kend) {
      if (mrow) mb_next = mask_byte(kt + kBN);
      issue(kt + kBN, ST ^ 1);
    }
    if (causal && kt > wq0 + kQW - 1) return;   // the whole tile is in this wave's future
    compute(Kb + ST * kTileBytes, Vb + ST * kTileBytes, kt, mw);
  };
  for (int kt = kt0; kt < kend; kt += 2 * kBN) {
    tile(kt, std::integral_constant<int, 0>{});
    if (kt + kBN < kend) tile(kt + kBN, std::integral_constant<int, 1>{});
  }

  // output row (b, qi) holds 2*H*64 bf16: hi of every head, then lo of every head (row-major,
  // or in the bf16 MFMA tile layout, where each 4-column group stays contiguous)
  const int64_t d = static_cast<int64_t>(H) * kHeadDim;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (qi[j] >= S || qi[j] < qlo) continue;
    const float l = lsum[j][0];     // every row of the ones product holds the query's sum
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t orow = qbase + qi[j];
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int col = h * kHeadDim + 16 * db + 4 * g;
      uint16_t* oh = out_tiled ? out + tile_off(orow, col, static_cast<int>(2 * d))
                               : out + orow * 2 * d + col;
      uint16_t* ol = out_tiled ? out + tile_off(orow, static_cast<int>(d) + col,
                                                static_cast<int>(2 * d))
                               : oh + d;
      const float t[4] = {o[j][db][0] * inv, o[j][db][1] * inv, o[j][db][2] * inv,
                          o[j][db][3] * inv};
      // v_cvt_pk_bf16_f32 rounds to nearest even, as f2bf does for every non-NaN value
      const bf16x4_t hv = {(__bf16)t[0], (__bf16)t[1], (__bf16)t[2], (__bf16)t[3]};
      const bf16x4_t lv = {(__bf16)(t[0] - (float)hv[0]), (__bf16)(t[1] - (float)hv[1]),
                           (__bf16)(t[2] - (float)hv[2]), (__bf16)(t[3] - (float)hv[3])};
      *reinterpret_cast<bf16x4_t*>(oh) = hv;
      *reinterpret_cast<bf16x4_t*>(ol) = lv;
    }
  }
}

// K4c -- exact attention for the lead queries of each row.
//
// The first queries of a row attend to few keys: query kv_start + r sees at most r + 1 of them,
// so the bf16 roundings of q, K, V and of the probabilities in K4a are not averaged away (at the
// first query the output is one bf16-rounded V row).  This pass recomputes, for each (b, h), the
// outputs of the kLead queries from kv_start on in fp32 from the projection GEMM's fp32 output:
// the same RMSNorm scale, 3D RoPE and softmax scale K2 applies, then exact masked softmax and PV.
// Those queries see only keys among the same kLead tokens (causal), so one block holds them all
// in LDS.  Later queries average over more than kLead keys and keep K4a's output.
//
// Block = one (b, h), 256 threads: thread t owns query t/4 and dims 16 (t%4) .. +15.  It first
// rotates those dims of its own token's q (kept in registers) and k (to LDS) -- RoPE pairs
// 8 (t%4) .. +7 -- and scales its v dims (to LDS).  Then, with K and V rows read as float4, one
// pass over the visible keys keeps the online softmax in fp32: the running maximum, and the sum
// and P V rescaled by exp(m_old - m_new) whenever a score passes it (measured against a pass
// for the maximum and a second for the sums: 142 -> 103 us at config 2's shape, together with
// the four-way dot product and the positions loaded once).  Each dot product is four partial
// sums, added, then summed over the query's 4 threads with 2 xor shuffles.  A wave's loop stops
// at the wave's last query (keys after it are in every query's future).
constexpr int kLead = 64;
constexpr int kLeadLd = kHeadDim + 4;   // LDS row stride (floats): 16-byte aligned rows

__global__ __launch_bounds__(256) void attn_lead_kernel(
    const float* __restrict__ qkv, int64_t ld, const float* __restrict__ rstd,
    const int64_t* __restrict__ pos, const float* __restrict__ tab, RopeArgs ra, float q_scale,
    int S, int H, const uint8_t* __restrict__ kmask, const int32_t* __restrict__ kv_start,
    const int32_t* __restrict__ q_offset, uint16_t* __restrict__ out, int out_tiled) {
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int kstart = kv_start ? min(max(kv_start[b], 0), S) : 0;
  const int n = min(kLead, S - kstart);
  if (n <= 0) return;
  // token row of position kstart + r in qkv / rstd / pos and out (packed or [batch, seq])
  const int64_t row0 = (q_offset ? static_cast<int64_t>(q_offset[b]) - kstart
                                 : static_cast<int64_t>(b) * S) + kstart;
  const int64_t d = static_cast<int64_t>(H) * kHeadDim;
  __shared__ __attribute__((aligned(16))) float ks[kLead * kLeadLd];
  __shared__ __attribute__((aligned(16))) float vs[kLead * kLeadLd];
  __shared__ uint8_t ok[kLead];
  const int t = threadIdx.x;
  const int r = t >> 2, part = t & 3;
  float q[16];
  if (r < n) {
    const int64_t row = row0 + r;
    const float rs = rstd[row];
    const float* src = qkv + row * ld + h * kHeadDim + 16 * part;
    float qa[16], ka[16], va[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      *reinterpret_cast<float4*>(qa + 4 * c) = *reinterpret_cast<const float4*>(src + 4 * c);
      *reinterpret_cast<float4*>(ka + 4 * c) = *reinterpret_cast<const float4*>(src + d + 4 * c);
      *reinterpret_cast<float4*>(va + 4 * c) =
          *reinterpret_cast<const float4*>(src + 2 * d + 4 * c);
    }
    float kr[16];
    // the token's three positions once, then the sixteen table entries as independent loads
    const int64_t* p3 = pos + row * 3;
    const int64_t P0 = p3[0], P1 = p3[1], P2 = p3[2];
    float csv[8], snv[8];
#pragma unroll
    for (int pp = 0; pp < 8; ++pp)
      rope_cos_sin3(part * 8 + pp, P0, P1, P2, tab, ra, csv[pp], snv[pp]);
#pragma unroll
    for (int pp = 0; pp < 8; ++pp) {
      const float cs = csv[pp], sn = snv[pp];
      const float q0 = qa[2 * pp] * rs, q1 = qa[2 * pp + 1] * rs;
      const float k0 = ka[2 * pp] * rs, k1 = ka[2 * pp + 1] * rs;
      q[2 * pp] = (q0 * cs - q1 * sn) * q_scale;
      q[2 * pp + 1] = (q1 * cs + q0 * sn) * q_scale;
      kr[2 * pp] = k0 * cs - k1 * sn;
      kr[2 * pp + 1] = k1 * cs + k0 * sn;
      va[2 * pp] *= rs;
      va[2 * pp + 1] *= rs;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      *reinterpret_cast<float4*>(ks + r * kLeadLd + 16 * part + 4 * c) =
          *reinterpret_cast<const float4*>(kr + 4 * c);
      *reinterpret_cast<float4*>(vs + r * kLeadLd + 16 * part + 4 * c) =
          *reinterpret_cast<const float4*>(va + 4 * c);
    }
    if (part == 0) ok[r] = !kmask || kmask[static_cast<int64_t>(b) * S + kstart + r] != 0;
  }
  __syncthreads();
  if (r >= n) return;   // no barrier follows; the rest of the 4-thread group returns with it
  // queries of this wave: 16 (t / 64) .. +15; no key after the wave's last query is visible
  const int jend = min(16 * (t >> 6) + 15, n - 1);

  auto dot = [&](int j) {
    const float4* kr = reinterpret_cast<const float4*>(ks + j * kLeadLd + 16 * part);
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 k4 = kr[c];
      a[c] = fmaf(q[4 * c], k4.x, a[c]);
      a[c] = fmaf(q[4 * c + 1], k4.y, a[c]);
      a[c] = fmaf(q[4 * c + 2], k4.z, a[c]);
      a[c] = fmaf(q[4 * c + 3], k4.w, a[c]);
    }
    float s = (a[0] + a[1]) + (a[2] + a[3]);
    s += __shfl_xor(s, 1, kWave);
    return s + __shfl_xor(s, 2, kWave);
  };
  // one pass, online: the running maximum m, the sum l and the output o are rescaled by
  // exp(m_old - m_new) when a visible score passes m
  float mx = -INFINITY, l = 0.f, o[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) o[e] = 0.f;
  for (int j = 0; j <= jend; ++j) {
    const float s = dot(j);
    if (j <= r && ok[j]) {
      if (s > mx) {
        const float alpha = expf(mx - s);   // 0 at the first visible key
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] *= alpha;
        mx = s;
      }
      const float pj = expf(s - mx);
      l += pj;
      const float4* vr = reinterpret_cast<const float4*>(vs + j * kLeadLd + 16 * part);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 v4 = vr[c];
        o[4 * c] = fmaf(pj, v4.x, o[4 * c]);
        o[4 * c + 1] = fmaf(pj, v4.y, o[4 * c + 1]);
        o[4 * c + 2] = fmaf(pj, v4.z, o[4 * c + 2]);
        o[4 * c + 3] = fmaf(pj, v4.w, o[4 * c + 3]);
      }
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;   // no visible key: 0, as in K4a
  const int64_t orow = row0 + r;
  const int col0 = h * kHeadDim + 16 * part;
#pragma unroll
  for (int e = 0; e < 16; e += 2) {
    uint32_t hi, lo;
    split_bf2(o[e] * inv, o[e + 1] * inv, hi, lo);
    uint16_t* oh = out_tiled ? out + tile_off(orow, col0 + e, static_cast<int>(2 * d))
                             : out + orow * 2 * d + col0 + e;
    uint16_t* ol = out_tiled ? out + tile_off(orow, static_cast<int>(d) + col0 + e,
                                              static_cast<int>(2 * d))
                             : oh + d;
    *reinterpret_cast<uint32_t*>(oh) = hi;
    *reinterpret_cast<uint32_t*>(ol) = lo;
  }
}

}  // namespace mdl

using namespace mdl;

namespace mdl {

int launch_prefill(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                   int batch, int seq, int n_heads, int head_dim, int cache_slots,
                   const uint8_t* key_mask, const uint8_t* row_holes, const int32_t* kv_start,
                   const int32_t* q_offset, int causal, uint16_t* out, int out_layout,
                   hipStream_t st) {
  if (!q || !k_cache || !v_cache || !out) return MDL_ERR_NULL;
  if (out_layout != MDL_LAYOUT_ROWS && out_layout != MDL_LAYOUT_TILES) return MDL_ERR_SHAPE;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || seq < 0 || n_heads <= 0 || n_heads > 65535 || batch > 65535)
    return MDL_ERR_SHAPE;
  if (seq > cache_slots) return MDL_ERR_CACHE;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned8(out))
    return MDL_ERR_ALIGN;
  if (batch == 0 || seq == 0) return MDL_OK;
  const int64_t heads = static_cast<int64_t>(batch) * n_heads;
  const int64_t nqt = (seq + kBM - 1) / kBM;
  const int64_t blocks = (heads + kXcds - 1) / kXcds * kXcds * nqt;
  if (blocks > 0x7fffffff) return MDL_ERR_SHAPE;
  attn_prefill_kernel<<<static_cast<unsigned>(blocks), 256, 0, st>>>(
      q, k_cache, v_cache, seq, n_heads, cache_slots, key_mask, row_holes, kv_start, q_offset,
      causal ? 1 : 0, out, out_layout == MDL_LAYOUT_TILES ? 1 : 0, static_cast<int>(nqt),
      static_cast<int>(heads));
  return launch_status();
}

}  // namespace mdl

extern "C" int mdl_attn_prefill(const uint16_t* q, const uint16_t* k_cache,
                                const uint16_t* v_cache, int batch, int seq, int n_heads,
                                int head_dim, int cache_slots, const uint8_t* key_mask,
                                const uint8_t* row_holes, const int32_t* kv_start, int causal,
                                uint16_t* out, int out_layout, void* stream) {
  return launch_prefill(q, k_cache, v_cache, batch, seq, n_heads, head_dim, cache_slots,
                        key_mask, row_holes, kv_start, nullptr, causal, out, out_layout,
                        static_cast<hipStream_t>(stream));
}

extern "C" int mdl_attn_prefill_packed(const uint16_t* q, const uint16_t* k_cache,
                                       const uint16_t* v_cache, int batch, int seq, int n_heads,
                                       int head_dim, int cache_slots, const uint8_t* key_mask,
                                       const uint8_t* row_holes, const int32_t* kv_start,
                                       const int32_t* q_offset, int causal, uint16_t* out,
                                       int out_layout, void* stream) {
  if (!kv_start || !q_offset) return MDL_ERR_NULL;
  return launch_prefill(q, k_cache, v_cache, batch, seq, n_heads, head_dim, cache_slots,
                        key_mask, row_holes, kv_start, q_offset, causal, out, out_layout,
                        static_cast<hipStream_t>(stream));
}

extern "C" int mdl_attn_prefill_lead(const float* qkv, int64_t qkv_ld, const float* rstd,
                                     const int64_t* pos, const float* rope_tab, int max_x,
                                     int max_y, int max_z, int px, int py, int pz, float q_scale,
                                     int batch, int seq, int n_heads, int head_dim,
                                     const uint8_t* key_mask, const int32_t* kv_start,
                                     const int32_t* q_offset, uint16_t* out, int out_layout,
                                     void* stream) {
  if (!qkv || !rstd || !pos || !rope_tab || !out) return MDL_ERR_NULL;
  if (out_layout != MDL_LAYOUT_ROWS && out_layout != MDL_LAYOUT_TILES) return MDL_ERR_SHAPE;
  if (q_offset && !kv_start) return MDL_ERR_NULL;
  if (head_dim != kHeadDim) return MDL_ERR_HEAD_DIM;
  if (batch < 0 || seq < 0 || n_heads <= 0 || max_x <= 0 || max_y <= 0 || max_z <= 0 ||
      px < 0 || py < 0 || pz < 0 || px + py + pz != kHeadDim / 2 ||
      qkv_ld < 3 * static_cast<int64_t>(n_heads) * kHeadDim)
    return MDL_ERR_SHAPE;
  if (!aligned16(qkv) || qkv_ld % 4 != 0 || !aligned4(out) || !aligned4(rope_tab))
    return MDL_ERR_ALIGN;
  const int64_t blocks = static_cast<int64_t>(batch) * n_heads;
  if (blocks == 0 || seq == 0) return MDL_OK;
  if (blocks > 0x7fffffff) return MDL_ERR_SHAPE;
  const RopeArgs ra{max_x, max_y, max_z, px, py, pz};
  attn_lead_kernel<<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
      qkv, qkv_ld, rstd, pos, rope_tab, ra, q_scale, seq, n_heads, key_mask, kv_start, q_offset,
      out, out_layout == MDL_LAYOUT_TILES ? 1 : 0);
  return launch_status();
}
