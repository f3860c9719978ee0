// Augmented prompt construction on the device: every (dihedral transform, colour permutation)
// variant of one task, tokenised, given its 3D positions and left-padded into one batch.
//
// A prompt is, for each demonstration pair, START input-grid IO_SEP output-grid END, then START
// test-grid IO_SEP; a grid is its rows, each closed by NEWLINE.  Positions: START (0,0,0),
// IO_SEP (0,0,2), END (0,0,4); a cell at row r, column c of a grid (x, y, z) = (c, r, 1) in an
// input / test grid and (c, r, 3) in an output grid; the NEWLINE closing row r is (0, r, z).
// (compute_positions_3d reduces to this on prompts of this shape; x and y clamp at 30 / 29.)
//
// One thread per output token: it finds its grid segment from the task's grid shapes (at most
// 11 grids), maps its (row, column) in the transformed grid back to the source cell, and applies
// the variant's colour permutation.  Cell reads are clamped to [0, n_cells) (a cell outside
// reads as colour 0); writes stay inside the row's [0, S).
#include "common.h"
#include "grid.h"

namespace mdl {

constexpr int kMaxGrids = 64;

// transformed dims and the source cell of transformed (r, c), for the 8 dihedral transforms in
// the order identity, rot90 (clockwise), rot180, rot270, flip_h, flip_v, transpose, anti-transpose
__device__ __forceinline__ bool swaps_dims(int d) { return d == 1 || d == 3 || d == 6 || d == 7; }

__device__ __forceinline__ int source_index(int d, int r, int c, int h, int w) {
  int sr, sc;
  switch (d) {
    case 0: sr = r; sc = c; break;
    case 1: sr = h - 1 - c; sc = r; break;
    case 2: sr = h - 1 - r; sc = w - 1 - c; break;
    case 3: sr = c; sc = w - 1 - r; break;
    case 4: sr = r; sc = w - 1 - c; break;
    case 5: sr = h - 1 - r; sc = c; break;
    case 6: sr = c; sc = r; break;
    default: sr = h - 1 - c; sc = w - 1 - r; break;
  }
  return sr * w + sc;
}

__global__ __launch_bounds__(256) void build_prompts_kernel(
    const uint8_t* __restrict__ cells, int64_t n_cells, const int32_t* __restrict__ grids,
    int n_grids,
    const int32_t* __restrict__ variants, const int32_t* __restrict__ perms, int n_perms,
    const int32_t* __restrict__ lengths, int seq, int64_t* __restrict__ ids,
    int64_t* __restrict__ pos, uint8_t* __restrict__ mask) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= seq) return;
  const int64_t o = static_cast<int64_t>(b) * seq + i;
  const int len = lengths[b];
  const int pad = seq - len;
  int64_t tok = kEnd, x = 0, y = 0, z = 0;
  if (i >= pad) {
    const int d = variants[2 * b] & 7;
    const int pr = clampi(variants[2 * b + 1], 0, n_perms - 1);
    int j = i - pad;                       // index inside the prompt
    // walk the segments: per pair START in IO_SEP out END, then START test IO_SEP
    for (int gi = 0; gi < n_grids; ++gi) {
      const bool output = (gi & 1) && gi != n_grids - 1;   // odd grids are outputs
      const bool first_of_example = !(gi & 1);             // START precedes inputs and test
      if (first_of_example) {
        if (j == 0) { tok = kStart; break; }
        --j;
      }
      const int h = grids[3 * gi + 1], w = grids[3 * gi + 2];
      const int th = swaps_dims(d) ? w : h, tw = swaps_dims(d) ? h : w;
      const int seg = th * (tw + 1);
      if (j < seg) {
        const int r = j / (tw + 1), c = j - r * (tw + 1);
        z = output ? 3 : 1;
        y = r < 29 ? r : 29;
        if (c == tw) {
          tok = kNewline;
        } else {
          const int64_t src = static_cast<int64_t>(grids[3 * gi]) + source_index(d, r, c, h, w);
          const int cell = (src >= 0 && src < n_cells) ? cells[src] % 10 : 0;
          tok = perms[pr * 10 + cell];
          x = c < 30 ? c : 30;
        }
        break;
      }
      j -= seg;
      if (!output) {                       // IO_SEP after an input / the test grid
        if (j == 0) { tok = kSep; z = 2; break; }
        --j;
      } else {                             // END after an output grid
        if (j == 0) { tok = kEnd; z = 4; break; }
        --j;
      }
    }
  }
  ids[o] = tok;
  pos[3 * o] = x;
  pos[3 * o + 1] = y;
  pos[3 * o + 2] = z;
  mask[o] = i >= pad ? 1 : 0;
}

}  // namespace mdl

using namespace mdl;

extern "C" int mdl_build_prompts(const uint8_t* cells, int64_t n_cells, const int32_t* grids,
                                 int n_grids, const int32_t* variants, int batch,
                                 const int32_t* perms, int n_perms, const int32_t* lengths,
                                 int seq, int64_t* ids_out, int64_t* pos_out, uint8_t* mask_out,
                                 void* stream) {
  if (!cells || !grids || !variants || !perms || !lengths || !ids_out || !pos_out || !mask_out)
    return MDL_ERR_NULL;
  if (batch < 0 || seq <= 0 || n_grids <= 0 || n_grids > kMaxGrids || (n_grids & 1) == 0 ||
      n_perms <= 0 || n_cells < 0 || static_cast<int64_t>(batch) * seq > (int64_t{1} << 40))
    return MDL_ERR_SHAPE;
  if (batch == 0) return MDL_OK;
  const dim3 grid((seq + 255) / 256, batch);
  if (grid.y > 65535) return MDL_ERR_SHAPE;
  build_prompts_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
      cells, n_cells, grids, n_grids, variants, perms, n_perms, lengths, seq, ids_out, pos_out,
      mask_out);
  return launch_status();
}
