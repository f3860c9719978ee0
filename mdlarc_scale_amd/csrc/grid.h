// Grid-position rule of the decode loop, shared by mdl_grid_step and mdl_decode_embed.
//
// State per row: column x, row y (int32, clamped to [0, max_x] / [0, max_y]) and whether the
// decoder is inside an output grid.  For the token just emitted, position() is where the model
// places it and advance() moves the state past it:
//   START   -> (0, 0, 0),  state x = y = 0, leaves the output
//   IO_SEP  -> (0, 0, 2),  state x = y = 0, enters the output
//   END     -> (0, 0, 4),  state unchanged
//   NEWLINE -> (0, y, 1|3), state x = 0, y = min(y + 1, max_y)
//   colour  -> (x, y, 1|3), state x = min(x + 1, max_x)
// (z = 3 inside an output grid, 1 otherwise) -- GridStateUpdater.update, src/inference.py:127-168.
#pragma once

#include <stdint.h>

namespace mdl {

constexpr int64_t kStart = 10, kNewline = 11, kSep = 12, kEnd = 13;

__device__ __forceinline__ int64_t clampi(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Writes the 3D position of token t into p[0..2] and advances (x, y, out).
__device__ __forceinline__ void grid_position_step(int64_t t, int max_x, int max_y, int32_t& gx,
                                                   int32_t& gy, uint8_t& io, int64_t* p) {
  const bool st = t == kStart, sp = t == kSep, en = t == kEnd, nl = t == kNewline;
  int64_t x = gx, y = gy;
  bool out = io != 0;
  int64_t z = out ? 3 : 1;
  if (st) z = 0;
  if (sp) z = 2;
  if (en) z = 4;
  p[0] = (st || sp || en || nl) ? 0 : clampi(x, 0, max_x);
  p[1] = (st || sp || en) ? 0 : clampi(y, 0, max_y);
  p[2] = z;
  if (st || sp) x = y = 0;
  if (st) out = false;
  if (sp) out = true;
  if (nl) {
    x = 0;
    y = y + 1 < max_y ? y + 1 : max_y;
  }
  if (t < 10) x = x + 1 < max_x ? x + 1 : max_x;
  gx = static_cast<int32_t>(clampi(x, 0, max_x));
  gy = static_cast<int32_t>(clampi(y, 0, max_y));
  io = out ? 1 : 0;
}

}  // namespace mdl
