// The sum of squares of a 7168-wide bf16 row in ONE order, shared by every path that
// forms it: the front's norm task (from the row in memory), and in a multi-layer launch
// the layer before's MoE final tasks (each from the 32 columns it writes) together with
// the next layer's stage A (from their tile sums). Each path adds the row's squares as
// the same balanced binary tree of correctly rounded f32 additions in column order,
// padded with zeros to 8192 columns (adding +0 is exact), so the RMSNorm factor of a
// row is bit-identical whichever path formed it. The reference sums a row's squares in
// its own reduction order (glm53/gfx950/kernel.py:1367-1398); its result is compared
// within tolerance, the paths here against each other bit for bit.
#pragma once

#include "common.h"

namespace mono {

constexpr int SSQ_COLS = 7168;
constexpr int SSQ_TILE = 32;                    // columns a tile: a MoE final task's
constexpr int SSQ_TILES = SSQ_COLS / SSQ_TILE;  // 224
constexpr int SSQ_PIECES = 1024;                // 16-byte pieces of the padded row

struct OpAddRn {
  MONO_DEV float operator()(float a, float b) const { return __fadd_rn(a, b); }
};

// tree levels 1-3: the squares of one 16-byte piece (8 consecutive columns)
MONO_DEV float piece_sum_of_squares(const u32x4& x) {
  float q[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    q[2 * e] = __fmul_rn(bf16_lo(x[e]), bf16_lo(x[e]));
    q[2 * e + 1] = __fmul_rn(bf16_hi(x[e]), bf16_hi(x[e]));
  }
  const OpAddRn add;
  return add(add(add(q[0], q[1]), add(q[2], q[3])), add(add(q[4], q[5]), add(q[6], q[7])));
}

// levels 4-5: four consecutive lanes holding a tile's four pieces in order (lane % 4 =
// piece % 4) -> the tile's sum, in each of the four lanes
MONO_DEV float tile_sum_of_pieces(float v) {
  v = __fadd_rn(v, dpp_f<DPP_XOR1>(v));
  return __fadd_rn(v, dpp_f<DPP_XOR2>(v));
}

// levels 1-5 with one column a lane: 32 consecutive lanes (a half wave, every lane
// active) each holding its column's value -> the tile's sum of squares in each of them
MONO_DEV float tile_sum_of_columns(float v) {
  const float t = row_reduce<16>(__fmul_rn(v, v), OpAddRn());
  return __fadd_rn(t, __shfl_xor(t, 16, WAVE));
}

// levels 6-13: the 256 tile sums (zeros past tile 223), lane l holding tiles 4 l ..
// 4 l + 3 -> the row's sum of squares (wave-uniform)
MONO_DEV float tiles_sum(float t0, float t1, float t2, float t3) {
  const OpAddRn add;
  return wave_reduce(add(add(t0, t1), add(t2, t3)), add);
}

}  // namespace mono
