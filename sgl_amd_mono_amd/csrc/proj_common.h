// Device pieces of the projection launches: block-scaled FP8 (and bf16) weight tiles
// against bf16 rows staged in LDS on the bf16 matrix cores, row-wise norms, RoPE and
// the FP4 index vectors.
//
// A weight tile is 16 rows x 128 k of a matrix in AITER's (16, 16) layout: lane
// (g = l / 16, r = l % 16) holds row r, k = 32 g + [0, 32) (32 FP8 bytes, two 16-byte
// loads 256 B apart; a wave's loads cover 2 KB of contiguous memory). The FP8 bytes
// are widened exactly to bf16 (v_cvt_scalef32_pk_bf16_fp8 with scale 1) and fed to
// four mfma_f32_16x16x32_bf16 against the LDS rows (samples as the N dimension); the
// 128-k partial is then scaled by the tile's f32 block scale into the accumulator
// (glm53/gfx950/kernel.py:30-37, 787-845, 1061-1172). Lane (g, r) ends with output
// rows 4 g + [0, 4) of sample r.
#pragma once

#include "common.h"

namespace mono {
namespace proj {

// the 8 bf16 of k = 8 q + [0, 8) of a lane's 32 FP8 bytes
MONO_DEV bf16x8 fp8x8_bf16(const i32x8& w, int q) {
  const uint32_t lo = (uint32_t)w[2 * q], hi = (uint32_t)w[2 * q + 1];
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  bf16x8 o;
  o[0] = a[0]; o[1] = a[1]; o[2] = b[0]; o[3] = b[1];
  o[4] = c[0]; o[5] = c[1]; o[6] = d[0]; o[7] = d[1];
  return o;
}

// one 128-k step of an FP8 tile against the lane's bf16 row at brow = &x[r][k0 + 32 g];
// the scheduling barrier keeps a step's LDS reads and conversions from being hoisted
// over earlier steps (which would hold every step's operands in registers at once)
MONO_DEV f32x4 step_fp8(const i32x8& w, const uint16_t* brow) {
  f32x4 p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 4; ++q) p = mfma_bf16(fp8x8_bf16(w, q), *reinterpret_cast<const bf16x8*>(brow + 8 * q), p);
  __builtin_amdgcn_sched_barrier(0);
  return p;
}

// one 128-k step of a bf16 tile (w[q]: the lane's 8 weights of k = 32 g + 8 q + [0, 8))
MONO_DEV f32x4 step_bf16(const u32x4 (&w)[4], const uint16_t* brow, f32x4 acc) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
    acc = mfma_bf16(__builtin_bit_cast(bf16x8, w[q]), *reinterpret_cast<const bf16x8*>(brow + 8 * q), acc);
  __builtin_amdgcn_sched_barrier(0);
  return acc;
}

MONO_DEV i32x8 join(const u32x4& lo, const u32x4& hi) {
  i32x8 v;
  v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
  v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
  return v;
}

// The lane's two 16-byte halves of 128-k step ks of 16-row group rg of a shuffled
// FP8 [N, K] matrix (kdiv32 = K / 32).
MONO_DEV void ld_fp8_tile(const uint8_t* wb, int kdiv32, int rg, int ks, int g, int r, u32x4& lo, u32x4& hi) {
  const uint8_t* p = wb + ((size_t)rg * kdiv32 + ks * 4 + g) * 512 + r * 16;
  lo = ld_nt_u32x4(p);
  hi = ld_nt_u32x4(p + 256);
}

// The lane's 16 bytes for MFMA q of 128-k step ks of 16-row group rg of a bf16 [N, K]
// matrix whose bytes are in the (16, 16) layout (kbytes32 = 2 K / 32 chunks a row):
// k = 128 ks + 32 g + 8 q + [0, 8) sits in 32-byte chunk 8 ks + 2 g + q / 2, half q % 2.
MONO_DEV u32x4 ld_bf16_tile(const uint8_t* wb, int kbytes32, int rg, int ks, int g, int r, int q) {
  return ld_nt_u32x4(wb + ((size_t)rg * kbytes32 * 2 + 16 * ks + 4 * g + q) * 256 + r * 16);
}

// products and sums rounded one at a time (no fused multiply-add), as the CPU
// restatement computes them
MONO_DEV float mul_rn(float a, float b) { return __fmul_rn(a, b); }
MONO_DEV float add_rn(float a, float b) { return __fadd_rn(a, b); }
MONO_DEV float sub_rn(float a, float b) { return __fsub_rn(a, b); }

// RoPE of one interleaved pair (glm53/gfx950/kernel.py:2072): (x0 c - x1 s, x0 s + x1 c)
MONO_DEV void rope_pair(float& x0, float& x1, float c, float s) {
  const float a = sub_rn(mul_rn(x0, c), mul_rn(x1, s));
  const float b = add_rn(mul_rn(x0, s), mul_rn(x1, c));
  x0 = a;
  x1 = b;
}

// biased exponent of the smallest power of two >= v (v > 0), clamped to [1, 254]
// (common/mx.py:26-32)
MONO_DEV uint32_t code_ceil(float v) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t e = ((b >> 23) & 0xffu) + ((b & 0x7fffffu) != 0u ? 1u : 0u);
  return min(max(e, 1u), 254u);
}
MONO_DEV float pow2_of(uint32_t code) { return __uint_as_float(code << 23); }

// E2M1 code of |q| <= 6, round to nearest, ties to the even code (the rounding the
// hardware FP4 converts apply)
MONO_DEV uint32_t e2m1_code(float q) {
  const float a = fabsf(q);
  uint32_t c;
  if (a <= 0.25f) c = 0;
  else if (a < 0.75f) c = 1;
  else if (a <= 1.25f) c = 2;
  else if (a < 1.75f) c = 3;
  else if (a <= 2.5f) c = 4;
  else if (a < 3.5f) c = 5;
  else if (a <= 5.0f) c = 6;
  else c = 7;
  return (q < 0.f && c != 0u) ? c + 8u : c;
}

// One 128-dim index vector held by a wave, lane l holding dims 2 l and 2 l + 1 (RoPE
// already applied): bf16, Walsh-Hadamard (Sylvester order, element stride 1 first),
// x 128^-1/2, bf16, then FP4 over 32-dim blocks (16 lanes) with a power-of-two scale
// (deepseek_v4/gfx950/kernels/stages/indexer.py:127-151 ``had_pair`` / ``fp4_block``).
// Returns the lane's byte (dim 2 l in the low nibble) and sets `e8` to its block's
// E8M0 scale code.
MONO_DEV uint32_t index_vec_fp4(float a, float b, int lane, uint32_t& e8) {
  a = bf16_round(a);
  b = bf16_round(b);
  float x = add_rn(a, b), y = sub_rn(a, b);  // element stride 1
#pragma unroll
  for (int m = 1; m < WAVE; m <<= 1) {
    const float px = __shfl_xor(x, m, WAVE), py = __shfl_xor(y, m, WAVE);
    const bool hi = (lane & m) != 0;
    x = hi ? sub_rn(px, x) : add_rn(x, px);
    y = hi ? sub_rn(py, y) : add_rn(y, py);
  }
  const float k = 0.08838834764831845f;  // 128^-1/2
  x = bf16_round(mul_rn(x, k));
  y = bf16_round(mul_rn(y, k));
  const float amax = row_reduce<16>(fmaxf(fabsf(x), fabsf(y)), OpMax());
  e8 = code_ceil(mul_rn(fmaxf(amax, 6.0f * 0x1p-126f), 1.0f / 6.0f));
  const float inv = pow2_of(254u - e8);
  const float qx = fminf(fmaxf(mul_rn(x, inv), -6.0f), 6.0f);
  const float qy = fminf(fmaxf(mul_rn(y, inv), -6.0f), 6.0f);
  return e2m1_code(qx) | (e2m1_code(qy) << 4);
}

}  // namespace proj
}  // namespace mono
