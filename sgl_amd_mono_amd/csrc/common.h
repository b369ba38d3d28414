// Device helpers shared by the gfx950 kernels of the decoder-layer path.
//
// Wave64 reductions, the FP8 / FP4 / bf16 converts of CDNA4, the 16x16 MFMA tiles
// the GEMVs use, and nontemporal weight loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MONO_DEV __device__ __forceinline__

// The thread's and the workgroup's indices. A translation unit that runs the phases in
// a loop over layers (the multi-layer launch) defines MONO_LAYER_LOOP first: the indices
// then pass an opaque copy at each use, so the compiler cannot hoist per-thread and
// per-workgroup arithmetic out of that loop (held across every phase, it spills).
MONO_DEV int thread_index() {
#ifdef MONO_LAYER_LOOP
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  __builtin_assume(t >= 0 && t < 1024);
  return t;
#else
  return (int)threadIdx.x;
#endif
}
MONO_DEV unsigned block_index() {
#ifdef MONO_LAYER_LOOP
  int b = (int)blockIdx.x;
  asm volatile("" : "+v"(b));
  b = __builtin_amdgcn_readfirstlane(b);  // uniform: scalar arithmetic and branches
  __builtin_assume(b >= 0 && b < 65536);
  return (unsigned)b;
#else
  return blockIdx.x;
#endif
}

// An opaque copy of a per-lane value: arithmetic derived from it inside a loop cannot be
// hoisted out of the loop and held in registers across it.
MONO_DEV int opaque_v(int v) {
  asm volatile("" : "+v"(v));
  return v;
}

typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

namespace mono {

constexpr int WAVE = 64;
constexpr float FP8_MAX = 448.0f;

// ------------------------------------------------------------------ lanes
MONO_DEV int lane_id() { return __lane_id(); }

// Cross-lane reductions without LDS traffic: DPP steps inside each 16-lane row
// (xor 1, xor 2, 8-lane half mirror, 16-lane mirror), then the four rows' results read
// into scalars. __shfl_xor would compile to ds_bpermute, an LDS round trip a step.
enum : int {
  DPP_XOR1 = 0xB1,         // quad_perm [1, 0, 3, 2]
  DPP_XOR2 = 0x4E,         // quad_perm [2, 3, 0, 1]
  DPP_HALF_MIRROR = 0x141, // lane i <-> 7 - i in each 8 lanes
  DPP_MIRROR = 0x140,      // lane i <-> 15 - i in each 16 lanes
};

template <int CTRL>
MONO_DEV float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
MONO_DEV uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Reduce over each group of WIDTH consecutive lanes (WIDTH in 2, 4, 8, 16); every
// lane of a group gets the group's result.
template <int WIDTH, class Op>
MONO_DEV float row_reduce(float v, Op op) {
  static_assert(WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16, "a DPP row is 16 lanes");
  v = op(v, dpp_f<DPP_XOR1>(v));
  if (WIDTH >= 4) v = op(v, dpp_f<DPP_XOR2>(v));
  if (WIDTH >= 8) v = op(v, dpp_f<DPP_HALF_MIRROR>(v));
  if (WIDTH >= 16) v = op(v, dpp_f<DPP_MIRROR>(v));
  return v;
}

template <class Op>
MONO_DEV float wave_reduce(float v, Op op) {
  v = row_reduce<16>(v, op);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return op(op(r0, r1), op(r2, r3));
}

struct OpAdd {
  MONO_DEV float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  MONO_DEV float operator()(float a, float b) const { return fmaxf(a, b); }
};

// sum / max over the wave, the same value in every lane (wave-uniform)
MONO_DEV float wave_sum(float v) { return wave_reduce(v, OpAdd()); }
MONO_DEV float wave_max(float v) { return wave_reduce(v, OpMax()); }

MONO_DEV uint32_t wave_umax(uint32_t v) {
  v = max(v, dpp_u<DPP_XOR1>(v));
  v = max(v, dpp_u<DPP_XOR2>(v));
  v = max(v, dpp_u<DPP_HALF_MIRROR>(v));
  v = max(v, dpp_u<DPP_MIRROR>(v));
  const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
  const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
  return max(a, b);
}

// Inclusive prefix sum over the wave, lane 0 first: DPP row shifts inside each 16-lane
// row (Hillis-Steele), then two row broadcasts carry the sums of row 0 and of rows
// 0..1 into the rows after them. Lanes whose DPP source lies outside the row add 0.
MONO_DEV int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return v;
}
// integer sum over the wave (wave-uniform)
MONO_DEV int wave_sum_i(int v) { return __builtin_amdgcn_readlane(wave_incl_scan(v), WAVE - 1); }

// max over groups of `WIDTH` consecutive lanes (WIDTH a power of two <= 16)
template <int WIDTH>
MONO_DEV float group_max(float v) {
  return row_reduce<WIDTH>(v, OpMax());
}

// ------------------------------------------------------------------ math
MONO_DEV float hw_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
MONO_DEV float hw_rsq(float x) { return __builtin_amdgcn_rsqf(x); }
MONO_DEV float hw_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
MONO_DEV float sigmoid(float x) { return hw_rcp(1.0f + hw_exp(-x)); }
MONO_DEV float silu(float x) { return x * sigmoid(x); }

// ------------------------------------------------------------------ bf16
MONO_DEV float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }
MONO_DEV float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
MONO_DEV float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
MONO_DEV uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;  // round to nearest even
  return __builtin_bit_cast(uint16_t, b);
}
MONO_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}
MONO_DEV float bf16_round(float f) { return (float)(__bf16)f; }
// a dword as two bf16 (low half first), taken by value: __builtin_bit_cast of an
// ext_vector element (v[i]) reads element 0 whatever i is (hipcc of ROCm 7.2)
MONO_DEV bf16x2 as_bf16x2(uint32_t u) { return __builtin_bit_cast(bf16x2, u); }

// ------------------------------------------------------------------ FP8 (OCP E4M3)
// two f32 (already clamped to +-448) -> two E4M3 bytes in the low 16 bits, RNE
MONO_DEV uint32_t fp8x2_pack(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}
// four f32 -> one dword of four E4M3 bytes
MONO_DEV uint32_t fp8x4_pack(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}
// bytes 0,1 (HI=false) or 2,3 (HI=true) of a dword -> two f32
template <bool HI>
MONO_DEV f32x2 fp8x2_unpack(uint32_t w) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)w, HI);
}

// ------------------------------------------------------------------ FP4 (E2M1) + E8M0
// byte `sel` (0..3) of `w` (two E2M1 codes, low nibble first) times `scale` -> two bf16
MONO_DEV bf16x2 fp4x2_to_bf16(uint32_t w, float scale, int sel) {
  switch (sel) {
    case 0: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
    case 1: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
    case 2: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
    default: return __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  }
}
// E8M0 code -> f32 2^(code-127) (code 0 -> 2^-127 is denormal: built from bits)
MONO_DEV float e8m0_to_f32(uint32_t code) {
  return code == 0 ? __uint_as_float(0x00400000u) : __uint_as_float(code << 23);
}

// ------------------------------------------------------------------ MFMA tiles
// C[16x16] += A[16x128] * B[128x16], E4M3 x E4M3, unit block scales.
// Lane l supplies row / column (l % 16) and one 32-element k group (l / 16).
MONO_DEV f32x4 mfma_fp8(const i32x8& a, const i32x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
// E2M1 x E2M1 with per-lane E8M0 scales (lane l: its row / column's scale of k group l / 16)
MONO_DEV f32x4 mfma_fp4(const i32x8& a, const i32x8& b, const f32x4& c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 4, 0, sa, 0, sb);
}
// C[16x16] += A[16x32] * B[32x16] in bf16; lane l: row / column l % 16, k 8*(l/16)..+7
MONO_DEV f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ memory
MONO_DEV u32x4 ld_nt_u32x4(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
MONO_DEV u32x4 ld_u32x4(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// Data no launch writes (weights and their scales) read at a wave-uniform address
// through the constant address space: a scalar load into SGPRs, outside the in-order
// vector memory queue.
typedef const __attribute__((address_space(4))) float const_f32;
MONO_DEV float ld_const_f32(const float* p) { return *(const_f32*)p; }
// 32 bytes (two dwordx4) straight into one MFMA operand tuple
MONO_DEV i32x8 ld_nt_i32x8(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const i32x8*>(p));
}
MONO_DEV i32x8 ld_i32x8(const void* p) { return *reinterpret_cast<const i32x8*>(p); }

}  // namespace mono
