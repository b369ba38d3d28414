// Device pieces shared by the persistent MoE launches (FP8 W8A8 and MXFP4 A16W4): the
// expert-selection order, a wave's top-k, the step's expert plan in LDS and the
// (16, 16)-shuffled weight loads.
#pragma once

#include "common.h"
#include "moe_plan.h"
#include "sync.h"

namespace mono {
namespace moe {

// f32 -> u32 key with the float order (larger key = larger value; +0 above -0)
// (glm53/check.py:94-97)
MONO_DEV uint32_t radix_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Sort a lane's 4 (key desc, id asc) candidates.
MONO_DEV void sort4(uint32_t (&k)[4], int (&id)[4], float (&raw)[4]) {
  const int pairs[5][2] = {{0, 1}, {2, 3}, {0, 2}, {1, 3}, {1, 2}};
#pragma unroll
  for (int p = 0; p < 5; ++p) {
    const int x = pairs[p][0], y = pairs[p][1];
    const bool first = (k[x] > k[y]) || (k[x] == k[y] && id[x] < id[y]);
    if (!first) {
      uint32_t tk = k[x]; k[x] = k[y]; k[y] = tk;
      int ti = id[x]; id[x] = id[y]; id[y] = ti;
      float tr = raw[x]; raw[x] = raw[y]; raw[y] = tr;
    }
  }
}

// The wave's top TOPK of 256 candidates (lane l holds candidates l + 64 i: key, id,
// and a value carried along) by key descending, lowest id on exact ties
// (glm53/gfx950/kernel.py:1575-1629). Lane k < TOPK gets pick k's id and value.
template <int TOPK>
MONO_DEV void wave_topk(uint32_t (&key)[4], int (&id)[4], float (&raw)[4], int n_ids, int& my_id, float& my_raw) {
  const int lane = lane_id();
  sort4(key, id, raw);
  my_raw = 0.f;
  my_id = 0;
  for (int k = 0; k < TOPK; ++k) {
    const uint32_t m = wave_umax(key[0]);
    uint64_t bal = __ballot(key[0] == m);
    if (__popcll(bal) > 1) {  // wave-uniform: an exact tie of keys, the lowest id wins
      const uint32_t cand = key[0] == m ? 0xffffu - (uint32_t)id[0] : 0u;
      const int low = (int)(0xffffu - wave_umax(cand));
      bal = __ballot(key[0] == m && id[0] == low);
    }
    const int src = __ffsll((long long)bal) - 1;
    const bool hit = lane == src;
    const int pick = min(__builtin_amdgcn_readlane(id[0], src), n_ids - 1);
    const float rv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, raw[0]), src));
    if (lane == k) {
      my_raw = rv;
      my_id = pick;
    }
    if (hit) {
      key[0] = key[1]; key[1] = key[2]; key[2] = key[3]; key[3] = 0u;
      id[0] = id[1]; id[1] = id[2]; id[2] = id[3]; id[3] = 0xffff;
      raw[0] = raw[1]; raw[1] = raw[2]; raw[2] = raw[3]; raw[3] = 0.f;
    }
  }
}

// The step's expert plan: slot 0 is the shared expert (id E, weight 1, every row);
// slots 1.. the distinct picked experts by ascending id.
template <int E, int TOPK>
struct PlanLds {
  int32_t expert[MAX_ACT];                 // expert id of each slot
  uint32_t rowmask[MAX_ACT];               // rows each slot serves
  int32_t dmap[E];                         // slot of a picked expert
  int32_t pick_id[MAX_ROWS][TOPK];
  float pick_w[MAX_ROWS][TOPK];
  int32_t rowslot[MAX_ROWS][TOPK + 1];     // a row's slots in plan order
  uint32_t used[E];
  int32_t wcount[16];
  int32_t n_act;
};

template <int E, int TOPK, int THREADS>
MONO_DEV void plan_from_picks(PlanLds<E, TOPK>& P, int S);

// The plan from the picks already in P.pick_id / P.pick_w (ids in [0, E)); all threads
// of the workgroup call it, after a barrier that orders the picks' writes.
template <int E, int TOPK, int THREADS>
MONO_DEV void plan_from_picks(PlanLds<E, TOPK>& P, int S) {
  static_assert(THREADS >= E && THREADS / WAVE <= 16, "one thread an expert");
  const int tid = thread_index(), lane = tid % WAVE, wave = tid / WAVE;
  for (int e = tid; e < E; e += THREADS) P.used[e] = 0u;
  __syncthreads();
  if (tid < S * TOPK) {
    const int s = tid / TOPK, k = tid % TOPK;
    atomicOr(&P.used[P.pick_id[s][k]], 1u << s);
  }
  __syncthreads();
  const bool f = tid < E && P.used[tid] != 0u;
  const uint64_t bal = __ballot(f);
  const int before = __popcll(bal & ((1ull << lane) - 1ull));
  if (lane == 0) P.wcount[wave] = __popcll(bal);
  __syncthreads();
  int off = 1;  // fixed trip count: the LDS reads issue together, not one wait a wave
#pragma unroll
  for (int w = 0; w < THREADS / WAVE; ++w) off += w < wave ? P.wcount[w] : 0;
  if (f) {
    const int d = off + before;
    P.expert[d] = tid;
    P.rowmask[d] = P.used[tid];
    P.dmap[tid] = d;
  }
  if (tid == 0) {
    P.expert[0] = E;
    P.rowmask[0] = (1u << S) - 1u;
    int n = 1;
    for (int w = 0; w < THREADS / WAVE; ++w) n += P.wcount[w];
    P.n_act = n;
  }
  __syncthreads();
  // a row's slots, ascending: thread (s, k) places pick k's slot at its rank among the
  // row's picks (equal slots ranked by k, so every place of the row is written once)
  static_assert(THREADS >= MAX_ROWS * TOPK, "one thread a pick");
  if (tid < S * TOPK) {
    const int s = tid / TOPK, k = tid % TOPK;
    int dd[TOPK];
#pragma unroll
    for (int k2 = 0; k2 < TOPK; ++k2) dd[k2] = P.dmap[P.pick_id[s][k2]];
    const int d = dd[k];
    int rank = 0;
#pragma unroll
    for (int k2 = 0; k2 < TOPK; ++k2) rank += (dd[k2] < d || (dd[k2] == d && k2 < k)) ? 1 : 0;
    P.rowslot[s][1 + rank] = d;
    if (k == 0) P.rowslot[s][0] = 0;
  }
  __syncthreads();
}

// Route weight of slot d for row s (0 if the slot does not serve the row).
template <int E, int TOPK>
MONO_DEV float route_weight(const PlanLds<E, TOPK>& P, int d, int s) {
  if (d == 0) return 1.0f;
  const int e = P.expert[d];
  float w = 0.f;
#pragma unroll
  for (int k = 0; k < TOPK; ++k) {  // unconditional reads: no branch a pick
    const float wk = P.pick_w[s][k];
    w = P.pick_id[s][k] == e ? wk : w;
  }
  return w;
}

// The 32 bytes lane (g, r) holds of 128-k block kb of 16-row group rg of a shuffled
// [N, K] E4M3 matrix at wb (kdiv32 = K / 32): k = 128 kb + 32 g + [0, 32) of row
// 16 rg + r, as two nontemporal dwordx4 loads 256 bytes apart.
MONO_DEV i32x8 ld_shuf(const uint8_t* wb, int kdiv32, int rg, int kb, int g, int r) {
  const uint8_t* p = wb + (size_t)(rg * kdiv32 + kb * 4 + g) * 512 + r * 16;
  const u32x4 lo = ld_nt_u32x4(p), hi = ld_nt_u32x4(p + 256);
  i32x8 v;
  v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
  v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
  return v;
}

// The 16 bytes lane l holds of 128-k step ks of 16-row group rg of a shuffled
// packed-E2M1 matrix [N, K/2] at wb (K = 32 kdiv32): row 16 rg + l % 16, k = 128 ks
// + 32 (l / 16) + [0, 32); a wave's loads cover 1 KB of contiguous memory
// (minimax_m31/a16w4.py:1-13).
MONO_DEV u32x4 ld_shuf_fp4(const uint8_t* wb, int kdiv32, int rg, int ks, int lane) {
  return ld_nt_u32x4(wb + ((size_t)rg * (kdiv32 / 4) + ks) * 1024 + lane * 16);
}

// 32 bytes of an LDS row as one MFMA operand
MONO_DEV i32x8 lds32(const uint8_t* p) {
  const u32x4 lo = *reinterpret_cast<const u32x4*>(p), hi = *reinterpret_cast<const u32x4*>(p + 16);
  i32x8 v;
  v[0] = lo[0]; v[1] = lo[1]; v[2] = lo[2]; v[3] = lo[3];
  v[4] = hi[0]; v[5] = hi[1]; v[6] = hi[2]; v[7] = hi[3];
  return v;
}

}  // namespace moe
}  // namespace mono
