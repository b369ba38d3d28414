// The FP8 MoE phase of a decode step as a workgroup-level class (Step), included by the
// MoE launch (moe_fp8.hip) and by the fused layer launch (layer.hip).
//
// This is the post-attention half of the reference's decoder-layer launch
// (sgl_amd_mono/glm53/gfx950/kernel.py stages router / ug / down, :4199-5187, W8A8 MoE
// mode) with the tensor-parallel reduce replaced by a local residual add. Stages hand
// data to each other through tagged mailbox words (sync.h); nothing waits at a grid
// barrier and every wait is bounded by the guard's deadline.
//
// Work, in the order each workgroup walks it:
//   ticket   one atomic add on the workgroup's own launch counter -> the launch's tag (sync.h)
//   norm     every workgroup: the RMSNorm statistics of all rows (kernel.py:1367-1415);
//            wave w keeps row w in registers for xq
//   router   task t < 16 * RK on workgroup t: 16 experts x a 512-wide K slice of the
//            bf16 router GEMV on the bf16-rounded normed rows (MFMA 16x16x32 bf16)
//            -> partial logits (mailbox rlog)
//   route    row s on workgroup G-1-s: the K slices summed in order, sigmoid, top-8 by
//            the f32 bits of (score + bias) with lowest-id ties, weights = score / sum
//            x route_scale (kernel.py:1575-1629) -> the row's picks (mailbox rsel)
//   xq       every workgroup: per-128 FP8 quantisation of the normed rows into LDS
//            (amax / 448 with a hardware reciprocal, kernel.py:1440-1450), after the
//            router and route so that neither waits for it
//   plan     every workgroup, before its first routed tile: the distinct experts of
//            the step; slot 0 is the shared expert (weight 1), slots 1.. the picked
//            experts by ascending id
//   tasks    one round-robin list over the workgroups:
//            up     (slot, 16-channel tile): FP8 x FP8 MFMA 16x16x128 with the 128x128
//                   weight block scale x the activation block scale per 128-k, the 8
//                   waves splitting K, SiLU(gate) * up -> mailbox mid
//            down   (slot, 256 output rows): the slot's mid quantised per 128 to FP8 in
//                   LDS (kernel.py:5118-5125), FP8 MFMA, x weight block scale x mid
//                   block scale x route weight -> mailbox ypart
//            final  (32 output rows): the row's slots summed in plan order + the
//                   residual -> bf16 out (kernel.py:5176-5185 without the peer reduce)
//
// Expert weights are read in place in AITER's (16, 16) shuffled layout
// ([N/16, K/32, 2, 16 rows, 16 B], glm53/gfx950/kernel.py:787-808): a lane's two
// 16-byte loads are exactly its MFMA operand, and a wave's pair covers 2 KB of
// contiguous HBM. Each workgroup issues a task's weight loads before it waits on or
// reduces the previous task, so weights stream while mailboxes are polled.
#pragma once

#include "common.h"
#include "moe_common.h"
#include "moe_ops.h"
#include "moe_plan.h"
#include "sync.h"

namespace mono {
namespace moe {

namespace {

constexpr int FT = 512;
constexpr int FW = FT / WAVE;  // 8 waves

// BASELINE config 2 geometry
constexpr int H = 7168, E = 256, I = 512, TOPK = 8;
constexpr int KB = H / 128;          // 128-k blocks of a hidden row
constexpr int IB = I / 128;          // 128-k blocks of a mid row
constexpr int NT = I / 16;           // up tiles a slot
constexpr int UP_KBW = KB / FW;      // k blocks a wave of an up tile
constexpr int UP_H0 = 4;             // of them in an up tile's first half (W[0..7]); the rest W[8..13]
constexpr int RK = 14;               // router K slices
constexpr int RKW = H / RK / FW;     // k a wave of a router task
constexpr int RSTEP = RKW / 32;      // bf16 MFMA steps a wave of a router task
constexpr int ROUTER_TASKS = (E / 16) * RK;
constexpr int DN_ROWS = 448;         // output rows of a down task: 28 16-row tiles x 4 k blocks
constexpr int DN_GROUPS = H / DN_ROWS;
constexpr int DN_PAIR = DN_ROWS / 16 / (FW / 2);  // row tiles of a wave pair
constexpr int FIN_ROWS = 32;
constexpr int FIN_TASKS = H / FIN_ROWS;
constexpr int NSLOT = TOPK + 1;      // slots a row uses: the shared expert and its picks
constexpr int PER_ROW = H / (8 * WAVE);  // 16-byte loads a lane makes of a hidden row
static_assert(KB % FW == 0 && RKW % 32 == 0 && H % (RK * FW) == 0, "tiling");
static_assert(UP_KBW * 2 == 14 && DN_PAIR * IB == 2 * 14 && H % DN_ROWS == 0, "14 weight tiles a wave");
static_assert(IB == 4 && DN_PAIR == 7, "a wave pair's row tiles: 3 whole and half of one each");
static_assert(I == 8 * WAVE && MAX_ROWS <= 2 * FW, "a down task's wave reads one or two mid rows, 8 channels a lane");
static_assert(MAX_ROWS * FIN_ROWS <= FT, "a final task's thread owns one (row, output)");

// wait sites (guard error word = site + 1), offset by the Step's site0 in a fused
// launch; W_A: the attention block's output rows (fused launch only)
enum { W_LOGITS = 0, W_PICKS = 1, W_MID = 2, W_YPART = 3, W_A = 4 };

struct Lds {
  uint8_t xq[MAX_ROWS][H];          // FP8 normed rows
  float xs[MAX_ROWS][KB];           // their block scales
  float rstd[MAX_ROWS];
  f32x4 red[2][FW][WAVE];           // cross-wave sums
  uint8_t bq[MAX_ROWS][I];          // a down task's FP8 mid
  float coef[MAX_ROWS][IB];         // its block scale x route weight
  PlanLds<E, TOPK> plan;
  uint32_t rkey[E];
  float rraw[E];
};

struct Args {
  const uint16_t* a;
  const uint16_t* g_post;
  const uint16_t* w_router;
  const float* bias;
  const uint8_t* w13;
  const float* s13;
  const uint8_t* w2;
  const float* s2;
  uint16_t* out;
  float* y_out;
  float* scores;
  int32_t* topk_ids;
  float* topk_w;
  int rows;
  float route_scale;
  float eps;
  // the fused layer's phase ticks ([grid][16], NULL: none): workgroup b stamps word
  // 16 b + k at MoE moment k (T_* below)
  int64_t* ticks;
  Mail mail;
  GuardArgs guard;
};

// bf16(a * rstd * gamma) of 8 consecutive k as one bf16 MFMA operand
// (stage_x_rmsnorm, kernel.py:1367-1400)
MONO_DEV bf16x8 normed8(const uint16_t* a, const uint16_t* g, float rstd) {
  const u32x4 av = ld_u32x4(a), gv = ld_u32x4(g);
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = pack_bf16x2(bf16_lo(av[q]) * rstd * bf16_lo(gv[q]), bf16_hi(av[q]) * rstd * bf16_hi(gv[q]));
  return __builtin_bit_cast(bf16x8, o);
}

// Task kinds of the round-robin list
enum { K_NONE = 0, K_UP = 1, K_DOWN = 2, K_FINAL = 3 };

// the MoE's moments in a fused layer's tick row (its other words are the layer's)
enum { T_PLAN = 4, T_A = 6, T_NORM = 7, T_ROUTER = 8, T_ROUTE = 9, T_QUANT = 10, T_ROW = 16 };

class Step {
 public:
  MONO_DEV Step(const Args& a, Lds& l) : A(a), L(l) {
    tid = threadIdx.x;
    lane = tid % WAVE;
    wave = tid / WAVE;
    g = lane / 16;
    r = lane % 16;
    G = gridDim.x;
    S = a.rows;
  }

  // Run under an earlier phase's guard in the same launch (its tag, deadline and fail
  // word, wait sites offset by `site_base`), on the residual stream `a` that phase's
  // n_done tasks announce with the done words at `done` (replicated, sync.h).
  MONO_DEV void adopt(const Guard& g, const uint64_t* done, int n_done, int site_base) {
    gd = g;
    a_done = done;
    n_a_done = n_done;
    site0 = site_base;
  }

  // The MoE of the step (false, workgroup-uniform: a wait failed; `refused`: the guard
  // refused the launch before anything ran).
  MONO_DEV bool run(bool& refused) {
    refused = false;
    if (!a_done && !guard_begin(A.guard, gd)) {  // a failed launch stops the guard until the host clears it
      refused = true;
      return false;
    }
    // the router task's weights go out before anything waits
    const int rt = blockIdx.x;
    u32x4 wr[RSTEP];
    if (rt < ROUTER_TASKS) router_load(rt, wr);
    if (a_done) {
      // every row of `a` is stored once its producers' done words carry the tag; `a` is
      // read with plain loads after that (no workgroup reads it earlier in the launch,
      // so no cache holds an older copy of its lines)
      const uint64_t* ad = done_copy(a_done);
      if (!hint_wait(n_a_done, [ad](int i) { return ad + i; }, site0 + W_A, gd)) return false;
      stamp(T_A);
    }

    u32x4 ar[PER_ROW];  // wave w's row w, kept for the quantisation
    norm_stats(ar);
    __syncthreads();
    stamp(T_NORM);
    if (rt < ROUTER_TASKS) router(rt, wr);
    stamp(T_ROUTER);
    if ((int)blockIdx.x >= G - S) {
      if (!route(G - 1 - (int)blockIdx.x)) return false;
      stamp(T_ROUTE);
    }
    quant_rows(ar);
    __syncthreads();
    stamp(T_QUANT);
    return tasks();
  }

  // NaN over the launch's output (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.out, (size_t)S * H, share); }

  // this workgroup's tick at MoE moment k (a fused layer with ticks only)
  MONO_DEV void stamp(int k) const {
    if (A.ticks && tid == 0) A.ticks[blockIdx.x * T_ROW + k] = (int64_t)now_ticks();
  }

 private:
  const Args& A;
  Lds& L;
  Guard gd;
  int tid, lane, wave, g, r, G, S;
  const uint64_t* a_done = nullptr;  // fused launch: the done words announcing `a`
  int n_a_done = 0;
  int site0 = 0;
  i32x8 W[14];  // weights of the next task: an up tile (14) or a down task (8)
  float SC[2 * UP_KBW];  // an up tile's block scales (gate, up a k block), read with each half

  // ---------------------------------------------------------------- norm
  // Wave w reads row w (lane: 8 consecutive k of each 512) into registers, which it
  // keeps for the quantisation; row w + 8 is read for its statistics.
  MONO_DEV void norm_stats(u32x4 (&ar)[PER_ROW]) {
    const uint16_t* row0 = A.a + (size_t)min(wave, S - 1) * H;
#pragma unroll
    for (int j = 0; j < PER_ROW; ++j) ar[j] = ld_u32x4(row0 + (j * WAVE + lane) * 8);
    if (wave + FW < S) {
      u32x4 w[PER_ROW];
      const uint16_t* row = A.a + (size_t)(wave + FW) * H;
#pragma unroll
      for (int j = 0; j < PER_ROW; ++j) w[j] = ld_u32x4(row + (j * WAVE + lane) * 8);
      row_rstd(wave + FW, w);
    }
    if (wave < S) row_rstd(wave, ar);
  }

  MONO_DEV void row_rstd(int s, const u32x4 (&w)[PER_ROW]) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < PER_ROW; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float lo = bf16_lo(w[j][q]), hi = bf16_hi(w[j][q]);
        ss += lo * lo + hi * hi;
      }
    ss = wave_sum(ss);
    if (lane == 0) L.rstd[s] = hw_rsq(ss * (1.0f / H) + A.eps);
  }

  // ---------------------------------------------------------------- router
  MONO_DEV void router_load(int t, u32x4 (&wr)[RSTEP]) {
    const int et = t % (E / 16), ks = t / (E / 16);
    const uint16_t* wrow = A.w_router + (size_t)(et * 16 + r) * H + ks * (H / RK) + wave * RKW + g * 8;
#pragma unroll
    for (int st = 0; st < RSTEP; ++st) wr[st] = ld_nt_u32x4(wrow + st * 32);
  }

  MONO_DEV void router(int t, const u32x4 (&wr)[RSTEP]) {
    const int et = t % (E / 16), ks = t / (E / 16);
    // columns r >= S compute on row S - 1 and are dropped: every load unconditional
    const int rr = min(r, S - 1);
    const float rj = L.rstd[rr];
    const uint16_t* arow = A.a + (size_t)rr * H;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < RSTEP; ++st) {
      const int k = ks * (H / RK) + wave * RKW + st * 32 + g * 8;
      acc = mfma_bf16(__builtin_bit_cast(bf16x8, wr[st]), normed8(arow + k, A.g_post + k, rj), acc);
    }
    L.red[0][wave][lane] = acc;
    __syncthreads();
    if (tid < 256) {
      const int l = tid % WAVE, i = tid / WAVE;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < FW; ++w) v += L.red[0][w][l][i];
      const int s = l % 16, e = et * 16 + 4 * (l / 16) + i;
      if (s < S) mb_putf(&A.mail.rlog[((size_t)ks * MAX_ROWS + s) * E + e], v, gd.tag);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- route
  MONO_DEV bool route(int s) {
    bool ok = true;
    const float bias = A.bias[min(tid, E - 1)];  // before the wait: no round trip after it
    if (tid < E) {
      const uint64_t* base = &A.mail.rlog[(size_t)s * E + tid];
      uint32_t v[RK];
      const auto at = [base](int ks) { return base + (size_t)ks * MAX_ROWS * E; };
      ok = poll_words<RK, decltype(at), false, false>(at, v, (1u << RK) - 1u, site0 + W_LOGITS, gd);
      float lg = 0.f;
#pragma unroll
      for (int ks = 0; ks < RK; ++ks) lg += __uint_as_float(v[ks]);
      const float raw = sigmoid(lg);
      L.rraw[tid] = raw;
      L.rkey[tid] = radix_key(raw + bias);
      if (A.scores && ok) A.scores[s * E + tid] = raw;
    }
    if (!block_all(ok)) return false;
    if (wave == 0) {
      uint32_t key[4];
      int id[4];
      float raw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        id[i] = lane + 64 * i;
        key[i] = L.rkey[id[i]];
        raw[i] = L.rraw[id[i]];
      }
      float my_raw;  // lane k < TOPK: the raw score and id of pick k
      int my_id;
      wave_topk<TOPK>(key, id, raw, E, my_id, my_raw);
      // sum of the picks' raw scores in the butterfly order of lanes 0..7
      float tot = lane < TOPK ? my_raw : 0.f;
      tot = row_reduce<TOPK>(tot, OpAdd());
      const float w = my_raw * (hw_rcp(tot) * A.route_scale);
      if (lane < TOPK) {
        mb_put(&A.mail.rsel[s * 2 * MAX_TOPK + lane], (uint32_t)my_id, gd.tag);
        mb_putf(&A.mail.rsel[s * 2 * MAX_TOPK + MAX_TOPK + lane], w, gd.tag);
        if (A.topk_ids) A.topk_ids[s * TOPK + lane] = my_id;
        if (A.topk_w) A.topk_w[s * TOPK + lane] = w;
      }
    }
    return true;
  }

  // ---------------------------------------------------------------- xq
  // Lane quantises 8 consecutive k of a row; 16 lanes make a 128-block. Row w comes
  // from the registers the norm filled; row w + 8 is read again.
  MONO_DEV void quant_rows(u32x4 (&ar)[PER_ROW]) {
    static_assert(MAX_ROWS <= 2 * FW, "two rows a wave at most");
    u32x4 gr[PER_ROW];
#pragma unroll
    for (int j = 0; j < PER_ROW; ++j) gr[j] = ld_u32x4(A.g_post + (j * WAVE + lane) * 8);
    if (wave < S) quant_row(wave, ar, gr);
    if (wave + FW < S) {
      const uint16_t* row = A.a + (size_t)(wave + FW) * H;
#pragma unroll
      for (int j = 0; j < PER_ROW; ++j) {
        ar[j] = ld_u32x4(row + (j * WAVE + lane) * 8);
        // gamma's bf16 -> f32 unpacking is redone for this row: shared with the first
        // row it would hold twice gamma's registers
        asm volatile("" : "+v"(gr[j]));
      }
      quant_row(wave + FW, ar, gr);
    }
  }

  MONO_DEV void quant_row(int s, const u32x4 (&av)[PER_ROW], const u32x4 (&gv)[PER_ROW]) {
    const float rj = L.rstd[s];
#pragma unroll
    for (int j = 0; j < PER_ROW; ++j) {
      const int k = (j * WAVE + lane) * 8;
      float x[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[2 * q] = bf16_lo(av[j][q]) * rj * bf16_lo(gv[j][q]);
        x[2 * q + 1] = bf16_hi(av[j][q]) * rj * bf16_hi(gv[j][q]);
      }
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[q]));
      const float amax = group_max<16>(m);
      const bool nz = amax > 0.f;
      const float inv = nz ? hw_rcp(amax) * FP8_MAX : 1.0f;
      u32x2 packed;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float q4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) q4[q] = fminf(fmaxf(x[4 * h + q] * inv, -FP8_MAX), FP8_MAX);
        packed[h] = fp8x4_pack(q4[0], q4[1], q4[2], q4[3]);
      }
      *reinterpret_cast<u32x2*>(&L.xq[s][k]) = packed;
      if ((lane % 16) == 0) L.xs[s][k / 128] = nz ? amax * (1.0f / FP8_MAX) : 1.0f;
      __builtin_amdgcn_sched_barrier(0);  // one chunk at a time: no interleaved live ranges
    }
  }

  // ---------------------------------------------------------------- plan
  MONO_DEV bool load_plan() { return build_plan<E, TOPK, FT>(L.plan, A.mail.rsel, S, site0 + W_PICKS, gd); }

  // ---------------------------------------------------------------- task list
  // kind of task T (the plan is loaded); K_NONE past the list
  MONO_DEV int classify(int T) const {
    const int n_up = L.plan.n_act * NT, n_dn = L.plan.n_act * DN_GROUPS;
    if (T < n_up) return K_UP;
    if (T < n_up + n_dn) return K_DOWN;
    if (T < n_up + n_dn + FIN_TASKS) return K_FINAL;
    return K_NONE;
  }

  // Issue task T's weight loads into W. Every entry of W is written on every path
  // (zero where the task has no weights), so none stays live into the next task.
  MONO_DEV void load_task(int kind, int T) {
    const i32x8 zero = {};
    if (kind == K_UP) {
      load_up<0>(T);
      load_up<1>(T);
    } else if (kind == K_DOWN) {
      load_down(T);
    } else {
#pragma unroll
      for (int q = 0; q < 14; ++q) W[q] = zero;
    }
  }

  // Each turn: consume the task's weights (waiting on its inputs), issue the next
  // task's weight loads, then publish the task's results while those loads fly.
  MONO_DEV bool tasks() {
    int T = blockIdx.x;
    // a shared-expert tile needs no plan: its loads go out before the plan is read
    if (T < NT) load_task(K_UP, T);
    if (!load_plan()) return false;
    stamp(T_PLAN);
    int kind = classify(T);
    if (T >= NT) load_task(kind, T);
    // consecutive up tiles, half by half: the next tile's first half goes out once this
    // tile's first half is consumed, its second half once this second half is, so one
    // half is always streaming while the other computes (vector memory returns in
    // order: consuming a half waits only for loads issued before it)
    while (kind == K_UP) {
      f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
      const int T2 = T + G;
      up_half<0>(ag, au);
      const int kind2 = classify(T2);
      if (kind2 != K_UP) {
        up_half<1>(ag, au);
        load_task(kind2, T2);
        up_publish(T, ag, au);
        T = T2;
        kind = kind2;
        break;
      }
      load_up<0>(T2);
      up_half<1>(ag, au);
      load_up<1>(T2);
      up_publish(T, ag, au);
      T = T2;
    }
    while (kind != K_NONE) {
      f32x4 acc[4];
      if (kind == K_DOWN) {
        if (!down_compute(T, acc)) return false;
      } else if (kind == K_UP) {
        acc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc[1] = acc[0];
        up_half<0>(acc[0], acc[1]);
        up_half<1>(acc[0], acc[1]);
      }
      const int T2 = T + G;
      const int kind2 = classify(T2);
      load_task(kind2, T2);
      if (kind == K_UP) {
        up_publish(T, acc[0], acc[1]);
      } else if (kind == K_DOWN) {
        down_publish(T, acc);
      } else {
        if (!final_task(T)) return false;
      }
      T = T2;
      kind = kind2;
    }
    return true;
  }

  // ---------------------------------------------------------------- up
  // Half HALF of up tile T (the wave's k blocks 0..3 or 4..6) into W, its block scales
  // into SC first.
  template <int HALF>
  MONO_DEV void load_up(int T) {
    constexpr int J0 = HALF == 0 ? 0 : UP_H0, J1 = HALF == 0 ? UP_H0 : UP_KBW;
    const int d = T / NT, c = T % NT;
    const int e = __builtin_amdgcn_readfirstlane(d == 0 ? E : L.plan.expert[d]);
    {  // the half's scales: scalar loads (one value a wave), apart from the vector queue
      const int wv = __builtin_amdgcn_readfirstlane(wave);
      const float* sg = A.s13 + ((size_t)e * (2 * I / 128) + c / 8) * KB + wv * UP_KBW;
#pragma unroll
      for (int j = J0; j < J1; ++j) {
        SC[2 * j] = ld_const_f32(sg + j);
        SC[2 * j + 1] = ld_const_f32(sg + (I / 128) * KB + j);
      }
    }
    const uint8_t* wb = A.w13 + (size_t)e * (2 * I) * H;
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      const int kb = wave * UP_KBW + j;
      W[2 * j] = ld_shuf(wb, H / 32, c, kb, g, r);
      W[2 * j + 1] = ld_shuf(wb, H / 32, NT + c, kb, g, r);
    }
  }
  // Half HALF of the up tile in W: FP8 x FP8 MFMA, block scale x activation scale.
  template <int HALF>
  MONO_DEV void up_half(f32x4& ag, f32x4& au) {
    constexpr int J0 = HALF == 0 ? 0 : UP_H0, J1 = HALF == 0 ? UP_H0 : UP_KBW;
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      const int kb = wave * UP_KBW + j;
      const i32x8 b = lds32(&L.xq[r][kb * 128 + g * 32]);
      const float xsj = L.xs[r][kb];
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 cg = mfma_fp8(W[2 * j], b, zero);
      const f32x4 cu = mfma_fp8(W[2 * j + 1], b, zero);
      ag += cg * (SC[2 * j] * xsj);
      au += cu * (SC[2 * j + 1] * xsj);
    }
  }

  MONO_DEV void up_publish(int T, const f32x4& ag, const f32x4& au) {
    const int d = T / NT, c = T % NT;
    const uint32_t mask = d == 0 ? (1u << S) - 1u : L.plan.rowmask[d];
    L.red[0][wave][lane] = ag;
    L.red[1][wave][lane] = au;
    __syncthreads();
    if (tid < 256) {
      const int l = tid % WAVE, i = tid / WAVE;
      float gs = 0.f, us = 0.f;
#pragma unroll
      for (int w = 0; w < FW; ++w) {
        gs += L.red[0][w][l][i];
        us += L.red[1][w][l][i];
      }
      const int s = l % 16, ch = c * 16 + 4 * (l / 16) + i;
      if ((mask >> s) & 1u) mb_putf(&A.mail.mid[((size_t)d * MAX_ROWS + s) * I + ch], silu(gs) * us, gd.tag);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- down
  // A down task (slot d, group grp) makes output rows grp * 448 .. + 448: 28 row tiles
  // of 16 x 4 128-k blocks = 112 weight tiles, 14 a wave. Wave pair p owns row tiles
  // 7p .. 7p + 6, i.e. tiles n = 0..27 of the pair in (row tile, k block) order: wave 2p
  // holds n = 0..13 (row tiles 0-2 whole, k blocks 0-1 of row tile 3), wave 2p + 1
  // n = 14..27; row tile 3's two halves meet in LDS.
  MONO_DEV void load_down(int T) {
    const int j = __builtin_amdgcn_readfirstlane(T - L.plan.n_act * NT);
    const int d = j / DN_GROUPS, grp = j % DN_GROUPS;
    const int e = __builtin_amdgcn_readfirstlane(L.plan.expert[d]);
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int n0 = (wv & 1) * 14, rt0 = grp * (DN_ROWS / 16) + (wv >> 1) * DN_PAIR;
    {  // block scales: scalar loads, apart from the vector queue
      const float* sb = A.s2 + (size_t)e * (H / 128) * IB;
#pragma unroll
      for (int i = 0; i < 14; ++i) {
        const int n = n0 + i, rt = rt0 + n / IB;
        SC[i] = ld_const_f32(sb + (rt / 8) * IB + n % IB);
      }
    }
    const uint8_t* wb = A.w2 + (size_t)e * H * I;
#pragma unroll
    for (int i = 0; i < 14; ++i) {
      const int n = n0 + i;
      W[i] = ld_shuf(wb, I / 32, rt0 + n / IB, n % IB, g, r);
    }
  }

  MONO_DEV bool down_compute(int T, f32x4 (&acc)[4]) {
    const int j = T - L.plan.n_act * NT;
    const int d = j / DN_GROUPS;
    const uint32_t mask = L.plan.rowmask[d];
    // wave w polls row w's mid (then row w + 8 when S > 8), lane l its 8 contiguous
    // channels 8l .. 8l + 7; 16 lanes make a 128-channel quantisation block
    constexpr int CG = I / WAVE;
    bool ok = true;
    for (int s = wave; s < S; s += FW) {  // wave-uniform trip count
      const bool in = (mask >> s) & 1u;
      const uint64_t* base = &A.mail.mid[((size_t)d * MAX_ROWS + s) * I + lane * CG];
      uint32_t v[CG];
#pragma unroll
      for (int q = 0; q < CG; ++q) v[q] = 0u;
      ok = poll_words<CG>([base](int q) { return base + q; }, v, in ? (1u << CG) - 1u : 0u, site0 + W_MID, gd) && ok;
      float m = 0.f;
#pragma unroll
      for (int q = 0; q < CG; ++q) m = fmaxf(m, fabsf(__uint_as_float(v[q])));
      const float am = group_max<128 / CG>(m);
      const bool nz = am > 0.f;
      const float inv = nz ? hw_rcp(am) * FP8_MAX : 1.0f;
      u32x2 packed;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float q4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) q4[q] = fminf(fmaxf(__uint_as_float(v[4 * h + q]) * inv, -FP8_MAX), FP8_MAX);
        packed[h] = fp8x4_pack(q4[0], q4[1], q4[2], q4[3]);
      }
      *reinterpret_cast<u32x2*>(&L.bq[s][lane * CG]) = packed;
      if ((lane % (128 / CG)) == 0)
        L.coef[s][lane / (128 / CG)] = in ? (nz ? am * (1.0f / FP8_MAX) : 1.0f) * route_weight(L.plan, d, s) : 0.f;
    }
    if (!block_all(ok)) return false;
    if (__builtin_amdgcn_readfirstlane(wave) & 1)
      down_mfma<1>(acc);
    else
      down_mfma<0>(acc);
    return true;
  }

  // acc[a]: the wave's a-th row tile (pair row tile a + 3 ODD)
  template <int ODD>
  MONO_DEV void down_mfma(f32x4 (&acc)[4]) {
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 14; ++i) {
      const int n = ODD * 14 + i, a = n / IB - 3 * ODD, kb = n % IB;
      const i32x8 bb = lds32(&L.bq[r][kb * 128 + g * 32]);
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 c = mfma_fp8(W[i], bb, zero);
      acc[a] += c * (SC[i] * L.coef[r][kb]);
    }
  }

  MONO_DEV void down_publish(int T, f32x4 (&acc)[4]) {
    const int j = T - L.plan.n_act * NT;
    const int d = j / DN_GROUPS, grp = j % DN_GROUPS;
    const uint32_t mask = L.plan.rowmask[d];
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const int odd = wv & 1, rt0 = grp * (DN_ROWS / 16) + (wv >> 1) * DN_PAIR;
    // the pair's row tile 3: the odd wave's k blocks 2-3 join the even wave's 0-1
    if (odd) L.red[0][wv][lane] = acc[0];
    __syncthreads();
    if (!odd) acc[3] += L.red[0][wv + 1][lane];
    if ((mask >> r) & 1u) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        if (odd && a == 0) continue;  // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int h = (rt0 + a + 3 * odd) * 16 + 4 * g + i;
          mb_putf(&A.mail.ypart[((size_t)d * MAX_ROWS + r) * H + h], acc[a][i], gd.tag);
        }
      }
    }
    __syncthreads();  // the next down task rewrites bq / coef / red
  }

  // ---------------------------------------------------------------- final
  MONO_DEV bool final_task(int T) {
    const int f = T - L.plan.n_act * (NT + DN_GROUPS);
    bool ok = true;
    // the thread's row and column re-derived from an opaque copy of its index: hoisted
    // out of the task loop, the row's offset would be held (and spilled) across tasks
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    if (t < S * FIN_ROWS) {
      const int s = t / FIN_ROWS, h = f * FIN_ROWS + t % FIN_ROWS;
      const uint64_t* base = &A.mail.ypart[(size_t)s * H + h];
      const int32_t* slots = L.plan.rowslot[s];
      uint32_t v[NSLOT];
      ok = poll_words<NSLOT>([base, slots](int k) { return base + (size_t)slots[k] * MAX_ROWS * H; }, v,
                             (1u << NSLOT) - 1u, site0 + W_YPART, gd);
      if (ok) {
        float y = 0.f;
#pragma unroll
        for (int k = 0; k < NSLOT; ++k) y += __uint_as_float(v[k]);
        const float res = bf16_bits_to_f32(A.a[(size_t)s * H + h]);
        A.out[(size_t)s * H + h] = f32_to_bf16_bits(res + y);
        if (A.y_out) A.y_out[(size_t)s * H + h] = y;
      }
    }
    return block_all(ok);
  }
};

// The kernel arguments of a launch (shared by k_moe_fp8 and the fused layer launch).
void fill_args(Args& a, const MoeFp8Args& g, const Mail& mail, const GuardArgs& guard) {
  a.a = static_cast<const uint16_t*>(g.a);
  a.g_post = static_cast<const uint16_t*>(g.g_post);
  a.w_router = static_cast<const uint16_t*>(g.w_router);
  a.bias = g.bias;
  a.w13 = static_cast<const uint8_t*>(g.w13);
  a.s13 = g.s13;
  a.w2 = static_cast<const uint8_t*>(g.w2);
  a.s2 = g.s2;
  a.out = static_cast<uint16_t*>(g.out);
  a.y_out = g.y;
  a.scores = g.scores;
  a.topk_ids = g.topk_ids;
  a.topk_w = g.topk_w;
  a.rows = g.rows;
  a.route_scale = g.route_scale;
  a.eps = g.eps;
  a.ticks = nullptr;
  a.mail = mail;
  a.guard = guard;
}

}  // namespace
}  // namespace moe
}  // namespace mono
