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
//   router   task t < 64 ceil(S / 2), on workgroups t, t + G, ...: experts 4 (t % 64) .. + 3
//            over rows 2 (t / 64) and 2 (t / 64) + 1, all of H in the task (the reference
//            gives a router task one row, kernel.py:4199-4330). The rows' RMSNorm
//            statistics (kernel.py:1367-1415), the bf16-rounded normed rows against the bf16
//            router rows (v_dot2 with f32 accumulation) -> sigmoid scores; and one 512-k
//            chunk of one of the rows quantised per 128 to FP8 (amax / 448 with a hardware
//            reciprocal, kernel.py:1440-1450) while it is in registers. Both go out
//            with device-coherent stores, then the task's done word (rdone)
//   gather   every workgroup, once every router task is done: the step's FP8 rows
//            straight into LDS (global_load_lds), their block scales, and each wave's
//            rows' scores into registers
//   route    every workgroup, wave w routing row w (and w + 8): top-8 by the f32 bits of
//            (score + bias) with lowest-id ties, weights = score / sum x route_scale
//            (kernel.py:1575-1629)
//   plan     the distinct experts of the step; slot 0 is the shared expert (weight 1),
//            slots 1.. the picked experts by ascending id
//   tasks    one round-robin list over the workgroups:
//            up     (slot, 16-channel tile): FP8 x FP8 MFMA 16x16x128 with the 128x128
//                   weight block scale x the activation block scale per 128-k, the 8
//                   waves splitting K, SiLU(gate) * up -> mailbox mid
//            down   (slot, 448 output rows): the slot's mid quantised per 128 to FP8 in
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
#include "row_ssq.h"
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
constexpr int RT_E = 4;              // experts a router task
constexpr int RT_S = 2;              // rows a router task
constexpr int RT_EG = E / RT_E;      // router tasks a row pair
constexpr int RCH = H / 512;         // 512-k chunks of a row: wave w holds chunks w and w + 8
constexpr int DN_ROWS = 448;         // output rows of a down task: 28 16-row tiles x 4 k blocks
constexpr int DN_GROUPS = H / DN_ROWS;
constexpr int DN_PAIR = DN_ROWS / 16 / (FW / 2);  // row tiles of a wave pair
constexpr int FIN_ROWS = 32;
constexpr int FIN_TASKS = H / FIN_ROWS;
constexpr int NSLOT = TOPK + 1;      // slots a row uses: the shared expert and its picks
static_assert(KB % FW == 0 && RCH > FW && RCH <= 2 * FW && E % RT_E == 0 && RT_EG >= RT_S * RCH, "tiling");
static_assert(H % (16 * WAVE) == 0 && E == 4 * WAVE && MAX_ROWS * KB <= 2 * FT, "the gather's copies");
static_assert(UP_KBW * 2 == 14 && DN_PAIR * IB == 2 * 14 && H % DN_ROWS == 0, "14 weight tiles a wave");
static_assert(IB == 4 && DN_PAIR == 7, "a wave pair's row tiles: 3 whole and half of one each");
static_assert(I == 8 * WAVE && MAX_ROWS <= 2 * FW, "a down task's wave reads one or two mid rows, 8 channels a lane");
static_assert(MAX_ROWS * FIN_ROWS <= FT, "a final task's thread owns one (row, output)");

// wait sites (guard error word = site + 1), offset by the Step's site0 in a fused
// launch; W_A: the attention block's output rows (fused launch only)
enum { W_ROUTER = 0, W_MID = 2, W_YPART = 3, W_A = 4 };

struct Lds {
  uint8_t xq[MAX_ROWS][H];          // FP8 normed rows
  float xs[MAX_ROWS][FW][8];        // their block scales: an up tile wave's UP_KBW, padded to 8
  union {
    f32x4 red[2][FW][WAVE];         // cross-wave sums of the expert tasks
    struct {
      float rss[FW][RT_S];            // a router task's sums of squares, a wave each
      float rlg[FW][4][RT_E * RT_S];  // its logits, a 16-lane row of a wave each (apart
                                      // from rss: fast waves write rlg while others read rss)
    } rt;
  };
  uint8_t bq[MAX_ROWS][I];          // a down task's FP8 mid
  float coef[MAX_ROWS][IB];         // its block scale x route weight
  PlanLds<E, TOPK> plan;
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
  // a later layer of the launch reads `out`: once its rows are stored, each final task
  // puts its 32 columns' sum of squares of every row as a tagged word
  // [MAX_ROWS][SSQ_TILES] (row_ssq.h; NULL: none)
  uint64_t* out_ssq;
  Mail mail;
  GuardArgs guard;
};

// Task kinds of the round-robin list
enum { K_NONE = 0, K_UP = 1, K_DOWN = 2, K_FINAL = 3 };

// the MoE's moments in a fused layer's tick row (its other words are the layer's): the
// attention block's rows seen, the first router task's statistics, the router tasks
// done, the gather done, the rows routed, the plan built
enum { T_PLAN = 4, T_A = 6, T_NORM = 7, T_ROUTER = 8, T_GATHER = 9, T_ROUTE = 10, T_ROW = 16 };

class Step {
 public:
  MONO_DEV Step(const Args& a, Lds& l) : A(a), L(l) {
    tid = thread_index();
    lane = tid % WAVE;
    wave = __builtin_amdgcn_readfirstlane(tid / WAVE);  // uniform: wave arithmetic stays scalar
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
    // the first router task's weights and the route's biases go out before anything waits
    const int n_rt = RT_EG * ((S + RT_S - 1) / RT_S);
    int t = block_index();
    u32x4 wr[RT_E][2], gr[2];
    if (t < n_rt) router_load(t, wr, gr);
    const f32x4 bias4 = *reinterpret_cast<const f32x4*>(A.bias + 4 * lane);
    const float bias[4] = {bias4[0], bias4[1], bias4[2], bias4[3]};
    if (a_done) {
      // every row of `a` is stored once its producers' done words carry the tag; `a` is
      // read with plain loads after that (no workgroup reads it earlier in the launch,
      // so no cache holds an older copy of its lines)
      const uint64_t* ad = done_copy(a_done);
      if (!hint_wait(n_a_done, [ad](int i) { return ad + i; }, site0 + W_A, gd)) return false;
      stamp(T_A);
    }
    for (; t < n_rt; t += G) {
      if (t != (int)block_index()) router_load(t, wr, gr);
      router_task(t, wr, gr);
    }
    stamp(T_ROUTER);
    f32x4 sc[2];
    if (!gather(n_rt, sc)) return false;
    stamp(T_GATHER);
    route_rows(sc, bias);
    stamp(T_ROUTE);
    __builtin_amdgcn_s_waitcnt(0);  // the gather's DMA into LDS (and the scale stores) done
    __syncthreads();
    // a shared-expert tile needs no plan: its loads go out before the plan is built
    if ((int)block_index() < NT) load_task(K_UP, block_index());
    plan_from_picks<E, TOPK, FT>(L.plan, S);
    stamp(T_PLAN);
    return tasks();
  }

  // NaN over the launch's output (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.out, (size_t)S * H, share); }

  // this workgroup's tick at MoE moment k (a fused layer with ticks only)
  MONO_DEV void stamp(int k) const {
    if (A.ticks && tid == 0) A.ticks[block_index() * T_ROW + k] = (int64_t)now_ticks();
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

  // ---------------------------------------------------------------- router
  // Router task t: experts RT_E (t % RT_EG) .. + RT_E - 1 over rows RT_S (t / RT_EG) ..;
  // wave w holds k chunks w and w + 8 (lane l: k = 512 j + 8 l .. + 7), the waves past
  // the last chunk load chunk RCH - 1 again and drop it.
  MONO_DEV static int chunk_k(int wv, int c, int ln) { return 512 * min(wv + FW * c, RCH - 1) + 8 * ln; }

  MONO_DEV void router_load(int t, u32x4 (&wr)[RT_E][2], u32x4 (&gr)[2]) {
    const int eg = t % RT_EG;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int k = chunk_k(wave, c, lane);
      gr[c] = ld_u32x4(A.g_post + k);
#pragma unroll
      for (int e = 0; e < RT_E; ++e) wr[e][c] = ld_nt_u32x4(A.w_router + (size_t)(RT_E * eg + e) * H + k);
    }
  }

  MONO_DEV void router_task(int t, const u32x4 (&wr)[RT_E][2], const u32x4 (&gr)[2]) {
    const int eg = t % RT_EG, s0 = (t / RT_EG) * RT_S;
    const bool two = wave + FW < RCH;  // wave-uniform: the wave's second chunk is a real one
    u32x4 av[RT_S][2];
#pragma unroll
    for (int si = 0; si < RT_S; ++si)
#pragma unroll
      for (int c = 0; c < 2; ++c) av[si][c] = ld_u32x4(A.a + (size_t)min(s0 + si, S - 1) * H + chunk_k(wave, c, lane));
    // sums of squares: the waves' in LDS, added in wave order
    float rstd[RT_S];
#pragma unroll
    for (int si = 0; si < RT_S; ++si) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bf16x2 v = as_bf16x2(av[si][c][q]);
          ss = (c == 0 || two) ? __builtin_amdgcn_fdot2_f32_bf16(v, v, ss, false) : ss;
        }
      ss = wave_sum(ss);
      if (lane == 0) L.rt.rss[wave][si] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int si = 0; si < RT_S; ++si) {
      float ss = 0.f;
#pragma unroll
      for (int w = 0; w < FW; ++w) ss += L.rt.rss[w][si];
      rstd[si] = hw_rsq(ss * (1.0f / H) + A.eps);
    }
    if (t == (int)block_index()) stamp(T_NORM);
    // the task's FP8 chunk: row s0 + cu / RCH, chunk cu % RCH (eg < RT_S RCH only)
    const int cu = eg < RT_S * RCH ? eg : -1;
    float acc[RT_E][RT_S];
#pragma unroll
    for (int e = 0; e < RT_E; ++e)
#pragma unroll
      for (int si = 0; si < RT_S; ++si) acc[e][si] = 0.f;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if (c == 1 && !two) break;
      float gf[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        gf[2 * q] = bf16_lo(gr[c][q]);
        gf[2 * q + 1] = bf16_hi(gr[c][q]);
      }
#pragma unroll
      for (int si = 0; si < RT_S; ++si) {
        // bf16(a * rstd * gamma): the router's operand (stage_x_rmsnorm, kernel.py:1367-1400)
        float x[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          x[2 * q] = bf16_lo(av[si][c][q]) * rstd[si] * gf[2 * q];
          x[2 * q + 1] = bf16_hi(av[si][c][q]) * rstd[si] * gf[2 * q + 1];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bf16x2 xb = as_bf16x2(pack_bf16x2(x[2 * q], x[2 * q + 1]));
#pragma unroll
          for (int e = 0; e < RT_E; ++e)
            acc[e][si] = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(wr[e][c][q]), xb, acc[e][si], false);
        }
        if (cu == si * RCH + wave + FW * c && s0 + si < S) quant_chunk(s0 + si, wave + FW * c, x);
      }
    }
    // logits: each 16-lane row's sum by DPP, then the 4 rows of the 8 waves in LDS, added
    // in a fixed order
#pragma unroll
    for (int e = 0; e < RT_E; ++e)
#pragma unroll
      for (int si = 0; si < RT_S; ++si) {
        const float v = row_reduce<16>(acc[e][si], OpAdd());
        if (r == 0) L.rt.rlg[wave][g][e * RT_S + si] = v;
      }
    __syncthreads();
    if (tid < RT_E * RT_S) {
      const int e = tid / RT_S, s = s0 + tid % RT_S;
      float lg = 0.f;
#pragma unroll
      for (int w = 0; w < FW; ++w)
#pragma unroll
        for (int q = 0; q < 4; ++q) lg += L.rt.rlg[w][q][tid];
      if (s < S) mb_putf(&A.mail.score[s * E + RT_E * eg + e], sigmoid(lg), gd.tag);
    }
    // the done word (for the FP8 rows) once every word of the task is stored
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    put_done(A.mail.rdone, t, gd.tag);
  }

  // Chunk j of row s (the wave's 8 normed values a lane, f32) per 128 to FP8: a lane's
  // 8 bytes and the 16-lane block's scale, device-coherent (read after the done word).
  MONO_DEV void quant_chunk(int s, int j, const float (&x)[8]) {
    float m = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[q]));
    const float amax = group_max<16>(m);
    const bool nz = amax > 0.f;
    const float inv = nz ? hw_rcp(amax) * FP8_MAX : 1.0f;
    uint32_t packed[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float q4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) q4[q] = fminf(fmaxf(x[4 * h + q] * inv, -FP8_MAX), FP8_MAX);
      packed[h] = fp8x4_pack(q4[0], q4[1], q4[2], q4[3]);
    }
    const u32x2 v = {packed[0], packed[1]};
    __builtin_amdgcn_raw_buffer_store_b64(v, coherent_rsrc(A.mail.xq, MAX_ROWS * H), s * H + 512 * j + 8 * lane, 0, SC1);
    if (r == 0) st_dev(&A.mail.xs[s * KB + 4 * j + g], nz ? amax * (1.0f / FP8_MAX) : 1.0f);
  }

  // ---------------------------------------------------------------- gather
  // Wave w's rows' scores (row w, and w + 8 when S > 8; lane l experts 4 l .. 4 l + 3)
  // polled as tagged words, and in the same pass (thread t < n_rt) every router task's
  // done word; then the step's FP8 rows into LDS by DMA (global_load_lds: no registers)
  // and their block scales. Plain cached loads for the rows: nothing reads these lines
  // in the launch before the done words, so no cache holds an older copy, and the
  // XCD's workgroups share its L2 for them. The caller waits for the DMA (s_waitcnt 0)
  // and meets the workgroup's barrier before reading the rows in LDS.
  MONO_DEV bool gather(int n_rt, f32x4 (&sc)[2]) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int s = wave + FW * k;
      uint32_t v[4] = {0u, 0u, 0u, 0u};
      if (s < S) {  // wave-uniform
        const uint64_t* row = A.mail.score + (size_t)s * E + 4 * lane;
        ok = poll_words<4>([row](int j) { return row + j; }, v, 0xfu, site0 + W_ROUTER, gd) && ok;
      }
      sc[k] = f32x4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
    }
    if (tid < n_rt) {
      uint32_t v;
      ok = poll_word(done_copy(A.mail.rdone) + tid, v, site0 + W_ROUTER, gd) && ok;
    }
    if (!block_all(ok)) return false;
    float xsv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) xsv[k] = A.mail.xs[min(tid + FT * k, S * KB - 1)];
    // 16 bytes a lane, a wave's 64 lanes one contiguous KB in both places
    const int n_xq = S * H / (16 * WAVE);  // wave-sized copies
    for (int c = wave; c < n_xq; c += FW)
      __builtin_amdgcn_global_load_lds(A.mail.xq + 16 * (WAVE * c + lane), &L.xq[0][0] + 16 * WAVE * c, 16, 0, 0);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = tid + FT * k, kb = i % KB;
      if (i < S * KB) L.xs[i / KB][kb / UP_KBW][kb % UP_KBW] = xsv[k];
    }
    return true;
  }

  // ---------------------------------------------------------------- route
  // Wave w routes row w (and w + 8) from its scores in registers: the top-TOPK of
  // (score + bias) -> the plan's picks; workgroup 0 also writes the debug outputs.
  MONO_DEV void route_rows(const f32x4 (&sc)[2], const float (&bias)[4]) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int s = wave + FW * k;
      if (s >= S) break;  // wave-uniform
      uint32_t key[4];
      int id[4];
      float raw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        id[i] = 4 * lane + i;
        raw[i] = sc[k][i];
        key[i] = radix_key(raw[i] + bias[i]);
      }
      if (A.scores && block_index() == 0) *reinterpret_cast<f32x4*>(&A.scores[s * E + 4 * lane]) = sc[k];
      float my_raw;  // lane k < TOPK: the raw score and id of pick k
      int my_id;
      wave_topk<TOPK>(key, id, raw, E, my_id, my_raw);
      // sum of the picks' raw scores in the butterfly order of lanes 0..7
      float tot = lane < TOPK ? my_raw : 0.f;
      tot = row_reduce<TOPK>(tot, OpAdd());
      const float w = my_raw * (hw_rcp(tot) * A.route_scale);
      if (lane < TOPK) {
        L.plan.pick_id[s][lane] = my_id;
        L.plan.pick_w[s][lane] = w;
        if (block_index() == 0) {
          if (A.topk_ids) A.topk_ids[s * TOPK + lane] = my_id;
          if (A.topk_w) A.topk_w[s * TOPK + lane] = w;
        }
      }
    }
  }

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
    int T = block_index();  // a shared-expert tile's loads (T < NT) went out before the plan
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
    static_assert(UP_H0 == 4 && UP_KBW <= 8, "a half's activation scales are one 16-byte read");
    const f32x4 xs4 = *reinterpret_cast<const f32x4*>(&L.xs[r][wave][4 * HALF]);
#pragma unroll
    for (int j = J0; j < J1; ++j) {
      const int kb = wave * UP_KBW + j;
      const i32x8 b = lds32(&L.xq[r][kb * 128 + g * 32]);
      const float xsj = xs4[j - J0];
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
    int t = thread_index();
    asm volatile("" : "+v"(t));
    float tile = 0.f;  // the row's sum of squares over this task's columns (out_ssq)
    if (t < S * FIN_ROWS) {
      const int s = t / FIN_ROWS, h = f * FIN_ROWS + t % FIN_ROWS;
      const uint64_t* base = &A.mail.ypart[(size_t)s * H + h];
      const int32_t* slots = L.plan.rowslot[s];
      uint32_t v[NSLOT];
      // every spin sweeps all missing words (no probe): the finals wait at the tail, when
      // the weight streams are over, and a probe's extra round trip is what costs there
      const auto at = [base, slots](int k) { return base + (size_t)slots[k] * MAX_ROWS * H; };
      ok = poll_words<NSLOT, decltype(at), false, false>(at, v,
                             (1u << NSLOT) - 1u, site0 + W_YPART, gd);
      if (ok) {
        float y = 0.f;
#pragma unroll
        for (int k = 0; k < NSLOT; ++k) y += __uint_as_float(v[k]);
        const float res = bf16_bits_to_f32(A.a[(size_t)s * H + h]);
        const uint16_t o = f32_to_bf16_bits(res + y);
        // write-through: a later layer of a multi-layer launch reads the rows
        __builtin_amdgcn_raw_buffer_store_b16(o, coherent_rsrc(A.out, (uint32_t)(S * H * 2)), (s * H + h) * 2, 0, SC1);
        if (A.y_out) A.y_out[(size_t)s * H + h] = y;
        if (A.out_ssq) tile = bf16_bits_to_f32(o);
      }
      static_assert(FIN_ROWS == SSQ_TILE && FIN_TASKS == SSQ_TILES, "a final task is a tile of the rows");
      if (A.out_ssq) tile = tile_sum_of_columns(tile);  // a row's 32 columns are a half wave
    }
    if (A.out_ssq) __builtin_amdgcn_s_waitcnt(0);  // the rows are stored before their tile sums
    const bool all = block_all(ok);
    if (all && A.out_ssq && t < S * FIN_ROWS && t % FIN_ROWS == 0)
      mb_put(&A.out_ssq[(size_t)(t / FIN_ROWS) * SSQ_TILES + f], __float_as_uint(tile), gd.tag);
    return all;
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
  a.out_ssq = nullptr;
  a.mail = mail;
  a.guard = guard;
}

}  // namespace
}  // namespace moe
}  // namespace mono
