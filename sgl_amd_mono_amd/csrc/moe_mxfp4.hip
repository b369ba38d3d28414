// MXFP4 (E2M1 + E8M0 per 32) routed + shared MoE of one decode step on gfx950 (A16W4:
// bf16 activations), as ONE persistent launch: one 512-thread workgroup per CU.
//
// The reference's A16W4 expert path (minimax_m31/a16w4.py:1-92 operands over AITER's
// (16, 16) layout; glm53/gfx950/kernel.py:966-970,1068-1085 ``unit_mxfp4_bf16``)
// behind a softmax router over given f32 logits. Work, in the order
// each workgroup walks it:
//   guard  the launch counter and error word (sync.h guard_fetch), then the logits and
//          the wave's slice of the rows (its MFMA B operands, kept in registers for the
//          whole launch), before any wait
//   route  every workgroup routes every row itself from the given logits: top-8 by the
//          f32 order (lowest id on ties), weights = softmax over the 8 picked logits;
//          no mailbox, so nothing waits before the first routed weights stream
//   plan   the step's distinct experts: slot 0 the shared expert (weight 1), slots 1..
//          the picked experts by ascending id
//   tasks  the workgroup's own stream, walked D tasks deep: each turn consumes a task's
//          weights (already in registers), issues the weight loads of the task D turns
//          later into the same registers, then publishes, so D - 1 to D tasks' weights
//          are always in flight (vector memory returns in order: a consume waits only
//          for the loads issued before it, and every task issues the same loads, so the
//          compiler's count of the later loads is exact). The stream:
//     up     (slot, 16-channel tile), tiles b, b + G, .. of the list of every slot's
//            tiles: a lane's 16 weight bytes are 32 E2M1 values of one row (row 16 rg +
//            l % 16, k 32 (l / 16) ..); v_cvt_scalef32_pk_bf16_fp4 widens them with the
//            row's E8M0 scale into four bf16 MFMA 16x16x32 operands against the
//            matching 8-k slices of the rows; the 8 waves split K. No barrier: each
//            wave leaves its partial sums in a ring of LDS buffers, and a complete
//            buffer is added up by the first wave that claims it (the waves ahead take
//            the reductions): mid = bf16(SiLU(gate) * up) -> mailbox mid
//     down   (slot, 256 output rows), a contiguous block of the list of every slot's
//            groups (so a workgroup stages its one or two slots' mids into LDS once),
//            blocks in reverse workgroup order (the workgroups that finish their up
//            tiles first take the slots whose mids are complete first): the same A16W4
//            MFMA, each wave its own 32 rows over the whole mid, x the route weight ->
//            mailbox ypart
//     final  (32 output rows) b, b + G, ..: the row's 9 slots summed in plan order ->
//            bf16 out
#include "common.h"
#include "moe_common.h"
#include "moe_ops.h"
#include "moe_plan.h"
#include "sync.h"

namespace mono {
namespace moe {

namespace {

constexpr int FT = 512;
constexpr int FW = FT / WAVE;

// BASELINE config 4 geometry
constexpr int H = 3072, E = 256, I = 384, TOPK = 8;
constexpr int HS = H / 128;          // 128-k steps of a hidden row
constexpr int IS = I / 128;          // 128-k steps of a mid row
constexpr int NT = I / 16;           // up tiles a slot
constexpr int UP_SW = HS / FW;       // k steps a wave of an up tile
constexpr int DN_ROWS = 256;
constexpr int DN_GROUPS = H / DN_ROWS;
constexpr int FIN_ROWS = 32;
constexpr int FIN_TASKS = H / FIN_ROWS;
constexpr int NSLOT = TOPK + 1;
constexpr int MSTRIDE = I + 8;       // bf16 a mid row in LDS
constexpr int MPT = MAX_ROWS * I / FT;  // mid words a thread polls when it stages a slot
constexpr int NW = 6;                // weight registers (u32x4) a task: up 2 x 3 steps, down 2 tiles x 3
constexpr int D = 2;                 // tasks a workgroup holds in flight (98 KB: enough for the
                                     // per-CU ingest with every CU streaming; a third sat in front
                                     // of the mid poll at the up -> down turn: 35.9 -> 34.2 us)
constexpr int RING = 4;              // LDS buffers of up partial sums
static_assert(HS % FW == 0 && I % 128 == 0 && I % MPT == 0 && MPT % 2 == 0, "tiling");
static_assert(2 * UP_SW == NW && 2 * IS == NW && DN_ROWS == FW * 32, "six 16-byte weight loads a lane a task");
static_assert(MAX_ROWS <= 2 * FW && MAX_ROWS == 16, "two rows a wave to route; an MFMA column a row");
static_assert(MAX_ROWS * FIN_ROWS <= FT, "a final task's thread owns one (row, output)");
// a workgroup's block of down groups holds at most ceil(slots * DN_GROUPS / grid) groups
// and spans at most two slots while that is at most DN_GROUPS + 1: grids of MIN_GRID
// workgroups and more (the launcher refuses smaller ones)
constexpr int MAX_SLOTS = MAX_ROWS * TOPK + 1;
constexpr int MIN_GRID = (MAX_SLOTS * DN_GROUPS + DN_GROUPS) / (DN_GROUPS + 1);
static_assert((MAX_SLOTS * DN_GROUPS + MIN_GRID - 1) / MIN_GRID <= DN_GROUPS + 1, "two slots a block");

// wait sites (guard error word = site + 1); W_RING: a wave waiting for an LDS buffer of
// up partial sums to be free, which ends once the other waves of its workgroup reach
// the same task (a failure there means a wave stopped early, which no path does)
enum { W_MID = 2, W_YPART = 3, W_RING = 4 };

struct Lds {
  f32x4 red[RING][2][FW][WAVE];     // up partial sums: (gate, up) of every wave
  uint32_t arrive[RING];            // waves that left their partial sums in a buffer
  uint32_t done[RING];              // uses of a buffer reduced so far
  uint32_t claim[RING];             // 1 while a wave reduces the buffer
  uint16_t mid[2][MAX_ROWS][MSTRIDE];  // the staged slots' bf16 mids (a block spans two)
  PlanLds<E, TOPK> plan;
};

struct Args {
  const uint16_t* x;
  const float* logits;
  const uint8_t* w13;
  const uint8_t* s13;
  const uint8_t* w2;
  const uint8_t* s2;
  uint16_t* out;
  float* y_out;
  int32_t* topk_ids;
  float* topk_w;
  int64_t* timeline;  // [tasks][4] or NULL
  int rows;
  Mail mail;
  GuardArgs guard;
};

// dword q of a lane's 16 weight bytes (8 E2M1 values) times 2^(e - 127) -> 8 bf16
MONO_DEV bf16x8 fp4x8_bf16(uint32_t w, float scale) {
  const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
  const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
  const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
  const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
  bf16x8 o;
  o[0] = a[0]; o[1] = a[1]; o[2] = b[0]; o[3] = b[1];
  o[4] = c[0]; o[5] = c[1]; o[6] = d[0]; o[7] = d[1];
  return o;
}

// acc += one 128-k step: weight word w (scale sc) against the lane's 4 B operands
MONO_DEV f32x4 a16w4_step(f32x4 acc, const u32x4& w, float sc, const bf16x8 (&b)[4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) acc = mfma_bf16(fp4x8_bf16(w[q], sc), b[q], acc);
  return acc;
}
MONO_DEV f32x4 a16w4_step(f32x4 acc, const u32x4& w, float sc, const uint16_t* brow) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
    acc = mfma_bf16(fp4x8_bf16(w[q], sc), *reinterpret_cast<const bf16x8*>(brow + 8 * q), acc);
  return acc;
}

enum { K_NONE = 0, K_UP = 1, K_DOWN = 2, K_FINAL = 3 };

// One task in flight: its place in the workgroup's stream, its list index (timeline
// row), kind, and the weight and scale words its loads fill.
struct Slot {
  u32x4 w[NW];
  uint32_t sw[NW];  // scale dwords: run h, step k in sw[3 h + k]
  int n, T, kind;
};

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

  MONO_DEV void run() {
    // the guard's two reads first, then the logits and the row slices: each wait below
    // waits only for what was issued before it (vector memory returns in order)
    const GuardFetch f = guard_fetch(A.guard);
    float lg[2][4];
    load_logits(lg);
    load_rows();
    if (!guard_begin(A.guard, gd, f)) return poison(true);
    if (!tasks(lg)) poison(false);
  }

  // NaN over the launch's output (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.out, (size_t)S * H, share); }

 private:
  const Args& A;
  Lds& L;
  Guard gd;
  int tid, lane, wave, g, r, G, S;
  uint64_t waited = 0;
  Slot P[D];
  bf16x8 xb[UP_SW][4];  // the wave's B operands: row r, k 128 (3 w + j) + 32 g + 8 q ..
  // the workgroup's stream: its up tiles, its block of down groups [v0, v0 + n_dn_b),
  // its final tasks
  int n_up = 0, n_dn = 0, n_up_b = 0, n_dn_b = 0, n_fin_b = 0, v0 = 0;

  // ---------------------------------------------------------------- rows
  // Lane (g, r)'s B operands for the wave's k steps, straight from the rows (row 0's
  // bytes for a lane past the step's rows, zeroed once they are back).
  MONO_DEV void load_rows() {
    const uint16_t* row = A.x + (size_t)(r < S ? r : 0) * H;  // every load issued
#pragma unroll
    for (int j = 0; j < UP_SW; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        xb[j][q] = __builtin_bit_cast(bf16x8, ld_u32x4(row + 128 * (wave * UP_SW + j) + 32 * g + 8 * q));
  }
  // Zero the lanes past the step's rows, then pass every operand through an empty
  // assembly statement: the compiler waits for the row loads there, before the first
  // weight loads are issued, and no longer counts them as pending inside the task loops
  // (where a wait of its own for them would also wait for the weights in flight).
  MONO_DEV void settle_rows() {
    const bool pad = r >= S;
#pragma unroll
    for (int j = 0; j < UP_SW; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x4 v = __builtin_bit_cast(u32x4, xb[j][q]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = pad ? 0u : v[e];
        __asm__ volatile("" : "+v"(v));
        xb[j][q] = __builtin_bit_cast(bf16x8, v);
      }
  }

  // ---------------------------------------------------------------- route
  // Wave w routes rows w and w + 8: lane l holds logits l + 64 i.
  MONO_DEV void load_logits(float (&lg)[2][4]) const {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int s = wave + FW * h;
#pragma unroll
      for (int i = 0; i < 4; ++i) lg[h][i] = A.logits[(size_t)(s < S ? s : 0) * E + lane + 64 * i];
    }
  }
  MONO_DEV void route(const float (&lg)[2][4]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int s = wave + FW * h;
      if (s >= S) continue;  // wave-uniform
      uint32_t key[4];
      int id[4];
      float raw[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        id[i] = lane + 64 * i;
        raw[i] = lg[h][i];
        key[i] = radix_key(raw[i]);
      }
      int my_id;
      float my_lg;
      wave_topk<TOPK>(key, id, raw, E, my_id, my_lg);
      // softmax over the picks: pick 0 holds the largest logit
      const float m = __shfl(my_lg, 0, WAVE);
      const float ex = lane < TOPK ? hw_exp(my_lg - m) : 0.f;
      float tot = ex;
#pragma unroll
      for (int o = 1; o < TOPK; o <<= 1) tot += __shfl_xor(tot, o, WAVE);
      const float w = ex / tot;
      if (lane < TOPK) {
        L.plan.pick_id[s][lane] = my_id;
        L.plan.pick_w[s][lane] = w;
        if (blockIdx.x == 0 && A.topk_ids) A.topk_ids[s * TOPK + lane] = my_id;
        if (blockIdx.x == 0 && A.topk_w) A.topk_w[s * TOPK + lane] = w;
      }
    }
  }

  // ---------------------------------------------------------------- the stream
  MONO_DEV void stream_init() {
    const int b = blockIdx.x;
    n_up = L.plan.n_act * NT;
    n_dn = L.plan.n_act * DN_GROUPS;
    n_up_b = b < n_up ? (n_up - b + G - 1) / G : 0;
    // down blocks in reverse workgroup order: the last workgroups finish their up tiles
    // first (the first ones hold the list's last round) and take the first slots, whose
    // mids are complete first
    const int rb = G - 1 - b;
    v0 = (int)((int64_t)rb * n_dn / G);
    n_dn_b = (int)((int64_t)(rb + 1) * n_dn / G) - v0;
    n_fin_b = b < FIN_TASKS ? (FIN_TASKS - b + G - 1) / G : 0;
  }
  // the workgroup's n-th task into slot p (kind, list index)
  MONO_DEV void task_of(Slot& p, int n) const {
    const int b = blockIdx.x;
    p.n = n;
    if (n < n_up_b) {
      p.kind = K_UP;
      p.T = b + n * G;
    } else if (n < n_up_b + n_dn_b) {
      p.kind = K_DOWN;
      p.T = n_up + v0 + (n - n_up_b);
    } else if (n < n_up_b + n_dn_b + n_fin_b) {
      p.kind = K_FINAL;
      p.T = n_up + n_dn + b + (n - n_up_b - n_dn_b) * G;
    } else {
      p.kind = K_NONE;
      p.T = 0;
    }
  }

  // Issue slot p's weight and scale loads for its task: the same six 16-byte weight
  // loads and two runs of three scale dwords for every kind (a task without weights
  // reads the shared expert's first bytes, cached, and ignores them), so the count of
  // loads between a task's issue and its use never depends on the kinds in between.
  //   up:   q = 2 j (gate rows 16 c..) and 2 j + 1 (up rows I + 16 c..), k step 3 w + j;
  //         scales: the gate row's and the up row's dwords of steps 3 w .. 3 w + 2
  //   down: q = 3 t + ks (rows (grp 256 + 32 w) + 16 t.., k step ks); scales: the two
  //         rows' dwords of steps 0 .. 2
  MONO_DEV void load_task(Slot& p) const {
    const uint8_t* wb = A.w13 + (size_t)E * (2 * I) * (H / 2);  // no weights: the shared expert's first bytes
    const uint8_t* sb = A.s13 + (size_t)E * (2 * I) * (H / 32);
    int rg[2] = {0, 0}, ks0 = 0, srow[2] = {0, 0}, sstride = 0, soff = 0, steps = 0;
    if (p.kind == K_UP) {
      const int d = p.T / NT, c = p.T % NT;
      const int e = d == 0 ? E : L.plan.expert[d];
      wb = A.w13 + (size_t)e * (2 * I) * (H / 2);
      sb = A.s13 + (size_t)e * (2 * I) * (H / 32);
      rg[0] = c;
      rg[1] = NT + c;
      ks0 = wave * UP_SW;
      srow[0] = 16 * c + r;
      srow[1] = I + 16 * c + r;
      sstride = H / 32;
      soff = 4 * ks0;
      steps = HS;
    } else if (p.kind == K_DOWN) {
      const int j = p.T - n_up;
      const int d = j / DN_GROUPS, grp = j % DN_GROUPS;
      const int e = L.plan.expert[d];
      wb = A.w2 + (size_t)e * H * (I / 2);
      sb = A.s2 + (size_t)e * H * (I / 32);
      rg[0] = (grp * DN_ROWS + wave * 32) / 16;
      rg[1] = rg[0] + 1;
      srow[0] = rg[0] * 16 + r;
      srow[1] = rg[1] * 16 + r;
      sstride = I / 32;
      steps = IS;
    }
    // weight q: up (rg[q & 1], ks0 + q / 2); down (rg[q / 3], q % 3)
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const bool up = p.kind == K_UP;
      const int g_q = up ? rg[q & 1] : rg[q / 3];
      const int k_q = up ? ks0 + q / 2 : q % 3;
      p.w[q] = ld_nt_u32x4(wb + ((size_t)g_q * steps + k_q) * 1024 + lane * 16);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t* sp = reinterpret_cast<const uint32_t*>(sb + (size_t)srow[h] * sstride + soff);
#pragma unroll
      for (int k = 0; k < 3; ++k) p.sw[3 * h + k] = sp[k];
    }
  }

  // Order this wave's LDS accesses across the point: no compiler motion across it, and
  // the wave's outstanding LDS operations complete (lgkmcnt 0) before it goes on. No
  // fence: a fence would also wait for the weight loads in flight (vmcnt 0).
  MONO_DEV static void lds_order() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // vmcnt 63 (no wait), expcnt 7, lgkmcnt 0
    __asm__ volatile("" ::: "memory");
  }

  // E8M0 byte `b` of a scale dword as an f32 power of two
  MONO_DEV static float scale_of(uint32_t word, int b) { return e8m0_to_f32((word >> (8 * b)) & 0xffu); }

  MONO_DEV bool tasks(const float (&lg)[2][4]) {
    route(lg);
    if (tid < RING) {
      L.arrive[tid] = 0u;
      L.done[tid] = 0u;
      L.claim[tid] = 0u;
    }
    plan_from_picks<E, TOPK, FT>(L.plan, S);  // its barriers also order the ring's zeros
    settle_rows();
    stream_init();
#pragma unroll
    for (int b = 0; b < D; ++b) {
      task_of(P[b], b);
      load_task(P[b]);
    }
    // the up tiles first (the stream holds every up tile before any other task), in a
    // loop of up turns alone: no turn in it waits on a mailbox or a barrier, so the
    // compiler's count of the loads issued since a slot's weights is exact and every
    // consume leaves the other slots' loads in flight
    int b = 0;
    bool ok = true;
    // rotations of two slots: the compiler's wait for the first slot consumed after the
    // loop header is conservative (it drains the loads in flight), so a pass of six
    // turns (three rotations) pays it once per six tasks (a straight-line first pass
    // measured no faster at 8 rows and slower at 16: the larger code)
    for (;;) {
      if (P[0].kind != K_UP) { b = 0; break; }
      ok &= up_turn<0>();
      if (P[1].kind != K_UP) { b = 1; break; }
      ok &= up_turn<1>();
      if (P[0].kind != K_UP) { b = 0; break; }
      ok &= up_turn<0>();
      if (P[1].kind != K_UP) { b = 1; break; }
      ok &= up_turn<1>();
      if (P[0].kind != K_UP) { b = 0; break; }
      ok &= up_turn<0>();
      if (P[1].kind != K_UP) { b = 1; break; }
      ok &= up_turn<1>();
    }
    if (!ok) gd.fail(W_RING);
    if (!block_all(ok)) return false;
    reduce_ready();  // every arrival is in: the uses still unreduced (claims keep each to one wave)
    // the down groups: the workgroup's block spans at most two slots; both mids are
    // staged into LDS at once (barriers and one poll), then down turns alone (no wait
    // in them)
    if (n_dn_b > 0) {
      const int d0 = v0 / DN_GROUPS, d1 = (v0 + n_dn_b - 1) / DN_GROUPS;
      if (!stage_mids(d0, d1)) return false;
      if (b == 1) {
        if (P[1].kind != K_DOWN) goto finals1;
        down_turn<1>(d0);
      }
      // three turns in straight-line code before the loop (a block holds at most three
      // groups up to 8 rows): at a loop header the waitcnt pass waits for every load in
      // flight (the copies between the unrolled rotations' registers), which here would
      // hold the next turn until the refills issued just before it are back
      if (P[0].kind != K_DOWN) goto finals0;
      down_turn<0>(d0);
      if (P[1].kind != K_DOWN) goto finals1;
      down_turn<1>(d0);
      if (P[0].kind != K_DOWN) goto finals0;
      down_turn<0>(d0);
      for (;;) {  // two rotations a pass, as the up loop
        if (P[1].kind != K_DOWN) goto finals1;
        down_turn<1>(d0);
        if (P[0].kind != K_DOWN) goto finals0;
        down_turn<0>(d0);
        if (P[1].kind != K_DOWN) goto finals1;
        down_turn<1>(d0);
        if (P[0].kind != K_DOWN) goto finals0;
        down_turn<0>(d0);
      }
    }
    if (b == 1) goto finals1;
    goto finals0;
    // the finals from the slot that holds the first of them
    int st;
  finals1:
    if ((st = turn<1>()) != 0) return st == 1;
  finals0:
    for (;;) {
      if ((st = turn<0>()) != 0) return st == 1;
      if ((st = turn<1>()) != 0) return st == 1;
    }
  }

  // One down turn on slot B (a down group of slot d0 or d0 + 1, both staged): consume,
  // refill, publish.
  template <int B>
  MONO_DEV void down_turn(int d0) {
    Slot& p = P[B];
    const uint64_t t0 = A.timeline ? now_ticks() : 0;
    const int d = (p.T - n_up) / DN_GROUPS;
    f32x4 acc[2];
    down_mfma(p, d, d - d0, acc);
    const int T = p.T;
    task_of(p, p.n + D);
    load_task(p);
    down_publish(T, acc);
    waited = 0;
    stamp(T, t0, K_DOWN);
  }

  // One turn of the up loop on slot B (an up task): consume, refill, publish. False if
  // the wave's wait for a free partial-sum buffer ran out of time.
  template <int B>
  MONO_DEV bool up_turn() {
    Slot& p = P[B];
    const uint64_t t0 = A.timeline ? now_ticks() : 0;
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = ag;
#pragma unroll
    for (int j = 0; j < UP_SW; ++j) {
      ag = a16w4_step(ag, p.w[2 * j], scale_of(p.sw[j], g), xb[j]);
      au = a16w4_step(au, p.w[2 * j + 1], scale_of(p.sw[3 + j], g), xb[j]);
    }
    const int T = p.T, n = p.n;
    task_of(p, n + D);
    load_task(p);
    const bool ok = up_publish(n, ag, au);
    waited = 0;
    stamp(T, t0, K_UP);
    return ok;
  }

  // One turn on slot B after the down groups (a final task): refill the slot with the
  // task D turns later, then run the final. 0: go on, 1: the stream is done, 2: a wait
  // failed.
  template <int B>
  MONO_DEV int turn() {
    static_assert(B < D, "slot");
    Slot& p = P[B];
    if (p.kind == K_NONE) return 1;
    const uint64_t t0 = A.timeline ? now_ticks() : 0;
    waited = 0;
    const int T = p.T;
    task_of(p, p.n + D);
    load_task(p);
    if (!final_task(T)) return 2;
    stamp(T, t0, K_FINAL);
    return 0;
  }

  // timeline row of task T: start, inputs-ready (0: waits on nothing) and end ticks,
  // workgroup << 8 | kind
  MONO_DEV void stamp(int T, uint64_t t0, int kind) const {
    if (A.timeline && tid == 0) {
      int64_t* tl = A.timeline + (size_t)T * 4;
      tl[0] = (int64_t)t0;
      tl[1] = (int64_t)waited;
      tl[2] = (int64_t)now_ticks();
      tl[3] = ((int64_t)blockIdx.x << 8) | kind;
    }
  }

  // ---------------------------------------------------------------- up
  // The wave's partial sums of its n-th up tile go to ring buffer n % RING (once the
  // buffer's previous use is reduced). A use whose 8 waves have all arrived is reduced by
  // whichever wave claims it first: every wave looks for complete buffers before each of
  // its arrivals and while it waits for a buffer, so the reductions (and their mid
  // stores) fall to the waves that are ahead, not to the last one to arrive. No
  // workgroup barrier: LDS serves one wave's operations in order, and each wave's writes
  // are complete (lgkmcnt 0) before its arrival is counted.
  MONO_DEV bool up_publish(int n, const f32x4& ag, const f32x4& au) {
    const int k = n % RING;
    const uint32_t use = (uint32_t)(n / RING);
    reduce_ready();  // before this wave's own arrival, so the last wave to arrive leaves its use to the next caller
    // the spin reads LDS and the clock only: no global memory operation in the up loop
    // but the weight loads and the mid stores, so the compiler's counts stay exact (the
    // caller records a failure after the loop)
    bool ok = true;
    while (__hip_atomic_load(&L.done[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != use) {
      if (now_ticks() > gd.deadline) {
        ok = false;
        break;
      }
      reduce_ready();
      __builtin_amdgcn_s_sleep(1);
    }
    lds_order();
    L.red[k][0][wave][lane] = ag;
    L.red[k][1][wave][lane] = au;
    lds_order();  // the partial sums are in LDS before the arrival is counted
    if (lane == 0) __hip_atomic_fetch_add(&L.arrive[k], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return ok;
  }

  // Reduce every ring buffer whose current use has all 8 arrivals and that this wave
  // claims (claim word 0 -> 1); the use's tile is the workgroup's up task done * RING + j.
  MONO_DEV void reduce_ready() {
#pragma unroll
    for (int j = 0; j < RING; ++j) {
      if (__hip_atomic_load(&L.arrive[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != FW) continue;
      uint32_t won = 0;
      if (lane == 0) {
        uint32_t expect = 0u;
        won = __hip_atomic_compare_exchange_strong(&L.claim[j], &expect, 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP) ? 1u : 0u;
      }
      if (!__builtin_amdgcn_readfirstlane((int)won)) continue;
      lds_order();
      // claimed: the use may have been reduced by another wave just before; reduce only
      // a buffer that is still complete (its use is then done[j])
      if (__hip_atomic_load(&L.arrive[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == FW)
        reduce_buffer(j, __hip_atomic_load(&L.done[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
      lds_order();
      if (lane == 0) __hip_atomic_store(&L.claim[j], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }

  // Buffer j's use `use` (all 8 partial sums in): lane l sums outputs (row l % 16,
  // channels 16 c + 4 (l / 16) + i), frees the buffer, and publishes the tile's mid.
  MONO_DEV void reduce_buffer(int j, uint32_t use) {
    const int T = (int)blockIdx.x + ((int)use * RING + j) * G;
    const int d = T / NT, c = T % NT;
    const uint32_t mask = d == 0 ? (1u << S) - 1u : L.plan.rowmask[d];
    f32x4 gs = {0.f, 0.f, 0.f, 0.f}, us = gs;
#pragma unroll
    for (int w = 0; w < FW; ++w) {
      gs += L.red[j][0][w][lane];
      us += L.red[j][1][w][lane];
    }
    lds_order();  // every read is back before the buffer is freed
    if (lane == 0) {
      __hip_atomic_store(&L.arrive[j], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_store(&L.done[j], use + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    const int s = lane % 16;
    if ((mask >> s) & 1u) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ch = c * 16 + 4 * (lane / 16) + i;
        // mid is staged as bf16 (glm53/gfx950/kernel.py:5111-5117)
        mb_putf(&A.mail.mid[((size_t)d * MAX_ROWS + s) * I + ch], bf16_round(silu(gs[i]) * us[i]), gd.tag);
      }
    }
    // the tile's done word, after its mid words: a hint for the down tasks' wait (their
    // poll of the tagged mid words stays the check)
    if (lane == 0) mb_put(&A.mail.mtile[T], 0u, gd.tag);
  }

  // ---------------------------------------------------------------- down
  // Stage the mids of slots d0 and d1 (= d0 or d0 + 1) into LDS: every thread of the
  // workgroup, one poll of both (the poll waits for every load issued before it, the
  // weights of the first down groups among them), then a barrier that publishes them.
  MONO_DEV bool stage_mids(int d0, int d1) {
    const int s = tid / (I / MPT), c0 = (tid % (I / MPT)) * MPT;
    const uint32_t m0 = L.plan.rowmask[d0], m1 = d1 != d0 ? L.plan.rowmask[d1] : 0u;
    const bool in0 = (m0 >> s) & 1u, in1 = (m1 >> s) & 1u;
    const uint64_t* b0 = &A.mail.mid[((size_t)d0 * MAX_ROWS + s) * I + c0];
    const uint64_t* b1 = &A.mail.mid[((size_t)d1 * MAX_ROWS + s) * I + c0];
    constexpr uint32_t ALL = (1u << MPT) - 1u;
    // first the slots' up tile done words (one a thread, the rest at the barrier): a
    // waiting workgroup then spins on at most 2 NT words instead of every mid word
    const uint64_t* tiles = &A.mail.mtile[(size_t)d0 * NT];
    if (!hint_wait((d1 - d0 + 1) * NT, [tiles](int i) { return tiles + i; }, W_MID, gd)) return false;
    uint32_t v[2 * MPT];
    const bool ok = poll_words<2 * MPT>([b0, b1](int q) { return q < MPT ? b0 + q : b1 + (q - MPT); }, v,
                                        (in0 ? ALL : 0u) | (in1 ? ALL << MPT : 0u), W_MID, gd);
    if (!block_all(ok)) return false;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const bool in = k == 0 ? in0 : in1;
#pragma unroll
      for (int q = 0; q < MPT; q += 2) {
        const float a = in ? __uint_as_float(v[k * MPT + q]) : 0.f, c = in ? __uint_as_float(v[k * MPT + q + 1]) : 0.f;
        *reinterpret_cast<uint32_t*>(&L.mid[k][s][c0 + q]) = pack_bf16x2(a, c);
      }
    }
    __syncthreads();
    if (A.timeline) waited = now_ticks();
    return true;
  }

  MONO_DEV void down_mfma(const Slot& p, int d, int k, f32x4 (&acc)[2]) const {
    const float wr = route_weight(L.plan, d, r);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < IS; ++ks)
        acc[t] = a16w4_step(acc[t], p.w[t * IS + ks], scale_of(p.sw[3 * t + ks], g), &L.mid[k][r][128 * ks + 32 * g]);
      acc[t] *= wr;
    }
  }

  MONO_DEV void down_publish(int T, const f32x4 (&acc)[2]) {
    const int j = T - n_up;
    const int d = j / DN_GROUPS, grp = j % DN_GROUPS;
    const uint32_t mask = L.plan.rowmask[d];
    if ((mask >> r) & 1u) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int h = grp * DN_ROWS + wave * 32 + t * 16 + 4 * g + i;
          mb_putf(&A.mail.ypart[((size_t)d * MAX_ROWS + r) * H + h], acc[t][i], gd.tag);
        }
    }
  }

  // ---------------------------------------------------------------- final
  MONO_DEV bool final_task(int T) {
    const int f = T - n_up - n_dn;
    bool ok = true;
    if (tid < S * FIN_ROWS) {
      const int s = tid / FIN_ROWS, h = f * FIN_ROWS + tid % FIN_ROWS;
      const uint64_t* base = &A.mail.ypart[(size_t)s * H + h];
      const int32_t* slots = L.plan.rowslot[s];
      uint32_t v[NSLOT];
      // every spin sweeps all missing words (no probe): the finals wait at the tail, when
      // the weight streams are over, and a probe's extra round trip is what costs there
      const auto at = [base, slots](int k) { return base + (size_t)slots[k] * MAX_ROWS * H; };
      ok = poll_words<NSLOT, decltype(at), false, false>(at, v,
                             (1u << NSLOT) - 1u, W_YPART, gd);
      if (ok) {
        float y = 0.f;
#pragma unroll
        for (int k = 0; k < NSLOT; ++k) y += __uint_as_float(v[k]);
        A.out[(size_t)s * H + h] = f32_to_bf16_bits(y);
        if (A.y_out) A.y_out[(size_t)s * H + h] = y;
      }
    }
    if (A.timeline) waited = now_ticks();
    return block_all(ok);
  }
};

__global__ __launch_bounds__(FT, 1) void k_moe_mxfp4(Args args) {
  __shared__ Lds lds;
  Step st(args, lds);
  st.run();
}

}  // namespace

bool moe_mxfp4_supported(const MoeGeom& geo) {
  return geo.hidden == H && geo.n_experts == E && geo.inter == I && geo.top_k == TOPK;
}

int moe_mxfp4_tasks(int max_act) { return max_act * (NT + DN_GROUPS) + FIN_TASKS; }

hipError_t moe_mxfp4_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_moe_mxfp4, FT, 0);
}

hipError_t moe_mxfp4_forward(const mono_moe_mxfp4_args& g, int grid, const Mail& mail, const GuardArgs& guard,
                             hipStream_t st) {
  if (grid < MIN_GRID || g.rows < 1 || g.rows > MAX_ROWS) return hipErrorInvalidConfiguration;
  Args a;
  a.x = static_cast<const uint16_t*>(g.x);
  a.logits = g.logits;
  a.w13 = static_cast<const uint8_t*>(g.w13);
  a.s13 = static_cast<const uint8_t*>(g.s13);
  a.w2 = static_cast<const uint8_t*>(g.w2);
  a.s2 = static_cast<const uint8_t*>(g.s2);
  a.out = static_cast<uint16_t*>(g.out);
  a.y_out = g.y;
  a.topk_ids = g.topk_ids;
  a.topk_w = g.topk_w;
  a.timeline = g.timeline;
  a.rows = g.rows;
  a.mail = mail;
  a.guard = guard;
  k_moe_mxfp4<<<grid, FT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace moe
}  // namespace mono
