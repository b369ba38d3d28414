// Sparse-attention phase of one decode step on gfx950, as ONE persistent launch (one
// 512-thread workgroup per CU). The reference runs it as stages of its decoder-layer
// launch: FP4 index scores (deepseek_v4/gfx950/kernels/stages/indexer.py:460-602 and
// the native-FP4 scorer deepseek_v41/gfx950/indexer/score_fp4.py:254-296), the exact
// top-2048 (indexer.py:604-802, glm53/gfx950/kernel.py:3000-3636), the sparse MLA
// split (kernel.py:3638-3973) and the split merge (kernel.py:3975-4123).
//
// Tasks, dealt round-robin over the workgroups in this order. A workgroup waits only on
// tasks earlier in the list or on its own top-k team, whose members share one round
// of the deal (teams never straddle a round), so the launch cannot deadlock while all
// workgroups are resident; every wait is guarded (sync.h):
//   score  (row, 1024 keys): 8 waves x 128 keys. The row's FP4 query (64 heads x 128
//          dims, E2M1 + E8M0 per 32) is the A operand and 16 keys of SGLang's FP4 index
//          plane the B operand of v_mfma_scale_f32_16x16x128_f8f6f4 with FP4 formats:
//          the plane's E8M0 bytes are the MFMA's per-lane B scales as they lie (a
//          lane's dword holds its key's scale for the page's four 16-key tiles).
//          score = sum_h w_h relu(q_h . k) -> mailbox score, and the task's histogram
//          of the keys' leading 8-bit digits -> mailbox hist1
//   topk   (row, member of a team of 16): the row's scores as order-preserving u32
//          keys, 2048 a member; an MSB-first 8-bit radix select of the 2048th largest
//          key: digit 1 from the chunk histograms, digit 2 from the sum of the members'
//          histograms (mailbox hist; a wave's most common digits go in as one atomic).
//          The keys sharing both digits with the threshold (mailbox cand) are ranked by
//          every member; a crowded bin (ties) takes digits 3 and 4 the same way as digit
//          2 and a stable compaction from the members' counts (mailbox cnt). Every key
//          above the threshold and the lowest positions equal to it, ascending -> cache
//          slots (page_table[p / 64] * 64 + p % 64) -> mailbox sel (glm53/check.py:100-117)
//   split  (row, 64 selected tokens): sub-tiles of 64 tokens gathered from the FP8
//          cache into LDS as they lie (q.k operands, widened exactly to bf16 in
//          registers) and, their value dims, widened and transposed (p.v operands); q
//          in registers; bf16 MFMA 16x16x32 for q.k (two waves a token tile, each half
//          of the 576 dims) and p.v, the per-token scale folded into the logit and the
//          probability, online softmax -> the split's partials (bf16, 32 KB in one
//          contiguous run) and (m, l), then its done word (mailbox sdone)
//   merge  (row, head): once every split of the row is done,
//          out = sum_j e^(m_j - M) acc_j / sum_j e^(m_j - M) l_j, bf16
#pragma once

#include "attn_ops.h"
#include "common.h"
#include "proj_ops.h"
#include "sync.h"

namespace mono {
namespace attn {

namespace {

#ifdef MONO_ATTN_LONG
constexpr bool kLongSplits = true;
constexpr int TMK = TEAM_LONG;  // members of a row's top-k team in this launch
#else
constexpr bool kLongSplits = false;
constexpr int TMK = TEAM;
#endif

constexpr int AT = 512;
constexpr int AW = AT / WAVE;
constexpr int KPM = MAX_CTX / TMK;           // keys a top-k team member owns
constexpr int KPT = KPM / AT;                // keys a thread of a member holds
constexpr int SUB = 64;                      // tokens a split sub-tile
constexpr int QK_HALF = DQK / 2;             // dims of q.k a wave sums (two waves a token tile)
constexpr int QK_STEPS = QK_HALF / 32;       // its bf16 MFMA k steps
// dwords a cached FP8 row in LDS: 16-byte aligned, and 20 banks (mod 64) from the next
// row, so the 16 rows of a q.k operand read fall on distinct banks
constexpr int KF_W = DQK / 4 + 4;
constexpr int VT_STRIDE = SUB + 8;           // bf16 a transposed value row (one dim) in LDS
constexpr int PF_STRIDE = SUB + 4;           // f32 a logit row in LDS
constexpr int PB_STRIDE = SUB + 8;           // bf16 a probability row in LDS
constexpr int ROPE_CH = (DQK - DV) / 16;     // 16-byte chunks of a row past the value dims
// 16-byte units a staged q row (one head): padded by one, so the 16 heads of a q
// operand read fall on distinct banks
constexpr int Q_UNITS = DQK / 8 + 1;
static_assert(DV / 16 * (SUB / 4) == AT && ROPE_CH * SUB <= AT && QK_HALF % 32 == 0, "gather tiling");
constexpr int KEYS_WAVE = CHUNK / AW;        // 128 keys a wave of a score task
constexpr int KTILES = KEYS_WAVE / 16;
constexpr float NEG_INF = -__builtin_huge_valf();
static_assert(KPM % AT == 0 && PAGE % KPT == 0 && TMK <= 16 && KPT % 4 == 0 && KEYS_WAVE % PAGE == 0 && SPLIT_MAX <= AT, "tiling");
static_assert(AT == NH * DV / 32, "tiling");

enum { W_SCORE = 0, W_SEL = 1, W_PART = 2, W_TEAM = 3 };



struct ScoreLds {
  uint32_t hist[256];  // the task's leading-digit histogram
};

struct TopkLds {
  int32_t pt[TOPK / PAGE];  // a short row's page table
  uint32_t hist[256];       // this member's digit histogram
  uint32_t tot[256];        // the team's
  uint32_t pre[256];        // the members' before this one
  uint32_t cu[CMAX];        // the team's threshold candidates, 0 past the last
  int32_t xw[TMK];          // the members' keys above the first digit
  int32_t cnt[TMK][2];      // the team's keys above / at the threshold
  uint32_t digit, uT;
  int32_t above, pre_above;
};

// Typed views of 16- and 8-byte units: an access through a pointer cast from a narrower
// element type is split by the compiler into 4-byte pairs (the cast's alignment is
// not known to it); through an array of the unit type it is one b128 / b64 access.
struct SplitLds {
  union {  // the sub-tile's cached rows as they lie (E4M3): q.k operands (8 dims a unit)
    u32x4 kf16[SUB][KF_W / 4];
    u32x2 kf8[SUB][KF_W / 2];
  };
  union {  // their first DV dims widened to bf16, a row a dim (vt_unit): p.v operands
    u32x4 vt16[DV][VT_STRIDE / 8];  // 8 tokens a unit
    u32x2 vt8[DV][VT_STRIDE / 4];   // 4 tokens a unit
    u32x4 q16[NH][Q_UNITS];         // before the first sub-tile: the row's q (bf16)
  };
  union {  // logits [dim half][head][token]: sums over dims [0, 288) and [288, 576)
    f32x4 pf4[2][NH][PF_STRIDE / 4];
    float pf[2][NH][PF_STRIDE];
  };
  union {  // probabilities times the tokens' scales, bf16 [head][token]
    u32x4 pb16[NH][PB_STRIDE / 8];
    u32x2 pb8[NH][PB_STRIDE / 4];
  };
  union {
    int32_t slot[SPLIT_MAX];
    i32x4 slot4[SPLIT_MAX / 4];
  };
  union {
    float kvs[SUB];
    f32x4 kvs4[SUB / 4];
  };
  float alpha[NH];
};
static_assert(KF_W % 4 == 0 && VT_STRIDE % 8 == 0 && PF_STRIDE % 4 == 0 && PB_STRIDE % 8 == 0, "16-byte units");
static_assert(NH * 16 == AT && SUB == 16 * 4, "softmax: a 16-lane row a head, 4 tokens a lane");

struct MergeLds {
  float w[8][SPLITS];  // each split's weight e^(m_j - M) a head of the task, 0 for an empty split
  float den[8];        // sum_j w_j l_j a head
};

struct Lds {
  union {
    ScoreLds sc;
    TopkLds t;
    SplitLds sp;
    MergeLds mg;
  } u;
  int32_t scan[AW];
};

struct Args {
  const uint8_t* iq;
  const uint8_t* iqs;
  const uint16_t* iw;
  const uint8_t* ikv;
  const uint8_t* iks;
  const uint16_t* q;
  const uint8_t* kv;
  const float* kv_scale;
  int kv_mask;  // slot & kv_mask indexes kv_scale (0: one scale for every row)
  const int32_t* pt;
  const int32_t* seq_lens;
  int pt_stride;
  int n_pages;
  uint16_t* out;
  int rows;
  float* scores;
  int32_t* topk;
  int64_t* timeline;
  float scale;
  // the front of the layer ran earlier in this launch: its replicated done words
  // (proj::Mail::fdone: FD_B + s row s's index key and head weights, FD_E + 8 s + j its
  // index query, FD_D + h head h of q), awaited at wait sites fsite and fsite + 1
  const uint64_t* fdone;
  int fsite;
  bool publish_out;  // a later stage of the launch reads `out`: each merge puts a done word
  // the row histograms: 1, two copies by launch parity (each launch clears its
  // successor's copy, the guard's flip words); 0, one copy that the launch's caller
  // clears once every reader is done (a layer of a multi-layer launch)
  int rowh_flip;
  Mail mail;
  GuardArgs guard;
};

MONO_DEV uint32_t radix_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// FP4 x FP4 16x16x128 with per-lane E8M0 scales; the B scale byte is picked by OPB.
template <int OPB>
MONO_DEV f32x4 mfma_fp4_opb(const u32x4& a, const u32x4& b, int sa, int sb) {
  const i32x8 A = {(int)a[0], (int)a[1], (int)a[2], (int)a[3], 0, 0, 0, 0};
  const i32x8 B = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, z, 4, 4, 0, sa, OPB, sb);
}

// E4M3 bytes 2 HW, 2 HW + 1 of a dword -> two bf16 as a dword, the first in the low half
// (exact: every E4M3 value is a bf16 value)
template <bool HW>
MONO_DEV uint32_t fp8x2_bf16(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HW));
}

// 8 E4M3 bytes (two dwords) -> 8 bf16: an MFMA operand of 8 consecutive k
MONO_DEV bf16x8 fp8x8_bf16x8(const u32x2& w) {
  const u32x4 o = {fp8x2_bf16<false>(w[0]), fp8x2_bf16<true>(w[0]), fp8x2_bf16<false>(w[1]), fp8x2_bf16<true>(w[1])};
  return __builtin_bit_cast(bf16x8, o);
}

class Step {
 public:
  MONO_DEV Step(const Args& a, Lds& l) : A(a), L(l) {
    tid = thread_index();
    lane = tid % WAVE;
    wave = tid / WAVE;
    g = lane / 16;
    r = lane % 16;
    G = gridDim.x;
    CH = a.mail.max_ctx / CHUNK;
  }

  MONO_DEV void run() {
    if (!begin()) return poison(true);
    if (!tasks()) poison(false);
  }

  // NaN over the launch's output (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.out, (size_t)A.rows * NH * DV, share); }

  // The launch's tag and deadline (false: the guard refused the launch or its epoch
  // scrub failed). The row histograms are the guard's flip accumulators: the launch
  // start clears the copy the next launch adds into.
  MONO_DEV bool begin() { return guard_begin(A.guard, gd); }

  // Run under a guard the caller set up (a layer of a multi-layer launch).
  MONO_DEV void adopt(const Guard& g) { gd = g; }

  MONO_DEV const Guard& guard() const { return gd; }

  // tasks in the list: score tasks padded to a multiple of TMK so no top-k team
  // straddles a round, then top-k members, splits, merges
  MONO_DEV int n_score() const { return (A.rows * CH + TMK - 1) / TMK * TMK; }
  // (a row's merges_of(rows) merges of 32 / merges_of(rows) heads each cover its NH heads)
  MONO_DEV int n_tasks() const { return n_score() + A.rows * TMK + A.rows * (splits_of(A.rows) + merges_of(A.rows)); }
  MONO_DEV int n_topk() const { return A.rows * TMK; }

  // This workgroup's tasks (false, workgroup-uniform: a wait failed).
  MONO_DEV bool tasks() {
    return tasks([] { return true; });
  }

  // The same with `between()` (workgroup-uniform; false: a wait failed) run after this
  // workgroup's top-k tasks and before its splits: the fused layer's deferred work.
  template <class Between>
  MONO_DEV bool tasks(Between&& between) {
    const int n_sc = n_score(), n_topk = A.rows * TMK;
    const int nsp = splits_of(A.rows);
    const int n_split = A.rows * nsp;
    if (!score_stage(block_index(), A.rows * CH)) return false;
    // a workgroup's list is ordered by stage: one loop a stage keeps each loop body to
    // one task kind (and its registers)
    int T = first_at_or_after(n_sc);
    for (; T < n_sc + n_topk; T += G) {
      const uint64_t t0 = now_ticks();
      const bool ok = topk_member((T - n_sc) / TMK, (T - n_sc) % TMK);
      stamp(T, t0, 1);
      if (!ok) return false;  // workgroup-uniform
    }
    if (!between()) return false;
    // one sub-tile a split up to LONG_ROWS rows (its loop over sub-tiles compiles away),
    // long splits above, in k_attn_long alone (MONO_ATTN_LONG): every other launch takes
    // at most LONG_ROWS rows.
    if (!kLongSplits || nsp == SPLITS) {
      for (T = first_at_or_after(n_sc + n_topk); T < n_sc + n_topk + n_split; T += G) {
        const uint64_t t0 = now_ticks();
        const int j = T - n_sc - n_topk;
        const bool ok = split_task<false>(j / SPLITS, j % SPLITS, SPLITS);
        stamp(T, t0, 2);
        if (!ok) return false;
      }
    } else {
      for (T = first_at_or_after(n_sc + n_topk); T < n_sc + n_topk + n_split; T += G) {
        const uint64_t t0 = now_ticks();
        const int j = T - n_sc - n_topk;
        const bool ok = split_task<true>(j / nsp, j % nsp, nsp);
        stamp(T, t0, 2);
        if (!ok) return false;
      }
    }
    if (!kLongSplits || nsp == SPLITS) return merges<SPLITS, 1>(n_sc + n_topk + n_split);
#ifdef MONO_ATTN_WIDE
    return nsp == 8 ? merges<8, 4>(n_sc + n_topk + n_split) : merges<4, 8>(n_sc + n_topk + n_split);
#else
    if (nsp == 8) return merges<8, 4>(n_sc + n_topk + n_split);
    return nsp == 5 ? merges<5, 8>(n_sc + n_topk + n_split) : merges<4, 8>(n_sc + n_topk + n_split);
#endif
  }

 private:
  const Args& A;
  Lds& L;
  Guard gd;
  int tid, lane, wave, g, r, G, CH;
  bool q_ready = false;  // the front's q has been awaited (a fused launch)
  uint64_t waited = 0;

  MONO_DEV int row_len(int s) const { return min(max(A.seq_lens[s], 0), A.mail.max_ctx); }
  // row s's leading-digit histogram of the launch with this tag: launches alternate
  // between two copies, and each launch clears the copy its successor uses
  MONO_DEV uint32_t* row_hist(uint32_t tag, int s) const {
    return A.mail.rowh + ((size_t)(A.rowh_flip ? tag & 1u : 0u) * A.mail.max_rows + s) * ROWH;
  }
  MONO_DEV int page_of(int s, int p) const {
    const int pg = A.pt[(size_t)s * A.pt_stride + p / PAGE];
    return min(max(pg, 0), A.n_pages - 1);
  }
  MONO_DEV int slot_of(int s, int p) const { return page_of(s, p) * PAGE + p % PAGE; }

  // this workgroup's first task at or after list index `at` (tasks are dealt round-robin)
  MONO_DEV int first_at_or_after(int at) const {
    const int b = block_index();
    return at <= b ? b : b + ((at - b + G - 1) / G) * G;
  }

  // timeline row of task T: start, inputs-ready and end ticks, workgroup << 8 | kind
  // (kind 0 score .. 3 merge); `waited` is 0 for a task that waits on nothing
  MONO_DEV void stamp(int T, uint64_t t0, int kind) const {
    if (A.timeline && tid == 0) {
      int64_t* tl = A.timeline + (size_t)T * 4;
      tl[0] = (int64_t)t0;
      tl[1] = (int64_t)waited;
      tl[2] = (int64_t)now_ticks();
      tl[3] = ((int64_t)block_index() << 8) | kind;
    }
  }
  MONO_DEV void mark_waited() { waited = now_ticks(); }

  // ---------------------------------------------------------------- score
  // A score task's operands for one wave: the row's FP4 query (head tile ht = heads
  // 16 ht ..), its head weights, and 128 keys = 2 pages = 8 tiles of 16 keys (lane
  // (g, r) holds chunk g of key 16 t + r) with their pages' E8M0 dwords.
  struct ScoreOps {
    int s, c, k0, n;
    u32x4 qa[IH / 16];
    int qsc[IH / 16];
    uint32_t w2[IH / 16][2];
    u32x4 kb[KTILES];
    uint32_t ks[KEYS_WAVE / PAGE];
    int pg[KEYS_WAVE / PAGE];
  };

  MONO_DEV void score_load(int T, ScoreOps& o) {
    score_where(T, o);
    if (o.k0 >= o.n) return;
    score_query(o);
    score_keys(o);
  }

  MONO_DEV void score_where(int T, ScoreOps& o) const {
    o.s = T / CH;
    o.c = T % CH;
    o.k0 = o.c * CHUNK + wave * KEYS_WAVE;
    o.n = row_len(o.s);
  }

  MONO_DEV void score_query(ScoreOps& o) const {
    if (o.k0 >= o.n) return;
#pragma unroll
    for (int ht = 0; ht < IH / 16; ++ht) {
      const size_t row = (size_t)o.s * IH + 16 * ht + r;
      o.qa[ht] = ld_u32x4(A.iq + row * (ID / 2) + g * 16);
      o.qsc[ht] = A.iqs[row * (ID / 32) + g];
      const u32x2 w4 = *reinterpret_cast<const u32x2*>(A.iw + (size_t)o.s * IH + 16 * ht + 4 * g);
      o.w2[ht][0] = w4[0];
      o.w2[ht][1] = w4[1];
    }
  }

  MONO_DEV void score_keys(ScoreOps& o) const {
    if (o.k0 >= o.n) return;
    int pg[KEYS_WAVE / PAGE];
#pragma unroll
    for (int i = 0; i < KEYS_WAVE / PAGE; ++i) pg[i] = page_of(o.s, o.k0 + i * PAGE);
#pragma unroll
    for (int kt = 0; kt < KTILES; ++kt)
      o.kb[kt] = ld_nt_u32x4(A.ikv + ((size_t)(pg[kt / 4] * 4 + g) * PAGE + (kt % 4) * 16 + r) * 16);
#pragma unroll
    for (int i = 0; i < KEYS_WAVE / PAGE; ++i)
      o.ks[i] = *reinterpret_cast<const uint32_t*>(A.iks + (size_t)(pg[i] * 4 + g) * PAGE + r * 4);
  }

  // The next task's query and page numbers; its key tiles and scales are issued from
  // inside the current task's compute (score_compute), so no wave sits in one 70 KB
  // issue burst (the CU's memory queue fills and stalls it) while it could compute.
  MONO_DEV void score_load_head(int T, ScoreOps& o) const {
    score_where(T, o);
    if (o.k0 >= o.n) return;
#pragma unroll
    for (int i = 0; i < KEYS_WAVE / PAGE; ++i) o.pg[i] = page_of(o.s, o.k0 + i * PAGE);
    score_query(o);  // after the page numbers: their wait does not wait for the query
  }
  MONO_DEV void score_key_tile(ScoreOps& o, int kt) const {
    o.kb[kt] = ld_nt_u32x4(A.ikv + ((size_t)(o.pg[kt / 4] * 4 + g) * PAGE + (kt % 4) * 16 + r) * 16);
  }
  MONO_DEV void score_key_scales(ScoreOps& o) const {
#pragma unroll
    for (int i = 0; i < KEYS_WAVE / PAGE; ++i)
      o.ks[i] = *reinterpret_cast<const uint32_t*>(A.iks + (size_t)(o.pg[i] * 4 + g) * PAGE + r * 4);
  }

  // key tile kt's logits against the four head tiles of the query
  MONO_DEV static void score_mfmas(const ScoreOps& o, int kt, f32x4 (&d)[IH / 16]) {
#pragma unroll
    for (int ht = 0; ht < IH / 16; ++ht) {
      switch (kt % 4) {
        case 0: d[ht] = mfma_fp4_opb<0>(o.qa[ht], o.kb[kt], o.qsc[ht], (int)o.ks[kt / 4]); break;
        case 1: d[ht] = mfma_fp4_opb<1>(o.qa[ht], o.kb[kt], o.qsc[ht], (int)o.ks[kt / 4]); break;
        case 2: d[ht] = mfma_fp4_opb<2>(o.qa[ht], o.kb[kt], o.qsc[ht], (int)o.ks[kt / 4]); break;
        default: d[ht] = mfma_fp4_opb<3>(o.qa[ht], o.kb[kt], o.qsc[ht], (int)o.ks[kt / 4]); break;
      }
    }
  }

  // The wave's 128 scores -> mailbox score (lane (g, r) ends with keys k0 + 16 g + r and
  // k0 + 64 + 16 g + r, so each store covers 64 consecutive positions), then the task's
  // histogram of their leading key digits, added into the row's histogram (the top-k's
  // first radix pass) before the chunk is marked done (mailbox cdone). Every wave
  // reaches the barriers; a wave past the row computes nothing.
  MONO_DEV void score_compute(const ScoreOps& o, ScoreOps& nx, bool more) {
    const bool live = o.k0 < o.n;  // wave-uniform
    // the next task's key tiles: two an iteration over this task's tiles 2-5 (its page
    // numbers, loaded first, have landed by then; tiles 4-7 measured 2.6 us slower at 48
    // rows, their loads still in flight at the task's acknowledgement wait)
    const bool nx_live = more && nx.k0 < nx.n;  // wave-uniform
    float sc[2] = {0.f, 0.f};
    if (live) {
      float wv[IH / 16][4];
#pragma unroll
      for (int ht = 0; ht < IH / 16; ++ht) {
        wv[ht][0] = bf16_lo(o.w2[ht][0]);
        wv[ht][1] = bf16_hi(o.w2[ht][0]);
        wv[ht][2] = bf16_lo(o.w2[ht][1]);
        wv[ht][3] = bf16_hi(o.w2[ht][1]);
      }
      // a key tile's four head-tile MFMAs are issued together and the next tile's before
      // this tile's results are consumed, so no MFMA's latency sits in front of its use
      // (32 MFMAs a wave, each consumed at once, cost ~1 us of exposed latency)
      f32x4 d[2][IH / 16];
      score_mfmas(o, 0, d[0]);
#pragma unroll
      for (int kt = 0; kt < KTILES; ++kt) {
        if (kt + 1 < KTILES) score_mfmas(o, kt + 1, d[(kt + 1) % 2]);
        static_assert(KTILES % 2 == 0, "two tiles an iteration");
        if (nx_live && kt >= 2 && kt < 2 + KTILES / 2) {
          score_key_tile(nx, 2 * kt - 4);
          score_key_tile(nx, 2 * kt - 3);
        }
        float part = 0.f;
#pragma unroll
        for (int ht = 0; ht < IH / 16; ++ht)
#pragma unroll
          for (int i = 0; i < 4; ++i) part += wv[ht][i] * (d[kt % 2][ht][i] > 0.f ? d[kt % 2][ht][i] : 0.f);
        part += __shfl_xor(part, 16, WAVE);  // every lane group now holds key 16 kt + r's sum
        part += __shfl_xor(part, 32, WAVE);
        if (kt % 4 == g) sc[kt / 4] = part;
      }
    } else if (nx_live) {
#pragma unroll
      for (int kt = 0; kt < KTILES; ++kt) score_key_tile(nx, kt);
    }
    if (nx_live) score_key_scales(nx);
    bool kl[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int pos = o.k0 + 64 * i + 16 * g + r;
      kl[i] = live && pos < o.n;
      if (kl[i]) {
        __hip_atomic_store(&A.mail.score[(size_t)o.s * A.mail.max_ctx + pos], __float_as_uint(sc[i]), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        if (A.scores) A.scores[(size_t)o.s * A.mail.max_ctx + pos] = sc[i];
      }
    }
    uint32_t* hist = L.u.sc.hist;
    __syncthreads();  // the previous task's histogram is added and cleared
#pragma unroll
    for (int i = 0; i < 2; ++i) hist_add(hist, kl[i], radix_key(sc[i]) >> 24);
    __syncthreads();
    if (o.c * CHUNK < o.n) {  // workgroup-uniform
      uint32_t* rh = row_hist(gd.tag, o.s);
      if (tid < 256 && hist[tid] != 0u)
        __hip_atomic_fetch_add(&rh[tid], hist[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);  // every add is performed before the chunk is marked done
      __syncthreads();
      if (tid == 0) mb_put(&A.mail.cdone[(size_t)o.s * CH + o.c], 0u, gd.tag);
    }
    if (tid < 256) hist[tid] = 0u;
  }

  // The workgroup's score tasks T0, T0 + G, ... < n_score, each task's loads issued
  // before the previous task computes.
  MONO_DEV bool score_stage(int T0, int n_score) {
    if (T0 >= n_score) return true;
    if (tid < 256) L.u.sc.hist[tid] = 0u;
    ScoreOps cur, nxt;
    if (A.fdone) {
      // the front of this launch writes each row's index query, head weights and new
      // key: the first task's keys stream before the wait, except a wave's whose 128
      // keys may hold a key written in this launch (the row's last `rows` positions: its
      // own new key and, for the rows of a verify chain, those of the chain's earlier
      // rows), then every row's front outputs are awaited
      score_where(T0, cur);
      const bool fresh = cur.k0 < cur.n && cur.k0 + KEYS_WAVE > cur.n - A.rows;  // wave-uniform
      if (!fresh) score_keys(cur);
      const uint64_t* fd = done_copy(A.fdone);
      const int nr = A.rows;
      if (!hint_wait(nr * (1 + IH / 8), [fd, nr](int i) { return fd + (i < nr ? proj::FD_B + i : proj::FD_E + i - nr); },
                     A.fsite, gd))
        return false;
      if (fresh) score_keys(cur);
      score_query(cur);
    } else {
      score_load(T0, cur);
    }
    for (int T = T0; T < n_score; T += G) {
      const uint64_t t0 = now_ticks();
      const bool more = T + G < n_score;
      if (more) score_load_head(T + G, nxt);
      score_compute(cur, nxt, more);
      stamp(T, t0, 0);
      if (more) cur = nxt;
    }
    __syncthreads();  // the top-k tasks reuse the LDS
    return true;
  }

  // ---------------------------------------------------------------- top-k
  // exclusive prefix sum of v over the workgroup (a full barrier)
  MONO_DEV int block_excl_scan(int v) {
    const int incl = wave_incl_scan(v);
    if (lane == WAVE - 1) L.scan[wave] = incl;
    __syncthreads();
    int before = 0;
#pragma unroll
    for (int w = 0; w < AW; ++w) before += w < wave ? L.scan[w] : 0;
    __syncthreads();
    return before + incl - v;
  }

  MONO_DEV void publish_sel(int s, int j, int slot) {
    mb_put(&A.mail.sel[(size_t)s * TOPK + j], (uint32_t)slot, gd.tag);
    if (A.topk) A.topk[(size_t)s * TOPK + j] = slot;
  }

  // Count a key digit into an LDS histogram: the lanes sharing the first live lane's
  // digit (scores share sign and exponent bits, so leading digits pile onto few bins)
  // as one atomic, every other live lane as a plain atomic (the LDS resolves spread
  // addresses quickly; a wave of same-address atomics would serialize).
  MONO_DEV void hist_add(uint32_t* hist, bool live, uint32_t d) {
    const uint64_t act = __ballot(live);
    if (act == 0) return;  // wave-uniform
    if (__popcll(act) <= 16) {  // few live lanes (wave-uniform): plain atomics, no scalar chain
      if (live) atomicAdd(&hist[d], 1u);
      return;
    }
    const int first = __builtin_ctzll(act);
    const uint32_t d0 = (uint32_t)__builtin_amdgcn_readlane((int)d, first);
    const uint64_t same = __ballot(live && d == d0);
    if (live && d != d0) atomicAdd(&hist[d], 1u);
    if (lane == first) atomicAdd(&hist[d0], (uint32_t)__popcll(same));
  }

  // Pick the next digit from a 256-bin histogram (wave 0): the highest digit d with
  // (keys above d) < need <= (keys above d) + hist[d] -> K.digit, K.above; with `pre`,
  // also K.pre_above = the sum of pre over the bins above d.
  MONO_DEV void pick_digit(TopkLds& K, const uint32_t* hist, int need, const uint32_t* pre) {
    if (wave != 0) return;
    int c[4], tot = 0;  // lane l holds bins 255 - 4l .. 252 - 4l, highest first
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = (int)hist[255 - 4 * lane - j];
      tot += c[j];
    }
    const int incl = wave_incl_scan(tot);
    const int excl = incl - tot;
    const bool mine = excl < need && need <= incl;
    int dg = 0, ab = 0, run = excl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (mine && dg == 0 && run + c[j] >= need) {
        dg = 256 + 255 - 4 * lane - j;  // + 256: found
        ab = run;
      }
      run += c[j];
    }
    const uint64_t who = __ballot(mine);
    const int src = who ? __ffsll((long long)who) - 1 : 0;
    dg = __builtin_amdgcn_readlane(dg, src) & 0xff;
    ab = __builtin_amdgcn_readlane(ab, src);
    if (pre) {
      int x = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) x += 255 - 4 * lane - j > dg ? (int)pre[255 - 4 * lane - j] : 0;
      x = wave_sum_i(x);
      if (lane == 0) K.pre_above = x;
    }
    if (lane == 0) {
      K.digit = (uint32_t)dg;
      K.above = ab;
    }
  }

  // One exchanged radix pass: member m's histogram of the digit at `shift` over its keys
  // matching prefix under mask -> mailbox hist as 128 words of two 16-bit bins (a member
  // holds at most KPM keys), plus `count` as word 128 when count >= 0; the team's sum
  // -> K.tot, the sum over the members before m -> K.pre, the members' counts -> K.xw.
  // Workgroup-uniform result.
  MONO_DEV bool exchange_hist(int s, int m, int pass, const uint32_t (&key)[KPT], int cnt, uint32_t prefix,
                              uint32_t mask, int shift, int count) {
    static_assert(KPM < 65536, "16-bit bins");
    TopkLds& K = L.u.t;
    if (tid < 256) K.hist[tid] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < KPT; ++q) hist_add(K.hist, q < cnt && (key[q] & mask) == prefix, (key[q] >> shift) & 0xffu);
    __syncthreads();
    uint64_t* hb = &A.mail.hist[((size_t)s * PASSES + pass) * TMK * HW];
    bool ok = true;
    if (tid < 128) {
      mb_put(&hb[m * HW + tid], K.hist[2 * tid] | (K.hist[2 * tid + 1] << 16), gd.tag);
      uint32_t v[TMK];
      const uint64_t* col = hb + tid;
      const auto at = [col](int j) { return col + j * HW; };
      ok = poll_words<TMK, decltype(at), false, false>(at, v, (1u << TMK) - 1u, W_TEAM, gd);
      uint32_t t = 0, p = 0;  // two 16-bit sums side by side (at most TMK KPM keys)
#pragma unroll
      for (int j = 0; j < TMK; ++j) {
        t += v[j];
        p += j < m ? v[j] : 0u;
      }
      K.tot[2 * tid] = t & 0xffffu;
      K.tot[2 * tid + 1] = t >> 16;
      K.pre[2 * tid] = p & 0xffffu;
      K.pre[2 * tid + 1] = p >> 16;
    } else if (count >= 0 && tid < 128 + TMK) {
      const int j = tid - 128;
      if (j == m) mb_put(&hb[m * HW + 128], (uint32_t)count, gd.tag);
      uint32_t v = 0;
      ok = poll_word(&hb[j * HW + 128], v, W_TEAM, gd);
      K.xw[j] = (int)v;
    }
    return block_all(ok);
  }

  // a threshold candidate's rank word: larger first = score desc, position asc (the
  // candidates share their keys' upper 16 bits)
  MONO_DEV static uint32_t cand_word(uint32_t key, int pos) { return (key << 16) | (uint32_t)(0x7fff - pos); }

  // Member m of row s's top-k team. The team selects the exact top-TOPK of the row
  // (score desc, position asc) -> cache slots, ascending. Member m owns positions
  // [m KPM, (m + 1) KPM), KPT of them in each thread's registers. An MSB-first 8-bit
  // radix select of the threshold key: digit 1 from the score tasks' chunk histograms,
  // digit 2 from the members' exchanged histograms. The keys left sharing both digits
  // with the threshold (the candidates, few unless scores tie) are exchanged as (low
  // key bits, position) and every member ranks them all; a crowded threshold bin
  // instead takes digits 3 and 4 the same way as digit 2 and then the members' counts
  // above / at the threshold (mailbox cnt). Each member writes its selected slots at
  // its offset in position order.
  MONO_DEV bool topk_member(int s, int m) {
    TopkLds& K = L.u.t;
    const int n = row_len(s);
    if (n <= TOPK) {  // every key is selected; no score is needed
      if (m == 0) {
        for (int i = tid; i < TOPK / PAGE; i += AT) K.pt[i] = i * PAGE < n ? page_of(s, i * PAGE) : 0;
        __syncthreads();
        for (int j = tid; j < TOPK; j += AT) publish_sel(s, j, j < n ? K.pt[j / PAGE] * PAGE + j % PAGE : -1);
        __syncthreads();  // the next task may rewrite the LDS page table
      }
      return true;
    }
    const int p0 = m * KPM + tid * KPT;
    const int cnt = min(max(n - p0, 0), KPT);
    const int page = cnt > 0 ? page_of(s, p0) : 0;  // a thread's keys share one page
    bool ok = true;
    // thread c < (scored chunks) waits for chunk c's scores and counts (done word)
    if (tid < (n + CHUNK - 1) / CHUNK) {
      uint32_t v;
      ok = poll_word(&A.mail.cdone[(size_t)s * CH + tid], v, W_SCORE, gd);
    }
    if (!block_all(ok)) return false;
    // then a thread's KPT consecutive scores: 16-byte device-coherent loads (the buffer
    // reads zeros past the row), and the row histogram
    uint32_t key[KPT];
    {
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(A.mail.score + (size_t)s * A.mail.max_ctx, 0, n * 4, BUF_DWORD3);
      u32x4 k4[KPT / 4];
#pragma unroll
      for (int i = 0; i < KPT / 4; ++i)
        k4[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (p0 + 4 * i) * 4, 0, SC1));
#pragma unroll
      for (int q = 0; q < KPT; ++q) key[q] = radix_key(__uint_as_float(k4[q / 4][q % 4]));
    }
    if (tid < 256) K.tot[tid] = ld_agent_u32(&row_hist(gd.tag, s)[tid]);
    __syncthreads();
    mark_waited();
    pick_digit(K, K.tot, TOPK, nullptr);
    __syncthreads();
    int need = TOPK - K.above;
    const uint32_t d1 = K.digit;
    uint32_t prefix = d1 << 24, mask = 0xff000000u;
    int above1 = 0;  // this member's keys above digit 1
#pragma unroll
    for (int q = 0; q < KPT; ++q) above1 += (q < cnt && (key[q] >> 24) > d1) ? 1 : 0;
    above1 = wave_sum_i(above1);
    if (lane == 0) L.scan[wave] = above1;
    __syncthreads();
    above1 = 0;
#pragma unroll
    for (int w = 0; w < AW; ++w) above1 += L.scan[w];
    if (!exchange_hist(s, m, 1, key, cnt, prefix, mask, 16, above1)) return false;
    pick_digit(K, K.tot, need, K.pre);
    __syncthreads();
    need -= K.above;
    int above_before = K.pre_above;  // the earlier members' keys above the threshold's upper 16 bits
    // a fixed trip count: the LDS reads issue together (a loop to m waits on each one;
    // 0.4-0.5 us of the top-k at 1 and 8 rows)
#pragma unroll
    for (int j = 0; j < TMK; ++j) above_before += j < m ? K.xw[j] : 0;
    prefix |= K.digit << 16;
    mask |= 0x00ff0000u;
    const int n_cand = (int)K.tot[K.digit], cand_before = (int)K.pre[K.digit];
    int sel_before;
    uint32_t uT = 0;  // candidates: the lowest selected rank word
    bool cand = n_cand <= CMAX;  // team-uniform
    if (cand) {
      const uint32_t P16 = prefix >> 16;
      int c_my = 0;
#pragma unroll
      for (int q = 0; q < KPT; ++q) c_my += (q < cnt && (key[q] >> 16) == P16) ? 1 : 0;
      int idx = cand_before + block_excl_scan(c_my);
      uint64_t* cb = &A.mail.cand[(size_t)s * CMAX];
#pragma unroll
      for (int q = 0; q < KPT; ++q)
        if (q < cnt && (key[q] >> 16) == P16) mb_put(&cb[idx++], cand_word(key[q], p0 + q), gd.tag);
      static_assert(CMAX == AT, "a thread a candidate");
      uint32_t u = 0;
      ok = true;
      if (tid < n_cand) ok = poll_word(&cb[tid], u, W_TEAM, gd);
      K.cu[tid] = u;
      if (!block_all(ok)) return false;
      if (wave * WAVE < n_cand) {  // wave-uniform
        // candidates ranked before this thread's, 32 a step with the step's LDS reads issued
        // together (K.cu holds zeros past the last candidate, and a step starting below
        // n_cand <= CMAX ends inside K.cu)
        static_assert(CMAX % 32 == 0, "whole steps");
        int rank = 0;
        for (int j = 0; j < n_cand; j += 32) {
          u32x4 x[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = *reinterpret_cast<const u32x4*>(&K.cu[j + 4 * i]);
#pragma unroll
          for (int i = 0; i < 8; ++i)
            rank += (x[i][0] > u ? 1 : 0) + (x[i][1] > u ? 1 : 0) + (x[i][2] > u ? 1 : 0) + (x[i][3] > u ? 1 : 0);
        }
        if (tid < n_cand && rank == need - 1) K.uT = u;
      }
      __syncthreads();
      uT = K.uT;
      sel_before = above_before + __syncthreads_count(tid < cand_before && u >= uT);
    } else {
#pragma unroll 1
      for (int pass = 2; pass < PASSES; ++pass) {
        const int shift = 24 - 8 * pass;
        __syncthreads();  // K.digit and K.tot are read
        if (!exchange_hist(s, m, pass, key, cnt, prefix, mask, shift, -1)) return false;
        pick_digit(K, K.tot, need, nullptr);
        __syncthreads();
        need -= K.above;
        prefix |= K.digit << shift;
        mask |= 0xffu << shift;
      }
      // the team's counts above / at T, then this member's offset
      int c_gt = 0, c_eq = 0;
#pragma unroll
      for (int q = 0; q < KPT; ++q) {
        c_gt += (q < cnt && key[q] > prefix) ? 1 : 0;
        c_eq += (q < cnt && key[q] == prefix) ? 1 : 0;
      }
      const int gt_in = block_excl_scan(c_gt), eq_in = block_excl_scan(c_eq);
      if (tid == AT - 1) {  // the last thread's inclusive sums are the member's totals
        mb_put(&A.mail.cnt[((size_t)s * TMK + m) * 2], (uint32_t)(gt_in + c_gt), gd.tag);
        mb_put(&A.mail.cnt[((size_t)s * TMK + m) * 2 + 1], (uint32_t)(eq_in + c_eq), gd.tag);
      }
      ok = true;
      if (tid < 2 * TMK) {
        uint32_t v = 0;
        ok = poll_word(&A.mail.cnt[(size_t)s * TMK * 2 + tid], v, W_TEAM, gd);
        K.cnt[tid / 2][tid % 2] = (int)v;
      }
      if (!block_all(ok)) return false;
      int eq_before = 0;  // over the members before m, in position order
      sel_before = 0;
      for (int j = 0; j < m; ++j) {
        const int take_j = min(max(need - eq_before, 0), K.cnt[j][1]);
        sel_before += K.cnt[j][0] + take_j;
        eq_before += K.cnt[j][1];
      }
      // this thread's share of the keys equal to T: the lowest positions first
      uT = (uint32_t)min(max(need - (eq_before + eq_in), 0), c_eq);
    }
    // the selected keys in position order: above the threshold prefix, and the
    // threshold's share (candidates ranked at or above uT / the first uT equal to T)
    bool take[KPT];
    int c_take = 0, te = 0;
#pragma unroll
    for (int q = 0; q < KPT; ++q) {
      if (cand) {
        const uint32_t hi = key[q] >> 16;
        take[q] = q < cnt && (hi > (prefix >> 16) || (hi == (prefix >> 16) && cand_word(key[q], p0 + q) >= uT));
      } else {
        const bool eq = q < cnt && key[q] == prefix;
        take[q] = (q < cnt && key[q] > prefix) || (eq && te < (int)uT);
        te += eq ? 1 : 0;
      }
      c_take += take[q] ? 1 : 0;
    }
    int idx = sel_before + block_excl_scan(c_take);
#pragma unroll
    for (int q = 0; q < KPT; ++q)
      if (take[q] && idx < TOPK) publish_sel(s, idx++, page * PAGE + (p0 + q) % PAGE);
    return true;
  }

  // ---------------------------------------------------------------- split
  // A thread's share of a sub-tile's rows: value chunk c = tid % 32 (dims 16 c .. 16 c +
  // 15) of the 4 tokens 4 m .. 4 m + 3, m = tid / 32 (a wave's load covers 512
  // contiguous bytes of each of 2 rows), and (the first SUB x ROPE_CH threads) one
  // 16-byte chunk past the value dims; the scale of token tid % SUB.
  struct Gather {
    u32x4 v[4];
    u32x4 rope;
    float sc;
  };

  // Issue sub-tile st's cache-row loads. Every load is unconditional (an empty slot reads
  // row 0, zeroed at the store): a load under a condition is waited for at the join,
  // which would serialize the gather's round trips.
  MONO_DEV void gather_load(const SplitLds& P, int st, Gather& gt) {
#pragma unroll
    for (int part = 0; part < 3; ++part) gather_load_part(P, st, gt, part);
  }
  // part 0: value chunks of tokens 4 m, 4 m + 1; part 1: of 4 m + 2, 4 m + 3; part 2: the
  // chunk past the value dims and the scale (a long split issues the next sub-tile's
  // parts between its phases, so no wave stalls in one burst)
  MONO_DEV void gather_load_part(const SplitLds& P, int st, Gather& gt, int part) {
    const int c = tid % (DV / 16), m = tid / (DV / 16);
    const int32_t* sl = P.slot + st * SUB;
    if (part < 2) {
#pragma unroll
      for (int k = 2 * part; k < 2 * part + 2; ++k)
        gt.v[k] = ld_nt_u32x4(A.kv + (size_t)max(sl[4 * m + k], 0) * DQK + 16 * c);
    } else {
      const int f = min(tid, ROPE_CH * SUB - 1);
      gt.rope = ld_nt_u32x4(A.kv + (size_t)max(sl[f / ROPE_CH], 0) * DQK + DV + 16 * (f % ROPE_CH));
      gt.sc = A.kv_scale[max(sl[tid % SUB], 0) & A.kv_mask];
    }
  }

  // The 16-byte unit of vt row d holding tokens 8 u .. 8 u + 7: a row's units XOR the
  // row's 16-dim group, so the 32 dim groups a wave's transposed store spans fall on 8
  // different bank groups instead of one (a p.v read stays one aligned unit).
  MONO_DEV static int vt_unit(int d, int u) { return u ^ ((d >> 4) & 7); }

  // Store sub-tile st's rows: as they lie into kf8, and the value dims widened to bf16
  // and transposed into vt (a thread writes one dim of its 4 tokens as 8 bytes); the
  // rows of empty slots as zeros.
  // (the rows as they lie, for q.k; the thread's value chunks stay in w. `vt_now`: the
  // transposed values now, else gather_store_vt later: a long split runs it under its q.k
  // MFMAs, 0.4-0.9 us faster at 24 and 48 rows; one-sub-tile splits measured 0.3-0.6 us
  // slower that way and transpose here)
  MONO_DEV void gather_store(SplitLds& P, int st, const Gather& gt, u32x4 (&w)[4], bool vt_now) {
    const int c = tid % (DV / 16), m = tid / (DV / 16);
    const int32_t* sl = P.slot + st * SUB;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const bool live = sl[4 * m + k] >= 0;
      w[k] = live ? gt.v[k] : u32x4{0u, 0u, 0u, 0u};
      P.kf16[4 * m + k][c] = w[k];
    }
    if (vt_now) gather_store_vt(P, w);
    if (tid < ROPE_CH * SUB) {
      const int t = tid / ROPE_CH;
      P.kf16[t][DV / 16 + tid % ROPE_CH] = sl[t] >= 0 ? gt.rope : u32x4{0u, 0u, 0u, 0u};
    }
    if (tid < SUB) P.kvs[tid] = sl[tid] >= 0 ? gt.sc : 0.f;
  }

  // The thread's value chunks widened to bf16 and transposed into vt.
  MONO_DEV void gather_store_vt(SplitLds& P, const u32x4 (&w)[4]) {
    const int c = tid % (DV / 16), m = tid / (DV / 16);
#pragma unroll
    for (int p = 0; p < 8; ++p) {  // dims 16 c + 2 p, 16 c + 2 p + 1
      uint32_t b[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) b[k] = p % 2 ? fp8x2_bf16<true>(w[k][p / 2]) : fp8x2_bf16<false>(w[k][p / 2]);
      const u32x2 lo = {__builtin_amdgcn_perm(b[1], b[0], 0x05040100u), __builtin_amdgcn_perm(b[3], b[2], 0x05040100u)};
      const u32x2 hi = {__builtin_amdgcn_perm(b[1], b[0], 0x07060302u), __builtin_amdgcn_perm(b[3], b[2], 0x07060302u)};
      const int h8 = 2 * vt_unit(16 * c, m / 2) + m % 2;
      P.vt8[16 * c + 2 * p][h8] = lo;
      P.vt8[16 * c + 2 * p + 1][h8] = hi;
    }
  }

  // Split j of row s's nsp: its selected tokens in sub-tiles of SUB, [32 j / nsp, 32 (j +
  // 1) / nsp) of the row's 32. LONG: a split may hold several sub-tiles (fewer than
  // SPLITS splits a row).
  template <bool LONG>
  MONO_DEV bool split_task(int s, int j, int nsp) {
    SplitLds& P = L.u.sp;
    const int nsel = min(row_len(s), TOPK);
#ifdef MONO_ATTN_WIDE
    const int len = LONG ? TOPK / nsp : TOPK / SPLITS;  // 4 even splits a row
    const int lo = j * len;
#else
    constexpr int NST = TOPK / SUB;  // sub-tiles a row
    const int lo = LONG ? (j * NST / nsp) * SUB : j * (TOPK / SPLITS);
    const int len = LONG ? ((j + 1) * NST / nsp) * SUB - lo : TOPK / SPLITS;
#endif
    const int cnt = min(max(nsel - lo, 0), len);
    const size_t mlb = ((size_t)s * SPLITS + j) * NH;
    if (cnt == 0) {  // an empty split contributes nothing to the merge
      if (tid < NH) {
        st_agent_f32(&A.mail.ml[(mlb + tid) * 2], NEG_INF);
        st_agent_f32(&A.mail.ml[(mlb + tid) * 2 + 1], 0.f);
      }
      split_done(s, j);
      return true;
    }
    if (A.fdone && !q_ready) {  // every head of q from the front of this launch
      const uint64_t* fd = done_copy(A.fdone) + proj::FD_D;
      if (!hint_wait(NH, [fd](int i) { return fd + i; }, A.fsite + 1, gd)) return false;
      q_ready = true;
    }
    {
      constexpr int QN = NH * DQK / 8, QL = (QN + AT - 1) / AT;
      u32x4 qv[QL];
#pragma unroll
      for (int i = 0; i < QL; ++i) qv[i] = ld_u32x4(A.q + (size_t)s * NH * DQK + (size_t)min(tid + i * AT, QN - 1) * 8);
#pragma unroll
      for (int i = 0; i < QL; ++i) {
        const int f = tid + i * AT;  // unconditional loads (see gather_load), guarded stores
        if (f < QN) P.q16[f / (DQK / 8)][f % (DQK / 8)] = qv[i];
      }
    }
    bool ok = true;
    if (tid < len) {
      int slot = -1;
      if (tid < cnt) {
        uint32_t v = 0;
        ok = poll_word(&A.mail.sel[(size_t)s * TOPK + lo + tid], v, W_SEL, gd);
        slot = (int)v;
        if (slot < 0 || slot >= A.n_pages * PAGE) slot = -1;
      }
      P.slot[tid] = slot;
    }
    if (!block_all(ok)) return false;
    mark_waited();

    // p.v of wave w: dims 64 w + 16 b + [0, 16) (b = 0..3) x heads 16 a + [0, 16) (a = 0, 1);
    // lane (g, r) holds dims 64 w + 16 b + 4 g + i of head 16 a + r. Softmax: each
    // 16-lane row of the workgroup one head (tid / 16), a lane 4 tokens; the head's
    // running maximum and sum (every lane of the row holds them).
    f32x4 acc[4][2];
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int a = 0; a < 2; ++a) acc[b][a] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = NEG_INF, l_run = 0.f;
    const int nsub = (cnt + SUB - 1) / SUB;
    Gather gt;
    gather_load(P, 0, gt);
    // q.k of wave (kh, tt): dims QK_HALF kh .. of tokens 16 tt .. 16 tt + 15 against every
    // head; its q operands (heads 16 a + r, 8 dims a k step) held in registers
    bf16x8 qa[2][QK_STEPS];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int ks = 0; ks < QK_STEPS; ++ks)
        qa[a][ks] = __builtin_bit_cast(bf16x8, P.q16[16 * a + r][QK_HALF / 8 * (wave / 4) + 4 * ks + g]);
    __syncthreads();  // every wave holds its q before the first sub-tile's rows overwrite it

#pragma unroll 1
    for (int st = 0; st < nsub; ++st) {
      // a long split: the lane's indices afresh each sub-tile (opaque copies), so the q.k,
      // softmax and p.v LDS addresses are derived inside the loop, not hoisted out of it
      // and held across it
      const int lane = LONG ? opaque_v(tid) % WAVE : this->lane, g = lane / 16, r = lane % 16;
      const int wv = LONG ? opaque_v(tid) / WAVE : wave;
      u32x4 w[4];
      gather_store(P, st, gt, w, !LONG);
      __syncthreads();
      // the next sub-tile's rows, in flight while this one computes (in three parts, one
      // before each phase)
      const bool next = st + 1 < nsub;
      if (next) gather_load_part(P, st + 1, gt, 0);
      // logits, transposed: A = 16 cached rows (FP8, widened in registers), B = 16 heads
      // of q; lane (g, r) ends with tokens 16 tt + 4 g + i of head 16 a + r
      {
        const u32x2* krow = &P.kf8[16 * (wv % 4) + r][QK_HALF / 8 * (wv / 4) + g];
        u32x2 kw[QK_STEPS];
#pragma unroll
        for (int ks = 0; ks < QK_STEPS; ++ks) kw[ks] = krow[4 * ks];
        f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int ks = 0; ks < QK_STEPS; ++ks) {
          const bf16x8 ka = fp8x8_bf16x8(kw[ks]);
          s0 = mfma_bf16(ka, qa[0][ks], s0);
          s1 = mfma_bf16(ka, qa[1][ks], s1);
        }
        P.pf4[wv / 4][r][4 * (wv % 4) + g] = s0;
        P.pf4[wv / 4][16 + r][4 * (wv % 4) + g] = s1;
      }
      if (LONG) gather_store_vt(P, w);  // under the q.k MFMAs (read by p.v, after the softmax's barrier)
      if (next) gather_load_part(P, st + 1, gt, 1);
      __syncthreads();
      // online softmax: head tid / 16, tokens 4 (tid % 16) .. + 3; the head's reductions
      // inside the lane's 16-lane row (DPP)
      {
        const int ti = LONG ? opaque_v(tid) : tid, h = ti / 16, tq = ti % 16;
        const f32x4 x0 = P.pf4[0][h][tq], x1 = P.pf4[1][h][tq], ks = P.kvs4[tq];
        const i32x4 sl = P.slot4[st * (SUB / 4) + tq];
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = sl[i] >= 0 ? (x0[i] + x1[i]) * (ks[i] * A.scale) : NEG_INF;
        const float mx = fmaxf(m_run, row_reduce<16>(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), OpMax()));
        float pr[4], ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[i] = (mx == NEG_INF || x[i] == NEG_INF) ? 0.f : hw_exp(x[i] - mx);
          ps += pr[i];
        }
        const float al = m_run == NEG_INF ? (mx == NEG_INF ? 1.f : 0.f) : hw_exp(m_run - mx);
        l_run = l_run * al + row_reduce<16>(ps, OpAdd());
        m_run = mx;
        P.pb8[h][tq] = u32x2{pack_bf16x2(pr[0] * ks[0], pr[1] * ks[1]), pack_bf16x2(pr[2] * ks[2], pr[3] * ks[3])};
        if (tq == 0) P.alpha[h] = al;
      }
      if (next) gather_load_part(P, st + 1, gt, 2);
      __syncthreads();
      // o^T[dims x heads] = alpha o^T + v^T p^T: A = 16 dims of the transposed values,
      // B = 16 heads' probabilities, k = 32 tokens a step
      {
        float alh[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) alh[a] = P.alpha[16 * a + r];
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[b][a][i] *= alh[a];
#pragma unroll
        for (int kt = 0; kt < SUB / 32; ++kt) {
          bf16x8 pv[2], va[4];  // every operand of the k step read before its MFMAs
#pragma unroll
          for (int a = 0; a < 2; ++a) pv[a] = __builtin_bit_cast(bf16x8, P.pb16[16 * a + r][4 * kt + g]);
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const int d = 64 * wv + 16 * b + r;
            va[b] = __builtin_bit_cast(bf16x8, P.vt16[d][vt_unit(d, 4 * kt + g)]);
          }
#pragma unroll
          for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int a = 0; a < 2; ++a) acc[b][a] = mfma_bf16(va[b], pv[a], acc[b][a]);
        }
      }
      __syncthreads();
    }
    // the partials (bf16, the reference's split partials, kernel.py:4040-4066) staged as
    // [head][dim] in LDS (a lane's 4 consecutive dims of a head as 8 bytes), then stored
    // as the split's contiguous 32 KB by 16-byte device-coherent stores (whole lines);
    // then (m, l); then the split's done word
    // (a head's row padded by 16 bytes: the 16 heads of a lane group's store fall on
    // distinct banks)
    constexpr int OT_ROW = DV / 8 + 1;  // 16-byte units a staged head row
    u32x2* ot = &P.vt8[0][0];           // free after the last p.v step's barrier
    static_assert(sizeof(P.vt8) >= NH * OT_ROW * 16, "partial staging");
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const u32x2 o = {pack_bf16x2(acc[b][a][0], acc[b][a][1]), pack_bf16x2(acc[b][a][2], acc[b][a][3])};
        ot[(16 * a + r) * 2 * OT_ROW + (64 * wave + 16 * b + 4 * g) / 4] = o;
      }
    __syncthreads();
    {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          A.mail.part + ((size_t)s * SPLITS + j) * NH * DV, 0, NH * DV * 2, BUF_DWORD3);
      const u32x4* ot16 = &P.vt16[0][0];
      constexpr int CH16 = NH * DV * 2 / 16;  // 16-byte chunks of the split's partials
#pragma unroll
      for (int q = 0; q < CH16 / AT; ++q) {
        const int c = tid + AT * q;
        __builtin_amdgcn_raw_buffer_store_b128(ot16[(c / (DV / 8)) * OT_ROW + c % (DV / 8)], rs, 16 * c, 0, SC1);
      }
    }
    if (tid % 16 == 0) {
      st_agent_f32(&A.mail.ml[(mlb + tid / 16) * 2], m_run);
      st_agent_f32(&A.mail.ml[(mlb + tid / 16) * 2 + 1], l_run);
    }
    split_done(s, j);  // its barrier also frees the LDS for the next task
    return true;
  }

  // every store of the split performed (each thread waits for its own), then its done word
  MONO_DEV void split_done(int s, int j) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) mb_put(&A.mail.sdone[(size_t)s * SPLITS + j], 0u, gd.tag);
  }

  // ---------------------------------------------------------------- merge
  // This workgroup's merges over a row's NSP splits: list index `at` + k is merge k (row
  // k / (32 / HM), heads (k % (32 / HM)) HM ..), HM heads a task.
  template <int NSP, int HM>
  MONO_DEV bool merges(int at) {
    constexpr int MPR = SPLITS / HM;  // merges a row
    const int n = A.rows * MPR;
    for (int T = first_at_or_after(at); T < at + n; T += G) {
      const uint64_t t0 = now_ticks();
      const int k = T - at;
      const bool ok = merge_task<NSP, HM>(k / MPR, k % MPR);
      stamp(T, t0, 3);
      if (!ok) return false;
    }
    return true;
  }

  // Merge (row s, heads hg HM .. hg HM + HM - 1) over the row's NSP splits: each thread
  // combines IPT channel pairs (a task takes in NSP x HM KB of partials, 32 or 40 KB).
  template <int NSP, int HM>
  MONO_DEV bool merge_task(int s, int hg) {
    constexpr int ITEMS = HM * DV / 2;                // channel pairs of the task
    constexpr int IPT = ITEMS > AT ? ITEMS / AT : 1;  // pairs a thread
    static_assert(NSP <= WAVE && HM <= AW && HM <= 8 && (ITEMS % AT == 0 || ITEMS < AT) && NH % HM == 0,
                  "a lane a split; a wave a head's weights");
    MergeLds& Q = L.u.mg;
    const int h0 = hg * HM;
    const size_t rb = (size_t)s * SPLITS;
    // every split of the row done: lane j of wave 0 polls split j's word
    bool ok = true;
    if (wave == 0 && lane < NSP) {
      uint32_t v;
      ok = poll_word(&A.mail.sdone[rb + lane], v, W_PART, gd);
    }
    if (!block_all(ok)) return false;
    mark_waited();
    // the split weights: wave w takes head h0 + w, lane j split j
    if (wave < HM) {
      const int h = h0 + wave;
      const int jl = min(lane, NSP - 1);
      const float m = ld_agent_f32(&A.mail.ml[((rb + jl) * NH + h) * 2]);
      const float l = lane < NSP ? ld_agent_f32(&A.mail.ml[((rb + jl) * NH + h) * 2 + 1]) : 0.f;
      const bool live = l > 0.f;
      const float M = wave_max(live ? m : NEG_INF);
      const float w = live ? hw_exp(m - M) : 0.f;
      const float den = wave_sum(w * l);
      if (lane < NSP) Q.w[wave][lane] = w;
      if (lane == 0) Q.den[wave] = den;
    }
    // the channel pairs of every split (unconditional loads; an empty split's words are
    // read and ignored)
    const bool mine = tid < ITEMS;  // wave-uniform
    uint32_t av[IPT][NSP];
    if (mine) {
#pragma unroll
      for (int k = 0; k < IPT; ++k) {
        const int it = tid + AT * k, h = h0 + it / (DV / 2), d0 = (it % (DV / 2)) * 2;
#pragma unroll
        for (int j = 0; j < NSP; ++j)
          av[k][j] = ld_agent_u32(reinterpret_cast<const uint32_t*>(&A.mail.part[((rb + j) * NH + h) * DV + d0]));
      }
    }
    __syncthreads();
    if (mine) {
#pragma unroll
      for (int k = 0; k < IPT; ++k) {
        const int it = tid + AT * k, hh = it / (DV / 2), h = h0 + hh, d0 = (it % (DV / 2)) * 2;
        float o[2] = {0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NSP; ++j) {
          const float w = Q.w[hh][j];
          if (w > 0.f) {
            o[0] += w * bf16_lo(av[k][j]);
            o[1] += w * bf16_hi(av[k][j]);
          }
        }
        const float den = Q.den[hh];
        const float inv = den > 0.f ? 1.0f / den : 0.f;
        uint32_t* po = reinterpret_cast<uint32_t*>(A.out + ((size_t)s * NH + h) * DV + d0);
        const uint32_t ov = pack_bf16x2(o[0] * inv, o[1] * inv);
        if (A.publish_out) {  // read in this launch: a device-coherent store, complete before the done word
          __hip_atomic_store(po, ov, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          *po = ov;
        }
      }
      if (A.publish_out) __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();  // (and the next task may rewrite the LDS weights)
    if (A.publish_out && tid < HM) mb_put(&A.mail.mdone[(size_t)s * NH + h0 + tid], 0u, gd.tag);
    return true;
  }
};

// The kernel arguments of a launch (shared by k_attn and the fused attention + back).
void fill_args(Args& a, const AttnArgs& g, const Mail& mail, const GuardArgs& guard) {
  a.iq = static_cast<const uint8_t*>(g.iq);
  a.iqs = static_cast<const uint8_t*>(g.iqs);
  a.iw = static_cast<const uint16_t*>(g.iw);
  a.ikv = static_cast<const uint8_t*>(g.ikv);
  a.iks = static_cast<const uint8_t*>(g.iks);
  a.q = static_cast<const uint16_t*>(g.q);
  a.kv = static_cast<const uint8_t*>(g.kv);
  a.kv_scale = g.kv_scale;
  a.kv_mask = g.kv_mask;
  a.pt = g.page_table;
  a.seq_lens = g.seq_lens;
  a.pt_stride = g.pt_stride;
  a.n_pages = g.n_pages;
  a.out = static_cast<uint16_t*>(g.out);
  a.rows = g.rows;
  a.scores = g.scores;
  a.topk = g.topk;
  a.timeline = g.timeline;
  a.scale = g.softmax_scale;
  a.publish_out = false;
  a.rowh_flip = 1;
  a.fdone = nullptr;
  a.fsite = 0;
  a.mail = mail;
  a.guard = guard;
}

}  // namespace
}  // namespace attn
}  // namespace mono
