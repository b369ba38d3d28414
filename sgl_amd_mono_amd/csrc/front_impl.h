// The front of the attention block as a workgroup-level class (Front), included by the
// front launch (front.hip) and by the fused layer launch (layer.hip).
//
// Front of the decoder layer on gfx950 as ONE persistent launch: one 512-thread
// workgroup per CU, tasks dealt round-robin, tagged mailboxes between stages.
//
// The reference's stages 1-4 (glm53/gfx950/kernel.py:1367-2443) with the FP4
// indexer of deepseek_v4/gfx950/kernels/stages/indexer.py:236-408:
//   N  (row): the input RMSNorm, bf16(x rstd gamma), once -> xn (untagged) and the
//      row's done word
//   A  (tile of 16 rows, K part) of [W_qkv (2112) | W_ik (128)] FP8 (whole K up to 8
//      rows, halves above) and W_iw (64) bf16 (K quarters) against the normed rows:
//      the weight burst goes out first, then the rows' done words are awaited and the
//      task's K part of every row arrives by DMA into LDS; its 128-k steps -> partial
//      sums (mailbox pa)
//   B  (row): the K parts summed in order; KV RMSNorm + k_pe RoPE -> one
//      power-of-two-scaled E4M3 row into the MLA cache; index key LayerNorm + RoPE +
//      Hadamard + FP4 into the index plane; head weights
//   C  (64-row tile) of W_qb (6144) and W_iq (8192) against q_an, the q_a RMSNorm that
//      every C task forms itself from stage A's q_a outputs (waiting on the q_a tiles,
//      not on a hand-off through B): q_nope (bf16 pairs), q_pe (RoPE, straight to q),
//      raw index query (bf16 pairs)
//   D  (head): q_lat = W_UK^T q_nope -> q[:, h, :512]
//   E  (row, 8 heads): index query RoPE + Hadamard + FP4 -> iq, iqs
// A workgroup waits only on tasks of earlier stages, and every workgroup is resident,
// so every wait ends (or its deadline fails it).
#pragma once

#include "common.h"
#include "proj_common.h"
#include "proj_ops.h"
#include "row_ssq.h"
#include "sync.h"

namespace mono {
namespace proj {
// the front's own names (the back of the block has its own Args / Lds in proj)
namespace fr {

namespace {

constexpr int FT = 512;
constexpr int FW = FT / WAVE;

constexpr int A_TILES = (N_QKV + ID) / 16;   // FP8 tiles of stage A
constexpr int W_TILES = IH / 16;             // bf16 tiles of stage A
constexpr int KPW = 4;                       // K parts of a bf16 tile
constexpr int QB_TILES = HEADS * QK / 64;
constexpr int NT_C = QB_TILES + IH * ID / 64;
constexpr int XA_ELEMS = MAX_ROWS * (HIDDEN / 2 + 8);  // 8 rows of K or 16 rows of K / 2
constexpr int XC = Q_LORA + 8;
constexpr int XD = NOPE + 8;
constexpr int ROW_PIECES = HIDDEN / 8;       // 16-byte pieces of an input row
constexpr int RPL = ROW_PIECES / WAVE;       // pieces a lane holds of a row
constexpr int MAX_STEPS_W = 7;               // 128-k steps a wave of a stage-A tile, at most
constexpr float EPS = 1e-6f;
constexpr float LN_EPS = 1e-6f;
constexpr float INDEX_W_SCALE = 0.011048543456039804f;  // 128^-1/2 * 64^-1/2
static_assert(SSQ_COLS == HIDDEN, "the shared sum-of-squares order covers the input rows");

// a row's input-RMSNorm factor from its sum of squares
MONO_DEV float row_rstd(float ssq) { return 1.0f / sqrtf(ssq / (float)HIDDEN + EPS); }
static_assert(ROW_PIECES % WAVE == 0 && KPW <= MAX_PARTS, "stage A split");

// FP8 tiles of stage A are split in K in kp_fp8(S) parts: whole (8 rows of K fit the
// LDS) up to 8 rows, halves above
MONO_DEV int kp_fp8(int S) { return S <= 8 ? 1 : 2; }
MONO_DEV int nt_a(int S) { return A_TILES * kp_fp8(S) + W_TILES * KPW; }

enum { W_PA = 0, W_QA = 1, W_QNOPE = 2, W_IQRAW = 3, W_XN = 5 };  // 4: the back's W_UV output

struct Lds {
  union {
    uint16_t xa[XA_ELEMS];  // stage A rows, stride = the part's k + 8
    uint16_t xc[MAX_ROWS][XC];
    uint16_t xd[MAX_ROWS][XD];
    float row[MAX_PARTS][N_A];
  } u;
  f32x4 red[FW][WAVE];
  float stat[FW][2];
  float tsum[SSQ_PIECES / 4];  // a norm task's tile sums of squares (zeros past the row)
  uint16_t gin[HIDDEN];  // the input RMSNorm weight, loaded once a launch
};

struct Args {
  mono_proj_weights w;
  mono_front_args a;
  Mail mail;
  GuardArgs guard;
  int kv_mask;  // -1: per-token power-of-two scales into a.kv_scale; 0: raw E4M3 rows
  int site0;    // the launch's first wait site (a layer's guard numbers the front's after its own)
  // the rows h come from the layer before in this launch: its final tasks' tile sums of
  // squares (tagged words [MAX_ROWS][SSQ_TILES], that layer's tag), awaited at wait site
  // h_site by the norm tasks, which take each row's rstd from them (NULL: the norm tasks
  // form it from the row)
  const uint64_t* h_ssq;
  int h_site;
};

class Front {
 public:
  MONO_DEV Front(const Args& args, Lds& l)
      : W(args.w), A(args.a), M(args.mail), L(l), kv_mask(args.kv_mask), h_ssq(args.h_ssq),
        h_site(args.h_site) {
    tid = thread_index();
    lane = tid % WAVE;
    wave = tid / WAVE;
    g = lane / 16;
    r = lane % 16;
    G = gridDim.x;
    S = A.rows;
    guard_args = args.guard;
    site0 = args.site0;
  }

  MONO_DEV void run() {
    if (!guard_begin(guard_args, gd)) return poison(true);
    if (!tasks()) poison(false);
  }

  // NaN over the launch's output q (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.q, (size_t)S * HEADS * (KV_LORA + PE_DIM), share); }

  // Run under another phase's guard in the same launch (its tag, deadline and fail
  // word; wait sites offset by site_base). `h_ready`: the rows h are known to be stored
  // (a grid barrier met since, whose scrub zeroed the tile sums), so the norm tasks
  // normalise them as in a one-layer launch.
  MONO_DEV void adopt(const Guard& g, int site_base, bool h_ready = false) {
    gd = g;
    site0 = site_base;
    if (h_ready) h_ssq = nullptr;
  }

  // Leave stage D (the absorbed query, whose output only the attention's splits read)
  // out of tasks(): the layer runs it later with deferred_d, on workgroups that would
  // otherwise wait for the top-k, so no score task waits behind it.
  MONO_DEV void set_defer_d(bool v) { defer_d = v; }

  // Stage-D task of head h outside tasks() (its timeline row as tasks() would stamp it).
  MONO_DEV bool deferred_d(int h) {
    relane();
    const uint64_t t0 = now_ticks();
    if (!stage_d(h)) return false;
    stamp(S + nt_a(S) + S + NT_C + h, t0, 3);
    return true;
  }

  // This workgroup's tasks (false, workgroup-uniform: a wait failed).
  MONO_DEV bool tasks() {
    for (int p = tid; p < ROW_PIECES; p += FT)
      *reinterpret_cast<u32x4*>(&L.gin[8 * p]) = ld_u32x4(static_cast<const uint16_t*>(W.g_in) + 8 * p);
    __syncthreads();
    for (int T = block_index();; T += G) {
      relane();
      int t = T, kind;
      bool ok = true;
      const uint64_t t0 = now_ticks();
      if (t < S) {
        kind = 5;
        ok = norm_row(t);
      } else if ((t -= S) < nt_a(S)) {
        kind = 0;
        ok = stage_a(t);
      } else if ((t -= nt_a(S)) < S) {
        kind = 1;
        ok = stage_b(t);
      } else if ((t -= S) < NT_C) {
        kind = 2;
        // the index-query tiles first: stage E, whose output the score tasks await,
        // waits on them; the q_b tiles feed only stage D (the splits' q)
        ok = stage_c(t < NT_C - QB_TILES ? QB_TILES + t : t - (NT_C - QB_TILES));
      } else if ((t -= NT_C) < HEADS) {
        kind = 3;
        if (defer_d) continue;  // run later, by deferred_d
        ok = stage_d(t);
      } else if ((t -= HEADS) < S * (IH / FW)) {
        kind = 4;
        ok = stage_e(t);
      } else {
        break;
      }
      if (!ok) return false;
      stamp(T, t0, kind);
    }
    return true;
  }

 private:
  const mono_proj_weights& W;
  const mono_front_args& A;
  const Mail& M;
  Lds& L;
  const int kv_mask;
  const uint64_t* h_ssq;
  const int h_site;
  bool defer_d = false;
  int site0;
  GuardArgs guard_args;
  Guard gd;
  int tid, lane, wave, g, r, G, S;
  uint64_t waited = 0;

  // Re-derive the thread's coordinates through an opaque copy at every task, so the
  // compiler cannot hoist each stage's per-thread address arithmetic out of the task
  // loop (held across all stages, it spills).
  MONO_DEV void relane() {
    int t = thread_index();
    asm volatile("" : "+v"(t));
    tid = t;
    lane = t % WAVE;
    wave = __builtin_amdgcn_readfirstlane(t / WAVE);  // wave-uniform: scalar branches
    g = lane / 16;
    r = lane % 16;
  }

  // timeline row of task T: start, inputs-ready and end ticks, workgroup << 8 | stage
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

  // ------------------------------------------------------------ row helpers
  // position of row s's new token and its cache slot (-1: a pad row writes nothing)
  MONO_DEV int position(int s) const { return A.seq_lens[s] - 1; }
  MONO_DEV int rope_row(int s) const {
    const int p = position(s);
    return (p >= 0 && p < A.max_pos) ? p : 0;
  }
  MONO_DEV int slot_of(int s) const {
    const int p = position(s);
    if (p < 0 || p >= A.max_pos || p >= A.pt_stride * 64) return -1;
    const int page = A.page_table[(size_t)s * A.pt_stride + p / 64];
    if (page < 0 || page >= A.n_pages) return -1;
    return page * 64 + p % 64;
  }

  // sums of two per-thread values over the workgroup, fixed order (a full barrier)
  MONO_DEV f32x2 block_sum2(float a, float b) {
    a = wave_sum(a);
    b = wave_sum(b);
    if (lane == 0) {
      L.stat[wave][0] = a;
      L.stat[wave][1] = b;
    }
    __syncthreads();
    f32x2 t = {0.f, 0.f};
#pragma unroll
    for (int w = 0; w < FW; ++w) {
      t[0] += L.stat[w][0];
      t[1] += L.stat[w][1];
    }
    __syncthreads();
    return t;
  }

  // ------------------------------------------------------------ stage A
  // A tile's weights go out first as one uninterrupted burst of loads (vector memory
  // completes in order, so nothing that must be waited for may sit between them); the
  // normed rows then go to LDS by DMA (global_load_lds, no registers).
  MONO_DEV bool stage_a(int t) {
    const int kp = kp_fp8(S);
    const bool bf16w = t >= A_TILES * kp;
    const int u = bf16w ? t - A_TILES * kp : t;
    const int parts = bf16w ? KPW : kp;
    const int tile = u / parts, part = u % parts;
    const int steps = HIDDEN / 128 / parts;  // 128-k steps of the part
    const int kw = steps * 128;
    const int nj = (steps - wave + FW - 1) / FW;  // this wave's steps: wave + 8 j
    // staged rows: k in [sk0, sk0 + skw), the FP8 part or the half holding a bf16 quarter
    const int spart = bf16w ? part / (KPW / kp) : part;
    const int skw = HIDDEN / kp, sk0 = spart * skw, sstride = skw + 8;
    const int koff = part * kw - sk0;

    // 1. weights (every load unconditional: surplus steps repeat the wave's last one
    // and are not computed; a load under a condition is waited for at the join)
    u32x4 WR[2 * MAX_STEPS_W];
    float SC[MAX_STEPS_W];
    if (!bf16w) {
      const bool qkv = tile < N_QKV / 16;
      const uint8_t* wb = static_cast<const uint8_t*>(qkv ? W.w_qkv : W.w_ik);
      const float* sb = qkv ? W.s_qkv : W.s_ik;
      const int rg = qkv ? tile : tile - N_QKV / 16;
#pragma unroll
      for (int j = 0; j < MAX_STEPS_W; ++j) {
        const int ks = part * steps + wave + FW * min(j, nj - 1);
        ld_fp8_tile(wb, HIDDEN / 32, rg, ks, g, r, WR[2 * j], WR[2 * j + 1]);
        SC[j] = sb[(rg * 16 / 128) * (HIDDEN / 128) + ks];
      }
    } else {
      const uint8_t* wb = static_cast<const uint8_t*>(W.w_iw);
#pragma unroll
      for (int j = 0; j < MAX_STEPS_W / 2; ++j) {
        const int ks = part * steps + wave + FW * min(j, nj - 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) WR[4 * j + q] = ld_bf16_tile(wb, HIDDEN * 2 / 32, tile, ks, g, r, q);
      }
#pragma unroll
      for (int q = 4 * (MAX_STEPS_W / 2); q < 2 * MAX_STEPS_W; ++q) WR[q] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < MAX_STEPS_W; ++j) SC[j] = 0.f;
    }
    __builtin_amdgcn_sched_barrier(0);
    if (!load_rows(sk0, skw, sstride)) return false;
    mark_waited();

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int rr = min(r, S - 1);  // rows past the step: copies of the last, dropped below
#pragma unroll
    for (int j = 0; j < MAX_STEPS_W; ++j) {
      if (j < nj && (!bf16w || j < MAX_STEPS_W / 2)) {
        const uint16_t* brow = &L.u.xa[rr * sstride + koff + 128 * (wave + FW * j) + 32 * g];
        if (!bf16w) {
          acc += SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), brow);
        } else {
          const u32x4 w4[4] = {WR[4 * j], WR[4 * j + 1], WR[4 * j + 2], WR[4 * j + 3]};
          acc = step_bf16(w4, brow, acc);
        }
      }
    }
    L.red[wave][lane] = acc;
    __syncthreads();
    if (tid < 4 * WAVE) {
      const int l = tid % WAVE, i = tid / WAVE;
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < FW; ++w) v += L.red[w][l][i];
      const int s = l % 16, row = (bf16w ? A_TILES * 16 : 0) + tile * 16 + 4 * (l / 16) + i;
      if (s < S) st_agent_f32(reinterpret_cast<float*>(&M.pa[((size_t)part * MAX_ROWS + s) * N_A + row]), v);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the partials are stored (and the next task rewrites the LDS)
    put_done(M.adone, t, gd.tag);
    return true;
  }

  // Stage N, row s: the input RMSNorm (glm53/gfx950/kernel.py:1367-1398) once for every
  // stage-A task (a stacked layer's from the layer before's tile sums, norm_from_tiles).
  // The row's sum of squares in the order every path shares
  // (row_ssq.h: a 16-byte piece a thread, four threads a tile, wave 0 the tiles); every
  // thread writes bf16(x rstd gamma) of its pieces to xn with device-coherent stores;
  // after they complete, the row's done word.
  MONO_DEV bool norm_row(int s) {
    if (h_ssq) return norm_from_tiles(s);
    const uint16_t* hrow = static_cast<const uint16_t*>(A.h) + (size_t)s * HIDDEN;
    static_assert(SSQ_PIECES == 2 * FT, "two 16-byte pieces a thread");
    u32x4 x[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int p = tid + FT * m;
      x[m] = ld_u32x4(hrow + 8 * min(p, ROW_PIECES - 1));
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int p = tid + FT * m;
      const float t = tile_sum_of_pieces(p < ROW_PIECES ? piece_sum_of_squares(x[m]) : 0.f);
      if (lane % 4 == 0) L.tsum[p / 4] = t;
    }
    __syncthreads();
    if (wave == 0) {
      const float r = row_rstd(tiles_sum(L.tsum[4 * lane], L.tsum[4 * lane + 1], L.tsum[4 * lane + 2],
                                         L.tsum[4 * lane + 3]));
      if (lane == 0) L.stat[0][0] = r;
    }
    __syncthreads();
    mark_waited();
    const float rstd = L.stat[0][0];
    const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(M.xn + (size_t)s * (HIDDEN / 2), HIDDEN * 2);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int p = tid + FT * m;
      if (p < ROW_PIECES) {
        const u32x4 gw = *reinterpret_cast<const u32x4*>(&L.gin[8 * p]);
        __builtin_amdgcn_raw_buffer_store_b128(normed8(x[m], gw, rstd), rs, p * 16, 0, SC1);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the row is stored (and L.stat is free again)
    put_done(M.xdone, s, gd.tag);
    return true;
  }

  // bf16(x rstd gamma) of 8 columns (the RMSNorm's rounding points, kernel.py:1367-1415)
  MONO_DEV static u32x4 normed8(const u32x4& x, const u32x4& gw, float rstd) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float y0 = mul_rn(mul_rn(bf16_lo(x[e]), rstd), bf16_lo(gw[e]));
      const float y1 = mul_rn(mul_rn(bf16_hi(x[e]), rstd), bf16_hi(gw[e]));
      o[e] = pack_bf16x2(y0, y1);
    }
    return o;
  }

  // Norm task of row s in a stacked layer: thread f < 224 polls the layer before's tile
  // sum f of the row (a tagged word of that layer's tag, wait site h_site; it certifies
  // the tile's 32 columns stored) and then loads those columns, so the row comes in
  // while the last tiles land; the row's rstd follows from the tile sums in the shared
  // order, and the normed tile goes to xn as norm_row writes it.
  MONO_DEV bool norm_from_tiles(int s) {
    Guard before = gd;
    before.tag = gd.tag - 1u;
    const uint16_t* hrow = static_cast<const uint16_t*>(A.h) + (size_t)s * HIDDEN;
    bool ok = true;
    u32x4 x[4];
    if (tid < SSQ_PIECES / 4) {
      uint32_t v = 0;
      if (tid < SSQ_TILES) ok = poll_word(&h_ssq[(size_t)s * SSQ_TILES + tid], v, h_site, before);
      L.tsum[tid] = __uint_as_float(v);
#pragma unroll
      for (int q = 0; q < 4; ++q) x[q] = ld_u32x4(hrow + 8 * (4 * min(tid, SSQ_TILES - 1) + q));
    }
    if (!block_all(ok)) return false;
    mark_waited();
    if (wave == 0) {
      const float r = row_rstd(tiles_sum(L.tsum[4 * lane], L.tsum[4 * lane + 1], L.tsum[4 * lane + 2],
                                         L.tsum[4 * lane + 3]));
      if (lane == 0) L.stat[0][0] = r;
    }
    __syncthreads();
    const float rstd = L.stat[0][0];
    if (tid < SSQ_TILES) {
      const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(M.xn + (size_t)s * (HIDDEN / 2), HIDDEN * 2);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p = 4 * tid + q;
        const u32x4 gw = *reinterpret_cast<const u32x4*>(&L.gin[8 * p]);
        __builtin_amdgcn_raw_buffer_store_b128(normed8(x[q], gw, rstd), rs, p * 16, 0, SC1);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the row is stored (and L.stat, L.tsum are free again)
    put_done(M.xdone, s, gd.tag);
    return true;
  }

  // The task's K part [k0, k0 + kw) of every normed row into LDS (row stride `stride`),
  // once every row's done word is in: device-coherent DMA, 1 KB a wave instruction.
  MONO_DEV bool load_rows(int k0, int kw, int stride) {
    const uint64_t* xd = done_copy(M.xdone);
    if (!hint_wait(S, [xd](int i) { return xd + i; }, site0 + W_XN, gd)) return false;
    const int m0 = k0 / (8 * WAVE), mw = kw / (8 * WAVE);  // 1 KB pieces a row
    for (int s = wave; s < S; s += FW) {
      const uint16_t* row = reinterpret_cast<const uint16_t*>(M.xn) + (size_t)s * HIDDEN;
      for (int m = 0; m < mw; ++m)
        __builtin_amdgcn_global_load_lds(row + 8 * (lane + WAVE * (m0 + m)), &L.u.xa[s * stride + 8 * WAVE * m], 16, 0, SC1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    return true;
  }

  // ------------------------------------------------------------ stage B
  MONO_DEV bool stage_b(int s) {
    constexpr int NW = (2 * (N_QKV + ID) + KPW * IH + FT - 1) / FT;  // words a thread polls, at most
    const int kp = kp_fp8(S);
    const int n_fp8 = kp * (N_QKV + ID), total = n_fp8 + KPW * IH;
    // everything but the partial sums is loaded before the wait
    const int slot = slot_of(s), pr = rope_row(s);
    const float cl = A.rope_cos[(size_t)pr * (PE_DIM / 2) + tid % (PE_DIM / 2)];
    const float sl = A.rope_sin[(size_t)pr * (PE_DIM / 2) + tid % (PE_DIM / 2)];
    const float gkv = bf16_bits_to_f32(static_cast<const uint16_t*>(W.g_kv)[tid]);
    const float gik0 = W.g_ik[2 * lane], gik1 = W.g_ik[2 * lane + 1];
    const float bik0 = W.b_ik[2 * lane], bik1 = W.b_ik[2 * lane + 1];
    {
      // every stage-A task's done word, then row s's partials in one pass
      const uint64_t* ad = done_copy(M.adone);
      if (!hint_wait(nt_a(S), [ad](int i) { return ad + i; }, site0 + W_PA, gd)) return false;
      mark_waited();
#pragma unroll
      for (int m = 0; m < NW; ++m) {
        const int w = tid + FT * m;
        int part, col;
        if (w < n_fp8) {
          part = w / (N_QKV + ID);
          col = w % (N_QKV + ID);
        } else {
          part = (w - n_fp8) / IH;
          col = N_QKV + ID + (w - n_fp8) % IH;
        }
        if (w < total) L.u.row[part][col] = ld_agent_f32(reinterpret_cast<const float*>(&M.pa[((size_t)part * MAX_ROWS + s) * N_A + col]));
      }
    }
    __syncthreads();
    // the K parts summed in part order
    for (int c = tid; c < N_A; c += FT) {
      const int np = c < N_QKV + ID ? kp : KPW;
      float v = L.u.row[0][c];
      for (int p = 1; p < np; ++p) v += L.u.row[p][c];
      L.u.row[0][c] = v;
    }
    __syncthreads();
    const float* row = L.u.row[0];

    // the KV latent's sum of squares (kernel.py:2005-2050); the q_a RMSNorm is stage C's
    const float kv = row[Q_LORA + tid];
    const float rk = 1.0f / sqrtf(block_sum2(0.f, kv * kv)[1] / (float)KV_LORA + EPS);

    // KV row: bf16 latent and RoPE'd k_pe, one power-of-two E4M3 scale
    const float kvn = bf16_round(mul_rn(mul_rn(kv, rk), gkv));
    float p0 = 0.f, p1 = 0.f;
    if (tid < PE_DIM / 2) {
      p0 = row[Q_LORA + KV_LORA + 2 * tid];
      p1 = row[Q_LORA + KV_LORA + 2 * tid + 1];
      rope_pair(p0, p1, cl, sl);
      p0 = bf16_round(p0);
      p1 = bf16_round(p1);
    }
    float am = fmaxf(fabsf(kvn), fmaxf(fabsf(p0), fabsf(p1)));
    am = wave_max(am);
    if (lane == 0) L.stat[wave][0] = am;
    __syncthreads();
    float amax = 0.f;
#pragma unroll
    for (int w = 0; w < FW; ++w) amax = fmaxf(amax, L.stat[w][0]);
    __syncthreads();
    // scale = 2^ceil(log2(max(amax, 1e-4) / 448)) (kernel.py:2137-2151); a cache
    // without a scale plane keeps raw E4M3 (scale 1, SGLang's HIP DSA row), values
    // clamped to the E4M3 range (a no-op under the power-of-two scale)
    const uint32_t e = kv_mask ? code_ceil(fmaxf(amax, 1e-4f) / FP8_MAX) : 127u;
    const float inv = pow2_of(254u - e);
    if (slot >= 0) {
      uint8_t* kvrow = static_cast<uint8_t*>(A.kv) + (size_t)slot * (KV_LORA + PE_DIM);
      const float q0 = fminf(fmaxf(mul_rn(kvn, inv), -FP8_MAX), FP8_MAX);
      const float q1 = __shfl_down(q0, 1, WAVE), q2 = __shfl_down(q0, 2, WAVE), q3 = __shfl_down(q0, 3, WAVE);
      if (tid % 4 == 0) st_dev(reinterpret_cast<uint32_t*>(kvrow + tid), fp8x4_pack(q0, q1, q2, q3));
      const float e0 = fminf(fmaxf(mul_rn(p0, inv), -FP8_MAX), FP8_MAX);
      const float e1 = fminf(fmaxf(mul_rn(p1, inv), -FP8_MAX), FP8_MAX);
      const float e2 = __shfl_down(e0, 1, WAVE), e3 = __shfl_down(e1, 1, WAVE);
      if (tid < PE_DIM / 2 && tid % 2 == 0)
        st_dev(reinterpret_cast<uint32_t*>(kvrow + KV_LORA + 2 * tid), fp8x4_pack(e0, e1, e2, e3));
      if (tid == 0) st_dev(&A.kv_scale[slot & kv_mask], pow2_of(e));
    }

    // index key: LayerNorm, RoPE on dims [0, 64), Hadamard, FP4 (kernel.py:2103-2131)
    if (wave == 1) {
      const float v0 = row[N_QKV + 2 * lane], v1 = row[N_QKV + 2 * lane + 1];
      const float mean = wave_sum(v0 + v1) / (float)ID;
      const float d0 = sub_rn(v0, mean), d1 = sub_rn(v1, mean);
      const float rs = 1.0f / sqrtf(wave_sum(d0 * d0 + d1 * d1) / (float)ID + LN_EPS);
      float y0 = add_rn(mul_rn(mul_rn(d0, rs), gik0), bik0);
      float y1 = add_rn(mul_rn(mul_rn(d1, rs), gik1), bik1);
      if (lane < PE_DIM / 2) rope_pair(y0, y1, cl, sl);
      uint32_t e8;
      const uint32_t byte = index_vec_fp4(y0, y1, lane, e8);
      if (slot >= 0) {
        const int page = slot / 64, t = slot % 64, blk = lane / 16;
        uint8_t* ikv = static_cast<uint8_t*>(A.ikv);
        uint8_t* iks = static_cast<uint8_t*>(A.iks);
        st_dev(&ikv[(((size_t)page * 4 + blk) * 64 + t) * 16 + lane % 16], (uint8_t)byte);
        // key t's scale byte sits at (t % 16) * 4 + t / 16 (score_fp4.py:212-241)
        if (lane % 16 == 0) st_dev(&iks[((size_t)page * 4 + blk) * 64 + (t % 16) * 4 + t / 16], (uint8_t)e8);
      }
    }
    // index head weights: bf16(W_iw x) * 128^-1/2 * 64^-1/2 (indexer.py:340-408)
    if (wave == 2) {
      const float raw = row[N_QKV + ID + lane];
      st_dev(&static_cast<uint16_t*>(A.iw)[(size_t)s * IH + lane],
             f32_to_bf16_bits(mul_rn(bf16_round(raw), INDEX_W_SCALE)));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // row s's KV row, index key and head weights are stored
    put_done(M.fdone, FD_B + s, gd.tag);
    return true;
  }

  // ------------------------------------------------------------ stage C
  static constexpr int QA_VL = Q_LORA / 4 / WAVE;  // 16-byte q_a pieces a lane holds of a row
  static_assert(Q_LORA % (4 * WAVE) == 0, "q_a rows split evenly over a wave's lanes");

  // q_an = bf16(q_a * rstd * g_q) of every row into L.u.xc (kernel.py:1978-2003), from
  // stage A's raw q_a (its K parts summed in part order): wave w normalises rows w, w + 8,
  // a lane 6 pieces of 4 consecutive columns, the row's sum of squares a wave sum. One
  // round of unconditional 16-byte loads: the second part's reads fall past the buffer
  // (zeros, no traffic) unless the step splits K.
  MONO_DEV void qa_norm(const u32x2 (&gq)[QA_VL]) {
    const bool two = kp_fp8(S) == 2;
    const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(M.pa, (uint32_t)((two ? 2 : 1) * MAX_ROWS * N_A * 4));
    for (int s = wave; s < S; s += FW) {  // wave-uniform
      u32x4 p0[QA_VL], p1[QA_VL];
#pragma unroll
      for (int j = 0; j < QA_VL; ++j) {
        const int c = 4 * (lane + WAVE * j);
        p0[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (s * N_A + c) * 4, 0, SC1));
        p1[j] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, ((MAX_ROWS + s) * N_A + c) * 4, 0, SC1));
      }
      float x[QA_VL][4];
      float sq = 0.f;
#pragma unroll
      for (int j = 0; j < QA_VL; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float a = __uint_as_float(p0[j][q]), b = __uint_as_float(p1[j][q]);
          x[j][q] = two ? a + b : a;
          sq += x[j][q] * x[j][q];
        }
      const float rq = 1.0f / sqrtf(wave_sum(sq) / (float)Q_LORA + EPS);
#pragma unroll
      for (int j = 0; j < QA_VL; ++j) {
        const int c = 4 * (lane + WAVE * j);
        u32x2 o;
        o[0] = pack_bf16x2(mul_rn(mul_rn(x[j][0], rq), bf16_lo(gq[j][0])), mul_rn(mul_rn(x[j][1], rq), bf16_hi(gq[j][0])));
        o[1] = pack_bf16x2(mul_rn(mul_rn(x[j][2], rq), bf16_lo(gq[j][1])), mul_rn(mul_rn(x[j][3], rq), bf16_hi(gq[j][1])));
        *reinterpret_cast<u32x2*>(&L.u.xc[s][c]) = o;
      }
    }
  }

  MONO_DEV bool stage_c(int c) {
    const bool qb = c < QB_TILES;
    const uint8_t* wb = static_cast<const uint8_t*>(qb ? W.w_qb : W.w_iq);
    const float* sb = qb ? W.s_qb : W.s_iq;
    const int rg = (qb ? c : c - QB_TILES) * 4 + wave / 2;
    u32x4 WR[12];
    float SC[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const int ks = (wave % 2) * 6 + j;
      ld_fp8_tile(wb, Q_LORA / 32, rg, ks, g, r, WR[2 * j], WR[2 * j + 1]);
      SC[j] = sb[(rg * 16 / 128) * (Q_LORA / 128) + ks];
    }
    // this thread's output pair (after the wave-pair reduction) and, for a q_pe tile,
    // its RoPE factors, loaded before the wait
    const int rgl = tid / 128, l = (tid / 2) % WAVE, pi = tid % 2;
    const int ch = 16 * rgl + 4 * (l / 16) + 2 * pi, so = l % 16;
    const int qrow = 64 * c + ch, qd = qrow % QK;
    const int prc = rope_row(min(so, S - 1)), ic = max(qd - NOPE, 0) / 2;
    const float rc = A.rope_cos[(size_t)prc * (PE_DIM / 2) + ic];
    const float rs = A.rope_sin[(size_t)prc * (PE_DIM / 2) + ic];
    // the q_a RMSNorm weight of this lane's columns, before the wait
    u32x2 gq[QA_VL];
#pragma unroll
    for (int j = 0; j < QA_VL; ++j)
      gq[j] = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(W.g_q) + 4 * (lane + WAVE * j));
    // the q_a tiles of stage A (task t holds tile t / kp), then q_an of every row
    const uint64_t* ad = done_copy(M.adone);
    if (!hint_wait((Q_LORA / 16) * kp_fp8(S), [ad](int i) { return ad + i; }, site0 + W_QA, gd)) return false;
    qa_norm(gq);
    __syncthreads();
    mark_waited();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const int ks = (wave % 2) * 6 + j;
      acc += SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), &L.u.xc[r][128 * ks + 32 * g]);
    }
    L.red[wave][lane] = acc;
    __syncthreads();
    {
      const float v0 = L.red[2 * rgl][l][2 * pi] + L.red[2 * rgl + 1][l][2 * pi];
      const float v1 = L.red[2 * rgl][l][2 * pi + 1] + L.red[2 * rgl + 1][l][2 * pi + 1];
      const int s = so;
      if (s < S) {
        if (qb) {
          const int row = qrow, head = row / QK, d = qd;
          if (d < NOPE) {
            __hip_atomic_store(&M.qnope[((size_t)s * HEADS + head) * (NOPE / 2) + d / 2], pack_bf16x2(v0, v1),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          } else {
            const int i = (d - NOPE) / 2;
            float x0 = v0, x1 = v1;
            rope_pair(x0, x1, rc, rs);
            st_dev(reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(A.q) + ((size_t)s * HEADS + head) * (KV_LORA + PE_DIM) +
                                               KV_LORA + 2 * i), pack_bf16x2(x0, x1));
          }
        } else {
          const int row = 64 * (c - QB_TILES) + ch, head = row / ID, d = row % ID;
          __hip_atomic_store(&M.iqraw[((size_t)s * IH + head) * (ID / 2) + d / 2], pack_bf16x2(v0, v1),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the tile's outputs are stored
    if (tid == 0) mb_put(&M.cdone[c], 0u, gd.tag);
    return true;
  }

  // ------------------------------------------------------------ stage D
  MONO_DEV bool stage_d(int h) {
    u32x4 WR[8];
    float SC[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rg = (KV_LORA / 16) * h + 4 * wave + j;
      ld_fp8_tile(static_cast<const uint8_t*>(W.w_uk), NOPE / 32, rg, 0, g, r, WR[2 * j], WR[2 * j + 1]);
      SC[j] = W.s_uk[rg * 16 / 128];
    }
    // head h's q_nope comes from q_b tiles 3h and 3h + 1 (QK = 192 rows a head); tile
    // 3h + 2 (its q_pe) is awaited too, so head h's done word covers all of its q
    static_assert(QK == 3 * 64 && NOPE == 2 * 64, "q_nope of a head = two q_b tiles");
    const uint64_t* cd = M.cdone + 3 * h;
    if (!hint_wait(3, [cd](int i) { return cd + i; }, site0 + W_QNOPE, gd)) return false;
    for (int w = tid; w < S * (NOPE / 2); w += FT) {
      const int s = w / (NOPE / 2), p = w % (NOPE / 2);
      *reinterpret_cast<uint32_t*>(&L.u.xd[s][2 * p]) = ld_agent_u32(&M.qnope[((size_t)s * HEADS + h) * (NOPE / 2) + p]);
    }
    __syncthreads();
    mark_waited();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v = SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), &L.u.xd[r][32 * g]);
      if (r < S) {
        const int cidx = 16 * (4 * wave + j) + 4 * g;
        u32x2 o;
        o[0] = pack_bf16x2(v[0], v[1]);
        o[1] = pack_bf16x2(v[2], v[3]);
        st_dev(reinterpret_cast<uint64_t*>(static_cast<uint16_t*>(A.q) + ((size_t)r * HEADS + h) * (KV_LORA + PE_DIM) + cidx),
               ((uint64_t)o[1] << 32) | o[0]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // head h of q is stored
    put_done(M.fdone, FD_D + h, gd.tag);
    return true;
  }

  // ------------------------------------------------------------ stage E
  MONO_DEV bool stage_e(int e) {
    const int s = e / (IH / FW), head = (e % (IH / FW)) * FW + wave;
    const int pr = rope_row(s);
    const float rc = A.rope_cos[(size_t)pr * (PE_DIM / 2) + lane % (PE_DIM / 2)];
    const float rs = A.rope_sin[(size_t)pr * (PE_DIM / 2) + lane % (PE_DIM / 2)];
    // index heads 8j .. 8j + 7 come from W_iq tiles 16j .. 16j + 15 (two a head)
    static_assert(ID == 2 * 64, "a raw index query head = two W_iq tiles");
    const uint64_t* cd = M.cdone + QB_TILES + 2 * (e % (IH / FW)) * FW;
    if (!hint_wait(2 * FW, [cd](int i) { return cd + i; }, site0 + W_IQRAW, gd)) return false;
    mark_waited();
    const uint32_t v = ld_agent_u32(&M.iqraw[((size_t)s * IH + head) * (ID / 2) + lane]);
    float a = bf16_lo(v), b = bf16_hi(v);
    if (lane < PE_DIM / 2) rope_pair(a, b, rc, rs);
    uint32_t e8;
    const uint32_t byte = index_vec_fp4(a, b, lane, e8);
    st_dev(&static_cast<uint8_t*>(A.iq)[((size_t)s * IH + head) * (ID / 2) + lane], (uint8_t)byte);
    if (lane % 16 == 0) st_dev(&static_cast<uint8_t*>(A.iqs)[((size_t)s * IH + head) * (ID / 32) + lane / 16], (uint8_t)e8);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the task's index-query heads are stored
    put_done(M.fdone, FD_E + e, gd.tag);
    return true;
  }
};

}  // namespace
}  // namespace fr
}  // namespace proj
}  // namespace mono
