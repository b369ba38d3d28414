// Back of the attention block on gfx950 as ONE persistent launch (one 512-thread
// workgroup per CU, tasks dealt round-robin, tagged mailboxes between the stages):
//   U  (head): o[:, h] = bf16(W_UV[h] o_lat[:, h]), 8 row groups of 16, one a wave,
//      K = 512 in 4 steps -> ob (untagged bf16 pairs) and the head's done word
//   O  (32-row tile) of W_o [7168, 4096]: 4 waves a row group, 8 128-k steps a wave,
//      against o staged in LDS; a = bf16(h + W_o o)
// (glm53/gfx950/kernel.py:3975-4197; the attention TP reduce there is the local
// residual add here.)
#pragma once

#include "common.h"
#include "proj_common.h"
#include "proj_ops.h"
#include "sync.h"

namespace mono {
namespace proj {

namespace {

constexpr int FT = 512;
constexpr int FW = FT / WAVE;
constexpr int O_K = HEADS * VDIM;         // 4096
constexpr int NT_O = HIDDEN / 32;         // 224 tiles of 32 rows
constexpr int XU = KV_LORA + 8;
constexpr int XO = O_K + 8;
constexpr int W_OB = 4;
constexpr int W_OLAT = 5;  // the attention's output, in the fused attention + back launch

struct Lds {
  union {
    uint16_t xu[MAX_ROWS][XU];
    uint16_t xo[MAX_ROWS][XO];
  } u;
  f32x4 red[FW][WAVE];
};

struct Args {
  mono_proj_weights w;
  mono_back_args a;
  Mail mail;
  GuardArgs guard;
};

class Back {
 public:
  MONO_DEV Back(const Args& args, Lds& l) : W(args.w), A(args.a), M(args.mail), L(l) {
    tid = thread_index();
    lane = tid % WAVE;
    wave = tid / WAVE;
    g = lane / 16;
    r = lane % 16;
    G = gridDim.x;
    S = A.rows;
    guard_args = args.guard;
  }

  MONO_DEV void run() {
    if (!begin()) return poison(true);
    if (!tasks(0)) poison(false);
  }

  // The launch's tag and deadline (false: the guard refused the launch).
  MONO_DEV bool begin() { return guard_begin(guard_args, gd); }

  // NaN over the launch's output `a` (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.a, (size_t)S * HIDDEN, share); }

  // Run under another launch's guard (a fused launch: its tag, deadline and fail word),
  // after that launch's attention merges: their done words [rows][HEADS].
  MONO_DEV void adopt(const Guard& g, const uint64_t* merge_done) {
    gd = g;
    merged = merge_done;
  }

  // A later phase of the launch reads `a`: each stage-O task stores its rows with
  // device-coherent stores and then puts done word t (of NT_O, replicated) at a_done.
  MONO_DEV void publish_a(uint64_t* done) { a_done = done; }

  static constexpr int N_TASKS = HEADS + NT_O;

  // This workgroup's tasks when the list's first task sits at index `base` of a longer
  // list dealt round-robin over the grid (false, workgroup-uniform: a wait failed).
  MONO_DEV bool tasks(int base) {
    const int b = block_index();
    int T = base <= b ? b : b + ((base - b + G - 1) / G) * G;
    for (; T < base + N_TASKS; T += G) {
      const int t = T - base;
      const uint64_t t0 = now_ticks();
      if (t < HEADS ? !stage_u(t) : !stage_o(t - HEADS)) return false;
      stamp(t, t0, t < HEADS ? 0 : 1);
    }
    return true;
  }

 private:
  const mono_proj_weights& W;
  const mono_back_args& A;
  const Mail& M;
  Lds& L;
  GuardArgs guard_args;
  Guard gd;
  int tid, lane, wave, g, r, G, S;
  uint64_t waited = 0;
  const uint64_t* merged = nullptr;  // the attention merges' done words (fused launch)
  uint64_t* a_done = nullptr;        // stage O's done words for a later phase (fused launch)

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

  MONO_DEV bool stage_u(int h) {
    u32x4 WR[8];
    float SC[4];
    const int rg = (VDIM / 16) * h + wave;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      ld_fp8_tile(static_cast<const uint8_t*>(W.w_uv), KV_LORA / 32, rg, j, g, r, WR[2 * j], WR[2 * j + 1]);
      SC[j] = W.s_uv[(rg * 16 / 128) * (KV_LORA / 128) + j];
    }
    if (merged) {  // in the same launch as the attention: every row's merge of this head
      const uint64_t* md = merged + h;
      if (!hint_wait(S, [md](int i) { return md + (size_t)i * HEADS; }, W_OLAT, gd)) return false;
    }
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(A.o_lat, S * HEADS * KV_LORA * 2);
    for (int f = tid; f < S * (KV_LORA / 8); f += FT) {
      const int s = f / (KV_LORA / 8), p = f % (KV_LORA / 8);
      *reinterpret_cast<u32x4*>(&L.u.xu[s][8 * p]) = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, (((s * HEADS + h) * KV_LORA) + 8 * p) * 2, 0, SC1));
    }
    __syncthreads();
    waited = now_ticks();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), &L.u.xu[r][128 * j + 32 * g]);
    if (r < S) {
      const int v = h * VDIM + 16 * wave + 4 * g;  // output channel of o
      u32x2 o;
      o[0] = pack_bf16x2(acc[0], acc[1]);
      o[1] = pack_bf16x2(acc[2], acc[3]);
      __builtin_amdgcn_raw_buffer_store_b64(o, coherent_rsrc(M.ob, MAX_ROWS * (O_K / 2) * 4),
                                            ((size_t)r * (O_K / 2) + v / 2) * 4, 0, SC1);
      if (A.o) *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(A.o) + (size_t)r * O_K + v) = o;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the head's o is stored (and the next task rewrites the LDS)
    put_done(M.odone, h, gd.tag);
    return true;
  }

  MONO_DEV bool stage_o(int t) {
    u32x4 WR[16];
    float SC[8];
    const int rg = 2 * t + wave / 4;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int ks = (wave % 4) * 8 + j;
      ld_fp8_tile(static_cast<const uint8_t*>(W.w_o), O_K / 32, rg, ks, g, r, WR[2 * j], WR[2 * j + 1]);
      SC[j] = W.s_o[(rg * 16 / 128) * (O_K / 128) + ks];
    }
    // every head's done word, then o of every row in one pass: thread t 16-byte units
    // t + 512 q (row q; rows past S read as 0 and are not kept)
    const uint64_t* od = done_copy(M.odone);
    if (!hint_wait(HEADS, [od](int i) { return od + i; }, W_OB, gd)) return false;
    {
      const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(M.ob, S * (O_K / 2) * 4);
      static_assert(O_K / 8 == FT, "a row of o is one 16-byte unit a thread");
      u32x4 v[MAX_ROWS];
#pragma unroll
      for (int q = 0; q < MAX_ROWS; ++q)
        v[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (q * FT + tid) * 16, 0, SC1));
#pragma unroll
      for (int q = 0; q < MAX_ROWS; ++q)
        if (q < S) *reinterpret_cast<u32x4*>(&L.u.xo[q][8 * tid]) = v[q];
    }
    __syncthreads();
    waited = now_ticks();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int ks = (wave % 4) * 8 + j;
      acc += SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), &L.u.xo[r][128 * ks + 32 * g]);
    }
    L.red[wave][lane] = acc;
    __syncthreads();
    {
      const int rgl = tid / 256, l = (tid / 4) % WAVE, i = tid % 4;
      float y = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) y += L.red[4 * rgl + k][l][i];
      const int s = l % 16, row = 32 * t + 16 * rgl + 4 * (l / 16) + i;
      if (s < S) {
        const size_t at = (size_t)s * HIDDEN + row;
        const float hv = bf16_bits_to_f32(static_cast<const uint16_t*>(A.h)[at]);
        const uint16_t av = f32_to_bf16_bits(__fadd_rn(hv, y));
        if (a_done)  // read by another workgroup of this launch: write through to memory
          __builtin_amdgcn_raw_buffer_store_b16(av, coherent_rsrc(A.a, S * HIDDEN * 2), at * 2, 0, SC1);
        else
          static_cast<uint16_t*>(A.a)[at] = av;
      }
    }
    if (a_done) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();  // every row of the tile is stored
      put_done(a_done, t, gd.tag);
    }
    __syncthreads();
    return true;
  }
};

}  // namespace
}  // namespace proj
}  // namespace mono
