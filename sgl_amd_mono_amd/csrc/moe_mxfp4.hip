// MXFP4 (E2M1 + E8M0 per 32) routed + shared MoE of one decode step on gfx950 (A16W4:
// bf16 activations), as ONE persistent launch: one 512-thread workgroup per CU.
//
// The reference's A16W4 expert path (minimax_m31/a16w4.py:1-92 operands over AITER's
// (16, 16) layout; glm53/gfx950/kernel.py:966-970,1068-1085 ``unit_mxfp4_bf16``)
// behind a softmax router over given f32 logits. Same shape of
// launch as moe_fp8.hip (tagged mailboxes, guarded waits, one round-robin task list):
//   route  row s on workgroup G-1-s: top-8 of the logits (f32 order, lowest id on
//          ties), weights = softmax over the 8 picked logits -> mailbox rsel
//   x      every workgroup: the rows' bf16 activations into LDS
//   up     (slot, 16-channel tile): a lane's 16 weight bytes are 32 E2M1 values of
//          one row (row 16 rg + l % 16, k 32 (l / 16) ..); v_cvt_scalef32_pk_bf16_fp4
//          widens them with the row's E8M0 scale into four bf16 MFMA 16x16x32
//          operands, against the matching 8-k slices of the bf16 rows; the 8 waves
//          split K; mid = bf16(SiLU(gate) * up) -> mailbox mid
//   down   (slot, 256 output rows): the slot's bf16 mid in LDS, the same A16W4 MFMA,
//          x the route weight -> mailbox ypart
//   final  (32 output rows): the row's 9 slots summed in plan order -> bf16 out
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
constexpr int XSTRIDE = H + 8;       // bf16 an activation row in LDS (rows in different banks)
constexpr int MSTRIDE = I + 8;       // bf16 a mid row in LDS
constexpr int MPT = MAX_ROWS * I / FT;  // mid words a thread polls in a down task
static_assert(HS % FW == 0 && I % 128 == 0 && I % MPT == 0 && MPT % 2 == 0, "tiling");
static_assert(2 * UP_SW <= 8 && 2 * IS <= 8, "weight registers");

enum { W_PICKS = 1, W_MID = 2, W_YPART = 3 };

struct Lds {
  uint16_t x[MAX_ROWS][XSTRIDE];    // the rows' bf16 activations
  uint16_t mid[MAX_ROWS][MSTRIDE];  // a down task's bf16 mid
  f32x4 red[2][FW][WAVE];
  PlanLds<E, TOPK> plan;
  uint32_t rkey[E];
  float rraw[E];
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
MONO_DEV f32x4 a16w4_step(f32x4 acc, const u32x4& w, float sc, const uint16_t* brow) {
#pragma unroll
  for (int q = 0; q < 4; ++q)
    acc = mfma_bf16(fp4x8_bf16(w[q], sc), *reinterpret_cast<const bf16x8*>(brow + 8 * q), acc);
  return acc;
}

enum { K_NONE = 0, K_UP = 1, K_DOWN = 2, K_FINAL = 3 };

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
    if (!guard_begin(A.guard, gd)) return poison(true);
    if ((int)blockIdx.x >= G - S) route(G - 1 - (int)blockIdx.x);
    load_rows();
    __syncthreads();
    if (!tasks()) poison(false);
  }

  // NaN over the launch's output (sync.h poison_bf16)
  MONO_DEV void poison(bool share) const { poison_bf16(A.out, (size_t)S * H, share); }

 private:
  const Args& A;
  Lds& L;
  Guard gd;
  int tid, lane, wave, g, r, G, S;
  bool plan_ready = false;
  u32x4 W[8];  // weights of the next task: an up tile (2 x 3 steps) or a down task (2 x 3)
  float SC[8];

  // ---------------------------------------------------------------- route
  MONO_DEV void route(int s) {
    if (tid < E) {
      const float lg = A.logits[(size_t)s * E + tid];
      L.rraw[tid] = lg;
      L.rkey[tid] = radix_key(lg);
    }
    __syncthreads();
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
        mb_put(&A.mail.rsel[s * 2 * MAX_TOPK + lane], (uint32_t)my_id, gd.tag);
        mb_putf(&A.mail.rsel[s * 2 * MAX_TOPK + MAX_TOPK + lane], w, gd.tag);
        if (A.topk_ids) A.topk_ids[s * TOPK + lane] = my_id;
        if (A.topk_w) A.topk_w[s * TOPK + lane] = w;
      }
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- rows
  MONO_DEV void load_rows() {
    constexpr int V = H / 8;  // 16-byte pieces of a row
    for (int f = tid; f < S * V; f += FT) {
      const int s = f / V, c = f % V;
      *reinterpret_cast<u32x4*>(&L.x[s][c * 8]) = ld_u32x4(A.x + (size_t)s * H + c * 8);
    }
  }

  // ---------------------------------------------------------------- task list
  MONO_DEV bool load_plan() {
    if (!build_plan<E, TOPK, FT>(L.plan, A.mail.rsel, S, W_PICKS, gd)) return false;
    plan_ready = true;
    return true;
  }

  MONO_DEV int classify(int T, bool& ok) {
    ok = true;
    if (T < NT) return K_UP;  // the shared expert's tiles need no plan
    if (!plan_ready && !(ok = load_plan())) return K_NONE;
    const int n_up = L.plan.n_act * NT, n_dn = L.plan.n_act * DN_GROUPS;
    if (T < n_up) return K_UP;
    if (T < n_up + n_dn) return K_DOWN;
    if (T < n_up + n_dn + FIN_TASKS) return K_FINAL;
    return K_NONE;
  }

  // E8M0 byte `b` of a scale dword as an f32 power of two
  MONO_DEV static float scale_of(uint32_t word, int b) { return e8m0_to_f32((word >> (8 * b)) & 0xffu); }

  // Issue task T's weight and scale loads into W / SC; every entry written on every path.
  MONO_DEV void load_task(int kind, int T) {
    if (kind == K_UP) {
      const int d = T / NT, c = T % NT;
      const int e = d == 0 ? E : L.plan.expert[d];
      const uint8_t* wb = A.w13 + (size_t)e * (2 * I) * (H / 2);
      const uint8_t* sb = A.s13 + (size_t)e * (2 * I) * (H / 32);
#pragma unroll
      for (int j = 0; j < UP_SW; ++j) {
        const int ks = wave * UP_SW + j;
        W[2 * j] = ld_shuf_fp4(wb, H / 32, c, ks, lane);            // gate rows 16c..
        W[2 * j + 1] = ld_shuf_fp4(wb, H / 32, NT + c, ks, lane);   // up rows I + 16c..
        const uint32_t sg = *reinterpret_cast<const uint32_t*>(sb + (size_t)(16 * c + r) * (H / 32) + 4 * ks);
        const uint32_t su = *reinterpret_cast<const uint32_t*>(sb + (size_t)(I + 16 * c + r) * (H / 32) + 4 * ks);
        SC[2 * j] = scale_of(sg, g);
        SC[2 * j + 1] = scale_of(su, g);
      }
#pragma unroll
      for (int q = 2 * UP_SW; q < 8; ++q) {
        W[q] = u32x4{0u, 0u, 0u, 0u};
        SC[q] = 0.f;
      }
    } else if (kind == K_DOWN) {
      const int j = T - L.plan.n_act * NT;
      const int d = j / DN_GROUPS, grp = j % DN_GROUPS;
      const int e = L.plan.expert[d];
      const uint8_t* wb = A.w2 + (size_t)e * H * (I / 2);
      const uint8_t* sb = A.s2 + (size_t)e * H * (I / 32);
      const int rg0 = (grp * DN_ROWS + wave * 32) / 16;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < IS; ++ks) {
          W[t * IS + ks] = ld_shuf_fp4(wb, I / 32, rg0 + t, ks, lane);
          const uint32_t sw = *reinterpret_cast<const uint32_t*>(sb + (size_t)((rg0 + t) * 16 + r) * (I / 32) + 4 * ks);
          SC[t * IS + ks] = scale_of(sw, g);
        }
#pragma unroll
      for (int q = 2 * IS; q < 8; ++q) {
        W[q] = u32x4{0u, 0u, 0u, 0u};
        SC[q] = 0.f;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        W[q] = u32x4{0u, 0u, 0u, 0u};
        SC[q] = 0.f;
      }
    }
  }

  MONO_DEV bool tasks() {
    int T = blockIdx.x;
    bool ok;
    int kind = classify(T, ok);
    if (!ok) return false;
    load_task(kind, T);
    while (kind != K_NONE) {
      f32x4 acc[2];
      if (kind == K_UP) {
        up_compute(acc[0], acc[1]);
      } else if (kind == K_DOWN) {
        if (!down_compute(T, acc)) return false;
      }
      const int T2 = T + G;
      const int kind2 = classify(T2, ok);
      if (!ok) return false;
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
  MONO_DEV void up_compute(f32x4& ag, f32x4& au) {
    ag = f32x4{0.f, 0.f, 0.f, 0.f};
    au = ag;
#pragma unroll
    for (int j = 0; j < UP_SW; ++j) {
      const int ks = wave * UP_SW + j;
      const uint16_t* brow = &L.x[r][128 * ks + 32 * g];
      ag = a16w4_step(ag, W[2 * j], SC[2 * j], brow);
      au = a16w4_step(au, W[2 * j + 1], SC[2 * j + 1], brow);
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
      // mid is staged as bf16 (glm53/gfx950/kernel.py:5111-5117)
      if ((mask >> s) & 1u) mb_putf(&A.mail.mid[((size_t)d * MAX_ROWS + s) * I + ch], bf16_round(silu(gs) * us), gd.tag);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- down
  MONO_DEV bool down_compute(int T, f32x4 (&acc)[2]) {
    const int j = T - L.plan.n_act * NT;
    const int d = j / DN_GROUPS;
    const uint32_t mask = L.plan.rowmask[d];
    // thread (row s, MPT contiguous channels) polls its mid words
    const int s = tid / (I / MPT), c0 = (tid % (I / MPT)) * MPT;
    const bool in = (mask >> s) & 1u;
    const uint64_t* base = &A.mail.mid[((size_t)d * MAX_ROWS + s) * I + c0];
    uint32_t v[MPT];
    const bool ok = poll_words<MPT>([base](int q) { return base + q; }, v, in ? (1u << MPT) - 1u : 0u, W_MID, gd);
    if (!block_all(ok)) return false;
#pragma unroll
    for (int q = 0; q < MPT; q += 2) {
      const float a = in ? __uint_as_float(v[q]) : 0.f, b = in ? __uint_as_float(v[q + 1]) : 0.f;
      *reinterpret_cast<uint32_t*>(&L.mid[s][c0 + q]) = pack_bf16x2(a, b);
    }
    __syncthreads();
    const float wr = route_weight(L.plan, d, r);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < IS; ++ks) acc[t] = a16w4_step(acc[t], W[t * IS + ks], SC[t * IS + ks], &L.mid[r][128 * ks + 32 * g]);
      acc[t] *= wr;
    }
    return true;
  }

  MONO_DEV void down_publish(int T, const f32x4 (&acc)[2]) {
    const int j = T - L.plan.n_act * NT;
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
    __syncthreads();  // the next down task rewrites the LDS mid
  }

  // ---------------------------------------------------------------- final
  MONO_DEV bool final_task(int T) {
    const int f = T - L.plan.n_act * (NT + DN_GROUPS);
    bool ok = true;
    if (tid < S * FIN_ROWS) {
      const int s = tid / FIN_ROWS, h = f * FIN_ROWS + tid % FIN_ROWS;
      const uint64_t* base = &A.mail.ypart[(size_t)s * H + h];
      const int32_t* slots = L.plan.rowslot[s];
      uint32_t v[NSLOT];
      ok = poll_words<NSLOT>([base, slots](int k) { return base + (size_t)slots[k] * MAX_ROWS * H; }, v,
                             (1u << NSLOT) - 1u, W_YPART, gd);
      if (ok) {
        float y = 0.f;
#pragma unroll
        for (int k = 0; k < NSLOT; ++k) y += __uint_as_float(v[k]);
        A.out[(size_t)s * H + h] = f32_to_bf16_bits(y);
        if (A.y_out) A.y_out[(size_t)s * H + h] = y;
      }
    }
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

hipError_t moe_mxfp4_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_moe_mxfp4, FT, 0);
}

hipError_t moe_mxfp4_forward(const mono_moe_mxfp4_args& g, int grid, const Mail& mail, const GuardArgs& guard,
                             hipStream_t st) {
  if (grid < MAX_ROWS || g.rows < 1 || g.rows > MAX_ROWS) return hipErrorInvalidConfiguration;
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
  a.rows = g.rows;
  a.mail = mail;
  a.guard = guard;
  k_moe_mxfp4<<<grid, FT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace moe
}  // namespace mono
