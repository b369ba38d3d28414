// Front of the decoder layer on gfx950 as ONE persistent launch: one 512-thread
// workgroup per CU, tasks dealt round-robin, tagged mailboxes between stages.
//
// The reference's stages 1-4 (glm53/gfx950/kernel.py:1367-2443) with the FP4
// indexer of deepseek_v4/gfx950/kernels/stages/indexer.py:236-408:
//   A  (tile of 16 rows, K half) of [W_qkv (2112) | W_ik (128)] FP8 and W_iw (64)
//      bf16 against the input-RMSNormed rows: every task sums each row's squares over
//      the whole row (one wave a row), stages its K half as bf16(x rstd gamma) in LDS,
//      and runs 3-4 128-k steps a wave -> partial sums (mailbox pa)
//   B  (row): the two halves summed; q_a RMSNorm -> q_an (bf16 pairs); KV RMSNorm +
//      k_pe RoPE -> one power-of-two-scaled E4M3 row into the MLA cache; index key
//      LayerNorm + RoPE + Hadamard + FP4 into the index plane; head weights
//   C  (64-row tile) of W_qb (6144) and W_iq (8192) against q_an: q_nope (bf16 pairs),
//      q_pe (RoPE, straight to q), raw index query (bf16 pairs)
//   D  (head): q_lat = W_UK^T q_nope -> q[:, h, :512]
//   E  (row, 8 heads): index query RoPE + Hadamard + FP4 -> iq, iqs
// A workgroup waits only on tasks of earlier stages, and every workgroup is resident,
// so every wait ends (or its deadline fails it).
#include "common.h"
#include "proj_common.h"
#include "proj_ops.h"
#include "sync.h"

namespace mono {
namespace proj {

namespace {

constexpr int FT = 512;
constexpr int FW = FT / WAVE;

constexpr int A_TILES = (N_QKV + ID) / 16;   // FP8 tiles of stage A
constexpr int W_TILES = IH / 16;             // bf16 tiles of stage A
constexpr int NT_A = (A_TILES + W_TILES) * KP;
constexpr int A_STEPS = HIDDEN / 128 / KP;   // 128-k steps a K part
constexpr int A_KW = HIDDEN / KP;            // k of a part
constexpr int XA = A_KW + 8;                 // LDS row stride (bf16): rows 4 banks apart
constexpr int QB_TILES = HEADS * QK / 64;
constexpr int NT_C = QB_TILES + IH * ID / 64;
constexpr int XC = Q_LORA + 8;
constexpr int XD = NOPE + 8;
constexpr int ROW_PIECES = HIDDEN / 8;       // 16-byte pieces of an input row
constexpr int PART_PIECES = ROW_PIECES / KP;
constexpr float EPS = 1e-6f;
constexpr float LN_EPS = 1e-6f;
constexpr float INDEX_W_SCALE = 0.011048543456039804f;  // 128^-1/2 * 64^-1/2
static_assert(A_STEPS == 3 * FW + 4 && PART_PIECES % WAVE == 0 && ROW_PIECES % WAVE == 0, "stage A split");

enum { W_PA = 0, W_QAN = 1, W_QNOPE = 2, W_IQRAW = 3 };

struct Lds {
  union {
    uint16_t xa[MAX_ROWS][XA];
    uint16_t xc[MAX_ROWS][XC];
    uint16_t xd[MAX_ROWS][XD];
    float row[KP][N_A];
  } u;
  f32x4 red[FW][WAVE];
  float stat[FW][2];
  uint32_t tag;
  uint32_t err;
};

struct Args {
  mono_proj_weights w;
  mono_front_args a;
  Mail mail;
  GuardArgs guard;
};

class Front {
 public:
  MONO_DEV Front(const Args& args, Lds& l) : W(args.w), A(args.a), M(args.mail), L(l) {
    tid = threadIdx.x;
    lane = tid % WAVE;
    wave = tid / WAVE;
    g = lane / 16;
    r = lane % 16;
    G = gridDim.x;
    S = A.rows;
    guard_args = args.guard;
  }

  MONO_DEV void run() {
    if (tid == 0) {
      const uint32_t ticket = __hip_atomic_fetch_add(&guard_args.words[G_TICKET], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
      L.tag = ticket / (uint32_t)G + 1u;
      L.err = ld_agent_u32(&guard_args.words[G_ERROR]);
    }
    __syncthreads();
    if (L.err != 0) return;
    gd.a = guard_args;
    gd.tag = L.tag;
    gd.deadline = now_ticks() + guard_args.deadline_ticks;
    for (int T = blockIdx.x;; T += G) {
      int t = T;
      bool ok = true;
      if (t < NT_A) {
        stage_a(t);
      } else if ((t -= NT_A) < S) {
        ok = stage_b(t);
      } else if ((t -= S) < NT_C) {
        ok = stage_c(t);
      } else if ((t -= NT_C) < HEADS) {
        ok = stage_d(t);
      } else if ((t -= HEADS) < S * (IH / FW)) {
        ok = stage_e(t);
      } else {
        break;
      }
      if (!ok) return;
    }
  }

 private:
  const mono_proj_weights& W;
  const mono_front_args& A;
  const Mail& M;
  Lds& L;
  GuardArgs guard_args;
  Guard gd;
  int tid, lane, wave, g, r, G, S;

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
  MONO_DEV void stage_a(int t) {
    const int tile = t / KP, part = t % KP;
    const bool bf16w = tile >= A_TILES;
    const int nj = wave < A_STEPS - 3 * FW ? 4 : 3;
    u32x4 WR[16];
    float SC[4];
    if (!bf16w) {
      const bool qkv = tile < N_QKV / 16;
      const uint8_t* wb = static_cast<const uint8_t*>(qkv ? W.w_qkv : W.w_ik);
      const float* sb = qkv ? W.s_qkv : W.s_ik;
      const int rg = qkv ? tile : tile - N_QKV / 16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ks = part * A_STEPS + wave + FW * j;
        if (j < nj) {
          ld_fp8_tile(wb, HIDDEN / 32, rg, ks, g, r, WR[2 * j], WR[2 * j + 1]);
          SC[j] = sb[(rg * 16 / 128) * (HIDDEN / 128) + ks];
        } else {
          WR[2 * j] = WR[2 * j + 1] = u32x4{0u, 0u, 0u, 0u};
          SC[j] = 0.f;
        }
      }
    } else {
      const uint8_t* wb = static_cast<const uint8_t*>(W.w_iw);
      const int rg = tile - A_TILES;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ks = part * A_STEPS + wave + FW * j;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          WR[4 * j + q] = j < nj ? ld_bf16_tile(wb, HIDDEN * 2 / 32, rg, ks, g, r, q) : u32x4{0u, 0u, 0u, 0u};
      }
    }
    stage_rows(part);
    __syncthreads();

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < nj) {
        const uint16_t* brow = &L.u.xa[r][128 * (wave + FW * j) + 32 * g];
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
      const int s = l % 16, row = tile * 16 + 4 * (l / 16) + i;
      if (s < S) mb_putf(&M.pa[((size_t)part * MAX_ROWS + s) * N_A + row], v, gd.tag);
    }
    __syncthreads();  // the next task rewrites the LDS
  }

  // Input RMSNorm (glm53/gfx950/kernel.py:1367-1398): wave w takes rows w, w + 8: the
  // whole row's squares (deterministic wave sum), then bf16(x rstd gamma) of the K
  // part into LDS.
  MONO_DEV void stage_rows(int part) {
    const uint16_t* gamma = static_cast<const uint16_t*>(W.g_in);
    for (int s = wave; s < S; s += FW) {
      const uint16_t* hrow = static_cast<const uint16_t*>(A.h) + (size_t)s * HIDDEN;
      u32x4 mine[PART_PIECES / WAVE], other[PART_PIECES / WAVE];
#pragma unroll
      for (int m = 0; m < PART_PIECES / WAVE; ++m) {
        mine[m] = ld_u32x4(hrow + 8 * (part * PART_PIECES + lane + WAVE * m));
        other[m] = ld_u32x4(hrow + 8 * ((1 - part) * PART_PIECES + lane + WAVE * m));
      }
      float ss = 0.f;
#pragma unroll
      for (int m = 0; m < PART_PIECES / WAVE; ++m) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a0 = bf16_lo(mine[m][e]), a1 = bf16_hi(mine[m][e]);
          const float b0 = bf16_lo(other[m][e]), b1 = bf16_hi(other[m][e]);
          ss += a0 * a0 + a1 * a1 + b0 * b0 + b1 * b1;
        }
        __builtin_amdgcn_sched_barrier(0);  // one piece at a time: the rest stay packed
      }
      ss = wave_sum(ss);
      const float rstd = 1.0f / sqrtf(ss / (float)HIDDEN + EPS);
#pragma unroll
      for (int m = 0; m < PART_PIECES / WAVE; ++m) {
        const int pc = lane + WAVE * m;
        const u32x4 gw = ld_u32x4(gamma + 8 * (part * PART_PIECES + pc));
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y0 = mul_rn(mul_rn(bf16_lo(mine[m][e]), rstd), bf16_lo(gw[e]));
          const float y1 = mul_rn(mul_rn(bf16_hi(mine[m][e]), rstd), bf16_hi(gw[e]));
          o[e] = pack_bf16x2(y0, y1);
        }
        *reinterpret_cast<u32x4*>(&L.u.xa[s][8 * pc]) = o;
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // ------------------------------------------------------------ stage B
  MONO_DEV bool stage_b(int s) {
    constexpr int NW = KP * N_A / FT;
    static_assert(KP * N_A % FT == 0, "row words");
    {
      uint32_t v[NW];
      const uint64_t* pa = M.pa;
      const int t0 = tid;
      const bool ok = poll_words<NW>(
          [pa, t0, s](int m) {
            const int w = t0 + FT * m, part = w / N_A, col = w % N_A;
            return pa + ((size_t)part * MAX_ROWS + s) * N_A + col;
          },
          v, (1u << NW) - 1u, W_PA, gd);
      if (!block_all(ok)) return false;
#pragma unroll
      for (int m = 0; m < NW; ++m) {
        const int w = tid + FT * m;
        L.u.row[w / N_A][w % N_A] = __uint_as_float(v[m]);
      }
    }
    __syncthreads();
    for (int c = tid; c < N_A; c += FT) L.u.row[0][c] = L.u.row[0][c] + L.u.row[1][c];
    __syncthreads();
    const float* row = L.u.row[0];

    // q_a and KV latent sums of squares (kernel.py:1978-2003, 2005-2050)
    float sq = 0.f;
    for (int c = tid; c < Q_LORA; c += FT) sq += row[c] * row[c];
    const float kv = row[Q_LORA + tid];
    const f32x2 ss = block_sum2(sq, kv * kv);
    const float rq = 1.0f / sqrtf(ss[0] / (float)Q_LORA + EPS);
    const float rk = 1.0f / sqrtf(ss[1] / (float)KV_LORA + EPS);

    // q_an, published as bf16 pairs
    const uint16_t* gq = static_cast<const uint16_t*>(W.g_q);
    for (int j = tid; j < Q_LORA / 2; j += FT) {
      const uint32_t gw = *reinterpret_cast<const uint32_t*>(gq + 2 * j);
      const float y0 = mul_rn(mul_rn(row[2 * j], rq), bf16_lo(gw));
      const float y1 = mul_rn(mul_rn(row[2 * j + 1], rq), bf16_hi(gw));
      mb_put(&M.qan[(size_t)s * (Q_LORA / 2) + j], pack_bf16x2(y0, y1), gd.tag);
    }

    // KV row: bf16 latent and RoPE'd k_pe, one power-of-two E4M3 scale
    const int slot = slot_of(s), pr = rope_row(s);
    const float c0 = tid < PE_DIM / 2 ? A.rope_cos[(size_t)pr * (PE_DIM / 2) + tid] : 0.f;
    const float s0 = tid < PE_DIM / 2 ? A.rope_sin[(size_t)pr * (PE_DIM / 2) + tid] : 0.f;
    const float kvn = bf16_round(mul_rn(mul_rn(kv, rk), bf16_bits_to_f32(static_cast<const uint16_t*>(W.g_kv)[tid])));
    float p0 = 0.f, p1 = 0.f;
    if (tid < PE_DIM / 2) {
      p0 = row[Q_LORA + KV_LORA + 2 * tid];
      p1 = row[Q_LORA + KV_LORA + 2 * tid + 1];
      rope_pair(p0, p1, c0, s0);
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
    // scale = 2^ceil(log2(max(amax, 1e-4) / 448)) (kernel.py:2137-2151)
    const uint32_t e = code_ceil(fmaxf(amax, 1e-4f) / FP8_MAX);
    const float inv = pow2_of(254u - e);
    if (slot >= 0) {
      uint8_t* kvrow = static_cast<uint8_t*>(A.kv) + (size_t)slot * (KV_LORA + PE_DIM);
      const float q0 = mul_rn(kvn, inv);
      const float q1 = __shfl_down(q0, 1, WAVE), q2 = __shfl_down(q0, 2, WAVE), q3 = __shfl_down(q0, 3, WAVE);
      if (tid % 4 == 0) *reinterpret_cast<uint32_t*>(kvrow + tid) = fp8x4_pack(q0, q1, q2, q3);
      const float e0 = mul_rn(p0, inv), e1 = mul_rn(p1, inv);
      const float e2 = __shfl_down(e0, 1, WAVE), e3 = __shfl_down(e1, 1, WAVE);
      if (tid < PE_DIM / 2 && tid % 2 == 0)
        *reinterpret_cast<uint32_t*>(kvrow + KV_LORA + 2 * tid) = fp8x4_pack(e0, e1, e2, e3);
      if (tid == 0) A.kv_scale[slot] = pow2_of(e);
    }

    // index key: LayerNorm, RoPE on dims [0, 64), Hadamard, FP4 (kernel.py:2103-2131)
    if (wave == 1) {
      const float v0 = row[N_QKV + 2 * lane], v1 = row[N_QKV + 2 * lane + 1];
      const float mean = wave_sum(v0 + v1) / (float)ID;
      const float d0 = sub_rn(v0, mean), d1 = sub_rn(v1, mean);
      const float rs = 1.0f / sqrtf(wave_sum(d0 * d0 + d1 * d1) / (float)ID + LN_EPS);
      float y0 = add_rn(mul_rn(mul_rn(d0, rs), W.g_ik[2 * lane]), W.b_ik[2 * lane]);
      float y1 = add_rn(mul_rn(mul_rn(d1, rs), W.g_ik[2 * lane + 1]), W.b_ik[2 * lane + 1]);
      if (lane < PE_DIM / 2)
        rope_pair(y0, y1, A.rope_cos[(size_t)pr * (PE_DIM / 2) + lane], A.rope_sin[(size_t)pr * (PE_DIM / 2) + lane]);
      uint32_t e8;
      const uint32_t byte = index_vec_fp4(y0, y1, lane, e8);
      if (slot >= 0) {
        const int page = slot / 64, t = slot % 64, blk = lane / 16;
        uint8_t* ikv = static_cast<uint8_t*>(A.ikv);
        uint8_t* iks = static_cast<uint8_t*>(A.iks);
        ikv[(((size_t)page * 4 + blk) * 64 + t) * 16 + lane % 16] = (uint8_t)byte;
        // key t's scale byte sits at (t % 16) * 4 + t / 16 (score_fp4.py:212-241)
        if (lane % 16 == 0) iks[((size_t)page * 4 + blk) * 64 + (t % 16) * 4 + t / 16] = (uint8_t)e8;
      }
    }
    // index head weights: bf16(W_iw x) * 128^-1/2 * 64^-1/2 (indexer.py:340-408)
    if (wave == 2) {
      const float raw = row[N_QKV + ID + lane];
      static_cast<uint16_t*>(A.iw)[(size_t)s * IH + lane] = f32_to_bf16_bits(mul_rn(bf16_round(raw), INDEX_W_SCALE));
    }
    __syncthreads();
    return true;
  }

  // ------------------------------------------------------------ stage C
  // poll S rows of n words (bf16 pairs) from `mb` (row stride `stride` words) into
  // LDS rows of `xs` (stride `xstride` bf16)
  template <int XS>
  MONO_DEV bool stage_pairs(const uint64_t* mb, int n, size_t stride, uint16_t (*xs)[XS], int site) {
    const int total = S * n;
    for (int base = 0; base < total; base += FT * 8) {
      uint32_t v[8];
      uint32_t pending = 0;
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (base + tid + FT * q < total) pending |= 1u << q;
      const int t0 = base + tid;
      const bool ok = poll_words<8>(
          [mb, t0, n, stride](int q) {
            const int w = t0 + FT * q;
            return mb + (size_t)(w / n) * stride + w % n;
          },
          v, pending, site, gd);
      if (!block_all(ok)) return false;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int w = t0 + FT * q;
        if (w < total) *reinterpret_cast<uint32_t*>(&xs[w / n][2 * (w % n)]) = v[q];
      }
    }
    return true;
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
    if (!stage_pairs<XC>(M.qan, Q_LORA / 2, Q_LORA / 2, L.u.xc, W_QAN)) return false;
    __syncthreads();
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const int ks = (wave % 2) * 6 + j;
      acc += SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), &L.u.xc[r][128 * ks + 32 * g]);
    }
    L.red[wave][lane] = acc;
    __syncthreads();
    {
      const int rgl = tid / 128, l = (tid / 2) % WAVE, pi = tid % 2;
      const float v0 = L.red[2 * rgl][l][2 * pi] + L.red[2 * rgl + 1][l][2 * pi];
      const float v1 = L.red[2 * rgl][l][2 * pi + 1] + L.red[2 * rgl + 1][l][2 * pi + 1];
      const int ch = 16 * rgl + 4 * (l / 16) + 2 * pi, s = l % 16;
      if (s < S) {
        if (qb) {
          const int row = 64 * c + ch, head = row / QK, d = row % QK;
          if (d < NOPE) {
            mb_put(&M.qnope[((size_t)s * HEADS + head) * (NOPE / 2) + d / 2], pack_bf16x2(v0, v1), gd.tag);
          } else {
            const int i = (d - NOPE) / 2, pr = rope_row(s);
            float x0 = v0, x1 = v1;
            rope_pair(x0, x1, A.rope_cos[(size_t)pr * (PE_DIM / 2) + i], A.rope_sin[(size_t)pr * (PE_DIM / 2) + i]);
            *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(A.q) + ((size_t)s * HEADS + head) * (KV_LORA + PE_DIM) +
                                         KV_LORA + 2 * i) = pack_bf16x2(x0, x1);
          }
        } else {
          const int row = 64 * (c - QB_TILES) + ch, head = row / ID, d = row % ID;
          mb_put(&M.iqraw[((size_t)s * IH + head) * (ID / 2) + d / 2], pack_bf16x2(v0, v1), gd.tag);
        }
      }
    }
    __syncthreads();
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
    if (!stage_pairs<XD>(M.qnope + (size_t)h * (NOPE / 2), NOPE / 2, (size_t)HEADS * (NOPE / 2), L.u.xd, W_QNOPE))
      return false;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v = SC[j] * step_fp8(join(WR[2 * j], WR[2 * j + 1]), &L.u.xd[r][32 * g]);
      if (r < S) {
        const int cidx = 16 * (4 * wave + j) + 4 * g;
        u32x2 o;
        o[0] = pack_bf16x2(v[0], v[1]);
        o[1] = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(A.q) + ((size_t)r * HEADS + h) * (KV_LORA + PE_DIM) + cidx) = o;
      }
    }
    __syncthreads();
    return true;
  }

  // ------------------------------------------------------------ stage E
  MONO_DEV bool stage_e(int e) {
    const int s = e / (IH / FW), head = (e % (IH / FW)) * FW + wave;
    uint32_t v;
    const bool ok = poll_word(&M.iqraw[((size_t)s * IH + head) * (ID / 2) + lane], v, W_IQRAW, gd);
    if (!block_all(ok)) return false;
    float a = bf16_lo(v), b = bf16_hi(v);
    if (lane < PE_DIM / 2) {
      const int pr = rope_row(s);
      rope_pair(a, b, A.rope_cos[(size_t)pr * (PE_DIM / 2) + lane], A.rope_sin[(size_t)pr * (PE_DIM / 2) + lane]);
    }
    uint32_t e8;
    const uint32_t byte = index_vec_fp4(a, b, lane, e8);
    static_cast<uint8_t*>(A.iq)[((size_t)s * IH + head) * (ID / 2) + lane] = (uint8_t)byte;
    if (lane % 16 == 0) static_cast<uint8_t*>(A.iqs)[((size_t)s * IH + head) * (ID / 32) + lane / 16] = (uint8_t)e8;
    return true;
  }
};

__global__ __launch_bounds__(FT, 1) void k_front(Args args) {
  __shared__ Lds lds;
  Front f(args, lds);
  f.run();
}

}  // namespace

hipError_t front_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_front, FT, 0);
}

hipError_t front_forward(const mono_proj_weights& w, const mono_front_args& a, int grid, const Mail& mail,
                         const GuardArgs& guard, hipStream_t st) {
  if (a.rows < 1 || a.rows > MAX_ROWS || grid < 1) return hipErrorInvalidConfiguration;
  Args args;
  args.w = w;
  args.a = a;
  args.mail = mail;
  args.guard = guard;
  k_front<<<grid, FT, 0, st>>>(args);
  return hipGetLastError();
}

}  // namespace proj
}  // namespace mono
