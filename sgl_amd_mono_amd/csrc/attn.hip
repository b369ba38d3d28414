// Sparse-attention phase of one decode step on gfx950, as ONE persistent launch (one
// 512-thread workgroup per CU). The reference runs it as stages of its decoder-layer
// launch: FP4 index scores (deepseek_v4/gfx950/kernels/stages/indexer.py:460-602 and
// the native-FP4 scorer deepseek_v41/gfx950/indexer/score_fp4.py:254-296), the exact
// top-2048 (indexer.py:604-802, glm53/gfx950/kernel.py:3000-3636), the sparse MLA
// split (kernel.py:3638-3973) and the split merge (kernel.py:3975-4123).
//
// Tasks, dealt round-robin over the workgroups in this order (a workgroup only ever
// waits on tasks that come earlier in every workgroup's list, so the launch cannot
// deadlock while all workgroups are resident; every wait is guarded, sync.h):
//   score  (row, 1024 keys): 8 waves x 128 keys. The row's FP4 query (64 heads x 128
//          dims, E2M1 + E8M0 per 32) is the A operand and 16 keys of SGLang's FP4 index
//          plane the B operand of v_mfma_scale_f32_16x16x128_f8f6f4 with FP4 formats:
//          the plane's E8M0 bytes are the MFMA's per-lane B scales as they lie (a
//          lane's dword holds its key's scale for the page's four 16-key tiles).
//          score = sum_h w_h relu(q_h . k) -> mailbox score
//   topk   (row): the row's scores as order-preserving u32 keys in LDS, an MSB-first
//          8-bit radix select of the 2048th key, then a stable compaction: every key
//          above it and the lowest positions equal to it, ascending -> cache slots
//          (page_table[p / 64] * 64 + p % 64) -> mailbox sel (glm53/check.py:100-117)
//   split  (row, 256 selected tokens): 4 sub-tiles of 64 tokens gathered from the FP8
//          cache into LDS (row-major for q.k, transposed latent for p.v), bf16 MFMA
//          16x16x32 with the FP8 values widened exactly, the per-token scale folded
//          into the logit and the probability, online softmax -> mailboxes part, ml
//   merge  (row, 4 heads): out = sum_j e^(m_j - M) acc_j / sum_j e^(m_j - M) l_j, bf16
#include "attn_ops.h"
#include "common.h"
#include "sync.h"

namespace mono {
namespace attn {

namespace {

constexpr int AT = 512;
constexpr int AW = AT / WAVE;
constexpr int KPT = MAX_CTX / AT;            // keys a thread holds in the top-k
constexpr int KL_WORDS = MAX_CTX + AT;       // one pad word a thread range: no bank conflicts
constexpr int SUB = 64;                      // tokens a split sub-tile
constexpr int NSUB = SPLIT / SUB;
constexpr int Q_STRIDE = DQK + 8;            // bf16 a q row in LDS
constexpr int KV_STRIDE = DQK + 16;          // bytes a cached row in LDS
constexpr int VT_STRIDE = SUB + 8;           // bytes a transposed latent row in LDS
constexpr int PB_STRIDE = SUB + 8;           // bf16 a probability row in LDS
constexpr int KEYS_WAVE = CHUNK / AW;        // 128 keys a wave of a score task
constexpr int KTILES = KEYS_WAVE / 16;
constexpr float NEG_INF = -__builtin_huge_valf();
static_assert(KPT % 16 == 0 && KEYS_WAVE % PAGE == 0 && SPLIT % SUB == 0, "tiling");
static_assert(AT == NH * DV / 32, "a merge thread owns 4 outputs of one head");

enum { W_SCORE = 0, W_SEL = 1, W_PART = 2 };

struct TopkLds {
  uint32_t kl[KL_WORDS];
  uint32_t hist[256];
  uint32_t digit;
  int32_t above;
};

struct SplitLds {
  uint16_t q[NH][Q_STRIDE];
  uint8_t kv[SUB][KV_STRIDE];
  uint8_t vt[DV][VT_STRIDE];
  float pf[NH][SUB];
  uint16_t pb[NH][PB_STRIDE];
  int32_t slot[SPLIT];
  float kvs[SUB];
  float alpha[NH];
};

struct Lds {
  union {
    TopkLds t;
    SplitLds sp;
  } u;
  int32_t scan[AW];
  uint32_t tag;
  uint32_t err;
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
  const int32_t* pt;
  const int32_t* seq_lens;
  int pt_stride;
  int n_pages;
  uint16_t* out;
  int rows;
  float* scores;
  int32_t* topk;
  float scale;
  Mail mail;
  GuardArgs guard;
};

MONO_DEV uint32_t radix_key(float f) {
  const uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
MONO_DEV float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// FP4 x FP4 16x16x128 with per-lane E8M0 scales; the B scale byte is picked by OPB.
template <int OPB>
MONO_DEV f32x4 mfma_fp4_opb(const u32x4& a, const u32x4& b, int sa, int sb) {
  const i32x8 A = {(int)a[0], (int)a[1], (int)a[2], (int)a[3], 0, 0, 0, 0};
  const i32x8 B = {(int)b[0], (int)b[1], (int)b[2], (int)b[3], 0, 0, 0, 0};
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, z, 4, 4, 0, sa, OPB, sb);
}

// 8 E4M3 bytes -> 8 bf16 (exact: every E4M3 value is a bf16 value)
MONO_DEV bf16x8 fp8x8_bf16(u32x2 w) {
  u32x4 o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const f32x2 lo = fp8x2_unpack<false>(w[h]), hi = fp8x2_unpack<true>(w[h]);
    o[2 * h] = (__float_as_uint(lo[0]) >> 16) | (__float_as_uint(lo[1]) & 0xffff0000u);
    o[2 * h + 1] = (__float_as_uint(hi[0]) >> 16) | (__float_as_uint(hi[1]) & 0xffff0000u);
  }
  return __builtin_bit_cast(bf16x8, o);
}

class Step {
 public:
  MONO_DEV Step(const Args& a, Lds& l) : A(a), L(l) {
    tid = threadIdx.x;
    lane = tid % WAVE;
    wave = tid / WAVE;
    g = lane / 16;
    r = lane % 16;
    G = gridDim.x;
    CH = a.mail.max_ctx / CHUNK;
  }

  MONO_DEV void run() {
    if (tid == 0) {
      const uint32_t ticket = __hip_atomic_fetch_add(&A.guard.words[G_TICKET], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
      L.tag = ticket / (uint32_t)G + 1u;
      L.err = ld_agent_u32(&A.guard.words[G_ERROR]);
    }
    __syncthreads();
    if (L.err != 0) return;
    gd.a = A.guard;
    gd.tag = L.tag;
    gd.deadline = now_ticks() + A.guard.deadline_ticks;
    const int n_score = A.rows * CH, n_topk = A.rows, n_split = A.rows * SPLITS, n_merge = A.rows * (NH / 4);
    const int total = n_score + n_topk + n_split + n_merge;
    for (int T = blockIdx.x; T < total; T += G) {
      bool ok = true;
      if (T < n_score) {
        score_task(T / CH, T % CH);
      } else if (T < n_score + n_topk) {
        ok = topk_task(T - n_score);
      } else if (T < n_score + n_topk + n_split) {
        const int j = T - n_score - n_topk;
        ok = split_task(j / SPLITS, j % SPLITS);
      } else {
        const int j = T - n_score - n_topk - n_split;
        ok = merge_task(j / (NH / 4), j % (NH / 4));
      }
      if (!ok) return;  // workgroup-uniform
    }
  }

 private:
  const Args& A;
  Lds& L;
  Guard gd;
  int tid, lane, wave, g, r, G, CH;

  MONO_DEV int row_len(int s) const { return min(max(A.seq_lens[s], 0), A.mail.max_ctx); }
  MONO_DEV int page_of(int s, int p) const {
    const int pg = A.pt[(size_t)s * A.pt_stride + p / PAGE];
    return min(max(pg, 0), A.n_pages - 1);
  }
  MONO_DEV int slot_of(int s, int p) const { return page_of(s, p) * PAGE + p % PAGE; }

  // ---------------------------------------------------------------- score
  MONO_DEV void score_task(int s, int c) {
    const int n = row_len(s);
    const int k0 = c * CHUNK + wave * KEYS_WAVE;
    if (k0 >= n) return;  // wave-uniform; the task has no barrier
    // the row's query: head tile ht is rows 16 ht .. of the 64 heads
    u32x4 qa[IH / 16];
    int qsc[IH / 16];
    float wv[IH / 16][4];
#pragma unroll
    for (int ht = 0; ht < IH / 16; ++ht) {
      const size_t row = (size_t)s * IH + 16 * ht + r;
      qa[ht] = ld_u32x4(A.iq + row * (ID / 2) + g * 16);
      qsc[ht] = A.iqs[row * (ID / 32) + g];
      const u32x2 w4 = *reinterpret_cast<const u32x2*>(A.iw + (size_t)s * IH + 16 * ht + 4 * g);
      wv[ht][0] = bf16_lo(w4[0]);
      wv[ht][1] = bf16_hi(w4[0]);
      wv[ht][2] = bf16_lo(w4[1]);
      wv[ht][3] = bf16_hi(w4[1]);
    }
    // 128 keys = 2 pages = 8 tiles of 16 keys: lane (g, r) holds chunk g of key 16 t + r
    const int p0 = k0 / PAGE;
    int pg[KEYS_WAVE / PAGE];
    uint32_t ks[KEYS_WAVE / PAGE];
#pragma unroll
    for (int i = 0; i < KEYS_WAVE / PAGE; ++i) pg[i] = page_of(s, (p0 + i) * PAGE);
    u32x4 kb[KTILES];
#pragma unroll
    for (int kt = 0; kt < KTILES; ++kt) {
      const int page = pg[kt / 4];
      kb[kt] = ld_nt_u32x4(A.ikv + ((size_t)(page * 4 + g) * PAGE + (kt % 4) * 16 + r) * 16);
    }
#pragma unroll
    for (int i = 0; i < KEYS_WAVE / PAGE; ++i)
      ks[i] = *reinterpret_cast<const uint32_t*>(A.iks + (size_t)(pg[i] * 4 + g) * PAGE + r * 4);
#pragma unroll
    for (int kt = 0; kt < KTILES; ++kt) {
      float part = 0.f;
#pragma unroll
      for (int ht = 0; ht < IH / 16; ++ht) {
        f32x4 d;
        switch (kt % 4) {
          case 0: d = mfma_fp4_opb<0>(qa[ht], kb[kt], qsc[ht], (int)ks[kt / 4]); break;
          case 1: d = mfma_fp4_opb<1>(qa[ht], kb[kt], qsc[ht], (int)ks[kt / 4]); break;
          case 2: d = mfma_fp4_opb<2>(qa[ht], kb[kt], qsc[ht], (int)ks[kt / 4]); break;
          default: d = mfma_fp4_opb<3>(qa[ht], kb[kt], qsc[ht], (int)ks[kt / 4]); break;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) part += wv[ht][i] * fmaxf(d[i], 0.f);
      }
      part += __shfl_xor(part, 16, WAVE);
      part += __shfl_xor(part, 32, WAVE);
      const int pos = k0 + kt * 16 + r;
      if (g == 0 && pos < n) {
        mb_putf(&A.mail.score[(size_t)s * A.mail.max_ctx + pos], part, gd.tag);
        if (A.scores) A.scores[(size_t)s * A.mail.max_ctx + pos] = part;
      }
    }
  }

  // ---------------------------------------------------------------- top-k
  // exclusive prefix sum of v over the workgroup (a full barrier); total to *tot
  MONO_DEV int block_excl_scan(int v, int* tot) {
    int incl = v;
#pragma unroll
    for (int o = 1; o < WAVE; o <<= 1) {
      const int y = __shfl_up(incl, o, WAVE);
      if (lane >= o) incl += y;
    }
    if (lane == WAVE - 1) L.scan[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < AW; ++w) {
      const int t = L.scan[w];
      before += w < wave ? t : 0;
      all += t;
    }
    __syncthreads();
    if (tot) *tot = all;
    return before + incl - v;
  }

  MONO_DEV void publish_sel(int s, int j, int slot) {
    mb_put(&A.mail.sel[(size_t)s * TOPK + j], (uint32_t)slot, gd.tag);
    if (A.topk) A.topk[(size_t)s * TOPK + j] = slot;
  }

  MONO_DEV bool topk_task(int s) {
    const int n = row_len(s);
    if (n <= TOPK) {  // every key is selected; no score is needed
      for (int j = tid; j < TOPK; j += AT) publish_sel(s, j, j < n ? slot_of(s, j) : -1);
      return true;
    }
    uint32_t* kl = L.u.t.kl;
    const int p0 = tid * KPT;
    const int cnt = min(max(n - p0, 0), KPT);
    const int kb = p0 + tid;  // padded LDS base of this thread's range
    const uint64_t* sc = &A.mail.score[(size_t)s * A.mail.max_ctx + p0];
    bool ok = true;
#pragma unroll 1
    for (int b = 0; b < KPT / 16; ++b) {
      const int have = min(max(cnt - b * 16, 0), 16);
      const uint32_t pending = have >= 16 ? 0xffffu : (1u << have) - 1u;
      uint32_t v[16];
      const uint64_t* base = sc + b * 16;
      if (ok) ok = poll_words<16>([base](int q) { return base + q; }, v, pending, W_SCORE, gd);
#pragma unroll
      for (int q = 0; q < 16; ++q)
        if (q < have) kl[kb + b * 16 + q] = radix_key(__uint_as_float(v[q]));
    }
    if (!block_all(ok)) return false;
    // MSB-first 8-bit radix select of the TOPK-th largest key
    uint32_t prefix = 0, mask = 0;
    int need = TOPK;
#pragma unroll 1
    for (int shift = 24; shift >= 0; shift -= 8) {
      if (tid < 256) L.u.t.hist[tid] = 0u;
      __syncthreads();
      for (int q = 0; q < cnt; ++q) {
        const uint32_t k = kl[kb + q];
        if ((k & mask) == prefix) atomicAdd(&L.u.t.hist[(k >> shift) & 0xffu], 1u);
      }
      __syncthreads();
      if (wave == 0) {
        int c[4], tot = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c[j] = (int)L.u.t.hist[255 - 4 * lane - j];
          tot += c[j];
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < WAVE; o <<= 1) {
          const int y = __shfl_up(incl, o, WAVE);
          if (lane >= o) incl += y;
        }
        const int excl = incl - tot;
        if (excl < need && need <= incl) {
          int run = excl;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (run + c[j] >= need) {
              L.u.t.digit = (uint32_t)(255 - 4 * lane - j);
              L.u.t.above = run;
              break;
            }
            run += c[j];
          }
        }
      }
      __syncthreads();
      need -= L.u.t.above;
      prefix |= L.u.t.digit << shift;
      mask |= 0xffu << shift;
      __syncthreads();
    }
    // stable compaction: keys above the threshold, then the lowest positions equal to it
    const uint32_t T = prefix;
    int c_gt = 0, c_eq = 0;
    for (int q = 0; q < cnt; ++q) {
      const uint32_t k = kl[kb + q];
      c_gt += k > T;
      c_eq += k == T;
    }
    const int eq_before = block_excl_scan(c_eq, nullptr);
    const int take = min(max(need - eq_before, 0), c_eq);
    int idx = block_excl_scan(c_gt + take, nullptr);
    int te = 0;
    for (int q = 0; q < cnt; ++q) {
      const uint32_t k = kl[kb + q];
      const bool eq = k == T;
      if ((k > T || (eq && te < take)) && idx < TOPK) {
        te += eq;
        publish_sel(s, idx++, slot_of(s, p0 + q));
      }
    }
    __syncthreads();  // the LDS keys are reused by the next task
    return true;
  }

  // ---------------------------------------------------------------- split
  MONO_DEV bool split_task(int s, int j) {
    SplitLds& P = L.u.sp;
    const int nsel = min(row_len(s), TOPK);
    const int lo = j * SPLIT;
    const int cnt = min(max(nsel - lo, 0), SPLIT);
    const size_t mlb = ((size_t)s * SPLITS + j) * NH;
    if (cnt == 0) {  // an empty split contributes nothing to the merge
      if (tid < NH) {
        mb_putf(&A.mail.ml[(mlb + tid) * 2], NEG_INF, gd.tag);
        mb_putf(&A.mail.ml[(mlb + tid) * 2 + 1], 0.f, gd.tag);
      }
      return true;
    }
    for (int f = tid; f < NH * DQK / 8; f += AT) {
      const int h = f / (DQK / 8), c8 = f % (DQK / 8);
      *reinterpret_cast<u32x4*>(&P.q[h][c8 * 8]) = ld_u32x4(A.q + ((size_t)s * NH + h) * DQK + c8 * 8);
    }
    bool ok = true;
    if (tid < SPLIT) {
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

    const int ht = wave / 4, tt = wave % 4;  // logit tile of this wave
    f32x4 acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[4] = {NEG_INF, NEG_INF, NEG_INF, NEG_INF}, l_run[4] = {0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
    for (int st = 0; st < NSUB && st * SUB < cnt; ++st) {
      // gather 64 cached rows: consecutive lanes read consecutive 16-byte chunks of a row
      for (int f = tid; f < SUB * (DQK / 16); f += AT) {
        const int t = f / (DQK / 16), c = f % (DQK / 16);
        const int slot = P.slot[st * SUB + t];
        u32x4 v = {0u, 0u, 0u, 0u};
        if (slot >= 0) v = ld_nt_u32x4(A.kv + (size_t)slot * DQK + c * 16);
        *reinterpret_cast<u32x4*>(&P.kv[t][c * 16]) = v;
        if (c < DV / 16) {
#pragma unroll
          for (int b = 0; b < 16; ++b) P.vt[c * 16 + b][t] = (uint8_t)(v[b / 4] >> (8 * (b % 4)));
        }
      }
      if (tid < SUB) {
        const int slot = P.slot[st * SUB + tid];
        P.kvs[tid] = slot >= 0 ? A.kv_scale[slot] : 0.f;
      }
      __syncthreads();
      // logits of 16 heads x 16 tokens a wave: K = 576 in 18 bf16 steps
      {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < DQK / 32; ++ks) {
          const bf16x8 qa = *reinterpret_cast<const bf16x8*>(&P.q[16 * ht + r][32 * ks + 8 * g]);
          const bf16x8 kb = fp8x8_bf16(*reinterpret_cast<const u32x2*>(&P.kv[16 * tt + r][32 * ks + 8 * g]));
          d = mfma_bf16(qa, kb, d);
        }
        const int t = 16 * tt + r;
        const bool valid = st * SUB + t < cnt && P.slot[st * SUB + t] >= 0;
        const float sc = P.kvs[t] * A.scale;
#pragma unroll
        for (int i = 0; i < 4; ++i) P.pf[16 * ht + 4 * g + i][t] = valid ? d[i] * sc : NEG_INF;
      }
      __syncthreads();
      // online softmax of heads 4 wave .. 4 wave + 3; lane = token
#pragma unroll
      for (int hh = 0; hh < 4; ++hh) {
        const int h = 4 * wave + hh;
        const float x = P.pf[h][lane];
        const float m_new = fmaxf(m_run[hh], wave_max(x));
        const float p = (m_new == NEG_INF || x == NEG_INF) ? 0.f : hw_exp(x - m_new);
        const float alpha = m_run[hh] == NEG_INF ? (m_new == NEG_INF ? 1.f : 0.f) : hw_exp(m_run[hh] - m_new);
        l_run[hh] = l_run[hh] * alpha + wave_sum(p);
        m_run[hh] = m_new;
        P.pb[h][lane] = f32_to_bf16_bits(p * P.kvs[lane]);
        if (lane == 0) P.alpha[h] = alpha;
      }
      __syncthreads();
      // o[32 heads x 64 dims of this wave] = alpha o + p . v
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) al[i] = P.alpha[16 * a + 4 * g + i];
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[a][b][i] *= al[i];
      }
#pragma unroll
      for (int kt = 0; kt < SUB / 32; ++kt) {
        bf16x8 pa[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) pa[a] = *reinterpret_cast<const bf16x8*>(&P.pb[16 * a + r][32 * kt + 8 * g]);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const bf16x8 vb = fp8x8_bf16(*reinterpret_cast<const u32x2*>(&P.vt[16 * (4 * wave + b) + r][32 * kt + 8 * g]));
#pragma unroll
          for (int a = 0; a < 2; ++a) acc[a][b] = mfma_bf16(pa[a], vb, acc[a][b]);
        }
      }
      __syncthreads();
    }
    const size_t pb = ((size_t)s * SPLITS + j) * NH;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int h = 16 * a + 4 * g + i, dim = 16 * (4 * wave + b) + r;
          mb_putf(&A.mail.part[(pb + h) * DV + dim], acc[a][b][i], gd.tag);
        }
    if (lane < 4) {
      const float m = lane == 0 ? m_run[0] : lane == 1 ? m_run[1] : lane == 2 ? m_run[2] : m_run[3];
      const float l = lane == 0 ? l_run[0] : lane == 1 ? l_run[1] : lane == 2 ? l_run[2] : l_run[3];
      const int h = 4 * wave + lane;
      mb_putf(&A.mail.ml[(mlb + h) * 2], m, gd.tag);
      mb_putf(&A.mail.ml[(mlb + h) * 2 + 1], l, gd.tag);
    }
    return true;
  }

  // ---------------------------------------------------------------- merge
  MONO_DEV bool merge_task(int s, int hg) {
    const int h = 4 * hg + tid / 128, d0 = (tid % 128) * 4;
    const size_t rb = (size_t)s * SPLITS;
    uint32_t ml[2 * SPLITS];
    const uint64_t* mlp = &A.mail.ml[(rb * NH + h) * 2];
    bool ok = poll_words<2 * SPLITS>([mlp](int q) { return mlp + (size_t)(q / 2) * NH * 2 + q % 2; }, ml,
                                     (1u << (2 * SPLITS)) - 1u, W_PART, gd);
    float M = NEG_INF;
    uint32_t live = 0;
#pragma unroll
    for (int j = 0; j < SPLITS; ++j) {
      if (__uint_as_float(ml[2 * j + 1]) > 0.f) {
        M = fmaxf(M, __uint_as_float(ml[2 * j]));
        live |= 0xfu << (4 * j);
      }
    }
    uint32_t av[4 * SPLITS];
    const uint64_t* ap = &A.mail.part[(rb * NH + h) * DV + d0];
    if (ok) ok = poll_words<4 * SPLITS>([ap](int q) { return ap + (size_t)(q / 4) * NH * DV + q % 4; }, av, live, W_PART, gd);
    float o[4] = {0.f, 0.f, 0.f, 0.f}, den = 0.f;
#pragma unroll
    for (int j = 0; j < SPLITS; ++j) {
      if ((live >> (4 * j)) & 1u) {
        const float w = hw_exp(__uint_as_float(ml[2 * j]) - M);
        den += w * __uint_as_float(ml[2 * j + 1]);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] += w * __uint_as_float(av[4 * j + i]);
      }
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    u32x2 packed;
    packed[0] = pack_bf16x2(o[0] * inv, o[1] * inv);
    packed[1] = pack_bf16x2(o[2] * inv, o[3] * inv);
    if (ok) *reinterpret_cast<u32x2*>(A.out + ((size_t)s * NH + h) * DV + d0) = packed;
    return block_all(ok);
  }
};

__global__ __launch_bounds__(AT, 1) void k_attn(Args args) {
  __shared__ Lds lds;
  Step st(args, lds);
  st.run();
}

}  // namespace

hipError_t attn_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_attn, AT, 0);
}

hipError_t attn_forward(const AttnArgs& g, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st) {
  if (g.rows < 1 || g.rows > MAX_ROWS || grid < 1 || mail.max_ctx % CHUNK || mail.max_ctx > MAX_CTX)
    return hipErrorInvalidConfiguration;
  Args a;
  a.iq = static_cast<const uint8_t*>(g.iq);
  a.iqs = static_cast<const uint8_t*>(g.iqs);
  a.iw = static_cast<const uint16_t*>(g.iw);
  a.ikv = static_cast<const uint8_t*>(g.ikv);
  a.iks = static_cast<const uint8_t*>(g.iks);
  a.q = static_cast<const uint16_t*>(g.q);
  a.kv = static_cast<const uint8_t*>(g.kv);
  a.kv_scale = g.kv_scale;
  a.pt = g.page_table;
  a.seq_lens = g.seq_lens;
  a.pt_stride = g.pt_stride;
  a.n_pages = g.n_pages;
  a.out = static_cast<uint16_t*>(g.out);
  a.rows = g.rows;
  a.scores = g.scores;
  a.topk = g.topk;
  a.scale = g.softmax_scale;
  a.mail = mail;
  a.guard = guard;
  k_attn<<<grid, AT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace attn
}  // namespace mono
