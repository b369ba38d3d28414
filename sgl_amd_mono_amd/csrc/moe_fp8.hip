// FP8 (128 x 128 block-scaled) routed + shared MoE of one decode step on gfx950.
//
// The post-attention half of the decoder layer (reference: glm53/gfx950/kernel.py
// stages 8-10, :4199-5187, W8A8 mode) as four stream-ordered kernels:
//
//   prep    one workgroup a row: RMSNorm statistics, FP8 quantisation of the normed
//           row in 128-blocks (amax / 448, hardware rcp, kernel.py:1440-1450)
//   router  bf16 MFMA GEMV split over 16-expert x 896-k tiles; the last workgroup to
//           arrive sums the K slices, applies the sigmoid, picks each row's top-8 by
//           f32(score + bias) with lowest-id ties (kernel.py:1575-1629) and writes the
//           step's plan: the distinct experts (shared expert last), their row masks
//           and route weights
//   up      persistent loop over (expert, 16-channel tile): FP8 x FP8 MFMA
//           (v_mfma_scale_f32_16x16x128_f8f6f4, unit E8M0 scales) with the f32 block
//           scales applied per 128-k, SiLU(gate) * up; the last tile of a 128-channel
//           block to arrive quantises that block of mid to FP8 (kernel.py:5118-5125)
//   down    one workgroup per 16 output rows, looping over the plan's experts: FP8
//           MFMA, x weight block scale x (mid scale x route weight), summed in plan
//           order, + the residual, bf16 out (kernel.py:5001-5187, TP reduce dropped)
//
// Weights stream once with nontemporal dwordx4 loads issued in batches before the
// MFMAs that consume them. Activation columns of rows that do not route to an expert
// load nothing and contribute zero.
#include "common.h"
#include "moe_plan.h"
#include "moe_ops.h"

namespace mono {
namespace moe {

constexpr int THREADS = 256;
constexpr int WAVES = THREADS / WAVE;

// ------------------------------------------------------------------ prep
template <int H>
__global__ __launch_bounds__(THREADS) void k_prep_w8a8(const uint16_t* __restrict__ a,
                                                       const uint16_t* __restrict__ gamma,
                                                       float eps, Scratch sc) {
  const int s = blockIdx.x;
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const uint16_t* row = a + (size_t)s * H;
  __shared__ float red[WAVES];
  float ss = 0.f;
  for (int v = threadIdx.x; v < H / 8; v += THREADS) {
    u32x4 w = ld_u32x4(row + v * 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float lo = bf16_lo(w[q]), hi = bf16_hi(w[q]);
      ss += lo * lo + hi * hi;
    }
  }
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float rstd = hw_rsq((red[0] + red[1] + red[2] + red[3]) * (1.0f / H) + eps);
  if (threadIdx.x == 0) sc.rstd[s] = rstd;
  uint16_t* xq = reinterpret_cast<uint16_t*>(sc.xq + (size_t)s * H);
  for (int b = wave; b < H / 128; b += WAVES) {
    const int k = b * 128 + lane * 2;
    const uint32_t av = *reinterpret_cast<const uint32_t*>(row + k);
    const uint32_t gv = *reinterpret_cast<const uint32_t*>(gamma + k);
    const float x0 = bf16_lo(av) * rstd * bf16_lo(gv);
    const float x1 = bf16_hi(av) * rstd * bf16_hi(gv);
    const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
    const bool nz = amax > 0.f;
    const float qs = nz ? amax * (1.0f / FP8_MAX) : 1.0f;
    const float inv = nz ? hw_rcp(amax) * FP8_MAX : 1.0f;
    const float q0 = fminf(fmaxf(x0 * inv, -FP8_MAX), FP8_MAX);
    const float q1 = fminf(fmaxf(x1 * inv, -FP8_MAX), FP8_MAX);
    xq[k / 2] = (uint16_t)fp8x2_pack(q0, q1);
    if (lane == 0) sc.xs[s * (H / 128) + b] = qs;
  }
}

// ------------------------------------------------------------------ router
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

// Every row's top-k of the finished logits and the step's plan (one workgroup).
// logit(s, e) = sum over the K slices in slice order; the candidates of lane l are
// experts l + 64 i.
template <int E, int TOPK>
MONO_DEV void finish_route_sigmoid(const MoeRouteOut& ro, const float* __restrict__ bias,
                                   int rows, float route_scale, Scratch sc) {
  static_assert(E == 256, "the lane layout holds 4 candidates a lane");
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  __shared__ uint32_t used[E + 1];
  __shared__ int pick_id[MAX_ROWS][TOPK];
  __shared__ float pick_w[MAX_ROWS][TOPK];
  for (int x = threadIdx.x; x <= E; x += THREADS) used[x] = 0;
  __syncthreads();
  for (int s = wave; s < rows; s += WAVES) {
    uint32_t key[4];
    int id[4];
    float raw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane + 64 * i;
      float lg = 0.f;
#pragma unroll
      for (int ks = 0; ks < ROUTER_SLICES; ++ks) lg += sc.rpart[(ks * MAX_ROWS + s) * E + e];
      raw[i] = sigmoid(lg);
      if (ro.scores) ro.scores[s * E + e] = raw[i];
      key[i] = radix_key(raw[i] + bias[e]);
      id[i] = e;
    }
    sort4(key, id, raw);
    float my_raw = 0.f;  // lane k < TOPK: the raw score and id of pick k
    int my_id = 0;
    for (int k = 0; k < TOPK; ++k) {
      const uint32_t m = wave_umax(key[0]);
      const uint32_t cand = key[0] == m ? 0xffffu - (uint32_t)id[0] : 0u;
      const int expert = (int)(0xffffu - wave_umax(cand));
      const bool hit = key[0] == m && id[0] == expert;
      const uint64_t bal = __ballot(hit);
      const int src = __ffsll((long long)bal) - 1;
      const float r = __shfl(raw[0], src, WAVE);
      if (lane == k) {
        my_raw = r;
        my_id = expert;
      }
      if (hit) {
        key[0] = key[1]; key[1] = key[2]; key[2] = key[3]; key[3] = 0u;
        id[0] = id[1]; id[1] = id[2]; id[2] = id[3]; id[3] = 0xffff;
        raw[0] = raw[1]; raw[1] = raw[2]; raw[2] = raw[3]; raw[3] = 0.f;
      }
    }
    // sum of the picks' raw scores in the butterfly order of lanes 0..7
    float tot = lane < TOPK ? my_raw : 0.f;
#pragma unroll
    for (int o = 1; o < TOPK; o <<= 1) tot += __shfl_xor(tot, o, WAVE);
    const float w = my_raw * (hw_rcp(tot) * route_scale);
    if (lane < TOPK) {
      pick_id[s][lane] = my_id;
      pick_w[s][lane] = w;
      atomicOr(&used[my_id], 1u << s);
      if (ro.topk_ids) ro.topk_ids[s * TOPK + lane] = my_id;
      if (ro.topk_w) ro.topk_w[s * TOPK + lane] = w;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) used[E] = rows >= 32 ? 0xffffffffu : ((1u << rows) - 1u);
  __syncthreads();
  // compact the used experts in ascending id order
  __shared__ int wcount[WAVES];
  __shared__ int dmap[E + 1];
  int base = 0;
  for (int c0 = 0; c0 <= E; c0 += THREADS) {
    const int e = c0 + threadIdx.x;
    const bool f = e <= E && used[e] != 0u;
    const uint64_t bal = __ballot(f);
    const int before = __popcll(bal & ((1ull << lane) - 1ull));
    if (lane == 0) wcount[wave] = __popcll(bal);
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += wcount[w];
    if (f) {
      const int d = off + before;
      dmap[e] = d;
      sc.plan->expert[d] = e;
      sc.plan->rowmask[d] = used[e];
    }
    base += wcount[0] + wcount[1] + wcount[2] + wcount[3];
    __syncthreads();
  }
  const int n_act = base;
  for (int idx = threadIdx.x; idx < n_act * MAX_ROWS; idx += THREADS) {
    const int d = idx / MAX_ROWS, s = idx % MAX_ROWS;
    float w = 0.f;
    if (s < rows) {
      // the shared expert is the last slot
      if (d == n_act - 1) {
        w = 1.0f;
      } else {
        for (int k = 0; k < TOPK; ++k)
          if (dmap[pick_id[s][k]] == d) w = pick_w[s][k];
      }
    }
    sc.plan->weight[idx] = w;
  }
  if (threadIdx.x == 0) {
    sc.plan->n_act = n_act;
    sc.plan->rows = rows;
  }
}

// bf16(a * rstd * gamma) of 8 consecutive k, as one MFMA operand (stage_x_rmsnorm,
// kernel.py:1367-1400)
MONO_DEV bf16x8 normed8(const uint16_t* a, const uint16_t* g, float rstd) {
  const u32x4 av = ld_u32x4(a), gv = ld_u32x4(g);
  u32x4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    o[q] = pack_bf16x2(bf16_lo(av[q]) * rstd * bf16_lo(gv[q]), bf16_hi(av[q]) * rstd * bf16_hi(gv[q]));
  return __builtin_bit_cast(bf16x8, o);
}

template <int H, int E, int TOPK>
__global__ __launch_bounds__(THREADS) void k_router_sigmoid(
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ gamma,
    const uint16_t* __restrict__ w_router, const float* __restrict__ bias, int rows,
    float route_scale, MoeRouteOut ro, Scratch sc) {
  constexpr int ET = E / 16;
  constexpr int KSL = H / ROUTER_SLICES;
  constexpr int STEPS = KSL / 32 / WAVES;
  static_assert(KSL % (32 * WAVES) == 0, "router K slice");
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int et = blockIdx.x % ET, ks = blockIdx.x / ET;
  const int r = lane % 16, grp = lane / 16;
  const bool live = r < rows;
  const float rj = live ? sc.rstd[r] : 0.f;
  const uint16_t* wrow = w_router + (size_t)(et * 16 + r) * H;
  const uint16_t* arow = a + (size_t)r * H;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  u32x4 wa[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st)
    wa[st] = ld_nt_u32x4(wrow + ks * KSL + (wave * STEPS + st) * 32 + grp * 8);
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int k = ks * KSL + (wave * STEPS + st) * 32 + grp * 8;
    bf16x8 b = {};
    if (live) b = normed8(arow + k, gamma + k, rj);
    acc = mfma_bf16(__builtin_bit_cast(bf16x8, wa[st]), b, acc);
  }
  __shared__ f32x4 red[WAVES][WAVE];
  __shared__ uint32_t flag;
  red[wave][lane] = acc;
  __syncthreads();
  {
    const int l = threadIdx.x % WAVE, i = threadIdx.x / WAVE;
    const float v = red[0][l][i] + red[1][l][i] + red[2][l][i] + red[3][l][i];
    const int col = l % 16, rowi = 4 * (l / 16) + i;
    if (col < rows) sc.rpart[(ks * MAX_ROWS + col) * E + et * 16 + rowi] = v;
  }
  if (!last_arrival(sc.rcount, gridDim.x, &flag)) return;
  finish_route_sigmoid<E, TOPK>(ro, bias, rows, route_scale, sc);
}

// ------------------------------------------------------------------ up / gate

// FP8 quantisation of one 128-block of mid for every row of expert slot d (one wave a
// row), folding the route weight into the block's coefficient (kernel.py:5118-5125).
template <int I>
MONO_DEV void quant_mid_block(int d, int b, uint32_t mask, Scratch sc) {
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  for (int s = wave; s < MAX_ROWS; s += WAVES) {
    if (!((mask >> s) & 1u)) continue;
    const size_t base = ((size_t)d * MAX_ROWS + s) * I + b * 128;
    const f32x2 m = *reinterpret_cast<const f32x2*>(sc.mid + base + lane * 2);
    const float amax = wave_max(fmaxf(fabsf(m[0]), fabsf(m[1])));
    const bool nz = amax > 0.f;
    const float qs = nz ? amax * (1.0f / FP8_MAX) : 1.0f;
    const float inv = nz ? hw_rcp(amax) * FP8_MAX : 1.0f;
    const float q0 = fminf(fmaxf(m[0] * inv, -FP8_MAX), FP8_MAX);
    const float q1 = fminf(fmaxf(m[1] * inv, -FP8_MAX), FP8_MAX);
    reinterpret_cast<uint16_t*>(sc.mq + base)[lane] = (uint16_t)fp8x2_pack(q0, q1);
    if (lane == 0) sc.mcoef[((size_t)d * MAX_ROWS + s) * (I / 128) + b] = qs * sc.plan->weight[d * MAX_ROWS + s];
  }
}

template <int H, int I>
__global__ __launch_bounds__(THREADS) void k_up_w8a8(const uint8_t* __restrict__ w13,
                                                     const float* __restrict__ s13, Scratch sc) {
  constexpr int NT = I / 16;    // 16-channel tiles an expert
  constexpr int KB = H / 128;   // 128-k blocks
  constexpr int KBW = KB / WAVES;
  constexpr int BATCH = KBW % 7 == 0 ? 7 : (KBW % 4 == 0 ? 4 : (KBW % 2 == 0 ? 2 : 1));
  static_assert(KB % WAVES == 0, "K blocks split evenly over the waves");
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int r = lane % 16, grp = lane / 16;
  __shared__ f32x4 redg[WAVES][WAVE], redu[WAVES][WAVE];
  __shared__ uint32_t flag;
  const int n_items = sc.plan->n_act * NT;
  for (int t = blockIdx.x; t < n_items; t += gridDim.x) {
    const int d = t / NT, c = t % NT;
    const int e = sc.plan->expert[d];
    const uint32_t mask = sc.plan->rowmask[d];
    const uint8_t* wg = w13 + ((size_t)e * 2 * I + c * 16 + r) * H;
    const uint8_t* wu = wg + (size_t)I * H;
    const float* sg = s13 + ((size_t)e * (2 * I / 128) + (c * 16) / 128) * KB;
    const float* su = s13 + ((size_t)e * (2 * I / 128) + (I + c * 16) / 128) * KB;
    const uint8_t* xrow = sc.xq + (size_t)r * H;
    const float* xsr = sc.xs + r * KB;
    f32x4 accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int b0 = 0; b0 < KBW; b0 += BATCH) {
      // columns of rows this expert does not serve load their (finite) row anyway and
      // are never stored
      i32x8 ag[BATCH], au[BATCH], bx[BATCH];
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int k = (wave * KBW + b0 + q) * 128 + grp * 32;
        ag[q] = ld_nt_i32x8(wg + k);
        au[q] = ld_nt_i32x8(wu + k);
        bx[q] = ld_i32x8(xrow + k);
      }
#pragma unroll
      for (int q = 0; q < BATCH; ++q) {
        const int kb = wave * KBW + b0 + q;
        const float xsj = xsr[kb];
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4 cg = mfma_fp8(ag[q], bx[q], zero);
        const f32x4 cu = mfma_fp8(au[q], bx[q], zero);
        accg += cg * (sg[kb] * xsj);
        accu += cu * (su[kb] * xsj);
      }
    }
    redg[wave][lane] = accg;
    redu[wave][lane] = accu;
    __syncthreads();
    {
      const int l = threadIdx.x % WAVE, i = threadIdx.x / WAVE;
      const float g = redg[0][l][i] + redg[1][l][i] + redg[2][l][i] + redg[3][l][i];
      const float u = redu[0][l][i] + redu[1][l][i] + redu[2][l][i] + redu[3][l][i];
      const int col = l % 16, ch = 4 * (l / 16) + i;
      if ((mask >> col) & 1u) sc.mid[((size_t)d * MAX_ROWS + col) * I + c * 16 + ch] = silu(g) * u;
    }
    if (last_arrival(&sc.mcount[d * (I / 128) + c / 8], 8, &flag)) quant_mid_block<I>(d, c / 8, mask, sc);
    __syncthreads();
  }
}

// ------------------------------------------------------------------ down
template <int H, int I>
__global__ __launch_bounds__(THREADS) void k_down_w8a8(const uint8_t* __restrict__ w2,
                                                       const float* __restrict__ s2,
                                                       const uint16_t* __restrict__ a,
                                                       uint16_t* __restrict__ out,
                                                       float* __restrict__ y_out, int rows,
                                                       Scratch sc) {
  constexpr int NB = I / 128;
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int r = lane % 16, grp = lane / 16;
  const int h0 = blockIdx.x * 16;
  const int n_act = sc.plan->n_act;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int d0 = wave; d0 < n_act; d0 += 2 * WAVES) {
    // two experts' tiles in flight a wave; the second is skipped past the plan (uniform)
    i32x8 A[2][NB], B[2][NB];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int d = d0 + p * WAVES;
      if (d < n_act) {
        const int e = sc.plan->expert[d];
        const uint8_t* wrow = w2 + ((size_t)e * H + h0 + r) * I;
        const uint8_t* mrow = sc.mq + ((size_t)d * MAX_ROWS + r) * I;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          A[p][b] = ld_nt_i32x8(wrow + b * 128 + grp * 32);
          B[p][b] = ld_i32x8(mrow + b * 128 + grp * 32);
        }
      }
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int d = d0 + p * WAVES;
      if (d < n_act) {
        const int e = sc.plan->expert[d];
        // a row the expert does not serve adds nothing (a select, so stale mid bytes
        // of that row cannot reach the sum)
        const bool lv = (sc.plan->rowmask[d] >> r) & 1u;
        const float* ws = s2 + ((size_t)e * (H / 128) + h0 / 128) * NB;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float coef = sc.mcoef[((size_t)d * MAX_ROWS + r) * NB + b];
          const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
          const f32x4 c = mfma_fp8(A[p][b], B[p][b], zero);
          const f32x4 t = acc + c * (ws[b] * coef);
          acc = lv ? t : acc;
        }
      }
    }
  }
  __shared__ f32x4 red[WAVES][WAVE];
  red[wave][lane] = acc;
  __syncthreads();
  const int l = threadIdx.x % WAVE, i = threadIdx.x / WAVE;
  const float y = red[0][l][i] + red[1][l][i] + red[2][l][i] + red[3][l][i];
  const int col = l % 16, h = h0 + 4 * (l / 16) + i;
  if (col < rows) {
    const float res = bf16_bits_to_f32(a[(size_t)col * H + h]);
    out[(size_t)col * H + h] = f32_to_bf16_bits(res + y);
    if (y_out) y_out[(size_t)col * H + h] = y;
  }
}

// ------------------------------------------------------------------ host
template <int H, int E, int I, int TOPK>
static hipError_t launch_w8a8(const MoeFp8Args& g, int n_cu, Scratch sc, hipStream_t st) {
  const uint16_t* a = static_cast<const uint16_t*>(g.a);
  const uint16_t* gp = static_cast<const uint16_t*>(g.g_post);
  k_prep_w8a8<H><<<g.rows, THREADS, 0, st>>>(a, gp, g.eps, sc);
  MoeRouteOut ro{g.scores, g.topk_ids, g.topk_w};
  k_router_sigmoid<H, E, TOPK><<<(E / 16) * ROUTER_SLICES, THREADS, 0, st>>>(
      a, gp, static_cast<const uint16_t*>(g.w_router), g.bias, g.rows, g.route_scale, ro, sc);
  const int max_act = (g.rows * TOPK < E ? g.rows * TOPK : E) + 1;
  int grid_up = max_act * (I / 16);
  if (grid_up > 2 * n_cu) grid_up = 2 * n_cu;
  k_up_w8a8<H, I><<<grid_up, THREADS, 0, st>>>(static_cast<const uint8_t*>(g.w13), g.s13, sc);
  k_down_w8a8<H, I><<<H / 16, THREADS, 0, st>>>(static_cast<const uint8_t*>(g.w2), g.s2, a,
                                                static_cast<uint16_t*>(g.out), g.y, g.rows, sc);
  return hipGetLastError();
}

hipError_t moe_fp8_forward(const MoeFp8Args& g, const MoeGeom& geo, int n_cu, Scratch sc, hipStream_t st) {
  if (geo.hidden == 7168 && geo.n_experts == 256 && geo.inter == 512 && geo.top_k == 8)
    return launch_w8a8<7168, 256, 512, 8>(g, n_cu, sc, st);
  return hipErrorInvalidValue;
}

bool moe_fp8_supported(const MoeGeom& geo) {
  return geo.hidden == 7168 && geo.n_experts == 256 && geo.inter == 512 && geo.top_k == 8;
}

}  // namespace moe
}  // namespace mono
