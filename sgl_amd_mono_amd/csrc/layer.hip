// The decoder layer after its projections' front as ONE persistent launch: the sparse
// attention (attn_step.h), the back of the attention block (back_impl.h: W_UV, o_proj,
// residual) and the FP8 MoE with its residual (moe_fp8_step.h), dealt to every
// workgroup in that order. The reference runs the same phases inside its single
// decoder-layer launch (glm53/gfx950/kernel.py:2684-5187).
//
// Hand-offs between the phases: each merge puts a done word for the back's W_UV (as
// in attn_back.hip); each o_proj tile stores its rows of `a` with device-coherent
// stores and then a replicated done word, which every workgroup's MoE waits for before
// reading `a`. A workgroup done with its attention and back tasks issues its router
// weight loads (and, for the shared expert's up tiles, its first expert weights) while
// the last o_proj tiles still run. All phases run under the attention runtime's guard
// and tag; the back's sites are 4 and 5, the MoE's are MOE_SITE0 + 0..4.
#include "attn_step.h"
#include "back_impl.h"
#include "front_impl.h"
#include "layer_ops.h"
#include "moe_fp8_step.h"

namespace mono {
namespace layer {

namespace {

struct Args {
  attn::Args at;
  proj::Args bk;
  moe::Args mo;
  uint64_t* a_done;
  int64_t* ticks;  // [grid][16] phase ticks (NULL: none)
};

// the layer's moments in a workgroup's tick row (4 and 6-10: the MoE's, moe_fp8_step.h)
enum { T_BEGIN = 0, T_FRONT = 1, T_ATTN = 2, T_BACK = 3, T_END = 5, T_WORDS = 16 };

MONO_DEV void stamp(int64_t* ticks, int k) {
  if (ticks && threadIdx.x == 0) ticks[blockIdx.x * T_WORDS + k] = (int64_t)now_ticks();
}

union Lds {
  attn::Lds at;
  proj::Lds bk;
  moe::Lds mo;
};

struct LayerArgs {
  proj::fr::Args fr;
  Args tail;
};

union LayerLds {
  Lds tail;
  proj::fr::Lds fr;
};

// A failed or refused launch writes NaN over the layer's output x_out (sync.h).
MONO_DEV void poison(const Args& args, bool share) {
  poison_bf16(args.mo.out, (size_t)args.mo.rows * moe::H, share);
}

// The back and the MoE after the attention, on the attention's guard (false: a wait
// failed).
MONO_DEV bool back_moe(const Args& args, Lds& lds, const attn::Step& st, const Guard& g) {
  __syncthreads();  // the LDS passes from the attention's layout to the back's
  {
    proj::Back bk(args.bk, lds.bk);
    bk.adopt(g, args.at.mail.mdone);
    bk.publish_a(args.a_done);
    if (!bk.tasks(st.n_tasks())) return false;
  }
  stamp(args.ticks, T_BACK);
  __syncthreads();  // and to the MoE's
  moe::Step ms(args.mo, lds.mo);
  ms.adopt(g, args.a_done, proj::NT_O, MOE_SITE0);
  bool refused;
  if (!ms.run(refused)) return false;
  stamp(args.ticks, T_END);
  return true;
}

__global__ __launch_bounds__(512, 1) void k_layer_tail(Args args) {
  __shared__ Lds lds;
  attn::Step st(args.at, lds.at);
  if (!st.begin()) return poison(args, true);
  stamp(args.ticks, T_BEGIN);
  const Guard g = st.guard();
  if (!st.tasks()) return poison(args, false);
  stamp(args.ticks, T_ATTN);
  if (!back_moe(args, lds, st, g)) poison(args, false);
}

// The whole decoder layer: the front's tasks first (under the attention's tag), then
// the attention, whose score tasks and splits wait on the front's done words.
__global__ __launch_bounds__(512, 1) void k_layer(LayerArgs args) {
  __shared__ LayerLds lds;
  attn::Step st(args.tail.at, lds.tail.at);
  if (!st.begin()) return poison(args.tail, true);  // the tag lives in registers from here on
  stamp(args.tail.ticks, T_BEGIN);
  const Guard g = st.guard();
  {
    proj::fr::Front f(args.fr, lds.fr);
    f.adopt(g, FRONT_SITE0);
    if (!f.tasks()) return poison(args.tail, false);
  }
  stamp(args.tail.ticks, T_FRONT);
  __syncthreads();  // the LDS passes from the front's layout to the attention's
  if (!st.tasks()) return poison(args.tail, false);
  stamp(args.tail.ticks, T_ATTN);
  if (!back_moe(args.tail, lds.tail, st, g)) poison(args.tail, false);
}

}  // namespace

hipError_t tail_occupancy(int* blocks_per_cu) {
  int a = 0, b = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k_layer_tail, 512, 0);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_layer, 512, 0);
  *blocks_per_cu = a < b ? a : b;
  return e;
}

hipError_t tail_forward(const attn::AttnArgs& g, const attn::Mail& amail, const GuardArgs& guard,
                        const mono_proj_weights& w, const mono_back_args& b, const proj::Mail& bmail,
                        const moe::MoeFp8Args& m, const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks, int grid,
                        hipStream_t st) {
  if (g.rows < 1 || g.rows > attn::MAX_ROWS || g.rows > proj::MAX_ROWS || g.rows > moe::MAX_ROWS || b.rows != g.rows ||
      m.rows != g.rows || grid < 1 || amail.max_ctx % attn::CHUNK || amail.max_ctx > attn::MAX_CTX)
    return hipErrorInvalidConfiguration;
  Args a;
  attn::fill_args(a.at, g, amail, guard);
  a.at.publish_out = true;
  a.bk.w = w;
  a.bk.a = b;
  a.bk.mail = bmail;
  a.bk.guard = guard;
  moe::fill_args(a.mo, m, mmail, guard);
  a.a_done = a_done;
  a.ticks = ticks;
  a.mo.ticks = ticks;
  k_layer_tail<<<grid, 512, 0, st>>>(a);
  return hipGetLastError();
}

hipError_t layer_forward(const mono_proj_weights& w, const mono_front_args& f, const proj::Mail& fmail,
                         int kv_mask, const attn::AttnArgs& g, const attn::Mail& amail, const GuardArgs& guard,
                         const mono_back_args& b, const proj::Mail& bmail, const moe::MoeFp8Args& m,
                         const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks, int grid, hipStream_t st) {
  if (f.rows != g.rows || f.rows < 1 || f.rows > proj::MAX_ROWS || g.rows > attn::MAX_ROWS || g.rows > moe::MAX_ROWS ||
      b.rows != g.rows || m.rows != g.rows || grid < 1 || amail.max_ctx % attn::CHUNK || amail.max_ctx > attn::MAX_CTX)
    return hipErrorInvalidConfiguration;
  LayerArgs a;
  a.fr.w = w;
  a.fr.a = f;
  a.fr.mail = fmail;
  a.fr.guard = guard;
  a.fr.kv_mask = kv_mask;
  a.fr.site0 = FRONT_SITE0;
  attn::fill_args(a.tail.at, g, amail, guard);
  a.tail.at.publish_out = true;
  a.tail.at.fdone = fmail.fdone;
  a.tail.at.fsite = ATTN_FRONT_SITE;
  a.tail.bk.w = w;
  a.tail.bk.a = b;
  a.tail.bk.mail = bmail;
  a.tail.bk.guard = guard;
  moe::fill_args(a.tail.mo, m, mmail, guard);
  a.tail.a_done = a_done;
  a.tail.ticks = ticks;
  a.tail.mo.ticks = ticks;
  k_layer<<<grid, 512, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace layer
}  // namespace mono
