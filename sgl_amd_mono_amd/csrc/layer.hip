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
#include <algorithm>

#include "layer_impl.h"

namespace mono {
namespace layer {

namespace {

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

// The whole decoder layer as one launch.
__global__ __launch_bounds__(512, 1) void k_layer(LayerArgs args) {
  __shared__ LayerLds lds;
  Guard g;
  if (!guard_begin(args.tail.at.guard, g)) return poison(args.tail, true);
  if (!run_layer(args, lds, g, false)) poison(args.tail, false);
}

}  // namespace

hipError_t tail_occupancy(int* blocks_per_cu) {
  int a = 0, b = 0, c = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k_layer_tail, 512, 0);
  if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k_layer, 512, 0);
  if (e == hipSuccess) e = stack_occupancy(&c);
  *blocks_per_cu = std::min(a, std::min(b, c));
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
  if (grid < 1) return hipErrorInvalidConfiguration;
  LayerArgs a;
  const hipError_t e = fill_layer(a, w, f, fmail, kv_mask, g, amail, guard, b, bmail, m, mmail, a_done, ticks);
  if (e != hipSuccess) return e;
  k_layer<<<grid, 512, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace layer
}  // namespace mono
