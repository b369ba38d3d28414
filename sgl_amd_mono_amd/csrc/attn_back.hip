// The sparse attention and the back of the attention block (W_UV, o_proj, residual) as
// ONE persistent launch: every workgroup walks its attention tasks (attn_step.h), then
// its back tasks (back_impl.h), dealt round-robin from one list in which the back's
// tasks follow the attention's. A workgroup whose attention work is done starts its
// back task at once: W_UV and W_o go out while the last splits and merges still run,
// and nothing waits for a launch boundary. The back's mailboxes are the attention
// runtime's own and carry the attention launch's tag; a failed wait in either part
// stops the launch through the attention runtime's guard.
#include "attn_back_ops.h"
#include "attn_step.h"
#include "back_impl.h"

namespace mono {
namespace fused {

namespace {

// the launches that hold the attention with other phases take at most proj::MAX_ROWS
// rows: their attention has one sub-tile a split (no long splits compiled in)
static_assert(proj::MAX_ROWS <= attn::LONG_ROWS, "fused launches: short splits only");

struct Args {
  attn::Args at;
  proj::Args bk;
};

union Lds {
  attn::Lds at;
  proj::Lds bk;
};

__global__ __launch_bounds__(512, 1) void k_attn_back(Args args) {
  __shared__ Lds lds;
  attn::Step st(args.at, lds.at);
  // a failed or refused launch writes NaN over its output `a`
  const auto poison = [&](bool share) { poison_bf16(args.bk.a.a, (size_t)args.bk.a.rows * proj::HIDDEN, share); };
  if (!st.begin()) return poison(true);
  const Guard g = st.guard();
  if (!st.tasks()) return poison(false);
  __syncthreads();  // the LDS passes from the attention's layout to the back's
  proj::Back bk(args.bk, lds.bk);
  bk.adopt(g, args.at.mail.mdone);
  if (!bk.tasks(st.n_tasks())) poison(false);
}

}  // namespace

hipError_t attn_back_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_attn_back, 512, 0);
}

hipError_t attn_back_forward(const attn::AttnArgs& g, const attn::Mail& mail, const GuardArgs& guard,
                             const mono_proj_weights& w, const mono_back_args& b, const proj::Mail& bmail, int grid,
                             hipStream_t st) {
  if (g.rows < 1 || g.rows > attn::MAX_ROWS || g.rows > proj::MAX_ROWS || b.rows != g.rows || grid < 1 ||
      mail.max_ctx % attn::CHUNK || mail.max_ctx > attn::MAX_CTX)
    return hipErrorInvalidConfiguration;
  Args a;
  attn::fill_args(a.at, g, mail, guard);
  a.at.publish_out = true;
  a.bk.w = w;
  a.bk.a = b;
  a.bk.mail = bmail;
  a.bk.guard = guard;
  k_attn_back<<<grid, 512, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace fused
}  // namespace mono
