// FP8 (128 x 128 block-scaled) routed + shared MoE of one decode step on gfx950, as ONE
// persistent launch: one 512-thread workgroup per CU, every workgroup resident at once.
// The phase itself (stages, task list, mailboxes) is moe_fp8_step.h.
#include "moe_fp8_step.h"

namespace mono {
namespace moe {

namespace {

__global__ __launch_bounds__(FT, 1) void k_moe_fp8(Args args) {
  __shared__ Lds lds;
  Step st(args, lds);
  bool refused;
  if (!st.run(refused)) st.poison(refused);
}

}  // namespace

bool moe_fp8_supported(const MoeGeom& geo) {
  return geo.hidden == H && geo.n_experts == E && geo.inter == I && geo.top_k == TOPK;
}

hipError_t moe_fp8_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_moe_fp8, FT, 0);
}

hipError_t moe_fp8_forward(const MoeFp8Args& g, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st) {
  if (grid < 1 || g.rows < 1 || g.rows > MAX_ROWS) return hipErrorInvalidConfiguration;
  Args a;
  fill_args(a, g, mail, guard);
  k_moe_fp8<<<grid, FT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace moe
}  // namespace mono
