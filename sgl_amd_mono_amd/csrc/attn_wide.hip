// The sparse-attention launch for steps above WIDE_ROWS rows (k_attn_wide): attn_step.h's
// long-split phase built with 4 even splits a row only (attn_long.hip holds 8 or 5).
#define MONO_ATTN_LONG 1
#define MONO_ATTN_WIDE 1
#include "attn_step.h"

namespace mono {
namespace attn {

namespace {

__global__ __launch_bounds__(AT, 1) void k_attn_wide(Args args) {
  __shared__ Lds lds;
  Step st(args, lds);
  st.run();
}

}  // namespace

hipError_t attn_wide_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_attn_wide, AT, 0);
}

hipError_t attn_wide_forward(const AttnArgs& g, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st) {
  if (g.rows <= WIDE_ROWS || g.rows > MAX_ROWS || grid < 1 || mail.max_ctx % CHUNK || mail.max_ctx > MAX_CTX)
    return hipErrorInvalidConfiguration;
  Args a;
  fill_args(a, g, mail, guard);
  k_attn_wide<<<grid, AT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace attn
}  // namespace mono
