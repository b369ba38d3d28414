// The sparse-attention launch for steps above LONG_ROWS rows (k_attn_long): the phase
// of attn_step.h with fewer, longer splits (splits_of) and merges of several heads, so
// a step's splits and its merges each fill one round of the grid. A kernel of its own:
// the long splits' sub-tile loop would otherwise share registers and code with the
// one-sub-tile splits of the smaller steps.
#define MONO_ATTN_LONG 1
#include "attn_step.h"

namespace mono {
namespace attn {

namespace {

__global__ __launch_bounds__(AT, 1) void k_attn_long(Args args) {
  __shared__ Lds lds;
  Step st(args, lds);
  st.run();
}

}  // namespace

hipError_t attn_long_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_attn_long, AT, 0);
}

hipError_t attn_long_forward(const AttnArgs& g, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st) {
  if (g.rows <= LONG_ROWS || g.rows > WIDE_ROWS || grid < 1 || mail.max_ctx % CHUNK || mail.max_ctx > MAX_CTX)
    return hipErrorInvalidConfiguration;
  Args a;
  fill_args(a, g, mail, guard);
  k_attn_long<<<grid, AT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace attn
}  // namespace mono
