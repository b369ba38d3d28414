// The sparse-attention launch (k_attn) and its host side; the stages are in
// attn_step.h.
#include "attn_step.h"

namespace mono {
namespace attn {

namespace {

__global__ __launch_bounds__(AT, 1) void k_attn(Args args) {
  __shared__ Lds lds;
  Step st(args, lds);
  st.run();
}

}  // namespace

hipError_t attn_occupancy(int* blocks_per_cu) {
  int a = 0, b = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k_attn, AT, 0);
  int c = 0;
  if (e == hipSuccess) e = attn_long_occupancy(&b);
  if (e == hipSuccess) e = attn_wide_occupancy(&c);
  *blocks_per_cu = a < b ? (a < c ? a : c) : (b < c ? b : c);
  return e;
}

// Steps above LONG_ROWS rows go to k_attn_long (attn_long.hip), whose splits are long.
hipError_t attn_forward(const AttnArgs& g, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st) {
  if (g.rows < 1 || g.rows > MAX_ROWS || grid < 1 || mail.max_ctx % CHUNK || mail.max_ctx > MAX_CTX)
    return hipErrorInvalidConfiguration;
  if (g.rows > WIDE_ROWS) return attn_wide_forward(g, grid, mail, guard, st);
  if (g.rows > LONG_ROWS) return attn_long_forward(g, grid, mail, guard, st);
  Args a;
  fill_args(a, g, mail, guard);
  k_attn<<<grid, AT, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace attn
}  // namespace mono
