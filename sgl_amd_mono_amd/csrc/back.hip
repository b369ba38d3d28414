// The back launch (k_back) and its host side; the stages are in back_impl.h.
#include "back_impl.h"

namespace mono {
namespace proj {

namespace {

__global__ __launch_bounds__(FT, 1) void k_back(Args args) {
  __shared__ Lds lds;
  Back b(args, lds);
  b.run();
}

}  // namespace

hipError_t back_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_back, FT, 0);
}

hipError_t back_forward(const mono_proj_weights& w, const mono_back_args& a, int grid, const Mail& mail,
                        const GuardArgs& guard, hipStream_t st) {
  if (a.rows < 1 || a.rows > MAX_ROWS || grid < 1) return hipErrorInvalidConfiguration;
  Args args;
  args.w = w;
  args.a = a;
  args.mail = mail;
  args.guard = guard;
  k_back<<<grid, FT, 0, st>>>(args);
  return hipGetLastError();
}

}  // namespace proj
}  // namespace mono
