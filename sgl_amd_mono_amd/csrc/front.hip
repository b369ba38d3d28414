// The front of the attention block (input RMSNorm through the index query) as ONE
// persistent launch; the phase itself is front_impl.h.
#include "front_impl.h"

namespace mono {
namespace proj {

using namespace fr;

namespace {

__global__ __launch_bounds__(FT, 1) void k_front(Args args) {
  __shared__ Lds lds;
  Front f(args, lds);
  f.run();
}

}  // namespace

hipError_t front_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_front, FT, 0);
}

hipError_t front_forward(const mono_proj_weights& w, const mono_front_args& a, int grid, const Mail& mail,
                         const GuardArgs& guard, int kv_mask, int site0, hipStream_t st) {
  if (a.rows < 1 || a.rows > MAX_ROWS || grid < 1) return hipErrorInvalidConfiguration;
  Args args;
  args.w = w;
  args.a = a;
  args.mail = mail;
  args.guard = guard;
  args.kv_mask = kv_mask;
  args.site0 = site0;
  args.h_ssq = nullptr;
  args.h_site = 0;
  k_front<<<grid, FT, 0, st>>>(args);
  return hipGetLastError();
}

}  // namespace proj
}  // namespace mono
