// Host-side declarations of the MoE phase's launchers (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "mono.h"
#include "moe_plan.h"

namespace mono {
namespace moe {

struct MoeGeom {
  int hidden, n_experts, top_k, inter;
};

// The C-ABI argument blocks, with the runtime's scalars folded in.
struct MoeFp8Args : mono_moe_fp8_args {
  float route_scale;
  float eps;
  MoeFp8Args(const mono_moe_fp8_args& a, float rs, float e) : mono_moe_fp8_args(a), route_scale(rs), eps(e) {}
  const uint16_t* a16() const { return static_cast<const uint16_t*>(a); }
};

// Optional routing outputs of the router's last workgroup.
struct MoeRouteOut {
  float* scores;
  int32_t* topk_ids;
  float* topk_w;
};

bool moe_fp8_supported(const MoeGeom& geo);
hipError_t moe_fp8_forward(const MoeFp8Args& g, const MoeGeom& geo, int n_cu, Scratch sc, hipStream_t st);

}  // namespace moe
}  // namespace mono
