// Host-side declarations of the MoE phase's launchers (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "mono.h"
#include "moe_plan.h"
#include "sync.h"

namespace mono {
namespace moe {

struct MoeGeom {
  int hidden, n_experts, top_k, inter;
};

// The C-ABI argument block with the runtime's scalars folded in.
struct MoeFp8Args : mono_moe_fp8_args {
  float route_scale;
  float eps;
  MoeFp8Args(const mono_moe_fp8_args& a, float rs, float e) : mono_moe_fp8_args(a), route_scale(rs), eps(e) {}
};

bool moe_fp8_supported(const MoeGeom& geo);
// Workgroups of the persistent launch that fit on one CU (must be >= 1).
hipError_t moe_fp8_occupancy(int* blocks_per_cu);
// Enqueue the one persistent launch on `st` with `grid` workgroups (one a CU).
hipError_t moe_fp8_forward(const MoeFp8Args& g, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st);

bool moe_mxfp4_supported(const MoeGeom& geo);
// Tasks in the MXFP4 launch's list at most, for max_act expert slots (timeline rows).
int moe_mxfp4_tasks(int max_act);
hipError_t moe_mxfp4_occupancy(int* blocks_per_cu);
hipError_t moe_mxfp4_forward(const mono_moe_mxfp4_args& g, int grid, const Mail& mail, const GuardArgs& guard,
                             hipStream_t st);

}  // namespace moe
}  // namespace mono
