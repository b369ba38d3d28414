// Host-side declarations of the fused attention + back launch (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "attn_ops.h"
#include "proj_ops.h"

namespace mono {
namespace fused {

hipError_t attn_back_occupancy(int* blocks_per_cu);
hipError_t attn_back_forward(const attn::AttnArgs& g, const attn::Mail& mail, const GuardArgs& guard,
                             const mono_proj_weights& w, const mono_back_args& b, const proj::Mail& bmail, int grid,
                             hipStream_t st);

}  // namespace fused
}  // namespace mono
