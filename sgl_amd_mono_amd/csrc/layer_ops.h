// Host-side declarations of the fused layer launch (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "attn_ops.h"
#include "moe_ops.h"
#include "proj_ops.h"

namespace mono {
namespace layer {

// first guard wait site of the MoE phase in the fused launch (the attention's are 0-3,
// the back's 4-5)
constexpr int MOE_SITE0 = 6;
// the front's wait sites in the one-launch layer (its own 0-5 + FRONT_SITE0) and the
// attention's waits on the front (index outputs, then q)
constexpr int FRONT_SITE0 = 11;
constexpr int ATTN_FRONT_SITE = 17;

hipError_t tail_occupancy(int* blocks_per_cu);
// the sparse attention, the back and the FP8 MoE of one step as one launch; a_done is
// the o_proj tiles' replicated done words (DONE_BYTES)
hipError_t tail_forward(const attn::AttnArgs& g, const attn::Mail& amail, const GuardArgs& guard,
                        const mono_proj_weights& w, const mono_back_args& b, const proj::Mail& bmail,
                        const moe::MoeFp8Args& m, const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks, int grid,
                        hipStream_t st);
// the whole layer as one launch: the front (its mailboxes fmail, kv_mask as front_forward)
// and then tail_forward's phases, all under `guard`
hipError_t layer_forward(const mono_proj_weights& w, const mono_front_args& f, const proj::Mail& fmail,
                         int kv_mask, const attn::AttnArgs& g, const attn::Mail& amail, const GuardArgs& guard,
                         const mono_back_args& b, const proj::Mail& bmail, const moe::MoeFp8Args& m,
                         const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks, int grid, hipStream_t st);

}  // namespace layer
}  // namespace mono
