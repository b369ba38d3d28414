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
// a layer of a multi-layer launch: the wait on the layer before's output rows
constexpr int STACK_H_SITE = 19;

// A layer's own buffers in a multi-layer launch (its table entry points at them): its
// row histograms, its MoE FP8 rows and their scales (read with plain loads, so no two
// layers of a launch share them), the tile sums of squares its final tasks put (NULL:
// the last layer) and those its norm tasks await (NULL: the first layer).
struct StackLayer {
  uint32_t* rowh;
  uint8_t* xq;
  float* xs;
  uint64_t* out_ssq;
  const uint64_t* h_ssq;
};

// workgroups a CU holds of the least of the layer's launches (the multi-layer one too)
hipError_t tail_occupancy(int* blocks_per_cu);
hipError_t stack_occupancy(int* blocks_per_cu);
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
// bytes of one layer's entry in a multi-layer launch's table
size_t stack_entry_bytes();
// Fill a table entry (host memory of stack_entry_bytes()) with one layer's arguments,
// as layer_forward takes them, on the layer's own buffers `sl`.
hipError_t stack_fill(void* entry, const StackLayer& sl, const mono_proj_weights& w, const mono_front_args& f,
                      const proj::Mail& fmail, int kv_mask, const attn::AttnArgs& g, const attn::Mail& amail,
                      const GuardArgs& guard, const mono_back_args& b, const proj::Mail& bmail,
                      const moe::MoeFp8Args& m, const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks);
// Every layer of a table (device memory, n_layers entries) as one launch; rowh_words:
// words of a layer's row histograms.
hipError_t stack_forward(const void* table, int n_layers, uint32_t rowh_words, const GuardArgs& guard, int grid,
                         hipStream_t st);

}  // namespace layer
}  // namespace mono
