// Shapes, mailboxes and limits of the MoE phase, shared by the host and the kernels.
#pragma once

#include <stdint.h>

namespace mono {
namespace moe {

constexpr int MAX_ROWS = 16;      // MFMA N: one column a decode row
constexpr int MAX_EXPERTS = 256;  // routed experts; the shared expert is id n_experts
constexpr int MAX_ACT = MAX_EXPERTS + 1;
constexpr int MAX_TOPK = 8;

// Mailboxes of one MoE runtime (tagged 64-bit words, see sync.h), sized for the
// runtime's max_rows: at most max_act = min(max_rows * top_k, E) + 1 expert slots.
struct Mail {
  uint64_t* rlog;   // [RK][MAX_ROWS][E]     router partial logits, one K slice each
  uint64_t* rsel;   // [MAX_ROWS][2 * TOPK]  a row's picks: ids, then weights
  uint64_t* mid;    // [max_act][MAX_ROWS][I]  silu(gate) * up, f32
  uint64_t* ypart;  // [max_act][MAX_ROWS][H]  an expert's weighted down output, f32
  uint32_t* guard;  // [G_WORDS]
};

}  // namespace moe
}  // namespace mono
