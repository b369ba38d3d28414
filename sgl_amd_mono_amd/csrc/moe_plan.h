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
  // the FP8 kernel's router tasks' outputs: tagged scores, and plain rows behind the
  // tasks' done words
  uint64_t* score;  // [MAX_ROWS][E]       routing scores, f32 (tagged)
  uint8_t* xq;      // [MAX_ROWS][H]       the normed rows in FP8
  float* xs;        // [MAX_ROWS][H / 128] their block scales
  uint64_t* rdone;  // DONE_BYTES: router task t's done word, replicated
  uint64_t* mid;    // [max_act][MAX_ROWS][I]  silu(gate) * up, f32
  uint64_t* mtile;  // [max_act][I / 16]     the MXFP4 kernel's up tile done words (hints)
  uint64_t* ypart;  // [max_act][MAX_ROWS][H]  an expert's weighted down output, f32
  uint32_t* guard;  // [G_WORDS]
};

}  // namespace moe
}  // namespace mono
