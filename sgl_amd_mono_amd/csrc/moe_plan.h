// The step's expert plan and scratch of the MoE phase, shared by the FP8 and MXFP4
// expert paths.
#pragma once

#include <stdint.h>

namespace mono {
namespace moe {

constexpr int MAX_ROWS = 16;      // MFMA N: one column a decode row
constexpr int MAX_EXPERTS = 256;  // routed experts; the shared expert is id n_experts
constexpr int MAX_ACT = MAX_EXPERTS + 1;
constexpr int MAX_TOPK = 8;
constexpr int ROUTER_SLICES = 8;  // K slices of the router GEMV

// Written once a step by the router's last workgroup; read by up/gate and down.
struct Plan {
  int32_t n_act;                        // distinct experts this step, the shared one last
  int32_t rows;
  int32_t pad[2];
  int32_t expert[MAX_ACT];              // ascending expert ids
  uint32_t rowmask[MAX_ACT];            // bit s: row s routes to the expert
  float weight[MAX_ACT * MAX_ROWS];     // route weight of (expert slot, row), 0 if unused
};

// Device scratch of one MoE runtime (offsets into one allocation).
struct Scratch {
  Plan* plan;
  float* rstd;        // [MAX_ROWS]
  uint8_t* xq;        // [MAX_ROWS][H] E4M3 activation (W8A8)
  float* xs;          // [MAX_ROWS][H/128] its block scales
  float* rpart;       // [ROUTER_SLICES][MAX_ROWS][E] router partial logits
  uint32_t* rcount;   // router arrivals
  float* mid;         // [MAX_ACT][MAX_ROWS][I] f32 silu(gate) * up
  uint32_t* mcount;   // [MAX_ACT][I/128] up/gate arrivals a 128-block
  uint8_t* mq;        // [MAX_ACT][MAX_ROWS][I] E4M3 mid (W8A8) or bf16 mid pairs (A16W4)
  float* mcoef;       // [MAX_ACT][MAX_ROWS][I/128] mid block scale x route weight
};

}  // namespace moe
}  // namespace mono
