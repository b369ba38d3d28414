// Host-side declarations of the projection launches (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "mono.h"
#include "sync.h"

namespace mono {
namespace proj {

constexpr int MAX_ROWS = 16;
constexpr int HIDDEN = 7168, Q_LORA = 1536, KV_LORA = 512, PE_DIM = 64;
constexpr int HEADS = 32, NOPE = 128, QK = NOPE + PE_DIM, VDIM = 128;
constexpr int IH = 64, ID = 128;
constexpr int N_QKV = Q_LORA + KV_LORA + PE_DIM;  // 2112 rows of q_a | kv_a
constexpr int N_A = N_QKV + ID + IH;              // stage-A outputs a row: q_a | kv_a | index k | index w
constexpr int MAX_PARTS = 4;                      // K parts of a stage-A tile, at most
constexpr int MAX_A_TASKS = 2 * (N_QKV + ID) / 16 + MAX_PARTS * IH / 16;  // stage-A tasks, at most
constexpr int C_TASKS = HEADS * QK / 64 + IH * ID / 64;                   // stage-C tiles

// Mailboxes of one projection runtime: untagged data, each read after its producers'
// tagged done words (see sync.h).
struct Mail {
  uint32_t* pa;     // [MAX_PARTS][MAX_ROWS][N_A]    stage-A partial sums, f32
  uint64_t* adone;  // [MAX_A_TASKS], replicated     a stage-A task's partials are stored
  uint32_t* qnope;  // [MAX_ROWS][HEADS][NOPE / 2]   q_nope, bf16 pairs
  uint32_t* iqraw;  // [MAX_ROWS][IH][ID / 2]        raw index query, bf16 pairs
  uint64_t* cdone;  // [C_TASKS]                     a stage-C tile's outputs are stored
  uint32_t* xn;     // [MAX_ROWS][HIDDEN / 2]        input-RMSNormed rows, bf16 pairs
                    //                                (untagged; read after xdone)
  uint64_t* xdone;  // [MAX_ROWS], replicated        row s of xn is stored
  uint32_t* ob;     // [MAX_ROWS][HEADS * VDIM / 2]  W_UV o_lat, bf16 pairs (untagged; read
                    //                                after odone)
  uint64_t* odone;  // [HEADS], replicated           a head's ob is stored
  uint64_t* fdone;  // [FD_WORDS], replicated         the front's outputs are stored, for a
                    //                                later phase of the launch: FD_B + s (row
                    //                                s's KV row, index key and head weights),
                    //                                FD_E + e (index-query task e), FD_D + h
                    //                                (head h of q: q_lat and q_pe)
  uint32_t* guard;  // [G_WORDS]
};
constexpr int FD_B = 0, FD_E = MAX_ROWS, FD_D = MAX_ROWS + MAX_ROWS * 8, FD_WORDS = FD_D + 32;
// words of the untagged mailboxes pa, qnope, iqraw, ob
constexpr size_t MAIL_WORDS[4] = {(size_t)MAX_PARTS * MAX_ROWS * N_A, (size_t)MAX_ROWS * HEADS * NOPE / 2,
                                  (size_t)MAX_ROWS * IH * ID / 2, (size_t)MAX_ROWS * HEADS * VDIM / 2};
static_assert(MAX_A_TASKS <= 512, "stage-A done words fit one replicated array");

hipError_t front_occupancy(int* blocks_per_cu);
hipError_t back_occupancy(int* blocks_per_cu);
// kv_mask: -1 writes per-token scales into a.kv_scale; 0 writes raw E4M3 rows (scale 1)
// and a.kv_scale points at one f32 word; site0: the number of the launch's first wait
// site under `guard`
hipError_t front_forward(const mono_proj_weights& w, const mono_front_args& a, int grid, const Mail& mail,
                         const GuardArgs& guard, int kv_mask, int site0, hipStream_t st);
hipError_t back_forward(const mono_proj_weights& w, const mono_back_args& a, int grid, const Mail& mail,
                        const GuardArgs& guard, hipStream_t st);

}  // namespace proj
}  // namespace mono
