// Host-side declarations of the sparse-attention phase (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "mono.h"
#include "sync.h"

namespace mono {
namespace attn {

constexpr int IH = 64;          // index heads
constexpr int ID = 128;         // index head dim (4 E2M1 chunks of 32)
constexpr int NH = 32;          // attention heads of this GPU's share
constexpr int DQK = 576;        // latent 512 + RoPE 64
constexpr int DV = 512;         // latent dims attended as values
constexpr int PAGE = 64;        // tokens a cache page
constexpr int TOPK = 2048;      // tokens a row attends
constexpr int MAX_ROWS = 64;
constexpr int MAX_CTX = 32768;  // keys a row at most (2048 a top-k team member)
constexpr int CHUNK = 1024;     // keys a score task
constexpr int SPLITS = 32;      // attention splits a row at most (64 selected tokens each)
constexpr int SPLIT_MAX = TOPK / 4;  // selected tokens a split at most
// Attention splits a row: 32 up to 16 rows (the layer's widest step), then fewer and
// longer ones, so a step's splits (rows x splits <= 256) fill one round of a 256-CU
// grid (split j of n takes the 64-token sub-tiles [32 j / n, 32 (j + 1) / n)); a row's
// merges are as many, of 32 / splits heads each, except with 5 splits: 4 merges of 8.
__host__ __device__ constexpr int splits_of(int rows) { return rows <= 16 ? 32 : rows <= 32 ? 8 : rows <= 48 ? 5 : 4; }
__host__ __device__ constexpr int merges_of(int rows) { return splits_of(rows) == 5 ? 4 : splits_of(rows); }
constexpr int LONG_ROWS = 16;  // steps above this take long splits (only k_attn holds them)
constexpr int WIDE_ROWS = 48;  // steps above this take 4 even splits a row (k_attn_wide)
constexpr int TEAM = 16;        // workgroups selecting one row's top-k together
constexpr int TEAM_LONG = 4;    // the same above LONG_ROWS rows (k_attn_long): one round of teams
constexpr int PASSES = 4;       // 8-bit radix digits of a 32-bit key
constexpr int CMAX = 512;       // threshold candidates a row exchanged as (key, position)
constexpr int HW = 136;         // words a member's histogram: 128 of two 16-bit bins, 1 count
constexpr int ROWH = 256;       // words a row histogram

// Mailboxes of one attention runtime (tagged 64-bit words, see sync.h).
struct Mail {
  uint32_t* score;  // [max_rows][max_ctx]           index scores, f32 (untagged; read after cdone)
  uint64_t* sel;    // [max_rows][TOPK]               selected slots, i32
  uint32_t* rowh;   // [2][max_rows][ROWH]           leading-digit histogram of a row's scores
                    //                                 (untagged counts; launch parity tag & 1)
  uint64_t* cdone;  // [max_rows][max_ctx / CHUNK]   a score chunk's scores are stored and
                    //                                 its counts are in rowh
  uint64_t* hist;   // [max_rows][PASSES][TEAM][HW]   a team member's digit histogram, packed
  uint64_t* cand;   // [max_rows][CMAX]               threshold candidates (low key bits, position)
  uint64_t* cnt;    // [max_rows][TEAM][2]            a member's keys above / at the threshold
  uint16_t* part;   // [max_rows][SPLITS][NH][DV]     a split's unnormalised output, bf16
                    //                                 (untagged; read after sdone)
  float* ml;        // [max_rows][SPLITS][NH][2]      a split's max logit and sum (untagged)
  uint64_t* sdone;  // [max_rows][SPLITS]             a split's part and ml are stored
  uint64_t* mdone;  // [max_rows][NH]                 a merge's output is stored (the fused
                    //                                 attention + back launch only)
  uint32_t* guard;  // [G_WORDS]
  int max_ctx;
  int max_rows;
};

struct AttnArgs : mono_attn_args {
  float softmax_scale;
  // index mask of kv_scale: -1 with a per-token scale plane; 0 when the caller passed
  // none and kv_scale points at one f32 1.0 (raw E4M3 rows)
  int kv_mask = -1;
  AttnArgs(const mono_attn_args& a, float sc) : mono_attn_args(a), softmax_scale(sc) {}
};

hipError_t attn_occupancy(int* blocks_per_cu);
hipError_t attn_forward(const AttnArgs& a, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st);
// the launch of a step above LONG_ROWS rows (attn_forward dispatches to it)
hipError_t attn_long_occupancy(int* blocks_per_cu);
hipError_t attn_long_forward(const AttnArgs& a, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st);
// the launch of a step above WIDE_ROWS rows (the same phase built with 4 even splits a
// row only: the 5-split merges cost these steps 1.3-1.9 us in one kernel)
hipError_t attn_wide_occupancy(int* blocks_per_cu);
hipError_t attn_wide_forward(const AttnArgs& a, int grid, const Mail& mail, const GuardArgs& guard, hipStream_t st);

}  // namespace attn
}  // namespace mono
