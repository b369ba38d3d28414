/* C-ABI of the MI355X (gfx950) decoder-layer monokernel path.
 *
 * One shared library, libmono_gfx950.so, exports the entry points below. Every
 * argument is a plain pointer, integer or float: device pointers to tensors the
 * caller owns (SGLang's weights and caches, read in place), sizes, and a HIP stream
 * passed as `void*` (a hipStream_t; NULL is the null stream). Every call is
 * stream-ordered and performs no host synchronisation, so a caller may capture it
 * in a HIP graph.
 *
 * Errors: every int-returning call returns MONO_OK (0) or a MONO_E* code and leaves
 * a message for `mono_last_error()` (per host thread) naming the argument and what
 * was expected, in the manner of the reference's ValueError / RuntimeError
 * (sgl_amd_mono/glm53/gfx950/runner.py:218-273).
 *
 * Reference interfaces replaced (yuychang/sgl-amd-mono):
 *   - Glm53Runtime(key, rank, group, device)            glm53/gfx950/runner.py:133-215
 *       -> mono_moe_create / mono_attn_create (scratch, counters, guard words)
 *   - Glm53Runtime.set_deadline / advance_step          glm53/gfx950/runner.py:197-210
 *       -> mono_set_deadline / mono_advance_step
 *   - Glm53LayerOp.launch(h, caches, cos, sin, step)    glm53/gfx950/runner.py:240-321
 *       (rt.dispatch of 42 raw data_ptr() ints + stream)
 *       -> mono_moe_fp8_forward  (its MoE half, stages 8-10, kernel.py:4199-5187)
 *       -> mono_attn_forward     (its sparse-attention half, kernel.py:2684-4123)
 *   - minimax_m31 FFN launch, A16W4 experts              minimax_m31/ffn.py:1182-1378
 *       -> mono_moe_mxfp4_forward
 *   - guard error words read back by tests              common/guard.py:16-30,100-241
 *       -> mono_read_error_words
 */
#ifndef MONO_GFX950_H
#define MONO_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MONO_ABI_VERSION 1

enum {
  MONO_OK = 0,
  MONO_EINVAL = 1, /* an argument is out of range / the wrong shape */
  MONO_EHIP = 2,   /* a HIP runtime call failed */
  MONO_ESTATE = 3, /* wrong device current, destroyed handle, ... */
  MONO_ENOMEM = 4,
};

enum { MONO_ROUTER_SIGMOID_BIAS = 0, MONO_ROUTER_SOFTMAX = 1 };

/* Guard words a runtime exposes (mono_*_read_errors), after the reference's guard
 * block (sgl_amd_mono/common/guard.py:16-30):
 *   [0] launch tickets (workgroups x launches so far)
 *   [1] 0, or 1 + the id of the first inter-workgroup wait that passed its deadline;
 *       sticky: every later launch of the runtime exits at once (fail-stop) until
 *       mono_*_clear_errors
 *   [2] tag of the launch that failed
 *   [3] the workgroup that failed first
 * Wait sites of the MoE launch: 0 router logits, 1 route picks, 2 expert mid
 * activations, 3 expert outputs. */
#define MONO_GUARD_WORDS 4
enum { MONO_WEIGHT_FP8_BLOCK128 = 0, MONO_WEIGHT_MXFP4 = 1 };

/* Version of this ABI (MONO_ABI_VERSION of the library). */
int mono_abi_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* mono_last_error(void);

/* ------------------------------------------------------------------ MoE phase */

typedef struct mono_moe mono_moe;

typedef struct {
  int32_t device;        /* HIP device ordinal the runtime lives on */
  int32_t max_rows;      /* widest decode step served, 1..16 */
  int32_t hidden;        /* H */
  int32_t n_experts;     /* routed experts E; the shared expert is id E */
  int32_t top_k;         /* routed picks a row (8) */
  int32_t inter;         /* expert intermediate I of this GPU's share */
  int32_t weight_format; /* MONO_WEIGHT_* */
  int32_t router;        /* MONO_ROUTER_* */
  float route_scale;     /* routed_scaling_factor (2.5 sigmoid router, 1 softmax) */
  float eps;             /* RMSNorm epsilon of the post-attention norm */
} mono_moe_config;

/* Replaces Glm53Runtime's MoE scratch (runner.py:133-195): allocates the runtime's
 * mailboxes and guard words on `cfg->device` (which must be current) and checks that
 * the persistent kernel fits one workgroup on every CU. A runtime's launches must be
 * stream-ordered (one stream at a time), like the reference's single caller thread. */
int mono_moe_create(const mono_moe_config* cfg, mono_moe** out);
/* Frees the scratch. NULL is a no-op; idempotent like PeerBuffer.close
 * (common/peer.py:157-165). */
int mono_moe_destroy(mono_moe* moe);

/* FP8 MoE block of one decode step, one persistent launch (
 * glm53/gfx950/kernel.py:4199-5187, called through Glm53LayerOp.launch,
 * runner.py:240-321): out = a + sum_slots w * down_e(silu(gate_e(xq)) * up_e(xq)),
 * xq = FP8(RMSNorm(a) * g_post), sigmoid + bias top-k router, shared expert id E with
 * weight 1. Expert weights are read in place in AITER's (16, 16) shuffled layout
 * (glm53/gfx950/kernel.py:787-808): the [N, K] E4M3 matrix of an expert stored as
 * [N/16, K/32, 2, 16, 16] bytes. Optional outputs (NULL skips) expose the routing. */
typedef struct {
  const void* a;        /* bf16 [rows, H] residual stream after attention */
  const void* g_post;   /* bf16 [H] post-attention RMSNorm weight */
  const void* w_router; /* bf16 [E, H] gate weight */
  const float* bias;    /* f32 [E] e_score_correction_bias */
  const void* w13;      /* e4m3 [E+1, 2I, H] gate rows then up rows, (16,16)-shuffled */
  const float* s13;     /* f32 [E+1, 2I/128, H/128] */
  const void* w2;       /* e4m3 [E+1, H, I], (16,16)-shuffled */
  const float* s2;      /* f32 [E+1, H/128, I/128] */
  void* out;            /* bf16 [rows, H] */
  int32_t rows;         /* 1..max_rows */
  float* y;             /* optional f32 [rows, H]: the MoE sum before the residual */
  float* scores;        /* optional f32 [rows, E]: sigmoid scores */
  int32_t* topk_ids;    /* optional i32 [rows, top_k] in pick order */
  float* topk_w;        /* optional f32 [rows, top_k] */
} mono_moe_fp8_args;

int mono_moe_fp8_forward(mono_moe* moe, const mono_moe_fp8_args* args, void* stream);

/* Deadline of every inter-workgroup wait of the runtime's launches, in seconds (default
 * 2). Replaces Glm53Runtime.set_deadline (runner.py:197-204, guard.py:69-76). */
int mono_moe_set_deadline(mono_moe* moe, double seconds);
/* Synchronise the device and copy the MONO_GUARD_WORDS guard words to `words`. */
int mono_moe_read_errors(mono_moe* moe, int32_t* words);
/* Synchronise, then clear guard words 1.. so the runtime launches again. */
int mono_moe_clear_errors(mono_moe* moe);
/* Tests of the fail-stop path: every wait at site `site` of later launches fails at
 * once, as if its deadline had passed (the host-forced fault of guard.py:79-88); -1
 * turns it off. */
int mono_moe_set_fault(mono_moe* moe, int32_t site);

/* MXFP4 (E2M1 + E8M0 per 32) A16W4 MoE of one decode step, one persistent launch
 * (minimax_m31/a16w4.py:1-92, glm53/gfx950/kernel.py:966-970):
 * out = bf16(sum_slots w * down_e(bf16(silu(gate_e(x)) * up_e(x)))), softmax top-k
 * router on the given f32 logits (lowest id on ties, weights = softmax over the
 * picks), shared expert id E with weight 1. The packed E2M1 byte matrices are read in
 * place in AITER's (16, 16) layout ([N/16, K/64, 2, 16, 16] bytes, a wave's 128-k step
 * 1 KB contiguous); the E8M0 scales are row-major. Runtime: weight_format
 * MONO_WEIGHT_MXFP4, router MONO_ROUTER_SOFTMAX, H 3072, E 256, top_k 8, I 384. */
typedef struct {
  const void* x;        /* bf16 [rows, H] */
  const float* logits;  /* f32 [rows, E] gate logits */
  const void* w13;      /* u8 [E+1, 2I, H/2] E2M1 pairs (even k in the low nibble), (16,16)-shuffled */
  const void* s13;      /* u8 [E+1, 2I, H/32] E8M0 */
  const void* w2;       /* u8 [E+1, H, I/2], (16,16)-shuffled */
  const void* s2;       /* u8 [E+1, H, I/32] */
  void* out;            /* bf16 [rows, H] */
  int32_t rows;
  float* y;             /* optional f32 [rows, H] */
  int32_t* topk_ids;    /* optional i32 [rows, top_k] */
  float* topk_w;        /* optional f32 [rows, top_k] */
} mono_moe_mxfp4_args;

int mono_moe_mxfp4_forward(mono_moe* moe, const mono_moe_mxfp4_args* args, void* stream);

/* --------------------------------------------------- sparse-attention phase */

typedef struct mono_attn mono_attn;

typedef struct {
  int32_t device;
  int32_t max_rows;      /* widest decode step, 1..64 */
  int32_t max_ctx;       /* keys a row may hold, a multiple of 1024, <= 32768 */
  float softmax_scale;   /* (qk_nope + qk_rope)^-1/2 = 192^-1/2 for this path */
} mono_attn_config;

/* Replaces the sparse-attention scratch of Glm53Runtime (runner.py:133-195): the
 * runtime's mailboxes (scores, selections, split partials) and guard words. */
int mono_attn_create(const mono_attn_config* cfg, mono_attn** out);
int mono_attn_destroy(mono_attn* attn);

/* Sparse-attention phase of one decode step, one persistent launch (
 * glm53/gfx950/kernel.py:2684-4123 index score / top-k / split / merge, with the FP4
 * indexer of deepseek_v4/gfx950/kernels/stages/indexer.py:460-802):
 *   score[t] = sum_h w_h relu(q_h . k_t) over the row's FP4 index keys,
 *   sel = exact top-2048 positions by (score desc, position asc) -> cache slots,
 *   out = softmax((q . kv_j) * scale) . kv_j[:512] over the selected slots.
 * Caches are SGLang's, read in place: 64-token pages, a slot is page * 64 + offset. */
typedef struct {
  const void* iq;            /* u8 [rows, 64, 64] E2M1 index query (dim 2i in the low nibble) */
  const void* iqs;           /* u8 [rows, 64, 4] E8M0, one per 32 dims */
  const void* iw;            /* bf16 [rows, 64] index head weights */
  const void* ikv;           /* u8 [pages, 4, 64, 16] FP4 index keys: chunk, key, 16 B */
  const void* iks;           /* u8 [pages, 4, 64] E8M0; key t at byte (t % 16) * 4 + t / 16 */
  const void* q;             /* bf16 [rows, 32, 576] absorbed latent query then RoPE query */
  const void* kv;            /* u8 [pages * 64, 576] E4M3 latent then RoPE key */
  const float* kv_scale;     /* f32 [pages * 64] per-token dequantisation scale */
  const int32_t* page_table; /* i32 [rows, pt_stride] logical page -> cache page */
  const int32_t* seq_lens;   /* i32 [rows] keys of each row (clamped to [0, max_ctx]) */
  int32_t pt_stride;
  int32_t n_pages;           /* pages of the caches; page ids are clamped below it */
  void* out;                 /* bf16 [rows, 32, 512] */
  int32_t rows;
  float* scores;             /* optional f32 [rows, max_ctx] index scores */
  int32_t* topk;             /* optional i32 [rows, 2048] selected slots, -1 past the count */
  int64_t* timeline;         /* optional i64 [tasks, 4] per task of the launch: start,
                                inputs-ready and end s_memrealtime ticks (100 MHz), and
                                workgroup << 8 | kind (the reference's timeline stamps,
                                common/stamps.py:24-33) */
} mono_attn_args;

int mono_attn_forward(mono_attn* attn, const mono_attn_args* args, void* stream);

/* Guard controls of an attention runtime (as the MoE runtime's). Wait sites: 0 index
 * scores, 1 selected slots, 2 split partials, 3 top-k team histograms and counts. */
int mono_attn_set_deadline(mono_attn* attn, double seconds);
int mono_attn_read_errors(mono_attn* attn, int32_t* words);
int mono_attn_clear_errors(mono_attn* attn);
int mono_attn_set_fault(mono_attn* attn, int32_t site);

#ifdef __cplusplus
}
#endif

#endif /* MONO_GFX950_H */
