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
 *       -> mono_layer_create (and mono_moe_create / mono_attn_create / mono_proj_create
 *          for one phase): scratch, launch counters, guard words
 *   - Glm53Runtime.set_deadline                          glm53/gfx950/runner.py:197-204
 *       -> mono_layer_set_deadline (mono_*_set_deadline)
 *   - Glm53Runtime.advance_step (the step epoch)        glm53/gfx950/runner.py:205-210
 *       -> no call: every launch takes its tag from the guard's own launch counters
 *   - Glm53LayerOp.launch(h, caches, cos, sin, step)    glm53/gfx950/runner.py:240-321
 *       (rt.dispatch of 42 raw data_ptr() ints + stream)
 *       -> mono_layer_forward    (the whole decoder layer, kernel.py:6-45)
 *       -> mono_front_forward    (its projections up to the index query, kernel.py:1367-2443)
 *       -> mono_attn_forward     (its sparse-attention half, kernel.py:2684-4123)
 *       -> mono_back_forward     (W_UV, o_proj and the residual, kernel.py:3975-4197)
 *       -> mono_moe_fp8_forward  (its MoE half, stages 8-10, kernel.py:4199-5187)
 *   - minimax_m31 FFN launch, A16W4 experts              minimax_m31/ffn.py:1182-1378
 *       -> mono_moe_mxfp4_forward
 *   - guard error words read back by tests              common/guard.py:16-30,100-241
 *       -> mono_layer_read_errors (mono_*_read_errors), mono_layer_pending_error
 *   - test fault injection (SGLANG_AMD_MONO_FAULT_INJECT) common/guard.py:79-88
 *       -> mono_layer_set_fault (mono_*_set_fault)
 */
#ifndef MONO_GFX950_H
#define MONO_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MONO_ABI_VERSION 4

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
 *   [0] tag epochs completed (tags repeat every 2^32 - 2 launches; the first launch of
 *       each later epoch zeroes the guard's mailboxes before anything runs)
 *   [1] 0, or 1 + the id of the first inter-workgroup wait that passed its deadline
 *       (31: the epoch scrub's barrier); sticky: every later launch under the guard
 *       exits at once (fail-stop), writing NaN over its output, until
 *       mono_*_clear_errors
 *   [2] tag of the launch that failed
 *   [3] the workgroup that failed first
 *   [4..5] launches begun, u64 (each workgroup also counts them in its own counter)
 *   [6] scrub barrier arrivals
 *   [7] 0
 * Every launch that fails a wait, or that the sticky error refuses, also writes the
 * error to a pinned host word (mono_layer_pending_error) and NaN over its output.
 * Wait sites of the MoE launch: 0 router tasks (their done words), 2 expert mid
 * activations, 3 expert outputs (1 is not used). */
#define MONO_GUARD_WORDS 8
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
/* Synchronise, then clear guard words 1-3, zero every mailbox (no word of an earlier
 * launch survives, both row-histogram copies start at zero) and clear the host word, so
 * the runtime launches again. The same for every mono_*_clear_errors. */
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
  int64_t* timeline;    /* optional i64 [max_act * 36 + 96, 4], max_act = min(8 max_rows, 256) + 1:
                           per task of the list (up tiles, down groups, finals) start,
                           inputs-ready (0: no wait) and end ticks (100 MHz) and
                           workgroup << 8 | kind (1 up, 2 down, 3 final) */
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
  const float* kv_scale;     /* f32 [pages * 64] per-token dequantisation scale, or NULL:
                                the rows are raw E4M3 (scale 1), SGLang's HIP DSA MLA row */
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

/* mono_attn_forward without a runtime and without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The launch's mailboxes and
 * guard words live in the library's static device scratch, about 10 MiB that each GPU
 * the library runs on holds until the process ends, sized for at most 8 rows of at
 * most 32768 keys (rows beyond 8, or a page table narrower than 512 pages, are
 * refused with MONO_EINVAL). The first call on a device clears that scratch with a
 * fill kernel on `stream` and must not run under stream capture; no call allocates or
 * synchronises. Every call on one GPU shares its scratch: calls must be stream-ordered,
 * and calls that overlap on one GPU race. Results equal mono_attn_forward's on a
 * runtime of max_rows 8, max_ctx 32768 and the same softmax_scale. Errors are not
 * sticky (no handle exists to clear them): a launch whose wait passes its 2 s deadline
 * writes NaN over `out`, and the next call runs normally. */
int mono_attn_forward_noalloc(const mono_attn_args* args, float softmax_scale, void* stream);

/* Guard controls of an attention runtime (as the MoE runtime's). Wait sites: 0 index
 * scores (a row's score chunks), 1 selected slots, 2 split partials, 3 top-k team
 * histograms and candidates. */
int mono_attn_set_deadline(mono_attn* attn, double seconds);
int mono_attn_read_errors(mono_attn* attn, int32_t* words);
int mono_attn_clear_errors(mono_attn* attn);
int mono_attn_set_fault(mono_attn* attn, int32_t site);

/* ---------------------------------------------------------------- projections
 * The attention block's projections around the sparse-attention phase, one GPU's
 * TP=4 share of a DeepSeek-V3.2-shaped layer (hidden 7168, q_lora 1536, kv_lora 512,
 * 32 heads of 128 nope + 64 rope dims, value dim 128, FP4 indexer of 64 heads x 128).
 *
 * mono_front_forward: one persistent launch (glm53/gfx950/kernel.py:1367-2443 with the
 * FP4 indexer of deepseek_v4/gfx950/kernels/stages/indexer.py:236-408): input RMSNorm,
 * q_a | kv_a and index key / head-weight projections, q_a RMSNorm, q_b + RoPE, the
 * absorbed query W_UK^T q_nope, KV RMSNorm + k_pe RoPE + the FP8 MLA cache row, the
 * index key (LayerNorm, RoPE, Hadamard, FP4) into the index plane, and the index
 * query (RoPE, Hadamard, FP4) and head weights: exactly mono_attn_args' inputs.
 *
 * mono_back_forward: one persistent launch (kernel.py:3975-4197 after the split
 * merge): o = W_UV o_lat per head, then a = h + W_o o (the TP all-reduce is a local
 * residual add).
 *
 * FP8 matrices are E4M3 in AITER's (16, 16) layout ([N/16, K/32, 2, 16, 16] bytes)
 * with f32 128 x 128 block scales, row-major [ceil(N/128), K/128]; they are widened
 * exactly to bf16 and multiplied with bf16 activations, f32 accumulation. */
typedef struct mono_proj mono_proj;

typedef struct {
  int device;
  int max_rows; /* widest step, 1..16 */
} mono_proj_config;

typedef struct {
  const void* g_in;   /* bf16 [7168] input RMSNorm weight */
  const void* w_qkv;  /* e4m3 [2112, 7168]: q_a 1536 | kv latent 512 | k_pe 64 */
  const float* s_qkv; /* [17, 56] */
  const void* w_ik;   /* e4m3 [128, 7168] index key */
  const float* s_ik;  /* [1, 56] */
  const void* w_iw;   /* bf16 [64, 7168] index head weights, (16, 16) layout of its bytes */
  const void* g_q;    /* bf16 [1536] q_a RMSNorm weight */
  const void* g_kv;   /* bf16 [512] KV RMSNorm weight */
  const float* g_ik;  /* f32 [128] index key LayerNorm weight */
  const float* b_ik;  /* f32 [128] index key LayerNorm bias */
  const void* w_qb;   /* e4m3 [6144, 1536]: rows h*192 + (nope 0..127 | pe 128..191) */
  const float* s_qb;  /* [48, 12] */
  const void* w_iq;   /* e4m3 [8192, 1536]: rows h*128 + d */
  const float* s_iq;  /* [64, 12] */
  const void* w_uk;   /* e4m3 [16384, 128]: rows h*512 + c, W_UK^T (q_lat = W q_nope) */
  const float* s_uk;  /* [128, 1] */
  const void* w_uv;   /* e4m3 [4096, 512]: rows h*128 + v */
  const float* s_uv;  /* [32, 4] */
  const void* w_o;    /* e4m3 [7168, 4096] */
  const float* s_o;   /* [56, 32] */
} mono_proj_weights;

typedef struct {
  const void* h;             /* bf16 [rows, 7168] residual stream */
  const int32_t* seq_lens;   /* [rows] keys of a row counting this step's token, which
                                sits at position seq_len - 1; a row outside
                                [1, min(max_pos, pt_stride * 64)] is a pad row: it
                                writes no cache row */
  const int32_t* page_table; /* [rows, pt_stride] */
  int pt_stride;
  int n_pages;               /* pages of the caches (a page id >= n_pages: pad row) */
  const float* rope_cos;     /* f32 [max_pos, 32] */
  const float* rope_sin;     /* f32 [max_pos, 32] */
  int max_pos;
  void* ikv;                 /* u8 [n_pages, 4, 64, 16] index plane, written in place */
  void* iks;                 /* u8 [n_pages, 4, 64] */
  void* kv;                  /* u8 [n_pages * 64, 576] MLA cache, written in place */
  float* kv_scale;           /* f32 [n_pages * 64], or NULL: rows written as raw E4M3
                                (scale 1, values clamped to +-448) */
  void* q;                   /* out bf16 [rows, 32, 576] q_lat | q_pe */
  void* iq;                  /* out u8 [rows, 64, 64] E2M1 index query */
  void* iqs;                 /* out u8 [rows, 64, 4] E8M0 */
  void* iw;                  /* out bf16 [rows, 64] index head weights */
  int rows;
  int64_t* timeline;         /* optional i64 [tasks, 4] per task: start, inputs-ready, end
                                ticks (s_memrealtime, 100 MHz), workgroup << 8 | stage
                                (0 A, 1 B, 2 C, 3 D, 4 E, 5 N: the input RMSNorm of a
                                row); tasks = 140 (rows <= 8) or 280, + 272 + 10 rows */
} mono_front_args;

typedef struct {
  const void* o_lat; /* bf16 [rows, 32, 512] the attention phase's output */
  const void* h;     /* bf16 [rows, 7168] residual stream */
  void* a;           /* out bf16 [rows, 7168] h + W_o W_UV o_lat */
  void* o;           /* optional out bf16 [rows, 4096] W_UV o_lat (NULL: not written) */
  int rows;
  int64_t* timeline; /* optional i64 [256, 4] as in mono_front_args (stage 0 U, 1 O) */
} mono_back_args;

/* Wait sites of the projection launches: 0 stage-A partials, 1 stage-A q_a tiles, 2 q_nope,
 * 3 raw index query, 4 W_UV output, 5 normed input rows. */
int mono_proj_create(const mono_proj_config* cfg, mono_proj** out);
int mono_proj_destroy(mono_proj* proj);
int mono_front_forward(mono_proj* proj, const mono_proj_weights* w, const mono_front_args* args, void* stream);
int mono_back_forward(mono_proj* proj, const mono_proj_weights* w, const mono_back_args* args, void* stream);
int mono_proj_set_deadline(mono_proj* proj, double seconds);
int mono_proj_read_errors(mono_proj* proj, int32_t* words);
int mono_proj_clear_errors(mono_proj* proj);
int mono_proj_set_fault(mono_proj* proj, int32_t site);

/* mono_attn_back_forward: mono_attn_forward followed by mono_back_forward on its output
 * (back->o_lat NULL or args->out), as ONE persistent launch of the attention runtime:
 * the reference runs both in its single decoder-layer launch (kernel.py:2684-4197), so
 * the back's weight loads start while the last splits and merges run. Results equal
 * the two calls'. The launch uses the attention runtime's guard (its wait sites, 4 for
 * the W_UV output and 5 for the merges' output). */
int mono_attn_back_forward(mono_attn* attn, const mono_attn_args* args, const mono_proj_weights* w,
                           const mono_back_args* back, void* stream);

/* --------------------------------------------------- the decoder layer */

typedef struct mono_layer mono_layer;

typedef struct {
  int32_t device;
  int32_t max_rows;     /* widest decode step, 1..16 */
  int32_t max_ctx;      /* keys a row may hold, a multiple of 1024, <= 32768 */
  float softmax_scale;  /* (qk_nope + qk_rope)^-1/2 = 192^-1/2 */
  float route_scale;    /* routed_scaling_factor, 2.5 */
  float eps;            /* post-attention RMSNorm epsilon, 1e-6 */
  int32_t max_layers;   /* most layers of one mono_layer_stack_forward launch (0 or 1: none) */
} mono_layer_config;

/* One step of one layer: the four parts' arguments as their own entry points take
 * them. attn's q / iq / iqs / iw are the front's outputs and it reads the caches and
 * step the front writes; back->o_lat is NULL or attn->out; moe->a is back->a. */
typedef struct {
  const mono_front_args* front;
  const mono_attn_args* attn;
  const mono_back_args* back;
  const mono_moe_fp8_args* moe;
  /* optional i64 [grid, 16] (the layer's launches; NULL skips): per workgroup, the
   * s_memrealtime tick (100 MHz) at which it [0] began, finished its [1] front tasks,
   * [2] attention tasks, [3] back tasks, [4] had the MoE's expert plan, [5] finished;
   * and the MoE prologue's moments: [6] the attention block's output seen, [7] its
   * first router task's norm statistics, [8] its router tasks done, [9] the router
   * outputs gathered, [10] its rows routed; the rest 0. The reference's per-CTA stamps
   * (common/stamps.py:24-33). */
  int64_t* ticks;
} mono_layer_args;

/* Replaces Glm53Runtime (runner.py:133-215) for a whole decoder layer: the mailboxes
 * of the front, the attention, the back and the FP8 MoE, and ONE guard (one count of
 * launches, one set of error words) for every launch of the layer, whichever of
 * mono_layer_forward / _front_forward / _tail_forward the caller mixes. */
int mono_layer_create(const mono_layer_config* cfg, mono_layer** out);
int mono_layer_destroy(mono_layer* layer);
/* Glm53LayerOp.launch (runner.py:240-321): the whole decoder layer as ONE persistent
 * launch (glm53/gfx950/kernel.py:6-45, 1367-5187): the front (as mono_front_forward),
 * the sparse attention, W_UV, o_proj + residual and the FP8 MoE + residual; results
 * equal the four entry points'. Stream-ordered on `stream`; never synchronises. */
int mono_layer_forward(mono_layer* layer, const mono_proj_weights* w, const mono_layer_args* args, void* stream);
/* The two launches of mono_layer_forward on their own (same checks), for a caller that
 * times or records between them: the front, then the fused rest. No counterpart in the
 * reference, whose layer is one launch. */
int mono_layer_front_forward(mono_layer* layer, const mono_proj_weights* w, const mono_layer_args* args,
                             void* stream);
int mono_layer_tail_forward(mono_layer* layer, const mono_proj_weights* w, const mono_layer_args* args,
                            void* stream);
/* Deadline of every wait of the layer's launches (Glm53Runtime.set_deadline,
 * runner.py:197-204; a serving caller passes half its watchdog, at most 60 s). */
int mono_layer_set_deadline(mono_layer* layer, double seconds);
/* words: int32 [MONO_GUARD_WORDS], the layer's guard (synchronises). Wait sites: 0-3
 * the attention's (index scores, selected slots, split partials, top-k team), 4 W_UV
 * output, 5 attention output, 6 router tasks, 7 (not used), 8 expert mid, 9 expert
 * outputs, 10 the attention block's output rows, 11-16 the front's (stage-A partials,
 * q_an, q_nope, raw index query, -, normed input rows), 17 the front's index outputs,
 * 18 the front's q, 19 (a multi-layer launch) the layer before's output rows, 31 the
 * tag-epoch scrub (and a multi-layer launch's grid meeting before a layer's scrub). */
int mono_layer_read_errors(mono_layer* layer, int32_t* words);
/* The layer's pinned host error word, without synchronising: 0, or 1 + the wait site
 * of a launch that failed or was refused since the last clear (-1: not a live layer).
 * No counterpart in the reference, which stops a failed launch by a GPU fault
 * (common/guard.py:91-97); a serving caller watches it from a host thread (graph
 * replays run no host code a step) and ends the process on a hit. A failed launch's
 * output holds NaN where its failing workgroups wrote it but may keep rows that other
 * workgroups finished: the host word, not the output, is authoritative. */
int32_t mono_layer_pending_error(mono_layer* layer);
/* Synchronise, clear the sticky error, every mailbox and the host word so the layer
 * launches again. */
int mono_layer_clear_errors(mono_layer* layer);
/* Tests of the fail-stop path (the reference's SGLANG_AMD_MONO_FAULT_INJECT
 * rank:site:after, common/guard.py:79-88): every wait at `site` of every launch from
 * the `after`-th next launch on fails at once, as if its deadline had passed (after 0:
 * the next launch; synchronises when after > 0); site -1 turns it off. The fault and
 * the deadline travel as kernel arguments: a launch captured in a graph keeps the ones
 * set when it was captured. */
int mono_layer_set_fault(mono_layer* layer, int32_t site, int64_t after);
/* Every decoder layer of one step as ONE persistent launch, in two calls: _stack_set
 * checks n layers' arguments and keeps them on the device (it synchronises the device;
 * not during a stream capture), and each _stack_forward launches the layers last set
 * (stream-ordered, never synchronises; a graph that captured it reads the arguments
 * last set when it replays). Layer l runs as mono_layer_forward(layer, w[l], args[l])
 * would, results equal, and reads layer l - 1's output (args[l]->front->h must be
 * args[l - 1]->moe->out) once that layer's final tasks have announced its rows. No
 * counterpart in the reference, which launches each layer (glm53/gfx950/runner.py:
 * 240-321); it removes the launch gap and the launch-counter round trip between layers,
 * and a layer's front starts its weight loads while the layer before finishes. Every
 * layer takes its own tag (a launch counts as n launches, rounded up to even, for the
 * guard) and its own deadline from its start, and fails alone at a wait as its
 * one-layer launch would; a failed or refused launch writes NaN over the last layer's
 * output. Layer 0's front->h and every layer's q / iq / iqs / iw, back->a, moe->out and
 * caches must not overlap (no layer rereads a line a later layer rewrites); ticks,
 * timelines and debug outputs per layer as mono_layer_forward takes them.
 * n <= cfg.max_layers. */
int mono_layer_stack_set(mono_layer* layer, int32_t n_layers, const mono_proj_weights* const* w,
                         const mono_layer_args* const* args);
int mono_layer_stack_forward(mono_layer* layer, void* stream);
/* Tests of the tag epochs (synchronises): the next launch takes launch ordinal
 * `ordinal`, i.e. tag ordinal % (2^32 - 2) + 1. Every mailbox is zeroed as well, so a
 * jump of any length or direction (odd ones change the row histograms' parity) leaves
 * no stale word. No counterpart in the reference. */
int mono_layer_set_launch_ordinal(mono_layer* layer, uint64_t ordinal);

#ifdef __cplusplus
}
#endif

#endif /* MONO_GFX950_H */
