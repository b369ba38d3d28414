// The decoder layer's phases as device code shared by its launches (layer.hip: one
// layer a launch; layer_stack.hip: every layer of a step in one launch): the kernel
// arguments, the LDS union and the phase sequence of one layer.
#pragma once

#include "attn_step.h"
#include "back_impl.h"
#include "front_impl.h"
#include "layer_ops.h"
#include "moe_fp8_step.h"

namespace mono {
namespace layer {

namespace {

// the launches that hold the attention with other phases take at most proj::MAX_ROWS
// rows: their attention has one sub-tile a split (no long splits compiled in)
static_assert(proj::MAX_ROWS <= attn::LONG_ROWS, "fused launches: short splits only");

struct Args {
  attn::Args at;
  proj::Args bk;
  moe::Args mo;
  uint64_t* a_done;
  int64_t* ticks;  // [grid][16] phase ticks (NULL: none)
};

// the layer's moments in a workgroup's tick row (4 and 6-10: the MoE's, moe_fp8_step.h)
enum { T_BEGIN = 0, T_FRONT = 1, T_ATTN = 2, T_BACK = 3, T_END = 5, T_WORDS = 16 };

MONO_DEV void stamp(int64_t* ticks, int k) {
  if (ticks && thread_index() == 0) ticks[block_index() * T_WORDS + k] = (int64_t)now_ticks();
}

union Lds {
  attn::Lds at;
  proj::Lds bk;
  moe::Lds mo;
};

struct LayerArgs {
  proj::fr::Args fr;
  Args tail;
};


union LayerLds {
  Lds tail;
  proj::fr::Lds fr;
};

// A failed or refused launch writes NaN over the layer's output x_out (sync.h).
MONO_DEV void poison(const Args& args, bool share) {
  poison_bf16(args.mo.out, (size_t)args.mo.rows * moe::H, share);
}

// The back and the MoE after the attention, on the attention's guard (false: a wait
// failed).
MONO_DEV bool back_moe(const Args& args, Lds& lds, const attn::Step& st, const Guard& g) {
  __syncthreads();  // the LDS passes from the attention's layout to the back's
  {
    proj::Back bk(args.bk, lds.bk);
    bk.adopt(g, args.at.mail.mdone);
    bk.publish_a(args.a_done);
    if (!bk.tasks(st.n_tasks())) return false;
  }
  stamp(args.ticks, T_BACK);
  __syncthreads();  // and to the MoE's
  moe::Step ms(args.mo, lds.mo);
  ms.adopt(g, args.a_done, proj::NT_O, MOE_SITE0);
  bool refused;
  if (!ms.run(refused)) return false;
  stamp(args.ticks, T_END);
  return true;
}

// One decoder layer under the guard `g`: the front's tasks first (under the layer's
// tag), then the attention, whose score tasks and splits wait on the front's done
// words, then the back and the MoE. `h_ready`: the layer's input rows are known to be
// stored (a grid barrier met since the layer that wrote them). False on a failed wait.
MONO_DEV bool run_layer(const LayerArgs& args, LayerLds& lds, const Guard& g, bool h_ready) {
  stamp(args.tail.ticks, T_BEGIN);
  attn::Step st(args.tail.at, lds.tail.at);
  st.adopt(g);
  // Stage D (the absorbed query, read only by the splits) leaves the front when the
  // workgroups after the top-k teams can take it: head d runs on workgroup
  // (scores + top-k tasks + d) mod G between its score and split tasks, which holds no
  // top-k task, so no score task waits behind a D task.
  const int d0 = st.n_score() + st.n_topk();
  const bool defer_d = st.n_topk() + proj::HEADS <= (int)gridDim.x;
  {
    proj::fr::Front f(args.fr, lds.fr);
    f.adopt(g, FRONT_SITE0, h_ready);
    f.set_defer_d(defer_d);
    if (!f.tasks()) return false;
  }
  stamp(args.tail.ticks, T_FRONT);
  __syncthreads();  // the LDS passes from the front's layout to the attention's
  const auto deferred = [&]() -> bool {
    if (!defer_d) return true;
    const int G = (int)gridDim.x, b = (int)block_index();
    for (int d = ((b - d0) % G + G) % G; d < proj::HEADS; d += G) {
      __syncthreads();  // the LDS passes to the front's layout
      proj::fr::Front f(args.fr, lds.fr);
      f.adopt(g, FRONT_SITE0);
      if (!f.deferred_d(d)) return false;
      __syncthreads();  // and back to the attention's
    }
    return true;
  };
  if (!st.tasks(deferred)) return false;
  stamp(args.tail.ticks, T_ATTN);
  return back_moe(args.tail, lds.tail, st, g);
}


// One layer's kernel arguments (the one-launch layer's and a multi-layer table entry's).
hipError_t fill_layer(LayerArgs& a, const mono_proj_weights& w, const mono_front_args& f, const proj::Mail& fmail,
                      int kv_mask, const attn::AttnArgs& g, const attn::Mail& amail, const GuardArgs& guard,
                      const mono_back_args& b, const proj::Mail& bmail, const moe::MoeFp8Args& m,
                      const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks) {
  if (f.rows != g.rows || f.rows < 1 || f.rows > proj::MAX_ROWS || g.rows > attn::MAX_ROWS || g.rows > moe::MAX_ROWS ||
      b.rows != g.rows || m.rows != g.rows || amail.max_ctx % attn::CHUNK || amail.max_ctx > attn::MAX_CTX)
    return hipErrorInvalidConfiguration;
  a.fr.w = w;
  a.fr.a = f;
  a.fr.mail = fmail;
  a.fr.guard = guard;
  a.fr.kv_mask = kv_mask;
  a.fr.site0 = FRONT_SITE0;
  a.fr.h_ssq = nullptr;
  a.fr.h_site = 0;
  attn::fill_args(a.tail.at, g, amail, guard);
  a.tail.at.publish_out = true;
  a.tail.at.fdone = fmail.fdone;
  a.tail.at.fsite = ATTN_FRONT_SITE;
  a.tail.bk.w = w;
  a.tail.bk.a = b;
  a.tail.bk.mail = bmail;
  a.tail.bk.guard = guard;
  moe::fill_args(a.tail.mo, m, mmail, guard);
  a.tail.a_done = a_done;
  a.tail.ticks = ticks;
  a.tail.mo.ticks = ticks;
  return hipSuccess;
}

}  // namespace
}  // namespace layer
}  // namespace mono
