// Every decoder layer of a step as ONE persistent launch (k_layers): the grid walks
// the layers in order, each layer's phases as the one-layer launch runs them
// (layer_impl.h), each under its own guard tag. The layers' kernel arguments live in a
// device table the host packs once (stack_fill) and the launch reads through the
// constant address space.
//
// This file is compiled with MONO_LAYER_LOOP (below: opaque thread and workgroup
// indices, and a guard that tells a failure by the launch's first tag, which every
// layer of the launch shares) and without the machine loop-invariant code motion pass:
// the compiler then hoists none of the phases' per-thread, per-workgroup and constant
// operands out of the layer loop, where they would stay live across all phases and spill.
#define MONO_LAYER_LOOP 1
#include "layer_impl.h"

namespace mono {
namespace layer {

namespace {

// A multi-layer launch: the table of every layer's arguments (device memory the launch
// only reads) and the launch's guard (the layer runtime's, without flip words).
struct StackArgs {
  const __attribute__((address_space(4))) LayerArgs* table;
  int n_layers;
  uint64_t count;
  uint32_t rowh_words;  // words of a layer's row histograms
  GuardArgs guard;
};

// Zero n words (a layer's row histograms once every reader is done), a grid-strided
// share a workgroup, with device-coherent stores.
MONO_DEV void clear_words(uint32_t* p, uint32_t n) {
  for (uint32_t i = block_index() * blockDim.x + (uint32_t)thread_index(); i < n; i += gridDim.x * blockDim.x)
    __hip_atomic_store(&p[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every decoder layer of a step as ONE launch: layer l reads layer l - 1's output. The
// launch takes `count` guard ordinals (one tag a layer; count even, so a one-layer
// launch after this one finds its launch-parity copies as the launch before left them)
// and its grid walks the layers in order, each under its own tag and deadline. A layer
// starts in a workgroup once that workgroup is done with the layer before; it waits only
// on its own phases and on the layer before's final tasks (the done words of its input
// rows), and it clears the layer before's row histograms, whose readers the layer
// before's MoE plan has waited for. Each layer's buffers that a later layer rewrites
// differ from every other layer's (the table's packer checks it), so no cache holds a
// line a later layer of the launch rewrites.
__global__ __launch_bounds__(512, 1) void k_layers(StackArgs args) {
  __shared__ LayerLds lds;
  const GuardFetch f = guard_fetch(args.guard, args.count);
  const Args& last = ((const LayerArgs*)&args.table[args.n_layers - 1])->tail;
  for (int l = 0; l < args.n_layers; ++l) {
    const LayerArgs& la = *(const LayerArgs*)&args.table[l];
    Guard g;
    bool scrubbed = false;
    if (!guard_layer(args.guard, g, f, l, args.count, &scrubbed)) return poison(last, l == 0);
    if (l > 0) clear_words(args.table[l - 1].tail.at.mail.rowh, args.rowh_words);
    if (!run_layer(la, lds, g, scrubbed)) return poison(last, false);
    __syncthreads();  // the LDS passes from the MoE's layout to the next front's
  }
  clear_words(last.at.mail.rowh, args.rowh_words);
}

}  // namespace

hipError_t stack_occupancy(int* blocks_per_cu) {
  return hipOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, k_layers, 512, 0);
}

size_t stack_entry_bytes() { return sizeof(LayerArgs); }

hipError_t stack_fill(void* entry, const StackLayer& sl, const mono_proj_weights& w, const mono_front_args& f,
                      const proj::Mail& fmail, int kv_mask, const attn::AttnArgs& g, const attn::Mail& amail,
                      const GuardArgs& guard, const mono_back_args& b, const proj::Mail& bmail,
                      const moe::MoeFp8Args& m, const moe::Mail& mmail, uint64_t* a_done, int64_t* ticks) {
  LayerArgs& a = *static_cast<LayerArgs*>(entry);
  const hipError_t e = fill_layer(a, w, f, fmail, kv_mask, g, amail, guard, b, bmail, m, mmail, a_done, ticks);
  if (e != hipSuccess) return e;
  // the layer's own row histograms (one copy, cleared by the launch once read)
  a.tail.at.rowh_flip = 0;
  a.tail.at.mail.rowh = sl.rowh;
  // the MoE's FP8 rows and scales, read with plain loads: the layer's own copies
  a.tail.mo.mail.xq = sl.xq;
  a.tail.mo.mail.xs = sl.xs;
  a.tail.mo.out_ssq = sl.out_ssq;
  a.fr.h_ssq = sl.h_ssq;
  a.fr.h_site = STACK_H_SITE;
  return hipSuccess;
}

hipError_t stack_forward(const void* table, int n_layers, uint32_t rowh_words, const GuardArgs& guard, int grid,
                         hipStream_t st) {
  if (n_layers < 1 || grid < 1 || !table) return hipErrorInvalidConfiguration;
  StackArgs a;
  a.table = (const __attribute__((address_space(4))) LayerArgs*)table;
  a.n_layers = n_layers;
  a.count = (uint64_t)(n_layers + (n_layers & 1));
  a.rowh_words = rowh_words;
  a.guard = guard;
  a.guard.flip = nullptr;
  a.guard.flip_words = 0;
  k_layers<<<grid, 512, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace layer
}  // namespace mono
