// Inter-workgroup hand-off inside one persistent launch: tagged mailbox words and the
// guard that bounds every wait.
//
// A mailbox word is 64 bits: the payload (an f32 or i32's bits) in the low half and
// the launch's tag in the high half, written by one agent-scope relaxed atomic store
// (global_store_dwordx2 sc1) and read by agent-scope relaxed atomic loads
// (global_load_dwordx2 sc1). The tag makes every word self-validating, so a producer
// needs no release fence and a consumer no acquire fence: on gfx950 those are an L2
// writeback / invalidate of the XCD, which costs far more than the hand-off. This is
// the reference's tagged (value, tag) pair (sgl_amd_mono/common/sync.py:30-207,
// glm53/gfx950/kernel.py:29-35,636-647), restated for HIP.
//
// Tags: every workgroup of a launch counts the guard's launches itself: workgroup b
// adds one to its own 64-bit counter (tickets[b], one atomic add on a word no other
// workgroup touches, so the grid's adds never serialise on one address) and the value
// before the add is the launch's ordinal (launches sharing a guard are stream-ordered
// and each runs every workgroup of the same grid, so all counters stay equal); the tag
// is ordinal % TAG_PERIOD + 1. Workgroup 0 also stores ordinal + 1 at guard words 4-5
// for the host. A HIP-graph replay counts on, so it never sees a stale word as ready.
//
// Tag epochs: tags repeat every TAG_PERIOD launches, and a word left unwritten for
// exactly that long would read as fresh (the reference scrubs its mailboxes for the
// same reason, deepseek_v4/gfx950/kernels/layer.py:837-849). The first launch of every
// epoch after the first (tag 1, ordinal > 0) therefore zeroes every mailbox the guard's
// launches write (the guard's scrub table) and meets the whole grid at a barrier
// (guard word 6) before any workgroup goes on, so within an epoch a word either holds a
// tag of that epoch or 0. TAG_PERIOD is even, so a tag's parity alternates through the
// wrap as well (the flip accumulators below rely on it).
//
// Guard words (int32 [8] in device memory, common/guard.py:16-30 in the reference):
//   0  tag epochs completed (scrubs run)
//   1  error: 1 + the id of the first wait site that ran out of time (sticky: every
//      later launch of the guard exits at once until the host clears it)
//   2  tag of the failing launch (waits of that launch give up when they see it)
//   3  workgroup that failed first
//   4-5 launches begun, u64 (workgroup 0's count)
//   6  scrub barrier arrivals (u32, G more a scrub)
// Every wait polls its words until their tags match, checking the deadline
// (s_memrealtime, 100 MHz) after its first poll and then every POLL_CHECK polls, and
// the launch's fail tag every POLL_CHECK polls. On expiry it records the error (and
// copies it to the host's pinned error word), raises word 2 and returns false; the
// caller makes the failure workgroup-uniform and the workgroup exits after writing NaN
// over the launch's output. No wait ever blocks past the deadline and nothing faults:
// the launch drains, the host sees the error without synchronising, and a caller that
// reads the output anyway reads NaN (fail-stop without a GPU fault).
#pragma once

#include "common.h"

namespace mono {

enum GuardWord {
  G_EPOCH = 0,
  G_ERROR = 1,
  G_FAIL_TAG = 2,
  G_FAIL_BLOCK = 3,
  G_TICKET = 4,  // u64 at words 4-5: launches begun
  G_BARRIER = 6,
  G_WORDS = 8
};
constexpr int POLL_CHECK = 32;
// tags 1 .. TAG_PERIOD; 0 marks an empty mailbox word
constexpr uint64_t TAG_PERIOD = 0xFFFFFFFEull;
// the wait site of the scrub barrier
constexpr int SCRUB_SITE = 31;
constexpr int SCRUB_MAX = 5;

// A device region of mailboxes the scrub zeroes: n16 16-byte units at p.
struct ScrubRegion {
  uint32_t* p;
  uint64_t n16;
};

// Kernel-argument part of the guard.
struct GuardArgs {
  uint32_t* words;
  // [grid] per-workgroup launch counters (u64), outside every scrub region
  uint64_t* tickets;
  // [SCRUB_MAX] in device memory: the guard's mailboxes (p = NULL past the last region)
  const ScrubRegion* scrub;
  // atomic accumulators used by launch parity: [2][flip_words]; every launch zeroes
  // the copy of its successor's parity, (tag + 1) & 1 (NULL: none)
  uint32_t* flip;
  // a pinned host word (device-visible): 1 + the failed wait site of the first failure
  // or refused launch, so the host sees a stop without synchronising (NULL: none)
  uint32_t* host_err;
  uint64_t deadline_ticks;
  // the host-forced fault (tests of the error path): every wait at fault_site of a
  // launch whose ordinal is at least fault_from fails at once (-1: none)
  uint64_t fault_from;
  int32_t fault_site;
  int32_t flip_words;
  // 1: a failure refuses every later launch until the host clears it (a runtime
  // handle's guard); 0: later launches run (a guard no host call can clear)
  int32_t sticky;
};

MONO_DEV uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

MONO_DEV void mb_put(uint64_t* p, uint32_t bits, uint32_t tag) {
  __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
MONO_DEV void mb_putf(uint64_t* p, float v, uint32_t tag) { mb_put(p, __float_as_uint(v), tag); }
MONO_DEV uint64_t mb_load(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A plain (L2-cacheable) load of a mailbox word. Only a first pass after a hint wait
// uses it: a line cached before its producer wrote it returns an old tag, and that word
// is then polled with agent-scope loads, so a stale copy is never taken for data.
MONO_DEV uint64_t mb_load_cached(const uint64_t* p) { return *p; }
MONO_DEV uint32_t ld_agent_u32(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// device-coherent plain data (read after the tagged word that announces it)
MONO_DEV float ld_agent_f32(const float* p) { return __uint_as_float(ld_agent_u32(reinterpret_cast<const uint32_t*>(p))); }
MONO_DEV void st_agent_f32(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A device-coherent (write-through) store of 1, 2, 4 or 8 bytes: data another
// workgroup of the launch reads after a done word.
template <class T>
MONO_DEV void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Untagged data behind a tagged done word: the producer stores it with device-coherent
// buffer stores, waits for them (s_waitcnt 0) and a barrier, then puts the done word;
// the consumer polls the done word, then reads the data with device-coherent loads.
// Bytes past the resource's size read as 0 and are not stored.
constexpr int BUF_DWORD3 = 0x00020000;  // raw buffer resource word 3 (gfx9)
constexpr int SC1 = 16;                 // buffer cache policy: device-coherent
MONO_DEV __amdgpu_buffer_rsrc_t coherent_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, BUF_DWORD3);
}

// A done word that many workgroups poll is put in DONE_REPLICAS copies 4 KB apart
// (apart in the memory channels) and workgroup b polls copy b % DONE_REPLICAS, so no
// single line takes every workgroup's polls. An array of n replicated done words takes
// DONE_REPLICAS * 4 KB (n <= 512).
constexpr int DONE_REPLICAS = 16;
constexpr size_t DONE_STRIDE = 4096 / sizeof(uint64_t);
constexpr size_t DONE_BYTES = DONE_REPLICAS * 4096;
// thread k < DONE_REPLICAS of the calling workgroup puts copy k of done word i
MONO_DEV void put_done(uint64_t* base, int i, uint32_t tag) {
  const int t = thread_index();
  if (t < DONE_REPLICAS) mb_put(base + t * DONE_STRIDE + i, 0u, tag);
}
MONO_DEV const uint64_t* done_copy(const uint64_t* base) { return base + (block_index() % DONE_REPLICAS) * DONE_STRIDE; }

// Copy an error code to the host's pinned error word: a plain system-scope store (no
// atomic read-modify-write over the bus; the device's sticky error word keeps the
// first failure, this word any failure's code), which the host reads without
// synchronising.
MONO_DEV void report_host(uint32_t* host_err, uint32_t code) {
  if (host_err) __hip_atomic_store(host_err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A launch's guard once it has begun (guard_begin): what its waits need.
struct Guard {
  uint32_t* words;
  uint32_t* host_err;
  uint64_t deadline;  // absolute s_memrealtime tick
  uint32_t tag;
#ifdef MONO_LAYER_LOOP
  uint32_t ltag;  // the launch's first tag (its first layer's)
#endif
  int fault;  // this launch's host-forced fault site (-1: none)

  // What a failure records and the peers' check compares: the launch's first tag, the
  // same for every layer of a multi-layer launch (a one-layer launch has only `tag`).
  MONO_DEV uint32_t launch_tag() const {
#ifdef MONO_LAYER_LOOP
    return ltag;
#else
    return tag;
#endif
  }

  // Record a failure at `site` (first one wins) and raise the launch's fail tag.
  MONO_DEV void fail(int site) const {
    uint32_t expect = 0;
    if (__hip_atomic_compare_exchange_strong(&words[G_ERROR], &expect, (uint32_t)site + 1u, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      __hip_atomic_store(&words[G_FAIL_BLOCK], (uint32_t)block_index(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      report_host(host_err, (uint32_t)site + 1u);
    }
    __hip_atomic_store(&words[G_FAIL_TAG], launch_tag(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // True (and the failure recorded) once the deadline has passed; with `peers`, also
  // once another workgroup of this launch has failed, in any of its layers (one more
  // memory round trip).
  MONO_DEV bool expired(int site, bool peers) const {
    if (now_ticks() > deadline) {
      fail(site);
      return true;
    }
    return peers && ld_agent_u32(&words[G_FAIL_TAG]) == launch_tag();
  }
};

// Poll the mailbox words at(j) of this lane whose bit j is set in `pending` until each
// carries `tag`; their payloads go to v[j]. `at` computes an address from its index,
// so callers hold no arrays of pointers. False if the guard expired first.
//
// The first pass loads every pending word. While words are missing, a spin loads only
// the first missing one (the probe), keeps it once it carries the tag and then sweeps
// the rest (a single-word wait ends with its probe, one round trip after the word): a
// waiting workgroup then costs one load a thread a spin, not one a word, so early
// waiters do not flood the memory system the producers are streaming through.
//
// CACHED_FIRST: the first pass uses plain cacheable loads (after a hint wait has seen the
// producers finish, so many workgroups reading one broadcast payload share the L2 of
// their XCD instead of each fetching it from memory).
// PROBE = false: every spin sweeps all missing words (for small exchanges between a few
// workgroups, where a probe's extra round trip is the cost that matters).
template <int N, class At, bool CACHED_FIRST = false, bool PROBE = true>
MONO_DEV bool poll_words(At at, uint32_t (&v)[N], uint32_t pending, int site, const Guard& g) {
  if (pending && site == g.fault) {  // host-forced fault: the wait fails at once
    g.fail(site);
    return false;
  }
  if (CACHED_FIRST) {
    uint64_t w[N];
#pragma unroll
    for (int j = 0; j < N; ++j)
      if ((pending >> j) & 1u) w[j] = mb_load_cached(at(j));
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (((pending >> j) & 1u) && (uint32_t)(w[j] >> 32) == g.tag) {
        v[j] = (uint32_t)w[j];
        pending &= ~(1u << j);
      }
    if (!pending) return true;
  }
  const auto sweep = [&]() {
    uint64_t w[N];
#pragma unroll
    for (int j = 0; j < N; ++j)
      if ((pending >> j) & 1u) w[j] = mb_load(at(j));
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (((pending >> j) & 1u) && (uint32_t)(w[j] >> 32) == g.tag) {
        v[j] = (uint32_t)w[j];
        pending &= ~(1u << j);
      }
  };
  sweep();
  for (uint32_t spin = 1; pending; ++spin) {
    if (!PROBE) {
      if (spin % POLL_CHECK <= 1 && g.expired(site, spin % POLL_CHECK == 0)) return false;
      __builtin_amdgcn_s_sleep(1);
      sweep();
      continue;
    }
    uint64_t probe = 0;
    uint32_t pbit = 0u;
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (!pbit && ((pending >> j) & 1u)) {
        probe = mb_load(at(j));
        pbit = 1u << j;
      }
    if ((uint32_t)(probe >> 32) == g.tag) {
      // the probe word is in: keep it (a single-word wait ends here) and sweep the rest
#pragma unroll
      for (int j = 0; j < N; ++j)
        if (pbit == (1u << j)) v[j] = (uint32_t)probe;
      pending &= ~pbit;
      if (pending) sweep();
      continue;
    }
    // the deadline after the 1st, 33rd, ... miss; other workgroups' failures after the
    // 32nd, 64th, ... (that check is a memory round trip, kept off the first retry)
    if (spin % POLL_CHECK <= 1 && g.expired(site, spin % POLL_CHECK == 0)) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

MONO_DEV bool poll_word(const uint64_t* p, uint32_t& v, int site, const Guard& g) {
  uint32_t vs[1];
  const bool ok = poll_words<1>([p](int) { return p; }, vs, 1u, site, g);
  v = vs[0];
  return ok;
}

// Wait until each of n hint words carries the tag: thread i < n polls at(i), one word
// that producer i of the awaited data writes with (or after) the rest of its share,
// while the other threads wait at the barrier. The full poll that follows then mostly
// finds every word in place on its first pass; meanwhile a waiting workgroup costs n
// loads a spin instead of one a payload word. Workgroup-uniform result.
template <class At>
MONO_DEV bool hint_wait(int n, At at, int site, const Guard& g) {
  bool ok = true;
  for (int i = thread_index(); i < n; i += blockDim.x) {
    uint32_t v;
    ok = poll_word(at(i), v, site, g) && ok;
  }
  return __syncthreads_and(ok ? 1 : 0) != 0;
}

// Workgroup-uniform AND of a per-thread flag (a full barrier).
MONO_DEV bool block_all(bool ok) { return __syncthreads_and(ok ? 1 : 0) != 0; }

MONO_DEV bool grid_barrier(const Guard& gd, bool epoch);

// Zero the guard's mailboxes (the first launch or layer of a tag epoch), then meet every
// workgroup of the grid once its zeros are stored (grid_barrier). Workgroup-uniform
// result.
MONO_DEV bool scrub_mailboxes(const GuardArgs& a, const Guard& gd) {
  const uint32_t n_threads = gridDim.x * blockDim.x;
  const uint32_t me = block_index() * blockDim.x + (uint32_t)thread_index();
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int k = 0; k < SCRUB_MAX; ++k) {
    const ScrubRegion rg = a.scrub[k];
    if (!rg.p) break;  // uniform
    // device-coherent 16-byte stores (regions are far below 4 GB)
    const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(rg.p, (uint32_t)(rg.n16 * 16));
    for (uint64_t i = me; i < rg.n16; i += n_threads)
      __builtin_amdgcn_raw_buffer_store_b128(zero, rs, (int)(i * 16), 0, SC1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  return grid_barrier(gd, true);
}

// Meet every workgroup of the grid: each adds one to guard word 6 and waits until the
// meeting's G arrivals are in (every meeting adds exactly G, so the count is a multiple
// of G between meetings). `epoch` (a scrub): workgroup 0 first counts a tag epoch and
// clears the fail tag. Workgroup-uniform result.
MONO_DEV bool grid_barrier(const Guard& gd, bool epoch) {
  __shared__ uint32_t target;
  if (thread_index() == 0) {
    if (epoch && block_index() == 0) {
      (void)__hip_atomic_fetch_add(&gd.words[G_EPOCH], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // a failure's tag of the old epoch must not read as this epoch's (a guard that
      // runs on after a failure reaches the wrap); stored before this workgroup arrives
      __hip_atomic_store(&gd.words[G_FAIL_TAG], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
    }
    uint32_t* bar = &gd.words[G_BARRIER];
    const uint32_t before = __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    target = before - before % gridDim.x + gridDim.x;
  }
  __syncthreads();
  bool ok = true;
  if (thread_index() == 0) {
    const uint32_t want = target;
    for (uint32_t spin = 0;; ++spin) {
      if ((int32_t)(ld_agent_u32(&gd.words[G_BARRIER]) - want) >= 0) break;
      if (spin % POLL_CHECK == 0 && gd.expired(SCRUB_SITE, spin > 0)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return block_all(ok);
}

// The guard's two reads at a launch's start (thread 0's values; 0 elsewhere): the
// workgroup's launch ordinal (its counter's value before this launch's add) and the
// sticky error word. guard_fetch issues them; their first use in guard_begin waits, so
// a kernel that calls guard_fetch first and loads its own inputs before guard_begin
// overlaps the two round trips with those loads (vector memory returns in order).
struct GuardFetch {
  uint64_t ord;
  uint32_t err;
};
// A launch that runs `count` layers takes `count` ordinals at once (one tag a layer).
MONO_DEV GuardFetch guard_fetch(const GuardArgs& a, uint64_t count = 1) {
  GuardFetch f{0, 0u};
  if (thread_index() == 0) {
    f.ord = __hip_atomic_fetch_add(a.tickets + block_index(), count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    f.err = a.sticky ? ld_agent_u32(&a.words[G_ERROR]) : 0u;
  }
  return f;
}

// Layer l of a launch that took `count` ordinals from f (guard_fetch): layer l runs as
// ordinal f.ord + l, with its own tag, deadline and forced fault, and scrubs the
// mailboxes if its ordinal starts a tag epoch. The first layer also reports the launches
// begun to the host and refuses the launch under a standing sticky error. A guard with
// flip accumulators (a one-layer launch) also clears its successor's copy of them. A
// scrub at a later layer first meets the whole grid, so no workgroup still works on the
// layers before when the mailboxes are zeroed; `scrubbed` (if given) reports a scrub.
MONO_DEV bool guard_layer(const GuardArgs& a, Guard& gd, const GuardFetch& f, int l, uint64_t count,
                          bool* scrubbed = nullptr) {
  __shared__ uint32_t sh[5];
  if (thread_index() == 0) {
    const uint64_t ord = f.ord + (uint64_t)l;
#ifdef MONO_LAYER_LOOP
    sh[4] = (uint32_t)(f.ord % TAG_PERIOD) + 1u;
#endif
    if (block_index() == 0 && l == 0)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(&a.words[G_TICKET]), f.ord + count, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t in_epoch = ord % TAG_PERIOD;
    sh[0] = (uint32_t)in_epoch + 1u;
    sh[1] = l == 0 ? f.err : 0u;
    sh[2] = ord >= a.fault_from ? 1u : 0u;
    sh[3] = (in_epoch == 0 && ord != 0) ? 1u : 0u;
  }
  __syncthreads();
  gd.words = a.words;
  gd.host_err = a.host_err;
  gd.tag = sh[0];
#ifdef MONO_LAYER_LOOP
  gd.ltag = sh[4];
#endif
  gd.deadline = now_ticks() + a.deadline_ticks;
  gd.fault = sh[2] ? a.fault_site : -1;
  const uint32_t err = sh[1];
  const bool scrub = sh[3] != 0;
  __syncthreads();  // sh is read before any later layer's or launch's use of it
  if (err != 0) {
    if (thread_index() == 0) report_host(a.host_err, err);
    return false;
  }
  if (scrubbed) *scrubbed = scrub;
  if (scrub && l > 0 && !grid_barrier(gd, false)) return false;
  if (scrub && !scrub_mailboxes(a, gd)) return false;
  if (a.flip) {
    uint32_t* nx = a.flip + (size_t)((gd.tag + 1u) & 1u) * a.flip_words;
    for (int i = block_index() * blockDim.x + thread_index(); i < a.flip_words; i += gridDim.x * blockDim.x)
      __hip_atomic_store(&nx[i], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return true;
}

// The start of every launch, called by every thread of the workgroup with what
// guard_fetch returned: set up the guard (tag, deadline, this launch's forced fault),
// scrub the mailboxes at the start of a tag epoch and clear the successor's copy of the
// flip accumulators. False (workgroup-uniform) if the guard's sticky error refuses the
// launch (a refused launch reports the error to the host word) or the scrub failed.
MONO_DEV bool guard_begin(const GuardArgs& a, Guard& gd, const GuardFetch& f) { return guard_layer(a, gd, f, 0, 1); }
MONO_DEV bool guard_begin(const GuardArgs& a, Guard& gd) { return guard_begin(a, gd, guard_fetch(a)); }

// A launch that failed or was refused writes NaN over its bf16 output (n elements at p):
// `share` writes the workgroup's grid-strided share (every workgroup refuses together),
// otherwise the whole output (the workgroups that saw a failure). Workgroups whose
// waits succeeded may still store finished rows afterwards, so a failed launch's output
// can be partly plausible; the host error word is what tells a failure.
MONO_DEV void poison_bf16(void* p, size_t n, bool share) {
  if (!p) return;
  uint32_t* w = static_cast<uint32_t*>(p);
  const size_t words = n / 2;
  const size_t step = share ? (size_t)gridDim.x * blockDim.x : blockDim.x;
  for (size_t i = (share ? block_index() * blockDim.x : 0) + (size_t)thread_index(); i < words; i += step) w[i] = 0x7fc07fc0u;
}

}  // namespace mono
