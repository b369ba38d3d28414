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
// Tags: every workgroup of a launch takes a ticket from guard word 0 with one atomic
// add; ticket / gridDim.x is the launch's ordinal (launches of one runtime are
// stream-ordered, so their tickets never interleave) and the tag is ordinal + 1. A
// HIP-graph replay takes fresh tickets, so it never sees a stale word as ready.
//
// Guard words (int32 [8] in device memory, common/guard.py:16-30 in the reference):
//   0  launch tickets
//   1  error: 1 + the id of the first wait site that ran out of time (sticky: every
//      later launch of the runtime exits at once until the host clears it)
//   2  tag of the failing launch (waits of that launch give up when they see it)
//   3  workgroup that failed first
// Every wait polls its words until their tags match, checking the deadline
// (s_memrealtime, 100 MHz) after its first poll and then every POLL_CHECK polls, and
// the launch's fail tag every POLL_CHECK polls. On expiry it records the error,
// raises word 2 and returns false; the caller makes the failure workgroup-uniform and
// the workgroup exits. No wait ever blocks past the deadline and nothing faults: the
// launch drains and the host reads the error words (fail-stop without a GPU fault).
#pragma once

#include "common.h"

namespace mono {

enum GuardWord { G_TICKET = 0, G_ERROR = 1, G_FAIL_TAG = 2, G_FAIL_BLOCK = 3, G_WORDS = 8 };
constexpr int POLL_CHECK = 32;

// Kernel-argument part of the guard: the words, the deadline and the host-forced
// fault (a wait site whose waits the host makes fail at once, for tests of the error
// path; -1 = none).
struct GuardArgs {
  uint32_t* words;
  uint64_t deadline_ticks;
  int32_t fault_site;
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
  if ((int)threadIdx.x < DONE_REPLICAS) mb_put(base + threadIdx.x * DONE_STRIDE + i, 0u, tag);
}
MONO_DEV const uint64_t* done_copy(const uint64_t* base) { return base + (blockIdx.x % DONE_REPLICAS) * DONE_STRIDE; }

struct Guard {
  GuardArgs a;
  uint64_t deadline;  // absolute s_memrealtime tick
  uint32_t tag;

  // Record a failure at `site` (first one wins) and raise the launch's fail tag.
  MONO_DEV void fail(int site) const {
    uint32_t expect = 0;
    if (__hip_atomic_compare_exchange_strong(&a.words[G_ERROR], &expect, (uint32_t)site + 1u, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      __hip_atomic_store(&a.words[G_FAIL_BLOCK], (uint32_t)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&a.words[G_FAIL_TAG], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // True (and the failure recorded) once the deadline has passed; with `peers`, also
  // once another workgroup of this launch has failed (one more memory round trip).
  MONO_DEV bool expired(int site, bool peers) const {
    if (now_ticks() > deadline) {
      fail(site);
      return true;
    }
    return peers && ld_agent_u32(&a.words[G_FAIL_TAG]) == tag;
  }
};

// Poll the mailbox words at(j) of this lane whose bit j is set in `pending` until each
// carries `tag`; their payloads go to v[j]. `at` computes an address from its index,
// so callers hold no arrays of pointers. False if the guard expired first.
//
// The first pass loads every pending word. While words are missing, a spin loads only
// the first missing one (the probe) and sweeps the rest once the probe has arrived: a
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
  if (pending && site == g.a.fault_site) {  // host-forced fault: the wait fails at once
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
    bool sent = false;
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (!sent && ((pending >> j) & 1u)) {
        probe = mb_load(at(j));
        sent = true;
      }
    if ((uint32_t)(probe >> 32) == g.tag) {
      sweep();
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
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    uint32_t v;
    ok = poll_word(at(i), v, site, g) && ok;
  }
  return __syncthreads_and(ok ? 1 : 0) != 0;
}

// Workgroup-uniform AND of a per-thread flag (a full barrier).
MONO_DEV bool block_all(bool ok) { return __syncthreads_and(ok ? 1 : 0) != 0; }

}  // namespace mono
