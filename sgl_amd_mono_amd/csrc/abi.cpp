// The C-ABI of libmono_gfx950.so: runtime handles, argument checks, error strings.
//
// A handle owns its device scratch (one hipMalloc at create, freed at destroy): the
// mailboxes and guard words of its persistent launch, the way the reference's
// Glm53Runtime owns its scratch mailboxes and guard words
// (glm53/gfx950/runner.py:133-215). Forward calls validate their arguments on the
// host, then enqueue one launch on the caller's stream and return.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "abi_errors.h"
#include "attn_back_ops.h"
#include "layer_ops.h"
#include "attn_ops.h"
#include "mono.h"
#include "moe_ops.h"
#include "proj_ops.h"
#include "row_ssq.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return MONO_OK;
}

#define HIP_TRY(call)                                                                   \
  do {                                                                                  \
    hipError_t e_ = (call);                                                             \
    if (e_ != hipSuccess) return fail(MONO_EHIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

#define REQUIRE_PTR(p) \
  if (!(p)) return fail(MONO_EINVAL, "argument %s must be a device pointer, got NULL", #p)

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

int check_device(int device) {
  int cur = -1;
  HIP_TRY(hipGetDevice(&cur));
  if (cur != device) return fail(MONO_ESTATE, "the current HIP device is %d, the runtime lives on %d", cur, device);
  return MONO_OK;
}

const double TICKS_PER_S = 100e6;  // s_memrealtime runs at 100 MHz
const double DEFAULT_DEADLINE_S = 2.0;
const double MAX_DEADLINE_S = 3600.0;

// Carves one device allocation into 256-byte aligned pieces after the runtime's header
// (the guard words, the scrub table and the unit scale in its first 256 bytes, then the
// per-workgroup launch counters).
constexpr size_t SCRUB_OFF = 64;    // the guard's scrub table in the header
constexpr size_t UNIT_OFF = 192;    // the f32 1.0 in the header
constexpr size_t TICKETS_OFF = 256;  // u64 [MAX_GRID] launch counters, one a workgroup
constexpr int MAX_GRID = 1024;
constexpr size_t HEADER = TICKETS_OFF + MAX_GRID * sizeof(uint64_t);
struct Carve {
  size_t off = HEADER;
  size_t take(size_t bytes) {
    const size_t at = off;
    off += align256(bytes);
    return at;
  }
};

}  // namespace

namespace mono {
// the library's error string for entry points in other sources (abi_errors.h)
int abi_fail(int code, const char* msg) { return fail(code, "%s", msg); }
int abi_ok() { return ok(); }
}  // namespace mono

// A pinned host word the launches' guard copies its errors to (system scope), so the
// host sees a stopped launch without synchronising.
struct HostErr {
  uint32_t* host = nullptr;  // host address
  uint32_t* dev = nullptr;   // the device's address of it
  int alloc(const char* what) {
    void* p = nullptr;
    hipError_t e = hipHostMalloc(&p, 64, hipHostMallocCoherent | hipHostMallocMapped);
    if (e != hipSuccess) return fail(MONO_ENOMEM, "hipHostMalloc for the %s error word: %s", what, hipGetErrorString(e));
    host = static_cast<uint32_t*>(p);
    *host = 0;
    void* d = nullptr;
    e = hipHostGetDevicePointer(&d, p, 0);
    if (e != hipSuccess) return fail(MONO_EHIP, "hipHostGetDevicePointer: %s", hipGetErrorString(e));
    dev = static_cast<uint32_t*>(d);
    return MONO_OK;
  }
  uint32_t read() const { return host ? __atomic_load_n(host, __ATOMIC_ACQUIRE) : 0u; }
  void clear() {
    if (host) __atomic_store_n(host, 0u, __ATOMIC_RELEASE);
  }
  int release() {
    if (!host) return MONO_OK;
    hipError_t e = hipHostFree(host);
    host = dev = nullptr;
    return e == hipSuccess ? MONO_OK : fail(MONO_EHIP, "hipHostFree: %s", hipGetErrorString(e));
  }
};

// What every runtime handle has: its device, the persistent grid, the scratch blob
// and the guard (common/guard.py:100-241 in the reference).
struct RuntimeBase {
  uint32_t magic = 0;
  int device = 0;
  int grid = 0;  // workgroups of the persistent launch: one a CU
  void* blob = nullptr;
  size_t blob_bytes = 0;
  mono::GuardArgs guard{};
  HostErr herr;
  // one f32 1.0 in the header: the per-token scale of every row of an MLA cache passed
  // without a scale plane (raw E4M3 rows), read and written at index 0
  float* unit = nullptr;

  // Allocate and zero the header and `bytes` of mailboxes (a Carve's `off`), and write
  // the scrub table: every mailbox after the header. Tag 0 is never a launch's tag, so
  // zeroed mailboxes read as empty.
  int init(int dev, size_t bytes, int (*occupancy)(int*), const char* what) {
    device = dev;
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, dev));
    int per_cu = 0;
    if (int rc = occupancy(&per_cu)) return rc;
    if (per_cu < 1) return fail(MONO_ESTATE, "the persistent %s kernel does not fit on a CU (occupancy %d)", what, per_cu);
    grid = prop.multiProcessorCount;
    if (grid > MAX_GRID) return fail(MONO_ESTATE, "%d CUs: the launch counters hold at most %d workgroups", grid, MAX_GRID);
    const size_t total = align256(bytes);
    hipError_t e = hipMalloc(&blob, total);
    if (e != hipSuccess) {
      blob = nullptr;
      return fail(MONO_ENOMEM, "hipMalloc(%zu) for the %s mailboxes: %s", total, what, hipGetErrorString(e));
    }
    blob_bytes = total;
    if (int rc = herr.alloc(what)) return rc;
    unit = reinterpret_cast<float*>(at(UNIT_OFF));
    mono::ScrubRegion table[mono::SCRUB_MAX] = {};
    table[0] = mono::ScrubRegion{reinterpret_cast<uint32_t*>(at(HEADER)), (total - HEADER) / 16};
    const float one = 1.0f;
    e = hipMemset(blob, 0, total);
    if (e == hipSuccess) e = hipMemcpy(unit, &one, sizeof(one), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(at(SCRUB_OFF), table, sizeof(table), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return fail(MONO_EHIP, "clearing the %s mailboxes: %s", what, hipGetErrorString(e));
    guard.words = reinterpret_cast<uint32_t*>(at(0));
    guard.tickets = reinterpret_cast<uint64_t*>(at(TICKETS_OFF));
    guard.scrub = reinterpret_cast<const mono::ScrubRegion*>(at(SCRUB_OFF));
    guard.host_err = herr.dev;
    guard.deadline_ticks = (uint64_t)(DEFAULT_DEADLINE_S * TICKS_PER_S);
    guard.fault_site = -1;
    guard.fault_from = 0;
    guard.sticky = 1;
    return MONO_OK;
  }
  char* at(size_t off) const { return static_cast<char*>(blob) + off; }
  // the mailboxes after the header, as a scrub region
  mono::ScrubRegion mailboxes() const {
    return mono::ScrubRegion{reinterpret_cast<uint32_t*>(at(HEADER)), (blob_bytes - HEADER) / 16};
  }
  // Free the scratch; the handle is dead afterwards (idempotent like PeerBuffer.close,
  // common/peer.py:157-165).
  int release() {
    magic = 0;
    int rc = herr.release();
    if (!blob) return rc;
    hipError_t e = hipFree(blob);
    blob = nullptr;
    if (e != hipSuccess) return fail(MONO_EHIP, "hipFree: %s", hipGetErrorString(e));
    return rc;
  }
};

struct mono_moe : RuntimeBase {
  mono_moe_config cfg;
  mono::moe::Mail mail;
};

struct mono_attn : RuntimeBase {
  mono_attn_config cfg;
  mono::attn::Mail mail;
  mono::proj::Mail back_mail;  // the fused attention + back launch's W_UV output and done words
};

struct mono_proj : RuntimeBase {
  mono_proj_config cfg;
  mono::proj::Mail mail;
};

static const uint32_t MOE_MAGIC = 0x6d6f6531u;
static const uint32_t ATTN_MAGIC = 0x6174746eu;
static const uint32_t PROJ_MAGIC = 0x70726f6au;

namespace {

int occ_moe_fp8(int* n) {
  HIP_TRY(mono::moe::moe_fp8_occupancy(n));
  return MONO_OK;
}
int occ_moe_mxfp4(int* n) {
  HIP_TRY(mono::moe::moe_mxfp4_occupancy(n));
  return MONO_OK;
}
int occ_proj(int* n) {
  int a = 0, b = 0;
  HIP_TRY(mono::proj::front_occupancy(&a));
  HIP_TRY(mono::proj::back_occupancy(&b));
  *n = std::min(a, b);
  return MONO_OK;
}
int occ_attn(int* n) {
  HIP_TRY(mono::attn::attn_occupancy(n));
  return MONO_OK;
}

bool live(const RuntimeBase* r, uint32_t magic) { return r && r->magic == magic; }

// The guard controls, on a guard's kernel arguments, its device, grid and host word.
struct GuardRef {
  mono::GuardArgs* g;
  int device;
  int grid;
  HostErr* herr;
};
GuardRef ref(RuntimeBase* r) { return GuardRef{&r->guard, r->device, r->grid, &r->herr}; }

int guard_set_deadline(GuardRef r, double seconds) {
  if (!(seconds > 0.0) || seconds > MAX_DEADLINE_S)
    return fail(MONO_EINVAL, "deadline must be in (0, %.0f] seconds, got %g", MAX_DEADLINE_S, seconds);
  const double ticks = seconds * TICKS_PER_S;
  r.g->deadline_ticks = ticks < 1.0 ? 1u : (uint64_t)ticks;
  return ok();
}

// The launches' ordinal so far (synchronises): workgroup 0's launch counter.
int guard_ordinal(GuardRef r, uint64_t* ord) {
  if (int rc = check_device(r.device)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(ord, r.g->tickets, sizeof(*ord), hipMemcpyDeviceToHost));
  return MONO_OK;
}

// The host-forced fault at `site` for every launch from `after` launches on (-1: off).
int guard_set_fault(GuardRef r, int32_t site, int64_t after) {
  if (site < -1 || site > 31) return fail(MONO_EINVAL, "fault site must be -1 (none) or a wait site 0..31, got %d", site);
  if (after < 0) return fail(MONO_EINVAL, "after must be >= 0 launches, got %lld", (long long)after);
  uint64_t from = 0;
  if (site >= 0 && after > 0) {
    if (int rc = guard_ordinal(r, &from)) return rc;
    from += (uint64_t)after;
  }
  r.g->fault_site = site;
  r.g->fault_from = from;
  return ok();
}

int guard_read(GuardRef r, int32_t* words) {
  if (!words) return fail(MONO_EINVAL, "read_errors: words is NULL");
  if (int rc = check_device(r.device)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(words, r.g->words, MONO_GUARD_WORDS * sizeof(int32_t), hipMemcpyDeviceToHost));
  return ok();
}

// Zero every mailbox region of the guard's scrub table (callers have synchronised).
// Afterwards no word carries any earlier launch's tag and both copies of the flip
// accumulators start at zero, whichever launches were refused or skipped before: a
// refused first launch of a tag epoch never ran its scrub, and a refused launch never
// cleared its successor's flip copy.
int guard_scrub_all(GuardRef r) {
  mono::ScrubRegion table[mono::SCRUB_MAX];
  HIP_TRY(hipMemcpy(table, r.g->scrub, sizeof(table), hipMemcpyDeviceToHost));
  for (const mono::ScrubRegion& rg : table) {
    if (!rg.p) break;
    HIP_TRY(hipMemset(rg.p, 0, rg.n16 * 16));
  }
  return MONO_OK;
}

// Clear the sticky error (words 1-3, the tickets stay), every mailbox and the host word.
int guard_clear(GuardRef r) {
  if (int rc = check_device(r.device)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemset(r.g->words + mono::G_ERROR, 0, 3 * sizeof(int32_t)));
  if (int rc = guard_scrub_all(r)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  r.herr->clear();
  return ok();
}

// Move the launch ordinal to `ordinal` (synchronises; tests of the tag epochs): the next
// launch takes tag ordinal % TAG_PERIOD + 1. Every mailbox is zeroed too, so a jump of
// any length or direction leaves no word that reads as written under a coming tag and
// no flip copy holding an earlier launch's sums.
int guard_set_ordinal(GuardRef r, uint64_t ordinal) {
  if (ordinal == UINT64_MAX) return fail(MONO_EINVAL, "ordinal %llu is out of range", (unsigned long long)ordinal);
  if (int rc = check_device(r.device)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  if (int rc = guard_scrub_all(r)) return rc;
  std::vector<uint64_t> counters((size_t)r.grid, ordinal);
  HIP_TRY(hipMemcpy(r.g->tickets, counters.data(), counters.size() * sizeof(uint64_t), hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(r.g->words + mono::G_TICKET, &ordinal, sizeof(ordinal), hipMemcpyHostToDevice));
  HIP_TRY(hipDeviceSynchronize());
  return ok();
}

}  // namespace

extern "C" int mono_abi_version(void) { return MONO_ABI_VERSION; }

extern "C" const char* mono_last_error(void) { return g_error.c_str(); }

// ------------------------------------------------------------------ MoE runtime

extern "C" int mono_moe_create(const mono_moe_config* cfg, mono_moe** out) {
  using namespace mono::moe;
  if (!cfg || !out) return fail(MONO_EINVAL, "mono_moe_create: cfg and out must be non-NULL");
  *out = nullptr;
  const mono_moe_config& c = *cfg;
  if (c.max_rows < 1 || c.max_rows > MAX_ROWS)
    return fail(MONO_EINVAL, "max_rows must be in [1, %d], got %d", MAX_ROWS, c.max_rows);
  if (c.n_experts < 1 || c.n_experts > MAX_EXPERTS)
    return fail(MONO_EINVAL, "n_experts must be in [1, %d], got %d", MAX_EXPERTS, c.n_experts);
  if (c.top_k < 1 || c.top_k > MAX_TOPK) return fail(MONO_EINVAL, "top_k must be in [1, %d], got %d", MAX_TOPK, c.top_k);
  if (c.hidden <= 0 || c.hidden % 512) return fail(MONO_EINVAL, "hidden must be a positive multiple of 512, got %d", c.hidden);
  if (c.inter <= 0 || c.inter % 128) return fail(MONO_EINVAL, "inter must be a positive multiple of 128, got %d", c.inter);
  if (c.weight_format != MONO_WEIGHT_FP8_BLOCK128 && c.weight_format != MONO_WEIGHT_MXFP4)
    return fail(MONO_EINVAL, "unknown weight_format %d", c.weight_format);
  if (c.router != MONO_ROUTER_SIGMOID_BIAS && c.router != MONO_ROUTER_SOFTMAX)
    return fail(MONO_EINVAL, "unknown router %d", c.router);
  const MoeGeom geo{c.hidden, c.n_experts, c.top_k, c.inter};
  const bool fp8 = c.weight_format == MONO_WEIGHT_FP8_BLOCK128;
  if (fp8 && (!moe_fp8_supported(geo) || c.router != MONO_ROUTER_SIGMOID_BIAS))
    return fail(MONO_EINVAL,
                "FP8 MoE geometry H=%d E=%d top_k=%d I=%d router %d has no compiled kernel (built: H=7168 E=256 "
                "top_k=8 I=512, sigmoid + bias router)",
                c.hidden, c.n_experts, c.top_k, c.inter, c.router);
  if (!fp8 && (!moe_mxfp4_supported(geo) || c.router != MONO_ROUTER_SOFTMAX))
    return fail(MONO_EINVAL,
                "MXFP4 MoE geometry H=%d E=%d top_k=%d I=%d router %d has no compiled kernel (built: H=3072 E=256 "
                "top_k=8 I=384, softmax router)",
                c.hidden, c.n_experts, c.top_k, c.inter, c.router);
  if (int rc = check_device(c.device)) return rc;
  const size_t H = c.hidden, E = c.n_experts, I = c.inter;
  const size_t max_act = (size_t)std::min(c.max_rows * c.top_k, c.n_experts) + 1;
  Carve cv;
  const size_t o_xq = cv.take((size_t)MAX_ROWS * H);
  const size_t o_xs = cv.take((size_t)MAX_ROWS * (H / 128) * 4);
  const size_t o_score = cv.take((size_t)MAX_ROWS * E * 8);
  const size_t o_rdone = cv.take(mono::DONE_BYTES);
  const size_t o_mid = cv.take(max_act * MAX_ROWS * I * 8);
  const size_t o_mtile = cv.take(max_act * (I / 16) * 8);
  const size_t o_ypart = cv.take(max_act * MAX_ROWS * H * 8);
  mono_moe* m = new mono_moe();
  m->magic = MOE_MAGIC;
  m->cfg = c;
  if (int rc = m->init(c.device, cv.off, fp8 ? occ_moe_fp8 : occ_moe_mxfp4, "MoE")) {
    (void)m->release();
    delete m;
    return rc;
  }
  m->mail.guard = m->guard.words;
  m->mail.xq = reinterpret_cast<uint8_t*>(m->at(o_xq));
  m->mail.xs = reinterpret_cast<float*>(m->at(o_xs));
  m->mail.score = reinterpret_cast<uint64_t*>(m->at(o_score));
  m->mail.rdone = reinterpret_cast<uint64_t*>(m->at(o_rdone));
  m->mail.mid = reinterpret_cast<uint64_t*>(m->at(o_mid));
  m->mail.mtile = reinterpret_cast<uint64_t*>(m->at(o_mtile));
  m->mail.ypart = reinterpret_cast<uint64_t*>(m->at(o_ypart));
  *out = m;
  return ok();
}

extern "C" int mono_moe_destroy(mono_moe* m) {
  if (!m) return ok();
  if (!live(m, MOE_MAGIC)) return fail(MONO_ESTATE, "mono_moe_destroy: not a live MoE runtime");
  const int rc = m->release();
  delete m;
  return rc ? rc : ok();
}

static int check_moe(const mono_moe* m, int rows) {
  if (!live(m, MOE_MAGIC)) return fail(MONO_ESTATE, "not a live MoE runtime");
  if (rows < 1 || rows > m->cfg.max_rows)
    return fail(MONO_EINVAL, "rows must be in [1, %d] (the runtime's max_rows), got %d", m->cfg.max_rows, rows);
  return check_device(m->device);
}

static int check_moe_fp8(const mono_moe* m, const mono_moe_fp8_args* args) {
  if (!args) return fail(MONO_EINVAL, "mono_moe_fp8_forward: args is NULL");
  if (int rc = check_moe(m, args->rows)) return rc;
  if (m->cfg.weight_format != MONO_WEIGHT_FP8_BLOCK128 || m->cfg.router != MONO_ROUTER_SIGMOID_BIAS)
    return fail(MONO_ESTATE, "this runtime was created for another weight format / router");
  REQUIRE_PTR(args->a);
  REQUIRE_PTR(args->g_post);
  REQUIRE_PTR(args->w_router);
  REQUIRE_PTR(args->bias);
  REQUIRE_PTR(args->w13);
  REQUIRE_PTR(args->s13);
  REQUIRE_PTR(args->w2);
  REQUIRE_PTR(args->s2);
  REQUIRE_PTR(args->out);
  return MONO_OK;
}

extern "C" int mono_moe_fp8_forward(mono_moe* m, const mono_moe_fp8_args* args, void* stream) {
  using namespace mono::moe;
  if (int rc = check_moe_fp8(m, args)) return rc;
  MoeFp8Args g(*args, m->cfg.route_scale, m->cfg.eps);
  hipError_t e = moe_fp8_forward(g, m->grid, m->mail, m->guard, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the FP8 MoE: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_moe_mxfp4_forward(mono_moe* m, const mono_moe_mxfp4_args* args, void* stream) {
  using namespace mono::moe;
  if (!args) return fail(MONO_EINVAL, "mono_moe_mxfp4_forward: args is NULL");
  if (int rc = check_moe(m, args->rows)) return rc;
  if (m->cfg.weight_format != MONO_WEIGHT_MXFP4 || m->cfg.router != MONO_ROUTER_SOFTMAX)
    return fail(MONO_ESTATE, "this runtime was created for another weight format / router");
  REQUIRE_PTR(args->x);
  REQUIRE_PTR(args->logits);
  REQUIRE_PTR(args->w13);
  REQUIRE_PTR(args->s13);
  REQUIRE_PTR(args->w2);
  REQUIRE_PTR(args->s2);
  REQUIRE_PTR(args->out);
  hipError_t e = moe_mxfp4_forward(*args, m->grid, m->mail, m->guard, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the MXFP4 MoE: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_moe_set_deadline(mono_moe* m, double seconds) {
  if (!live(m, MOE_MAGIC)) return fail(MONO_ESTATE, "not a live MoE runtime");
  return guard_set_deadline(ref(m), seconds);
}

extern "C" int mono_moe_set_fault(mono_moe* m, int32_t site) {
  if (!live(m, MOE_MAGIC)) return fail(MONO_ESTATE, "not a live MoE runtime");
  return guard_set_fault(ref(m), site, 0);
}

extern "C" int mono_moe_read_errors(mono_moe* m, int32_t* words) {
  if (!live(m, MOE_MAGIC)) return fail(MONO_ESTATE, "not a live MoE runtime");
  return guard_read(ref(m), words);
}

extern "C" int mono_moe_clear_errors(mono_moe* m) {
  if (!live(m, MOE_MAGIC)) return fail(MONO_ESTATE, "not a live MoE runtime");
  return guard_clear(ref(m));
}

// ------------------------------------------------------------------ attention runtime

extern "C" int mono_attn_create(const mono_attn_config* cfg, mono_attn** out) {
  using namespace mono::attn;
  if (!cfg || !out) return fail(MONO_EINVAL, "mono_attn_create: cfg and out must be non-NULL");
  *out = nullptr;
  const mono_attn_config& c = *cfg;
  if (c.max_rows < 1 || c.max_rows > MAX_ROWS)
    return fail(MONO_EINVAL, "max_rows must be in [1, %d], got %d", MAX_ROWS, c.max_rows);
  if (c.max_ctx < CHUNK || c.max_ctx > MAX_CTX || c.max_ctx % CHUNK)
    return fail(MONO_EINVAL, "max_ctx must be a multiple of %d in [%d, %d], got %d", CHUNK, CHUNK, MAX_CTX, c.max_ctx);
  if (!(c.softmax_scale > 0.f)) return fail(MONO_EINVAL, "softmax_scale must be positive, got %g", c.softmax_scale);
  if (int rc = check_device(c.device)) return rc;
  const size_t R = c.max_rows;
  Carve cv;
  const size_t o_score = cv.take(R * c.max_ctx * 4);
  const size_t o_sel = cv.take(R * TOPK * 8);
  const size_t o_rowh = cv.take(2 * R * ROWH * 4);
  const size_t o_cdone = cv.take(R * (c.max_ctx / CHUNK) * 8);
  const size_t o_hist = cv.take(R * PASSES * TEAM * HW * 8);
  const size_t o_cand = cv.take(R * CMAX * 8);
  const size_t o_cnt = cv.take(R * TEAM * 2 * 8);
  const size_t o_part = cv.take(R * SPLITS * NH * DV * 2);
  const size_t o_ml = cv.take(R * SPLITS * NH * 2 * 4);
  const size_t o_sdone = cv.take(R * SPLITS * 8);
  const size_t o_mdone = cv.take(R * NH * 8);
  const size_t o_fob = cv.take((size_t)mono::proj::MAX_ROWS * mono::proj::HEADS * mono::proj::VDIM / 2 * 4);
  const size_t o_fodone = cv.take(mono::DONE_BYTES);
  mono_attn* a = new mono_attn();
  a->magic = ATTN_MAGIC;
  a->cfg = c;
  if (int rc = a->init(c.device, cv.off, occ_attn, "attention")) {
    (void)a->release();
    delete a;
    return rc;
  }
  if (a->grid % TEAM) {  // top-k teams must not straddle a round of the task list
    (void)a->release();
    delete a;
    return fail(MONO_ESTATE, "the attention launch needs a CU count divisible by %d, got %d", TEAM, a->grid);
  }
  a->mail.mdone = reinterpret_cast<uint64_t*>(a->at(o_mdone));
  a->back_mail = mono::proj::Mail{};
  a->back_mail.ob = reinterpret_cast<uint32_t*>(a->at(o_fob));
  a->back_mail.odone = reinterpret_cast<uint64_t*>(a->at(o_fodone));
  a->back_mail.guard = a->guard.words;
  a->mail.guard = a->guard.words;
  a->mail.score = reinterpret_cast<uint32_t*>(a->at(o_score));
  a->mail.sel = reinterpret_cast<uint64_t*>(a->at(o_sel));
  a->mail.rowh = reinterpret_cast<uint32_t*>(a->at(o_rowh));
  // the row histograms are atomic accumulators by launch parity: the guard's flip words
  a->guard.flip = a->mail.rowh;
  a->guard.flip_words = (int32_t)(R * ROWH);
  a->mail.cdone = reinterpret_cast<uint64_t*>(a->at(o_cdone));
  a->mail.hist = reinterpret_cast<uint64_t*>(a->at(o_hist));
  a->mail.cand = reinterpret_cast<uint64_t*>(a->at(o_cand));
  a->mail.cnt = reinterpret_cast<uint64_t*>(a->at(o_cnt));
  a->mail.part = reinterpret_cast<uint16_t*>(a->at(o_part));
  a->mail.ml = reinterpret_cast<float*>(a->at(o_ml));
  a->mail.sdone = reinterpret_cast<uint64_t*>(a->at(o_sdone));
  a->mail.max_ctx = c.max_ctx;
  a->mail.max_rows = c.max_rows;
  *out = a;
  return ok();
}

extern "C" int mono_attn_destroy(mono_attn* a) {
  if (!a) return ok();
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "mono_attn_destroy: not a live attention runtime");
  const int rc = a->release();
  delete a;
  return rc ? rc : ok();
}

// The kernel arguments of an attention launch: a NULL kv_scale (raw E4M3 MLA rows)
// reads the runtime's f32 1.0 for every row.
static mono::attn::AttnArgs attn_args(const mono_attn* a, const mono_attn_args& args) {
  mono::attn::AttnArgs g(args, a->cfg.softmax_scale);
  if (!args.kv_scale) {
    g.kv_scale = a->unit;
    g.kv_mask = 0;
  }
  return g;
}

extern "C" int mono_attn_forward(mono_attn* a, const mono_attn_args* args, void* stream) {
  using namespace mono::attn;
  if (!args) return fail(MONO_EINVAL, "mono_attn_forward: args is NULL");
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "not a live attention runtime");
  if (args->rows < 1 || args->rows > a->cfg.max_rows)
    return fail(MONO_EINVAL, "rows must be in [1, %d] (the runtime's max_rows), got %d", a->cfg.max_rows, args->rows);
  if (args->pt_stride < a->cfg.max_ctx / PAGE)
    return fail(MONO_EINVAL, "pt_stride must cover max_ctx / 64 = %d pages, got %d", a->cfg.max_ctx / PAGE,
                args->pt_stride);
  if (args->n_pages < 1) return fail(MONO_EINVAL, "n_pages must be positive, got %d", args->n_pages);
  if (int rc = check_device(a->device)) return rc;
  REQUIRE_PTR(args->iq);
  REQUIRE_PTR(args->iqs);
  REQUIRE_PTR(args->iw);
  REQUIRE_PTR(args->ikv);
  REQUIRE_PTR(args->iks);
  REQUIRE_PTR(args->q);
  REQUIRE_PTR(args->kv);
  REQUIRE_PTR(args->page_table);
  REQUIRE_PTR(args->seq_lens);
  REQUIRE_PTR(args->out);
  AttnArgs g = attn_args(a, *args);
  hipError_t e = attn_forward(g, a->grid, a->mail, a->guard, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the sparse attention: %s", hipGetErrorString(e));
  return ok();
}

static int check_attn_back(const mono_attn* a, const mono_attn_args* args, const mono_proj_weights* w,
                           const mono_back_args* back) {
  using namespace mono::attn;
  if (!args || !w || !back) return fail(MONO_EINVAL, "mono_attn_back_forward: args, w and back must be non-NULL");
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "not a live attention runtime");
  if (args->rows < 1 || args->rows > a->cfg.max_rows || args->rows > mono::proj::MAX_ROWS)
    return fail(MONO_EINVAL, "rows must be in [1, %d] (the runtime's max_rows), got %d",
                std::min(a->cfg.max_rows, mono::proj::MAX_ROWS), args->rows);
  if (back->rows != args->rows) return fail(MONO_EINVAL, "back->rows (%d) must equal args->rows (%d)", back->rows, args->rows);
  if (back->o_lat && back->o_lat != args->out)
    return fail(MONO_EINVAL, "back->o_lat must be NULL or args->out: the back reads the attention's output");
  if (args->pt_stride < a->cfg.max_ctx / PAGE)
    return fail(MONO_EINVAL, "pt_stride must cover max_ctx / 64 = %d pages, got %d", a->cfg.max_ctx / PAGE,
                args->pt_stride);
  if (args->n_pages < 1) return fail(MONO_EINVAL, "n_pages must be positive, got %d", args->n_pages);
  if (int rc = check_device(a->device)) return rc;
  REQUIRE_PTR(args->iq);
  REQUIRE_PTR(args->iqs);
  REQUIRE_PTR(args->iw);
  REQUIRE_PTR(args->ikv);
  REQUIRE_PTR(args->iks);
  REQUIRE_PTR(args->q);
  REQUIRE_PTR(args->kv);
  REQUIRE_PTR(args->page_table);
  REQUIRE_PTR(args->seq_lens);
  REQUIRE_PTR(args->out);
  REQUIRE_PTR(w->w_uv);
  REQUIRE_PTR(w->s_uv);
  REQUIRE_PTR(w->w_o);
  REQUIRE_PTR(w->s_o);
  REQUIRE_PTR(back->h);
  REQUIRE_PTR(back->a);
  return MONO_OK;
}

extern "C" int mono_attn_back_forward(mono_attn* a, const mono_attn_args* args, const mono_proj_weights* w,
                                      const mono_back_args* back, void* stream) {
  using namespace mono::attn;
  if (int rc = check_attn_back(a, args, w, back)) return rc;
  int per_cu = 0;
  HIP_TRY(mono::fused::attn_back_occupancy(&per_cu));
  if (per_cu < 1) return fail(MONO_ESTATE, "the fused attention + back kernel does not fit on a CU");
  mono_back_args b = *back;
  b.o_lat = args->out;
  AttnArgs g = attn_args(a, *args);
  hipError_t e = mono::fused::attn_back_forward(g, a->mail, a->guard, *w, b, a->back_mail, a->grid,
                                                static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the fused attention + back: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_attn_set_deadline(mono_attn* a, double seconds) {
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "not a live attention runtime");
  return guard_set_deadline(ref(a), seconds);
}

extern "C" int mono_attn_set_fault(mono_attn* a, int32_t site) {
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "not a live attention runtime");
  return guard_set_fault(ref(a), site, 0);
}

extern "C" int mono_attn_read_errors(mono_attn* a, int32_t* words) {
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "not a live attention runtime");
  return guard_read(ref(a), words);
}

extern "C" int mono_attn_clear_errors(mono_attn* a) {
  if (!live(a, ATTN_MAGIC)) return fail(MONO_ESTATE, "not a live attention runtime");
  // the scrub table covers every mailbox, the row histograms' two copies included
  return guard_clear(ref(a));
}

// ------------------------------------------------------------------ projection runtime

extern "C" int mono_proj_create(const mono_proj_config* cfg, mono_proj** out) {
  using namespace mono::proj;
  if (!cfg || !out) return fail(MONO_EINVAL, "mono_proj_create: cfg and out must be non-NULL");
  *out = nullptr;
  const mono_proj_config& c = *cfg;
  if (c.max_rows < 1 || c.max_rows > MAX_ROWS)
    return fail(MONO_EINVAL, "max_rows must be in [1, %d], got %d", MAX_ROWS, c.max_rows);
  if (int rc = check_device(c.device)) return rc;
  Carve cv;
  size_t o_mb[4];
  for (int i = 0; i < 4; ++i) o_mb[i] = cv.take(MAIL_WORDS[i] * 4);
  const size_t o_odone = cv.take(mono::DONE_BYTES);
  const size_t o_xn = cv.take((size_t)mono::proj::MAX_ROWS * mono::proj::HIDDEN * 2);
  const size_t o_xdone = cv.take(mono::DONE_BYTES);
  const size_t o_adone = cv.take(mono::DONE_BYTES);
  const size_t o_cdone = cv.take((size_t)mono::proj::C_TASKS * 8);
  const size_t o_fdone = cv.take(mono::DONE_BYTES);
  mono_proj* p = new mono_proj();
  p->magic = PROJ_MAGIC;
  p->cfg = c;
  if (int rc = p->init(c.device, cv.off, occ_proj, "projection")) {
    (void)p->release();
    delete p;
    return rc;
  }
  p->mail.guard = p->guard.words;
  p->mail.pa = reinterpret_cast<uint32_t*>(p->at(o_mb[0]));
  p->mail.qnope = reinterpret_cast<uint32_t*>(p->at(o_mb[1]));
  p->mail.iqraw = reinterpret_cast<uint32_t*>(p->at(o_mb[2]));
  p->mail.adone = reinterpret_cast<uint64_t*>(p->at(o_adone));
  p->mail.cdone = reinterpret_cast<uint64_t*>(p->at(o_cdone));
  p->mail.ob = reinterpret_cast<uint32_t*>(p->at(o_mb[3]));
  p->mail.odone = reinterpret_cast<uint64_t*>(p->at(o_odone));
  p->mail.xn = reinterpret_cast<uint32_t*>(p->at(o_xn));
  p->mail.xdone = reinterpret_cast<uint64_t*>(p->at(o_xdone));
  p->mail.fdone = reinterpret_cast<uint64_t*>(p->at(o_fdone));
  *out = p;
  return ok();
}

extern "C" int mono_proj_destroy(mono_proj* p) {
  if (!p) return ok();
  if (!live(p, PROJ_MAGIC)) return fail(MONO_ESTATE, "mono_proj_destroy: not a live projection runtime");
  const int rc = p->release();
  delete p;
  return rc ? rc : ok();
}

static int check_proj(const mono_proj* p, const mono_proj_weights* w, int rows) {
  if (!live(p, PROJ_MAGIC)) return fail(MONO_ESTATE, "not a live projection runtime");
  if (!w) return fail(MONO_EINVAL, "weights is NULL");
  if (rows < 1 || rows > p->cfg.max_rows)
    return fail(MONO_EINVAL, "rows must be in [1, %d] (the runtime's max_rows), got %d", p->cfg.max_rows, rows);
  return check_device(p->device);
}

static int check_front(const mono_proj* p, const mono_proj_weights* w, const mono_front_args* args) {
  if (!args) return fail(MONO_EINVAL, "mono_front_forward: args is NULL");
  if (int rc = check_proj(p, w, args->rows)) return rc;
  REQUIRE_PTR(w->g_in);
  REQUIRE_PTR(w->w_qkv);
  REQUIRE_PTR(w->s_qkv);
  REQUIRE_PTR(w->w_ik);
  REQUIRE_PTR(w->s_ik);
  REQUIRE_PTR(w->w_iw);
  REQUIRE_PTR(w->g_q);
  REQUIRE_PTR(w->g_kv);
  REQUIRE_PTR(w->g_ik);
  REQUIRE_PTR(w->b_ik);
  REQUIRE_PTR(w->w_qb);
  REQUIRE_PTR(w->s_qb);
  REQUIRE_PTR(w->w_iq);
  REQUIRE_PTR(w->s_iq);
  REQUIRE_PTR(w->w_uk);
  REQUIRE_PTR(w->s_uk);
  REQUIRE_PTR(args->h);
  REQUIRE_PTR(args->seq_lens);
  REQUIRE_PTR(args->page_table);
  REQUIRE_PTR(args->rope_cos);
  REQUIRE_PTR(args->rope_sin);
  REQUIRE_PTR(args->ikv);
  REQUIRE_PTR(args->iks);
  REQUIRE_PTR(args->kv);
  REQUIRE_PTR(args->q);
  REQUIRE_PTR(args->iq);
  REQUIRE_PTR(args->iqs);
  REQUIRE_PTR(args->iw);
  if (args->pt_stride < 1) return fail(MONO_EINVAL, "pt_stride must be positive, got %d", args->pt_stride);
  if (args->n_pages < 1) return fail(MONO_EINVAL, "n_pages must be positive, got %d", args->n_pages);
  if (args->max_pos < 1) return fail(MONO_EINVAL, "max_pos must be positive, got %d", args->max_pos);
  return MONO_OK;
}

extern "C" int mono_front_forward(mono_proj* p, const mono_proj_weights* w, const mono_front_args* args,
                                  void* stream) {
  if (int rc = check_front(p, w, args)) return rc;
  // a NULL kv_scale writes raw E4M3 rows (scale 1) and stores its 1.0 in the runtime's word
  mono_front_args fa = *args;
  int kv_mask = -1;
  if (!fa.kv_scale) {
    fa.kv_scale = p->unit;
    kv_mask = 0;
  }
  hipError_t e =
      mono::proj::front_forward(*w, fa, p->grid, p->mail, p->guard, kv_mask, 0, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the front projections: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_back_forward(mono_proj* p, const mono_proj_weights* w, const mono_back_args* args, void* stream) {
  if (!args) return fail(MONO_EINVAL, "mono_back_forward: args is NULL");
  if (int rc = check_proj(p, w, args->rows)) return rc;
  REQUIRE_PTR(w->w_uv);
  REQUIRE_PTR(w->s_uv);
  REQUIRE_PTR(w->w_o);
  REQUIRE_PTR(w->s_o);
  REQUIRE_PTR(args->o_lat);
  REQUIRE_PTR(args->h);
  REQUIRE_PTR(args->a);
  hipError_t e = mono::proj::back_forward(*w, *args, p->grid, p->mail, p->guard, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the output projections: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_proj_set_deadline(mono_proj* p, double seconds) {
  if (!live(p, PROJ_MAGIC)) return fail(MONO_ESTATE, "not a live projection runtime");
  return guard_set_deadline(ref(p), seconds);
}

extern "C" int mono_proj_set_fault(mono_proj* p, int32_t site) {
  if (!live(p, PROJ_MAGIC)) return fail(MONO_ESTATE, "not a live projection runtime");
  return guard_set_fault(ref(p), site, 0);
}

extern "C" int mono_proj_read_errors(mono_proj* p, int32_t* words) {
  if (!live(p, PROJ_MAGIC)) return fail(MONO_ESTATE, "not a live projection runtime");
  return guard_read(ref(p), words);
}

extern "C" int mono_proj_clear_errors(mono_proj* p) {
  if (!live(p, PROJ_MAGIC)) return fail(MONO_ESTATE, "not a live projection runtime");
  return guard_clear(ref(p));
}

// ------------------------------------------------------------------ decoder layer

// One decoder layer's runtimes: the projection, attention and FP8 MoE mailboxes,
// private to the layer (never handed out on their own), the o_proj tiles' done words of
// the fused launch, and the layer's guard. Every launch of the layer (the whole layer,
// or its front and the fused rest apart) runs under that one guard: the attention
// runtime's guard words and launch counters (one count of launches, so tags never collide between the
// launches, whichever the caller mixes) and host word, its row histograms as the flip
// words, and a scrub table of all four mailbox regions.
struct mono_layer {
  uint32_t magic = 0;
  mono_proj* p = nullptr;
  mono_attn* a = nullptr;
  mono_moe* m = nullptr;
  void* extra = nullptr;  // a_done, then the scrub table
  uint64_t* a_done = nullptr;
  mono::GuardArgs guard{};
  // multi-layer launches (max_layers > 1): each layer's own row histograms and MoE FP8
  // rows with their scales (stack_stride bytes a layer), then the final tasks' tagged tile sums
  // of squares (scrubbed with every other mailbox); the device table of the layers'
  // kernel arguments and the host copy of what it holds
  int max_layers = 0;
  void* stack_mail = nullptr;
  size_t stack_stride = 0;
  size_t stack_o_xq = 0, stack_o_xs = 0;
  uint64_t* x_ssq = nullptr;
  void* table = nullptr;
  std::vector<uint8_t> table_host;
  int stack_n = 0;  // layers of the table's last mono_layer_stack_set (0: none)
};
static const uint32_t LAYER_MAGIC = 0x6c617972u;
static bool layer_live(const mono_layer* L) { return L && L->magic == LAYER_MAGIC; }
static GuardRef layer_ref(mono_layer* L) { return GuardRef{&L->guard, L->a->device, L->a->grid, &L->a->herr}; }

static int layer_release(mono_layer* L) {
  int rc = MONO_OK;
  for (void** pp : {&L->stack_mail, &L->table}) {
    if (*pp) {
      hipError_t e = hipFree(*pp);
      if (e != hipSuccess) rc = fail(MONO_EHIP, "hipFree: %s", hipGetErrorString(e));
      *pp = nullptr;
    }
  }
  L->x_ssq = nullptr;
  if (L->extra) {
    hipError_t e = hipFree(L->extra);
    if (e != hipSuccess) rc = fail(MONO_EHIP, "hipFree: %s", hipGetErrorString(e));
    L->extra = nullptr;
    L->a_done = nullptr;
  }
  if (L->m) rc = mono_moe_destroy(L->m) ? MONO_EHIP : rc;
  if (L->a) rc = mono_attn_destroy(L->a) ? MONO_EHIP : rc;
  if (L->p) rc = mono_proj_destroy(L->p) ? MONO_EHIP : rc;
  L->m = nullptr;
  L->a = nullptr;
  L->p = nullptr;
  L->magic = 0;
  return rc;
}

constexpr int MAX_STACK_LAYERS = 256;

// A layer runtime's buffers for multi-layer launches: every layer's row histograms and
// MoE FP8 rows with their scales, the final tasks' tagged tile sums of squares (one
// zeroed allocation, the scrub region `rg`) and the device table of the layers' kernel
// arguments.
static int stack_alloc(mono_layer* L, int max_layers, mono::ScrubRegion& rg) {
  using namespace mono;
  const size_t R = (size_t)L->a->cfg.max_rows;
  Carve cv;  // a layer's share: rowh at 0, then the MoE's FP8 rows and scales
  cv.off = 0;
  cv.take(R * attn::ROWH * 4);
  L->stack_o_xq = cv.take((size_t)moe::MAX_ROWS * 7168);
  L->stack_o_xs = cv.take((size_t)moe::MAX_ROWS * (7168 / 128) * 4);
  L->stack_stride = align256(cv.off);
  const size_t ssq_bytes = (size_t)moe::MAX_ROWS * SSQ_TILES * sizeof(uint64_t);
  const size_t bytes = L->stack_stride * (size_t)max_layers + ssq_bytes;
  hipError_t e = hipMalloc(&L->stack_mail, bytes);
  if (e != hipSuccess) {
    L->stack_mail = nullptr;
    return fail(MONO_ENOMEM, "hipMalloc(%zu) for the multi-layer mailboxes: %s", bytes, hipGetErrorString(e));
  }
  e = hipMemset(L->stack_mail, 0, bytes);
  if (e != hipSuccess) return fail(MONO_EHIP, "clearing the multi-layer mailboxes: %s", hipGetErrorString(e));
  L->x_ssq = reinterpret_cast<uint64_t*>(static_cast<char*>(L->stack_mail) + L->stack_stride * (size_t)max_layers);
  const size_t tbytes = layer::stack_entry_bytes() * (size_t)max_layers;
  e = hipMalloc(&L->table, tbytes);
  if (e != hipSuccess) {
    L->table = nullptr;
    return fail(MONO_ENOMEM, "hipMalloc(%zu) for the layers' argument table: %s", tbytes, hipGetErrorString(e));
  }
  L->max_layers = max_layers;
  rg = ScrubRegion{static_cast<uint32_t*>(L->stack_mail), bytes / 16};
  return MONO_OK;
}

extern "C" int mono_layer_create(const mono_layer_config* cfg, mono_layer** out) {
  if (!cfg || !out) return fail(MONO_EINVAL, "mono_layer_create: cfg and out must be non-NULL");
  *out = nullptr;
  const mono_layer_config& c = *cfg;
  if (c.max_rows < 1 || c.max_rows > mono::moe::MAX_ROWS)
    return fail(MONO_EINVAL, "max_rows must be in [1, %d], got %d", mono::moe::MAX_ROWS, c.max_rows);
  if (c.max_layers < 0 || c.max_layers > MAX_STACK_LAYERS)
    return fail(MONO_EINVAL, "max_layers must be in [0, %d], got %d", MAX_STACK_LAYERS, c.max_layers);
  if (int rc = check_device(c.device)) return rc;
  int per_cu = 0;
  HIP_TRY(mono::layer::tail_occupancy(&per_cu));
  if (per_cu < 1) return fail(MONO_ESTATE, "the fused layer kernel does not fit on a CU");
  mono_layer* L = new mono_layer();
  const mono_proj_config pc{c.device, c.max_rows};
  const mono_attn_config ac{c.device, c.max_rows, c.max_ctx, c.softmax_scale};
  const mono_moe_config mc{c.device, c.max_rows, 7168, 256, 8, 512, MONO_WEIGHT_FP8_BLOCK128,
                           MONO_ROUTER_SIGMOID_BIAS, c.route_scale, c.eps};
  int rc = mono_proj_create(&pc, &L->p);
  if (!rc) rc = mono_attn_create(&ac, &L->a);
  if (!rc) rc = mono_moe_create(&mc, &L->m);
  const size_t table_off = mono::DONE_BYTES;
  if (!rc) {
    hipError_t e = hipMalloc(&L->extra, table_off + 256);
    if (e != hipSuccess) {
      L->extra = nullptr;
      rc = fail(MONO_ENOMEM, "hipMalloc(%zu) for the layer's done words: %s", (size_t)(table_off + 256),
                hipGetErrorString(e));
    } else {
      L->a_done = static_cast<uint64_t*>(L->extra);
      mono::ScrubRegion table[mono::SCRUB_MAX] = {L->a->mailboxes(), L->p->mailboxes(), L->m->mailboxes(),
                                                  mono::ScrubRegion{reinterpret_cast<uint32_t*>(L->a_done),
                                                                    mono::DONE_BYTES / 16}};
      if (c.max_layers > 1) rc = stack_alloc(L, c.max_layers, table[4]);
      char* tb = static_cast<char*>(L->extra) + table_off;
      if (!rc) e = hipMemset(L->extra, 0, table_off + 256);
      if (!rc && e == hipSuccess) e = hipMemcpy(tb, table, sizeof(table), hipMemcpyHostToDevice);
      if (!rc && e == hipSuccess) e = hipDeviceSynchronize();
      if (!rc && e != hipSuccess) rc = fail(MONO_EHIP, "clearing the layer's done words: %s", hipGetErrorString(e));
      L->guard = L->a->guard;
      L->guard.scrub = reinterpret_cast<const mono::ScrubRegion*>(tb);
    }
  }
  if (rc) {
    const std::string why = g_error;
    (void)layer_release(L);
    delete L;
    return fail(rc, "%s", why.c_str());
  }
  L->magic = LAYER_MAGIC;
  *out = L;
  return ok();
}

extern "C" int mono_layer_destroy(mono_layer* L) {
  if (!L) return ok();
  if (!layer_live(L)) return fail(MONO_ESTATE, "mono_layer_destroy: not a live layer runtime");
  const int rc = layer_release(L);
  delete L;
  return rc ? rc : ok();
}

// The checks every layer launch makes of one layer's arguments (the front's too with `front`).
static int check_layer(mono_layer* L, const mono_proj_weights* w, const mono_layer_args* args, bool front) {
  if (!args || !w || !args->front || !args->attn || !args->back || !args->moe)
    return fail(MONO_EINVAL, "mono_layer_forward: w, args and its four parts must be non-NULL");
  const mono_front_args& f = *args->front;
  const mono_attn_args& at = *args->attn;
  const int rows = f.rows;
  if (at.rows != rows || args->back->rows != rows || args->moe->rows != rows)
    return fail(MONO_EINVAL, "front, attn, back and moe must have the same rows (%d, %d, %d, %d)", rows, at.rows,
                args->back->rows, args->moe->rows);
  if (at.q != f.q || at.iq != f.iq || at.iqs != f.iqs || at.iw != f.iw)
    return fail(MONO_EINVAL, "attn's q, iq, iqs and iw must be the front's outputs");
  if (at.ikv != f.ikv || at.iks != f.iks || at.kv != f.kv || at.kv_scale != f.kv_scale ||
      at.page_table != f.page_table || at.seq_lens != f.seq_lens)
    return fail(MONO_EINVAL, "attn must read the caches and step the front writes");
  if (args->moe->a != args->back->a) return fail(MONO_EINVAL, "moe->a must be back->a: the MoE reads the back's output");
  if (int rc = check_attn_back(L->a, args->attn, w, args->back)) return rc;
  if (int rc = check_moe_fp8(L->m, args->moe)) return rc;
  if (front)
    if (int rc = check_front(L->p, w, args->front)) return rc;
  return MONO_OK;
}

static int layer_launch(mono_layer* L, const mono_proj_weights* w, const mono_layer_args* args, void* stream,
                        bool front, bool tail) {
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  if (int rc = check_layer(L, w, args, front)) return rc;
  const mono_attn_args& at = *args->attn;
  mono_back_args b = *args->back;
  b.o_lat = at.out;
  const mono::attn::AttnArgs g = attn_args(L->a, at);
  const mono::moe::MoeFp8Args m(*args->moe, L->m->cfg.route_scale, L->m->cfg.eps);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (front) {
    mono_front_args fa = *args->front;
    int kv_mask = -1;
    if (!fa.kv_scale) {  // raw E4M3 rows: the 1.0 the attention reads too
      fa.kv_scale = L->a->unit;
      kv_mask = 0;
    }
    if (tail)  // the whole layer as one launch
      e = mono::layer::layer_forward(*w, fa, L->p->mail, kv_mask, g, L->a->mail, L->guard, b, L->a->back_mail, m,
                                     L->m->mail, L->a_done, args->ticks, L->a->grid, st);
    else  // the front alone, under the layer's guard (its sites numbered as in the one launch)
      e = mono::proj::front_forward(*w, fa, L->a->grid, L->p->mail, L->guard, kv_mask, mono::layer::FRONT_SITE0, st);
  } else {
    e = mono::layer::tail_forward(g, L->a->mail, L->guard, *w, b, L->a->back_mail, m, L->m->mail, L->a_done,
                                  args->ticks, L->a->grid, st);
  }
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the layer: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_layer_forward(mono_layer* L, const mono_proj_weights* w, const mono_layer_args* args,
                                  void* stream) {
  return layer_launch(L, w, args, stream, true, true);
}

extern "C" int mono_layer_front_forward(mono_layer* L, const mono_proj_weights* w, const mono_layer_args* args,
                                        void* stream) {
  return layer_launch(L, w, args, stream, true, false);
}

extern "C" int mono_layer_tail_forward(mono_layer* L, const mono_proj_weights* w, const mono_layer_args* args,
                                       void* stream) {
  return layer_launch(L, w, args, stream, false, true);
}

namespace {

// A device range a multi-layer launch writes or rereads: [p, p + bytes), the layer and
// what it holds (for the error message).
struct Span {
  uintptr_t p;
  size_t bytes;
  int layer;
  const char* what;
};

}  // namespace

extern "C" int mono_layer_stack_set(mono_layer* L, int32_t n, const mono_proj_weights* const* w,
                                    const mono_layer_args* const* args) {
  using namespace mono;
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  if (L->max_layers < 2) return fail(MONO_ESTATE, "the layer runtime was created without max_layers (> 1)");
  if (n < 1 || n > L->max_layers)
    return fail(MONO_EINVAL, "n_layers must be in [1, %d] (the runtime's max_layers), got %d", L->max_layers, n);
  if (!w || !args) return fail(MONO_EINVAL, "mono_layer_stack_set: w and args must be non-NULL");
  std::vector<Span> spans;
  for (int l = 0; l < n; ++l) {
    if (int rc = check_layer(L, w[l], args[l], true)) {
      const std::string why = g_error;
      return fail(rc, "layer %d: %s", l, why.c_str());
    }
    const mono_front_args& f = *args[l]->front;
    const size_t r = (size_t)f.rows, pages = (size_t)f.n_pages;
    if (l > 0 && f.h != args[l - 1]->moe->out)
      return fail(MONO_EINVAL, "layer %d: front->h must be layer %d's moe->out", l, l - 1);
    if (l == 0) spans.push_back({(uintptr_t)f.h, r * 7168 * 2, l, "front->h"});
    spans.push_back({(uintptr_t)f.q, r * 32 * 576 * 2, l, "q"});
    spans.push_back({(uintptr_t)f.iq, r * 64 * 32, l, "iq"});
    spans.push_back({(uintptr_t)f.iqs, r * 64 * 4, l, "iqs"});
    spans.push_back({(uintptr_t)f.iw, r * 64 * 2, l, "iw"});
    spans.push_back({(uintptr_t)f.kv, pages * 64 * 576, l, "kv"});
    spans.push_back({(uintptr_t)f.ikv, pages * 4 * 64 * 16, l, "ikv"});
    spans.push_back({(uintptr_t)f.iks, pages * 4 * 64, l, "iks"});
    if (f.kv_scale) spans.push_back({(uintptr_t)f.kv_scale, pages * 64 * 4, l, "kv_scale"});
    spans.push_back({(uintptr_t)args[l]->back->a, r * 7168 * 2, l, "back->a"});
    spans.push_back({(uintptr_t)args[l]->moe->out, r * 7168 * 2, l, "moe->out"});
  }
  std::sort(spans.begin(), spans.end(), [](const Span& x, const Span& y) { return x.p < y.p; });
  for (size_t i = 1; i < spans.size(); ++i) {
    const Span& x = spans[i - 1];
    const Span& y = spans[i];
    if (x.p + x.bytes > y.p)
      return fail(MONO_EINVAL,
                  "layer %d's %s overlaps layer %d's %s: a multi-layer launch needs each layer's outputs and "
                  "caches in buffers of their own",
                  x.layer, x.what, y.layer, y.what);
  }
  const size_t eb = layer::stack_entry_bytes();
  std::vector<uint8_t> table(eb * (size_t)n, 0);
  for (int l = 0; l < n; ++l) {
    const mono_layer_args& la = *args[l];
    const mono_attn_args& at = *la.attn;
    mono_back_args b = *la.back;
    b.o_lat = at.out;
    const attn::AttnArgs g = attn_args(L->a, at);
    const moe::MoeFp8Args m(*la.moe, L->m->cfg.route_scale, L->m->cfg.eps);
    mono_front_args fa = *la.front;
    int kv_mask = -1;
    if (!fa.kv_scale) {
      fa.kv_scale = L->a->unit;
      kv_mask = 0;
    }
    char* mail = static_cast<char*>(L->stack_mail) + L->stack_stride * (size_t)l;
    const layer::StackLayer sl{reinterpret_cast<uint32_t*>(mail), reinterpret_cast<uint8_t*>(mail + L->stack_o_xq),
                               reinterpret_cast<float*>(mail + L->stack_o_xs), l + 1 < n ? L->x_ssq : nullptr,
                               l > 0 ? L->x_ssq : nullptr};
    hipError_t e = layer::stack_fill(table.data() + eb * (size_t)l, sl, *w[l], fa, L->p->mail, kv_mask, g,
                                     L->a->mail, L->guard, b, L->a->back_mail, m, L->m->mail, L->a_done, la.ticks);
    if (e != hipSuccess) return fail(MONO_EINVAL, "layer %d: %s", l, hipGetErrorString(e));
  }
  if (int rc = check_device(L->a->device)) return rc;
  // launches in flight may still read the table
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(L->table, table.data(), table.size(), hipMemcpyHostToDevice));
  L->table_host.swap(table);
  L->stack_n = n;
  return ok();
}

extern "C" int mono_layer_stack_forward(mono_layer* L, void* stream) {
  using namespace mono;
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  if (L->stack_n < 1) return fail(MONO_ESTATE, "mono_layer_stack_forward: no layers set (mono_layer_stack_set)");
  if (int rc = check_device(L->a->device)) return rc;
  const hipError_t e = layer::stack_forward(L->table, L->stack_n, (uint32_t)(L->a->cfg.max_rows * attn::ROWH),
                                            L->guard, L->a->grid, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the layers: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_layer_set_deadline(mono_layer* L, double seconds) {
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  return guard_set_deadline(layer_ref(L), seconds);
}

extern "C" int mono_layer_set_fault(mono_layer* L, int32_t site, int64_t after) {
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  return guard_set_fault(layer_ref(L), site, after);
}

extern "C" int mono_layer_read_errors(mono_layer* L, int32_t* words) {
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  return guard_read(layer_ref(L), words);
}

extern "C" int32_t mono_layer_pending_error(mono_layer* L) {
  if (!layer_live(L)) return -1;
  return (int32_t)L->a->herr.read();
}

extern "C" int mono_layer_clear_errors(mono_layer* L) {
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  // the scrub table covers every mailbox, the row histograms' two copies included
  return guard_clear(layer_ref(L));
}

extern "C" int mono_layer_set_launch_ordinal(mono_layer* L, uint64_t ordinal) {
  if (!layer_live(L)) return fail(MONO_ESTATE, "not a live layer runtime");
  return guard_set_ordinal(layer_ref(L), ordinal);
}
