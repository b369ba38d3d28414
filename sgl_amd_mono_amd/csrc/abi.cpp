// The C-ABI of libmono_gfx950.so: runtime handles, argument checks, error strings.
//
// A handle owns its device scratch (one hipMalloc at create, freed at destroy), the
// way the reference's Glm53Runtime owns its scratch mailboxes and guard words
// (glm53/gfx950/runner.py:133-215). Forward calls validate their arguments on the
// host, then enqueue the phase's kernels on the caller's stream and return.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <string>

#include "mono.h"
#include "moe_ops.h"

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

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

int check_device(int device) {
  int cur = -1;
  HIP_TRY(hipGetDevice(&cur));
  if (cur != device) return fail(MONO_ESTATE, "the current HIP device is %d, the runtime lives on %d", cur, device);
  return MONO_OK;
}

}  // namespace

struct mono_moe {
  mono_moe_config cfg;
  int grid;  // workgroups of the persistent launch: one a CU
  void* blob;
  size_t blob_bytes;
  mono::moe::Mail mail;
  mono::GuardArgs guard;
  uint32_t magic;
};

static const uint32_t MOE_MAGIC = 0x6d6f6531u;
static const double TICKS_PER_S = 100e6;  // s_memrealtime runs at 100 MHz
static const double DEFAULT_DEADLINE_S = 2.0;
static const double MAX_DEADLINE_S = 3600.0;

extern "C" int mono_abi_version(void) { return MONO_ABI_VERSION; }

extern "C" const char* mono_last_error(void) { return g_error.c_str(); }

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
  if (c.weight_format == MONO_WEIGHT_FP8_BLOCK128 && !moe_fp8_supported(geo))
    return fail(MONO_EINVAL,
                "FP8 MoE geometry H=%d E=%d top_k=%d I=%d has no compiled kernel (built: H=7168 E=256 top_k=8 I=512)",
                c.hidden, c.n_experts, c.top_k, c.inter);
  if (int rc = check_device(c.device)) return rc;
  const size_t H = c.hidden, E = c.n_experts, I = c.inter;
  const size_t max_act = (size_t)std::min(c.max_rows * c.top_k, c.n_experts) + 1;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off += align256(bytes);
    return at;
  };
  const size_t o_guard = take(mono::G_WORDS * 4);
  const size_t o_rlog = take((size_t)moe_fp8_router_slices() * MAX_ROWS * E * 8);
  const size_t o_rsel = take((size_t)MAX_ROWS * 2 * MAX_TOPK * 8);
  const size_t o_mid = take(max_act * MAX_ROWS * I * 8);
  const size_t o_ypart = take(max_act * MAX_ROWS * H * 8);

  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, c.device));
  int per_cu = 0;
  HIP_TRY(moe_fp8_occupancy(&per_cu));
  if (per_cu < 1)
    return fail(MONO_ESTATE, "the persistent MoE kernel does not fit on a CU (occupancy %d)", per_cu);
  mono_moe* m = new mono_moe();
  m->cfg = c;
  m->magic = MOE_MAGIC;
  m->blob_bytes = off;
  m->grid = prop.multiProcessorCount;
  hipError_t e = hipMalloc(&m->blob, off);
  if (e != hipSuccess) {
    delete m;
    return fail(MONO_ENOMEM, "hipMalloc(%zu) for the MoE mailboxes: %s", off, hipGetErrorString(e));
  }
  // tag 0 is never a launch's tag, so zeroed mailboxes read as empty
  e = hipMemset(m->blob, 0, off);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(m->blob);
    delete m;
    return fail(MONO_EHIP, "clearing the MoE mailboxes: %s", hipGetErrorString(e));
  }
  char* b = static_cast<char*>(m->blob);
  m->mail.guard = reinterpret_cast<uint32_t*>(b + o_guard);
  m->mail.rlog = reinterpret_cast<uint64_t*>(b + o_rlog);
  m->mail.rsel = reinterpret_cast<uint64_t*>(b + o_rsel);
  m->mail.mid = reinterpret_cast<uint64_t*>(b + o_mid);
  m->mail.ypart = reinterpret_cast<uint64_t*>(b + o_ypart);
  m->guard.words = m->mail.guard;
  m->guard.deadline_ticks = (uint64_t)(DEFAULT_DEADLINE_S * TICKS_PER_S);
  m->guard.fault_site = -1;
  *out = m;
  return ok();
}

extern "C" int mono_moe_destroy(mono_moe* m) {
  if (!m) return ok();
  if (m->magic != MOE_MAGIC) return fail(MONO_ESTATE, "mono_moe_destroy: not a live MoE runtime");
  m->magic = 0;
  if (m->blob) {
    hipError_t e = hipFree(m->blob);
    m->blob = nullptr;
    if (e != hipSuccess) {
      delete m;
      return fail(MONO_EHIP, "hipFree: %s", hipGetErrorString(e));
    }
  }
  delete m;
  return ok();
}

static int check_moe(const mono_moe* m, int rows) {
  if (!m || m->magic != MOE_MAGIC) return fail(MONO_ESTATE, "not a live MoE runtime");
  if (rows < 1 || rows > m->cfg.max_rows)
    return fail(MONO_EINVAL, "rows must be in [1, %d] (the runtime's max_rows), got %d", m->cfg.max_rows, rows);
  return check_device(m->cfg.device);
}

#define REQUIRE_PTR(p) \
  if (!(p)) return fail(MONO_EINVAL, "argument %s must be a device pointer, got NULL", #p)

extern "C" int mono_moe_fp8_forward(mono_moe* m, const mono_moe_fp8_args* args, void* stream) {
  using namespace mono::moe;
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
  MoeFp8Args g(*args, m->cfg.route_scale, m->cfg.eps);
  hipError_t e = moe_fp8_forward(g, m->grid, m->mail, m->guard, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the FP8 MoE: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_moe_set_deadline(mono_moe* m, double seconds) {
  if (!m || m->magic != MOE_MAGIC) return fail(MONO_ESTATE, "not a live MoE runtime");
  if (!(seconds > 0.0) || seconds > MAX_DEADLINE_S)
    return fail(MONO_EINVAL, "deadline must be in (0, %.0f] seconds, got %g", MAX_DEADLINE_S, seconds);
  const double ticks = seconds * TICKS_PER_S;
  m->guard.deadline_ticks = ticks < 1.0 ? 1u : (uint64_t)ticks;
  return ok();
}

extern "C" int mono_moe_set_fault(mono_moe* m, int32_t site) {
  if (!m || m->magic != MOE_MAGIC) return fail(MONO_ESTATE, "not a live MoE runtime");
  if (site < -1 || site > 15) return fail(MONO_EINVAL, "fault site must be -1 (none) or a wait site 0..15, got %d", site);
  m->guard.fault_site = site;
  return ok();
}

extern "C" int mono_moe_read_errors(mono_moe* m, int32_t* words) {
  if (!m || m->magic != MOE_MAGIC) return fail(MONO_ESTATE, "not a live MoE runtime");
  if (!words) return fail(MONO_EINVAL, "mono_moe_read_errors: words is NULL");
  if (int rc = check_device(m->cfg.device)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(words, m->mail.guard, MONO_GUARD_WORDS * sizeof(int32_t), hipMemcpyDeviceToHost));
  return ok();
}

extern "C" int mono_moe_clear_errors(mono_moe* m) {
  if (!m || m->magic != MOE_MAGIC) return fail(MONO_ESTATE, "not a live MoE runtime");
  if (int rc = check_device(m->cfg.device)) return rc;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemset(m->mail.guard + mono::G_ERROR, 0, (MONO_GUARD_WORDS - 1) * sizeof(int32_t)));
  HIP_TRY(hipDeviceSynchronize());
  return ok();
}

extern "C" int mono_moe_mxfp4_forward(mono_moe* m, const mono_moe_mxfp4_args* args, void* stream) {
  (void)m;
  (void)args;
  (void)stream;
  return fail(MONO_EINVAL, "mono_moe_mxfp4_forward: not built yet");
}
