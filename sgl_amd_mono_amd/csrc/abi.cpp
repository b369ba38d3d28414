// The C-ABI of libmono_gfx950.so: runtime handles, argument checks, error strings.
//
// A handle owns its device scratch (one hipMalloc at create, freed at destroy), the
// way the reference's Glm53Runtime owns its scratch mailboxes and guard words
// (glm53/gfx950/runner.py:133-215). Forward calls validate their arguments on the
// host, then enqueue the phase's kernels on the caller's stream and return.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
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
  int n_cu;
  void* blob;
  size_t blob_bytes;
  mono::moe::Scratch sc;
  uint32_t magic;
};

static const uint32_t MOE_MAGIC = 0x6d6f6531u;

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
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t at = off;
    off += align256(bytes);
    return at;
  };
  const size_t o_plan = take(sizeof(Plan));
  const size_t o_rstd = take(MAX_ROWS * 4);
  const size_t o_xq = take(MAX_ROWS * H);
  const size_t o_xs = take(MAX_ROWS * (H / 128) * 4);
  const size_t o_rpart = take((size_t)ROUTER_SLICES * MAX_ROWS * E * 4);
  const size_t o_rcount = take(4);
  const size_t o_mid = take((size_t)MAX_ACT * MAX_ROWS * I * 4);
  const size_t o_mcount = take((size_t)MAX_ACT * (I / 128) * 4);
  const size_t o_mq = take((size_t)MAX_ACT * MAX_ROWS * I * 2);
  const size_t o_mcoef = take((size_t)MAX_ACT * MAX_ROWS * (I / 128) * 4);

  mono_moe* m = new mono_moe();
  m->cfg = c;
  m->magic = MOE_MAGIC;
  m->blob_bytes = off;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, c.device);
  if (e != hipSuccess) {
    delete m;
    return fail(MONO_EHIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  }
  m->n_cu = prop.multiProcessorCount;
  e = hipMalloc(&m->blob, off);
  if (e != hipSuccess) {
    delete m;
    return fail(MONO_ENOMEM, "hipMalloc(%zu) for the MoE scratch: %s", off, hipGetErrorString(e));
  }
  // counters start at zero; every later launch leaves them at zero
  e = hipMemset(m->blob, 0, off);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    (void)hipFree(m->blob);
    delete m;
    return fail(MONO_EHIP, "clearing the MoE scratch: %s", hipGetErrorString(e));
  }
  char* b = static_cast<char*>(m->blob);
  m->sc.plan = reinterpret_cast<Plan*>(b + o_plan);
  m->sc.rstd = reinterpret_cast<float*>(b + o_rstd);
  m->sc.xq = reinterpret_cast<uint8_t*>(b + o_xq);
  m->sc.xs = reinterpret_cast<float*>(b + o_xs);
  m->sc.rpart = reinterpret_cast<float*>(b + o_rpart);
  m->sc.rcount = reinterpret_cast<uint32_t*>(b + o_rcount);
  m->sc.mid = reinterpret_cast<float*>(b + o_mid);
  m->sc.mcount = reinterpret_cast<uint32_t*>(b + o_mcount);
  m->sc.mq = reinterpret_cast<uint8_t*>(b + o_mq);
  m->sc.mcoef = reinterpret_cast<float*>(b + o_mcoef);
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
  const MoeGeom geo{m->cfg.hidden, m->cfg.n_experts, m->cfg.top_k, m->cfg.inter};
  MoeFp8Args g(*args, m->cfg.route_scale, m->cfg.eps);
  hipError_t e = moe_fp8_forward(g, geo, m->n_cu, m->sc, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(MONO_EHIP, "launching the FP8 MoE: %s", hipGetErrorString(e));
  return ok();
}

extern "C" int mono_moe_mxfp4_forward(mono_moe* m, const mono_moe_mxfp4_args* args, void* stream) {
  (void)m;
  (void)args;
  (void)stream;
  return fail(MONO_EINVAL, "mono_moe_mxfp4_forward: not built yet");
}
