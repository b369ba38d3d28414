// mono_attn_forward_noalloc: the sparse-attention launch of mono_attn_forward for a
// caller that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The launch's mailboxes and guard words live in one
// file-scope device array, `scratch`, sized for at most NA_ROWS rows of at most
// MAX_CTX keys; each GPU the library runs on holds its own copy until the process
// ends. The first call on a device takes the array's address with
// hipGetSymbolAddress (the array's host-side name is not a device address) and clears
// it with a fill kernel on the caller's stream; later calls allocate nothing and
// synchronise nothing.
//
// Every call on a GPU shares that GPU's array: calls must be stream-ordered (one
// stream at a time), and calls that overlap on one GPU race. The guard is not sticky,
// since no host call exists to clear it: a launch whose wait fails writes NaN over its
// output, and the next call runs normally (its tags are fresh, and the launch-parity
// histograms it adds into were cleared when the failed launch began).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "abi_errors.h"
#include "attn_ops.h"
#include "mono.h"
#include "sync.h"

namespace mono {
namespace attn {

namespace {

constexpr int NA_ROWS = 8;    // rows a call at most
constexpr int NA_CTX = MAX_CTX;
constexpr int MAX_DEVICES = 64;
constexpr size_t al256(size_t n) { return (n + 255) & ~size_t(255); }

// the carve of the array: a 256-byte header (guard words, scrub table, the f32 1.0 of
// raw E4M3 rows), the per-workgroup launch counters, then the mailboxes of a runtime
// with max_rows NA_ROWS, max_ctx NA_CTX
constexpr size_t O_SCRUB = 64, O_UNIT = 192, O_TICKETS = 256;
constexpr int MAX_GRID = 1024;
constexpr size_t O_SCORE = O_TICKETS + MAX_GRID * sizeof(uint64_t);
constexpr size_t O_SEL = O_SCORE + al256((size_t)NA_ROWS * NA_CTX * 4);
constexpr size_t O_ROWH = O_SEL + al256((size_t)NA_ROWS * TOPK * 8);
constexpr size_t O_CDONE = O_ROWH + al256((size_t)2 * NA_ROWS * ROWH * 4);
constexpr size_t O_HIST = O_CDONE + al256((size_t)NA_ROWS * (NA_CTX / CHUNK) * 8);
constexpr size_t O_CAND = O_HIST + al256((size_t)NA_ROWS * PASSES * TEAM * HW * 8);
constexpr size_t O_CNT = O_CAND + al256((size_t)NA_ROWS * CMAX * 8);
constexpr size_t O_PART = O_CNT + al256((size_t)NA_ROWS * TEAM * 2 * 8);
constexpr size_t O_ML = O_PART + al256((size_t)NA_ROWS * SPLITS * NH * DV * 2);
constexpr size_t O_SDONE = O_ML + al256((size_t)NA_ROWS * SPLITS * NH * 2 * 4);
constexpr size_t O_MDONE = O_SDONE + al256((size_t)NA_ROWS * SPLITS * 8);
constexpr size_t SCRATCH_BYTES = O_MDONE + al256((size_t)NA_ROWS * NH * 8);
static_assert(SCRATCH_BYTES <= 10u * 1024 * 1024, "the static scratch stays within 10 MiB");

}  // namespace

// The device-side scratch of every no-alloc call on a GPU (one copy per GPU).
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

namespace {

// Zero the mailboxes (every workgroup a grid-strided share), then, in workgroup 0 alone,
// the header: zeroed guard words, the scrub table (every mailbox) and the unit scale.
__global__ __launch_bounds__(256) void k_scratch_init(uint8_t* base) {
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4* p = reinterpret_cast<u32x4*>(base);
  for (size_t i = O_SCORE / 16 + blockIdx.x * blockDim.x + threadIdx.x; i < SCRATCH_BYTES / 16;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = zero;
  if (blockIdx.x == 0) {
    for (size_t i = threadIdx.x; i < O_SCORE / 16; i += blockDim.x) p[i] = zero;
    __syncthreads();
    if (threadIdx.x == 0) {
      ScrubRegion* t = reinterpret_cast<ScrubRegion*>(base + O_SCRUB);
      t[0] = ScrubRegion{reinterpret_cast<uint32_t*>(base + O_SCORE), (SCRATCH_BYTES - O_SCORE) / 16};
      *reinterpret_cast<float*>(base + O_UNIT) = 1.0f;
    }
  }
}

// A device's address of `scratch` and its persistent grid, set up once per device.
struct DeviceScratch {
  bool ready = false;
  uint8_t* ptr = nullptr;  // hipGetSymbolAddress of scratch on this device
  int grid = 0;
};
std::mutex g_mu;
DeviceScratch g_dev[MAX_DEVICES];

int failf(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int failf(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return abi_fail(code, buf);
}

// The current device's scratch (set up on its first call: address, grid, cleared
// array; the clear is a fill kernel on `st`, stream-ordered before the first launch).
int device_scratch(hipStream_t st, DeviceScratch* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return failf(MONO_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= MAX_DEVICES) return failf(MONO_ESTATE, "device %d is beyond the %d this library serves", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceScratch& d = g_dev[dev];
  if (!d.ready) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return failf(MONO_EHIP, "hipStreamIsCapturing: %s", hipGetErrorString(e));
    if (cs != hipStreamCaptureStatusNone)
      return failf(MONO_ESTATE, "the first mono_attn_forward_noalloc call on device %d must run outside stream "
                                "capture: it clears the device's scratch", dev);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return failf(MONO_EHIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    int cus = 0, per_cu = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess) e = attn_occupancy(&per_cu);
    if (e != hipSuccess) return failf(MONO_EHIP, "querying device %d: %s", dev, hipGetErrorString(e));
    if (per_cu < 1) return failf(MONO_ESTATE, "the persistent attention kernel does not fit on a CU");
    if (cus % TEAM) return failf(MONO_ESTATE, "the attention launch needs a CU count divisible by %d, got %d", TEAM, cus);
    if (cus > MAX_GRID) return failf(MONO_ESTATE, "%d CUs: the launch counters hold at most %d workgroups", cus, MAX_GRID);
    k_scratch_init<<<cus, 256, 0, st>>>(static_cast<uint8_t*>(p));
    e = hipGetLastError();
    if (e != hipSuccess) return failf(MONO_EHIP, "clearing the static scratch: %s", hipGetErrorString(e));
    d.ptr = static_cast<uint8_t*>(p);
    d.grid = cus;
    d.ready = true;
  }
  *out = d;
  return MONO_OK;
}

}  // namespace
}  // namespace attn
}  // namespace mono

extern "C" int mono_attn_forward_noalloc(const mono_attn_args* args, float softmax_scale, void* stream) {
  using namespace mono::attn;
  using mono::attn::failf;
  if (!args) return failf(MONO_EINVAL, "mono_attn_forward_noalloc: args is NULL");
  if (args->rows < 1 || args->rows > NA_ROWS)
    return failf(MONO_EINVAL, "rows must be in [1, %d] (the static scratch holds %d rows of %d keys), got %d", NA_ROWS,
                 NA_ROWS, NA_CTX, args->rows);
  if (!(softmax_scale > 0.f)) return failf(MONO_EINVAL, "softmax_scale must be positive, got %g", softmax_scale);
  if (args->pt_stride < NA_CTX / PAGE)
    return failf(MONO_EINVAL, "pt_stride must cover %d / 64 = %d pages, got %d", NA_CTX, NA_CTX / PAGE, args->pt_stride);
  if (args->n_pages < 1) return failf(MONO_EINVAL, "n_pages must be positive, got %d", args->n_pages);
  const void* need[] = {args->iq, args->iqs, args->iw, args->ikv, args->iks, args->q,
                        args->kv, args->page_table, args->seq_lens, args->out};
  const char* names[] = {"iq", "iqs", "iw", "ikv", "iks", "q", "kv", "page_table", "seq_lens", "out"};
  for (int i = 0; i < 10; ++i)
    if (!need[i]) return failf(MONO_EINVAL, "argument args->%s must be a device pointer, got NULL", names[i]);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  DeviceScratch d;
  if (int rc = device_scratch(st, &d)) return rc;
  uint8_t* base = d.ptr;  // the device address; never the array's host-side name
  Mail mail{};
  mail.guard = reinterpret_cast<uint32_t*>(base);
  mail.score = reinterpret_cast<uint32_t*>(base + O_SCORE);
  mail.sel = reinterpret_cast<uint64_t*>(base + O_SEL);
  mail.rowh = reinterpret_cast<uint32_t*>(base + O_ROWH);
  mail.cdone = reinterpret_cast<uint64_t*>(base + O_CDONE);
  mail.hist = reinterpret_cast<uint64_t*>(base + O_HIST);
  mail.cand = reinterpret_cast<uint64_t*>(base + O_CAND);
  mail.cnt = reinterpret_cast<uint64_t*>(base + O_CNT);
  mail.part = reinterpret_cast<uint16_t*>(base + O_PART);
  mail.ml = reinterpret_cast<float*>(base + O_ML);
  mail.sdone = reinterpret_cast<uint64_t*>(base + O_SDONE);
  mail.mdone = reinterpret_cast<uint64_t*>(base + O_MDONE);
  mail.max_ctx = NA_CTX;
  mail.max_rows = NA_ROWS;
  mono::GuardArgs guard{};
  guard.words = mail.guard;
  guard.tickets = reinterpret_cast<uint64_t*>(base + O_TICKETS);
  guard.scrub = reinterpret_cast<const mono::ScrubRegion*>(base + O_SCRUB);
  guard.flip = mail.rowh;
  guard.flip_words = NA_ROWS * ROWH;
  guard.host_err = nullptr;
  guard.deadline_ticks = 200000000ull;  // 2 s at the 100 MHz s_memrealtime clock
  guard.fault_from = 0;
  guard.fault_site = -1;
  guard.sticky = 0;
  AttnArgs g(*args, softmax_scale);
  if (!args->kv_scale) {  // raw E4M3 rows read at scale 1
    g.kv_scale = reinterpret_cast<const float*>(base + O_UNIT);
    g.kv_mask = 0;
  }
  const hipError_t e = attn_forward(g, d.grid, mail, guard, st);
  if (e != hipSuccess) return failf(MONO_EHIP, "launching the sparse attention: %s", hipGetErrorString(e));
  return mono::abi_ok();
}
