// Allocation-free Q4_K matvec entry point (no counterpart in the reference).
//
// For callers that cannot allocate device memory during a call: code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
// It runs the split-K matvec kernel (axh_q4k_matvec_sk_s16 in q4_matvec.hip:
// one-wave workgroups of 16 superblocks, the last one to finish adds the
// partial sums in workgroup order) with its workspace in `scratch`, a fixed
// per-device array of this file, instead of the per-stream workspace that
// axh_q4k_matvec allocates on first use.
//
// Set-up (axh_context_create, once per device, with that device current)
// resolves the array's device address with hipGetSymbolAddress, clears it and
// prepares the kernel; afterwards a call allocates nothing.  The host-side
// name `scratch` is only a stand-in: every kernel argument and clear uses the
// resolved address.  Workspace layout (as the kernel reads it): word 0 is the
// workgroup counter, which every call leaves at zero; partial sums start at
// float kSkPartials, 32 rows per workgroup.  Every call on a device shares its
// array, so calls that overlap on one GPU race: issue them on one stream, or
// order them.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "axh_internal.h"

namespace {

constexpr uint32_t kMaxRows = 32;      // the kernel's partial-sum rows per workgroup
constexpr uint32_t kSpw = 16;          // superblocks per workgroup
constexpr uint32_t kMaxSb = 256;       // at most 16 workgroups
constexpr uint32_t kPartials = 64;     // floats before the partial sums
constexpr size_t kScratchBytes = (kPartials + (kMaxSb / kSpw) * kMaxRows) * sizeof(float);

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

struct DeviceScratch {
  std::once_flag once;
  void *ptr = nullptr;
  hipError_t err = hipSuccess;
};
DeviceScratch g_scratch[kMaxDevices];

// Resolves (once per device) the address of this device's copy of `scratch`
// and zeroes it; must run with `device` current.
axh_status resolve_scratch(int device, void **out) {
  if (device < 0 || device >= kMaxDevices)
    return axh::fail(AXH_ERR_NO_SUPPORTED_DEVICE, "device index beyond the scratch table");
  DeviceScratch &d = g_scratch[device];
  std::call_once(d.once, [&d] {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) e = hipMemset(p, 0, kScratchBytes); // set-up time, not in a capture
    if (e == hipSuccess) e = hipDeviceSynchronize();
    d.err = e;
    d.ptr = e == hipSuccess ? p : nullptr;
  });
  if (d.err != hipSuccess || !d.ptr)
    return axh::fail(AXH_ERR_BUFFER_ALLOCATION,
                     std::string("no-alloc scratch set-up failed: ") + hipGetErrorString(d.err));
  *out = d.ptr;
  return AXH_OK;
}

constexpr const char *kKernel = "axh_q4k_matvec_sk_s16";

struct RowsArgs {
  uint32_t n_rows, units_per_row, tile_units, pad;
};

} // namespace

namespace axh {

// Called by axh_context_create with the context's device current.  A failure
// is remembered and reported by the entry point; the context stays usable.
void noalloc_setup(axh_context *ctx) {
  void *p = nullptr;
  if (resolve_scratch(ctx->core->device, &p) != AXH_OK) return;
  axh_kernel *k = nullptr;
  if (builtin_kernel(ctx, kKernel, 4, sizeof(RowsArgs), 64u, &k) != AXH_OK || !k) return;
  ctx->noalloc_kernel = k; // owned by ctx->ops until the context is destroyed
  ctx->noalloc_scratch = p;
}

} // namespace axh

extern "C" axh_status axh_q4k_matvec_noalloc(axh_context *ctx, const void *q, const float *x,
                                              float *y, uint32_t n_rows, uint32_t sb_per_row,
                                              void *stream) {
  using axh::fail;
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (n_rows == 0) return axh::ok();
  if (n_rows > kMaxRows || sb_per_row == 0 || sb_per_row > kMaxSb)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "axh_q4k_matvec_noalloc takes 1-32 rows of 1-256 superblocks (its scratch holds "
                "2304 bytes: the counter and 16 workgroups x 32 rows of partial sums)");
  if (!q || !x || !y) return fail(AXH_ERR_INVALID_ARGUMENT, "q, x and y must be device pointers");
  if (((uintptr_t)q & 15u) || ((uintptr_t)x & 15u))
    return fail(AXH_ERR_INVALID_ARGUMENT, "q and x must be 16-byte aligned");
  // Both resolved at context creation: no lookup, no host allocation here.
  axh_kernel *const k = ctx->noalloc_kernel;
  void *const ws = ctx->noalloc_scratch;
  if (!k || !ws) {
    void *p = nullptr;
    const axh_status s = resolve_scratch(ctx->core->device, &p); // reports a scratch failure
    if (s != AXH_OK) return s;
    return fail(AXH_ERR_PIPELINE_CREATION,
                "the split-K kernel was not prepared at context creation (see the last error of "
                "axh_context_create)");
  }
  hipSetDevice(ctx->core->device);
  const uint32_t grid[3] = {(sb_per_row + kSpw - 1) / kSpw, 1, 1};
  RowsArgs a{n_rows, sb_per_row, kSpw, 0};
  void *bufs[4] = {const_cast<void *>(q), const_cast<float *>(x), y, ws};
  const axh_status s =
      axh::launch_raw(k, grid, bufs, 4, &a, sizeof(a), 0, axh::pick_stream(ctx, stream));
  return s == AXH_OK ? axh::ok() : s;
}
