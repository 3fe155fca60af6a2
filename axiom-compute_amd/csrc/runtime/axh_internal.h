// Internal types shared by the runtime (axh_runtime.cpp) and the Q4
// operations (axh_ops.cpp).  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "axh.h"
#include "axh_tune.h"

namespace axh {

// Records `msg` as this thread's last error and returns `s`.
axh_status fail(axh_status s, const std::string &msg);
axh_status ok();

struct LoadedModule {
  hipModule_t module = nullptr;
  int refs = 0;
};

// Device-side state shared by a context and every handle prepared on it, so
// a handle may outlive the context that made it.
struct Core {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name;
  uint32_t max_wg[3] = {0, 0, 0};
  uint32_t max_lds = 0;
  uint32_t cu_count = 1;
  uint64_t fence_timeout_ms = 10000;
  std::string cache_dir;

  std::mutex staging_mu;
  void *staging = nullptr; // pinned host memory
  size_t staging_bytes = 0;
  // Staging buffers whose copy outlived a fence timeout (freed at teardown).
  std::vector<void *> retired_staging;

  std::mutex cache_mu; // guards modules and kernels
  std::unordered_map<uint64_t, LoadedModule> modules;
  std::unordered_map<uint64_t, axh_kernel *> kernels; // non-owning

  ~Core();
};

} // namespace axh

struct axh_kernel {
  std::atomic<int> refs{1};
  std::shared_ptr<axh::Core> core;
  uint64_t key = 0;
  uint64_t module_hash = 0;
  hipFunction_t fn = nullptr;
  std::string entry;
  std::vector<uint8_t> access;
  uint32_t pc_bytes = 0;
  uint32_t wg[3] = {1, 1, 1};
  uint32_t lds = 0;
  // Kernels of this library's own code objects take their push constants as
  // separate 32-bit arguments (preloaded into SGPRs): launches pass one
  // kernel parameter per word.  Other code objects take one by-value block.
  bool scalar_pc = false;
  std::mutex mu;              // serialises dispatch_handle on this handle
  std::vector<void *> pool;   // per-binding device buffers
  std::vector<size_t> pool_bytes;
};

struct axh_context {
  std::shared_ptr<axh::Core> core;
  std::mutex ops_mu;
  std::unordered_map<std::string, axh_kernel *> ops; // builtin kernels by entry name
  std::unordered_map<uint64_t, uint32_t> occupancy;  // (kernel, lds) -> workgroups per CU
  // Per-stream device workspaces of the kernels that reduce across
  // workgroups (split-K matvec): calls on one stream never overlap.
  std::unordered_map<void *, void *> workspaces;
  // Set when a capture on the context stream records a launch that uses the
  // context stream's workspace (the graph then replays on that stream only).
  std::atomic<bool> capture_uses_workspace{false};
  // Tuned winners consulted when a call passes no variant; loaded from and
  // saved to winners_path (empty: in memory only).
  std::mutex winners_mu;
  axh_winner_table *winners = nullptr;
  std::atomic<bool> has_winners{false};
  std::string winners_path;
  // The allocation-free matvec's kernel and this device's scratch address,
  // both resolved once at context creation (null if that set-up failed), so
  // its calls look nothing up and allocate nothing on the host either.
  axh_kernel *noalloc_kernel = nullptr;
  void *noalloc_scratch = nullptr;
};

namespace axh {
// Launch `k` with explicit kernel arguments; `lds` overrides the plan's
// dynamic LDS when non-zero.
axh_status launch_raw(axh_kernel *k, const uint32_t grid[3], void *const *buffers, size_t n_buffers,
                      const void *pc, size_t pc_bytes, uint32_t lds, hipStream_t stream);
// True for the code objects embedded in this library (their kernels take
// push constants as separate 32-bit arguments).
bool is_builtin_code_object(const void *co, size_t bytes);
// Builtin kernel by entry name, prepared once per context.
axh_status builtin_kernel(axh_context *ctx, const char *entry, uint32_t n_buffers,
                          uint32_t pc_bytes, uint32_t wg_x, axh_kernel **out);
hipStream_t pick_stream(axh_context *ctx, void *stream);
// Set-up of the allocation-free matvec (axh_noalloc.hip): resolves this
// device's scratch array and prepares its kernel.  Run by axh_context_create.
void noalloc_setup(axh_context *ctx);
// The tuned winner for (op, n_rows, units), if the context has one.
bool lookup_winner(axh_context *ctx, const char *op, uint32_t n_rows, uint32_t units,
                   axh_q4_variant *out);
// Loads (or starts) the context's winner table from `dir`; frees it.
void winners_attach(axh_context *ctx, const std::string &dir);
void winners_detach(axh_context *ctx);
uint64_t hash_bytes(const void *data, size_t n, uint64_t seed);
} // namespace axh
