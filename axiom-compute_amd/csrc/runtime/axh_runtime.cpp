// HIP runtime behind the axh C ABI: context, code-object module cache, kernel
// handles with pooled buffers, dispatch_handle semantics, resident buffers.
//
// Mirrors crates/axc-runtime (context.rs, kernel_handle.rs, dispatch.rs,
// error.rs) of rudybear/axiom-compute with HIP in place of Vulkan:
//   SPIR-V shader module      -> gfx950 code object (hipModuleLoadData)
//   pipeline (entry point)    -> hipFunction_t (hipModuleGetFunction)
//   descriptor set + PC       -> kernel arguments (pointers + push-constant struct)
//   staging buffers + copies  -> pinned host buffer + hipMemcpyAsync
//   fence wait                -> hipEventQuery polling with the fence timeout
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>

#include "axh_internal.h"

namespace axh {

static thread_local std::string t_last_error;

axh_status fail(axh_status s, const std::string &msg) {
  t_last_error = msg;
  return s;
}
axh_status ok() {
  t_last_error.clear();
  return AXH_OK;
}

static std::string hip_msg(const char *what, hipError_t e) {
  return std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
}

// FNV-1a 64 over bytes, chained by `seed`; used for cache keys only.
uint64_t hash_bytes(const void *data, size_t n, uint64_t seed) {
  const uint8_t *p = static_cast<const uint8_t *>(data);
  uint64_t h = 0xcbf29ce484222325ull ^ seed;
  for (size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

Core::~Core() {
  if (device >= 0) hipSetDevice(device);
  for (auto &kv : modules)
    if (kv.second.module) hipModuleUnload(kv.second.module);
  if (stream) hipStreamSynchronize(stream); // retired staging buffers may still be in use
  if (staging) hipHostFree(staging);
  for (void *p : retired_staging) hipHostFree(p);
  if (stream) hipStreamDestroy(stream);
}

hipStream_t pick_stream(axh_context *ctx, void *stream) {
  return stream ? static_cast<hipStream_t>(stream) : ctx->core->stream;
}

static uint64_t round_up_pow2(uint64_t v) {
  if (v <= 1) return 1;
  if (v > (1ull << 62)) return UINT64_MAX;
  uint64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Waits for all work queued on `stream` so far, polling an event so the wait
// is bounded by the context's fence timeout (reference: vkWaitForFences with
// AXC_FENCE_TIMEOUT_MS, kernel_handle.rs:672-686).
static axh_status wait_stream(Core &core, hipStream_t stream) {
  hipEvent_t ev;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventCreate", e));
  e = hipEventRecord(ev, stream);
  if (e != hipSuccess) {
    hipEventDestroy(ev);
    return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventRecord", e));
  }
  const auto t0 = std::chrono::steady_clock::now();
  const auto limit = std::chrono::milliseconds(core.fence_timeout_ms);
  int spins = 0;
  for (;;) {
    e = hipEventQuery(ev);
    if (e == hipSuccess) break;
    if (e != hipErrorNotReady) {
      hipEventDestroy(ev);
      return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventQuery", e));
    }
    if (std::chrono::steady_clock::now() - t0 > limit) {
      hipEventDestroy(ev);
      return fail(AXH_ERR_FENCE_TIMEOUT,
                  "completion wait timed out after " +
                      std::to_string(core.fence_timeout_ms * 1000000ull) + " ns");
    }
    if (++spins > 64) std::this_thread::sleep_for(std::chrono::microseconds(20));
  }
  hipEventDestroy(ev);
  return AXH_OK;
}

static axh_status ensure_staging(Core &core, size_t bytes) {
  if (core.staging_bytes >= bytes) return AXH_OK;
  if (core.staging) hipHostFree(core.staging);
  core.staging = nullptr;
  core.staging_bytes = 0;
  const size_t want = round_up_pow2(bytes);
  hipError_t e = hipHostMalloc(&core.staging, want, hipHostMallocDefault);
  if (e != hipSuccess) return fail(AXH_ERR_MEMORY_MAP, hip_msg("hipHostMalloc", e));
  core.staging_bytes = want;
  return AXH_OK;
}

static constexpr size_t kStagingChunk = size_t(32) << 20;

// A wait that timed out leaves its copy queued on the stream, still reading
// or writing the staging buffer.  The buffer is retired (freed when the core
// goes away) so the next staged copy fills a fresh one instead of handing
// the queued transfer the wrong bytes.
static axh_status staging_wait(Core &core) {
  const axh_status s = wait_stream(core, core.stream);
  if (s == AXH_ERR_FENCE_TIMEOUT && core.staging) {
    core.retired_staging.push_back(core.staging);
    core.staging = nullptr;
    core.staging_bytes = 0;
  }
  return s;
}

// Host -> device through the pinned staging buffer, in chunks.
static axh_status staged_upload(Core &core, void *dst, const void *src, size_t bytes,
                                uint32_t binding) {
  std::lock_guard<std::mutex> lk(core.staging_mu);
  axh_status s = ensure_staging(core, bytes < kStagingChunk ? bytes : kStagingChunk);
  if (s != AXH_OK) return s;
  for (size_t off = 0; off < bytes; off += kStagingChunk) {
    const size_t n = (bytes - off) < kStagingChunk ? (bytes - off) : kStagingChunk;
    std::memcpy(core.staging, static_cast<const uint8_t *>(src) + off, n);
    hipError_t e = hipMemcpyAsync(static_cast<uint8_t *>(dst) + off, core.staging, n,
                                  hipMemcpyHostToDevice, core.stream);
    if (e != hipSuccess)
      return fail(AXH_ERR_STAGING_COPY, "binding #" + std::to_string(binding) +
                                            " (HostToDevice): " + hip_msg("hipMemcpyAsync", e));
    s = staging_wait(core);
    if (s != AXH_OK) return s;
  }
  return AXH_OK;
}

static axh_status staged_download(Core &core, void *dst, const void *src, size_t bytes,
                                  uint32_t binding) {
  std::lock_guard<std::mutex> lk(core.staging_mu);
  axh_status s = ensure_staging(core, bytes < kStagingChunk ? bytes : kStagingChunk);
  if (s != AXH_OK) return s;
  for (size_t off = 0; off < bytes; off += kStagingChunk) {
    const size_t n = (bytes - off) < kStagingChunk ? (bytes - off) : kStagingChunk;
    hipError_t e = hipMemcpyAsync(core.staging, static_cast<const uint8_t *>(src) + off, n,
                                  hipMemcpyDeviceToHost, core.stream);
    if (e != hipSuccess)
      return fail(AXH_ERR_READBACK, "readback of binding #" + std::to_string(binding) +
                                        " failed: " + hip_msg("hipMemcpyAsync", e));
    s = staging_wait(core);
    if (s != AXH_OK) return s;
    std::memcpy(static_cast<uint8_t *>(dst) + off, core.staging, n);
  }
  return AXH_OK;
}

axh_status launch_raw(axh_kernel *k, const uint32_t grid[3], void *const *buffers,
                      size_t n_buffers, const void *pc, size_t pc_bytes, uint32_t lds,
                      hipStream_t stream) {
  // Kernel arguments: buffer pointers in binding order, then the push
  // constants as one by-value struct (16-byte aligned local copy), or as
  // one argument per 32-bit word for this library's own kernels.
  void *ptrs[64];
  void *params[64 + 64];
  alignas(16) uint8_t pcbuf[256];
  if (n_buffers > 64 || pc_bytes > sizeof(pcbuf))
    return fail(AXH_ERR_DESCRIPTOR_POOL, "too many kernel arguments");
  size_t np = 0;
  for (size_t i = 0; i < n_buffers; ++i) {
    ptrs[i] = buffers[i];
    params[np++] = &ptrs[i];
  }
  if (pc_bytes && k->scalar_pc) { // one 32-bit argument per word
    if (pc_bytes % 4u || np + pc_bytes / 4u > sizeof(params) / sizeof(params[0]))
      return fail(AXH_ERR_PUSH_CONSTANT_SIZE_MISMATCH,
                  "builtin kernels take push constants as whole 32-bit words");
    std::memcpy(pcbuf, pc, pc_bytes);
    for (size_t w = 0; w < pc_bytes / 4u; ++w) params[np++] = pcbuf + 4u * w;
  } else if (pc_bytes) {
    std::memcpy(pcbuf, pc, pc_bytes);
    params[np++] = pcbuf;
  }
  const uint32_t shmem = lds ? lds : k->lds;
  hipError_t e = hipModuleLaunchKernel(k->fn, grid[0], grid[1], grid[2], k->wg[0], k->wg[1],
                                       k->wg[2], shmem, stream, params, nullptr);
  if (e != hipSuccess)
    return fail(AXH_ERR_COMMAND_RECORD, hip_msg("hipModuleLaunchKernel", e) + " for '" +
                                            k->entry + "'");
  return AXH_OK;
}

static void release_module(Core &core, uint64_t h) {
  auto it = core.modules.find(h);
  if (it == core.modules.end()) return;
  if (--it->second.refs == 0) {
    hipSetDevice(core.device);
    hipModuleUnload(it->second.module);
    core.modules.erase(it);
  }
}

} // namespace axh

using namespace axh;

extern "C" {

const char *axh_last_error(void) { return t_last_error.c_str(); }

uint32_t axh_abi_version(void) { return AXH_ABI_VERSION; }

const char *axh_status_name(int s) {
  switch (s) {
  case AXH_OK: return "Ok";
  case AXH_ERR_RUNTIME_LOAD: return "VulkanEntryFailed";
  case AXH_ERR_NO_INSTANCE: return "NoVulkanInstance";
  case AXH_ERR_NO_SUPPORTED_DEVICE: return "NoSupportedDevice";
  case AXH_ERR_NO_COMPUTE_QUEUE: return "NoComputeQueue";
  case AXH_ERR_DEVICE_CREATION: return "DeviceCreationFailed";
  case AXH_ERR_MODULE_CREATION: return "ShaderModuleCreationFailed";
  case AXH_ERR_DESCRIPTOR_SET_LAYOUT: return "DescriptorSetLayoutFailed";
  case AXH_ERR_DESCRIPTOR_POOL: return "DescriptorPoolFailed";
  case AXH_ERR_PIPELINE_LAYOUT: return "PipelineLayoutFailed";
  case AXH_ERR_PIPELINE_CREATION: return "PipelineCreationFailed";
  case AXH_ERR_BUFFER_ALLOCATION: return "BufferAllocationFailed";
  case AXH_ERR_MEMORY_MAP: return "MemoryMapFailed";
  case AXH_ERR_NO_COMPATIBLE_MEMORY_TYPE: return "NoCompatibleMemoryType";
  case AXH_ERR_COMMAND_RECORD: return "CommandBufferRecordFailed";
  case AXH_ERR_QUEUE_SUBMIT: return "QueueSubmitFailed";
  case AXH_ERR_FENCE_TIMEOUT: return "FenceTimeout";
  case AXH_ERR_READBACK: return "ReadbackFailed";
  case AXH_ERR_BINDING_COUNT_MISMATCH: return "BindingCountMismatch";
  case AXH_ERR_PUSH_CONSTANT_SIZE_MISMATCH: return "PushConstantSizeMismatch";
  case AXH_ERR_WORKGROUP_COUNT_EXCEEDS_LIMIT: return "WorkgroupCountExceedsDeviceLimit";
  case AXH_ERR_METADATA_IO: return "MetadataIoError";
  case AXH_ERR_METADATA_PARSE: return "MetadataParseError";
  case AXH_ERR_METADATA_SCHEMA_MISMATCH: return "MetadataSchemaMismatch";
  case AXH_ERR_CODE_OBJECT_CACHE_LOAD: return "PipelineCacheLoadFailed";
  case AXH_ERR_STAGING_COPY: return "StagingCopyFailed";
  case AXH_ERR_INVALID_ARGUMENT: return "InvalidArgument";
  default: return "Unknown";
  }
}

axh_status axh_context_create(const axh_context_options *opts, axh_context **out) {
  if (!out) return fail(AXH_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  hipError_t e = hipInit(0);
  if (e != hipSuccess) return fail(AXH_ERR_NO_INSTANCE, hip_msg("hipInit", e));
  int count = 0;
  e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(AXH_ERR_NO_SUPPORTED_DEVICE, "no HIP device with a compute queue");

  int index = opts ? opts->device_index : -1;
  if (index < 0) {
    const char *env = std::getenv("AXH_DEVICE_INDEX");
    index = env ? std::atoi(env) : 0;
  }
  if (index < 0 || index >= count)
    return fail(AXH_ERR_NO_SUPPORTED_DEVICE, "device index " + std::to_string(index) +
                                                 " out of range (" + std::to_string(count) +
                                                 " devices)");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, index);
  if (e != hipSuccess) return fail(AXH_ERR_NO_SUPPORTED_DEVICE, hip_msg("hipGetDeviceProperties", e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(AXH_ERR_NO_SUPPORTED_DEVICE,
                std::string("device is ") + prop.gcnArchName + ", kernels are built for gfx950");
  e = hipSetDevice(index);
  if (e != hipSuccess) return fail(AXH_ERR_DEVICE_CREATION, hip_msg("hipSetDevice", e));

  auto core = std::make_shared<Core>();
  core->device = index;
  // The marketing name can be empty (it comes from a PCI id table that not
  // every install ships); the architecture string is always there.
  core->name = std::string(prop.name[0] ? prop.name : "AMD GPU") + " [" + prop.gcnArchName + "]";
  core->max_wg[0] = (uint32_t)prop.maxGridSize[0];
  core->max_wg[1] = (uint32_t)prop.maxGridSize[1];
  core->max_wg[2] = (uint32_t)prop.maxGridSize[2];
  core->max_lds = (uint32_t)prop.sharedMemPerBlock;
  core->cu_count = prop.multiProcessorCount > 0 ? (uint32_t)prop.multiProcessorCount : 1u;
  uint64_t timeout = opts ? opts->fence_timeout_ms : 0;
  if (timeout == 0) {
    const char *env = std::getenv("AXH_FENCE_TIMEOUT_MS");
    timeout = env ? std::strtoull(env, nullptr, 10) : 0;
    if (timeout == 0) timeout = 10000;
  }
  core->fence_timeout_ms = timeout;
  if (opts && opts->code_object_cache_dir) core->cache_dir = opts->code_object_cache_dir;
  e = hipStreamCreateWithFlags(&core->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    core->stream = nullptr;
    return fail(AXH_ERR_NO_COMPUTE_QUEUE, hip_msg("hipStreamCreate", e));
  }
  axh_context *ctx = new axh_context();
  ctx->core = core;
  winners_attach(ctx, core->cache_dir);
  noalloc_setup(ctx); // a failure there is reported by axh_q4k_matvec_noalloc
  *out = ctx;
  return ok();
}

void axh_context_destroy(axh_context *ctx) {
  if (!ctx) return;
  {
    std::lock_guard<std::mutex> lk(ctx->ops_mu);
    for (auto &kv : ctx->ops) axh_kernel_release(kv.second);
    ctx->ops.clear();
  }
  if (ctx->core && ctx->core->stream) {
    hipSetDevice(ctx->core->device);
    hipStreamSynchronize(ctx->core->stream);
  }
  if (!ctx->workspaces.empty()) {
    hipSetDevice(ctx->core->device);
    hipDeviceSynchronize(); // workspaces may be in use on caller streams
    for (auto &kv : ctx->workspaces) hipFree(kv.second);
  }
  winners_detach(ctx);
  delete ctx; // Core lives on while handles hold it
}

const char *axh_context_device_name(const axh_context *ctx) {
  return ctx ? ctx->core->name.c_str() : "";
}

void *axh_context_stream(const axh_context *ctx) { return ctx ? ctx->core->stream : nullptr; }

void axh_context_max_workgroup_count(const axh_context *ctx, uint32_t out[3]) {
  for (int i = 0; i < 3; ++i) out[i] = ctx ? ctx->core->max_wg[i] : 0;
}

axh_status axh_validate_request(const axh_binding_plan *plan, const uint32_t workgroups[3],
                                size_t n_inputs, size_t n_outputs, size_t pc_bytes,
                                const uint32_t max_wg[3]) {
  if (!plan || !workgroups) return fail(AXH_ERR_INVALID_ARGUMENT, "plan/workgroups is NULL");
  const size_t expected = plan->n_buffers;
  if (n_inputs != expected)
    return fail(AXH_ERR_BINDING_COUNT_MISMATCH, "binding count mismatch: expected " +
                                                    std::to_string(expected) + ", got " +
                                                    std::to_string(n_inputs));
  if (n_outputs != expected)
    return fail(AXH_ERR_BINDING_COUNT_MISMATCH, "binding count mismatch: expected " +
                                                    std::to_string(expected) + ", got " +
                                                    std::to_string(n_outputs));
  if (pc_bytes != plan->push_constant_total_bytes)
    return fail(AXH_ERR_PUSH_CONSTANT_SIZE_MISMATCH,
                "push constant size mismatch: expected " +
                    std::to_string(plan->push_constant_total_bytes) + " bytes, got " +
                    std::to_string(pc_bytes));
  if (max_wg) {
    for (int a = 0; a < 3; ++a)
      if (workgroups[a] > max_wg[a])
        return fail(AXH_ERR_WORKGROUP_COUNT_EXCEEDS_LIMIT,
                    "workgroup count [" + std::to_string(workgroups[0]) + ", " +
                        std::to_string(workgroups[1]) + ", " + std::to_string(workgroups[2]) +
                        "] exceeds device limit [" + std::to_string(max_wg[0]) + ", " +
                        std::to_string(max_wg[1]) + ", " + std::to_string(max_wg[2]) + "]");
  }
  return ok();
}

axh_status axh_prepare_kernel(axh_context *ctx, const void *code_object, size_t co_bytes,
                              const axh_binding_plan *plan, uint32_t pc_bytes, const char *entry,
                              axh_kernel **out) {
  if (!out) return fail(AXH_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  if (!ctx || !code_object || co_bytes == 0 || !plan || !entry)
    return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument to prepare_kernel");
  if (plan->n_buffers > 64 || (plan->n_buffers && !plan->access))
    return fail(AXH_ERR_DESCRIPTOR_SET_LAYOUT, "binding plan needs 0..64 buffers with access modes");
  for (uint32_t i = 0; i < plan->n_buffers; ++i)
    if (plan->access[i] > AXH_ACCESS_READ_WRITE)
      return fail(AXH_ERR_DESCRIPTOR_SET_LAYOUT, "binding #" + std::to_string(i) +
                                                     " has an unknown access mode");
  if (pc_bytes != plan->push_constant_total_bytes || pc_bytes > 256)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "push constant size " + std::to_string(pc_bytes) +
                                             " disagrees with the plan (" +
                                             std::to_string(plan->push_constant_total_bytes) +
                                             ") or exceeds 256 bytes");
  const uint32_t *w = plan->workgroup_size;
  if (w[0] == 0 || w[1] == 0 || w[2] == 0 || (uint64_t)w[0] * w[1] * w[2] > 1024)
    return fail(AXH_ERR_PIPELINE_LAYOUT, "workgroup size must be 1..1024 invocations");

  Core &core = *ctx->core;
  const uint64_t mh = hash_bytes(code_object, co_bytes, 0x51ull);
  uint64_t key = hash_bytes(entry, std::strlen(entry), mh);
  key = hash_bytes(plan->access, plan->n_buffers, key);
  const uint32_t facts[6] = {plan->n_buffers, pc_bytes, w[0], w[1], w[2], plan->dynamic_lds_bytes};
  key = hash_bytes(facts, sizeof(facts), key);

  {
    std::lock_guard<std::mutex> lk(core.cache_mu);
    auto it = core.kernels.find(key);
    if (it != core.kernels.end()) {
      int r = it->second->refs.load();
      while (r > 0 && !it->second->refs.compare_exchange_weak(r, r + 1)) {}
      if (r > 0) {
        *out = it->second;
        return ok();
      }
    }
  }
  if (hipSetDevice(core.device) != hipSuccess)
    return fail(AXH_ERR_DEVICE_CREATION, "hipSetDevice failed");

  std::lock_guard<std::mutex> lk(core.cache_mu);
  auto found = core.kernels.find(key); // second check under the lock
  if (found != core.kernels.end()) {
    int r = found->second->refs.load();
    while (r > 0 && !found->second->refs.compare_exchange_weak(r, r + 1)) {}
    if (r > 0) {
      *out = found->second;
      return ok();
    }
  }
  auto mit = core.modules.find(mh);
  if (mit == core.modules.end()) {
    LoadedModule lm;
    hipError_t e = hipModuleLoadData(&lm.module, code_object);
    if (e != hipSuccess) return fail(AXH_ERR_MODULE_CREATION, hip_msg("hipModuleLoadData", e));
    mit = core.modules.emplace(mh, lm).first;
  }
  hipFunction_t fn = nullptr;
  hipError_t e = hipModuleGetFunction(&fn, mit->second.module, entry);
  if (e != hipSuccess) {
    if (mit->second.refs == 0) {
      hipModuleUnload(mit->second.module);
      core.modules.erase(mit);
    }
    return fail(AXH_ERR_PIPELINE_CREATION,
                std::string("entry point '") + entry + "': " + hip_msg("hipModuleGetFunction", e));
  }
  mit->second.refs++;
  axh_kernel *k = new axh_kernel();
  k->core = ctx->core;
  k->key = key;
  k->module_hash = mh;
  k->fn = fn;
  k->entry = entry;
  k->access.assign(plan->access, plan->access + plan->n_buffers);
  k->pc_bytes = pc_bytes;
  k->wg[0] = w[0];
  k->wg[1] = w[1];
  k->wg[2] = w[2];
  k->lds = plan->dynamic_lds_bytes;
  k->scalar_pc = is_builtin_code_object(code_object, co_bytes);
  core.kernels[key] = k;
  *out = k;
  return ok();
}

void axh_kernel_retain(axh_kernel *k) {
  if (k) k->refs.fetch_add(1);
}

void axh_kernel_release(axh_kernel *k) {
  if (!k) return;
  if (k->refs.fetch_sub(1) != 1) return;
  std::shared_ptr<Core> core = k->core;
  {
    std::lock_guard<std::mutex> lk(core->cache_mu);
    auto it = core->kernels.find(k->key);
    if (it != core->kernels.end() && it->second == k) core->kernels.erase(it);
    hipSetDevice(core->device);
    for (void *p : k->pool)
      if (p) hipFree(p);
    release_module(*core, k->module_hash);
  }
  delete k; // the last holder of `core` may free the device state here
}

uint64_t axh_kernel_cache_key(const axh_kernel *k) { return k ? k->key : 0; }

uint64_t axh_kernel_pool_bytes(const axh_kernel *k, uint32_t binding) {
  if (!k || binding >= k->pool_bytes.size()) return 0;
  return k->pool_bytes[binding];
}

axh_status axh_dispatch_handle(axh_context *ctx, axh_kernel *k, const uint32_t workgroups[3],
                               const void *const *inputs, const size_t *input_sizes,
                               size_t n_inputs, const size_t *output_sizes, size_t n_outputs,
                               void *const *outputs, const void *pc, size_t pc_bytes) {
  if (!ctx || !k || !workgroups) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  axh_binding_plan plan{};
  plan.n_buffers = (uint32_t)k->access.size();
  plan.access = k->access.data();
  plan.push_constant_total_bytes = k->pc_bytes;
  axh_status s =
      axh_validate_request(&plan, workgroups, n_inputs, n_outputs, pc_bytes, ctx->core->max_wg);
  if (s != AXH_OK) return s;
  if (pc_bytes && !pc) return fail(AXH_ERR_INVALID_ARGUMENT, "push_constants is NULL");
  for (size_t i = 0; i < n_inputs; ++i)
    if (input_sizes[i] && !inputs[i])
      return fail(AXH_ERR_INVALID_ARGUMENT, "input #" + std::to_string(i) + " is NULL");
  for (size_t i = 0; i < n_outputs; ++i)
    if (output_sizes[i] && !outputs[i])
      return fail(AXH_ERR_INVALID_ARGUMENT, "output #" + std::to_string(i) + " is NULL");

  Core &core = *ctx->core;
  std::lock_guard<std::mutex> lk(k->mu);
  hipSetDevice(core.device);
  const size_t n = k->access.size();
  if (k->pool.size() < n) {
    k->pool.resize(n, nullptr);
    k->pool_bytes.resize(n, 0);
  }
  for (size_t i = 0; i < n; ++i) {
    uint64_t need = input_sizes[i];
    if (output_sizes[i] > need) need = output_sizes[i];
    if (need < 4) need = 4;
    if (k->pool_bytes[i] >= need) continue;
    const uint64_t sz = round_up_pow2(need);
    if (sz == UINT64_MAX)
      return fail(AXH_ERR_BUFFER_ALLOCATION, "buffer #" + std::to_string(i) + " allocation failed (" +
                                                 std::to_string(need) +
                                                 " bytes): requested size too large (> 2^62 bytes)");
    if (k->pool[i]) hipFree(k->pool[i]);
    k->pool[i] = nullptr;
    k->pool_bytes[i] = 0;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess)
      return fail(AXH_ERR_BUFFER_ALLOCATION, "buffer #" + std::to_string(i) + " allocation failed (" +
                                                 std::to_string(sz) + " bytes): " +
                                                 hip_msg("hipMalloc", e));
    k->pool[i] = p;
    k->pool_bytes[i] = sz;
  }
  for (size_t i = 0; i < n; ++i) {
    if (input_sizes[i] == 0) continue;
    s = staged_upload(core, k->pool[i], inputs[i], input_sizes[i], (uint32_t)i);
    if (s != AXH_OK) return s;
  }
  s = launch_raw(k, workgroups, k->pool.data(), n, pc, pc_bytes, 0, core.stream);
  if (s != AXH_OK) return s;
  s = wait_stream(core, core.stream);
  if (s != AXH_OK) return s;
  for (size_t i = 0; i < n; ++i) {
    if (output_sizes[i] == 0) continue;
    s = staged_download(core, outputs[i], k->pool[i], output_sizes[i], (uint32_t)i);
    if (s != AXH_OK) return s;
  }
  return ok();
}

axh_status axh_dispatch(axh_context *ctx, const void *code_object, size_t co_bytes,
                        const axh_binding_plan *plan, const uint32_t workgroups[3],
                        const void *const *inputs, const size_t *input_sizes, size_t n_inputs,
                        const size_t *output_sizes, size_t n_outputs, void *const *outputs,
                        const void *pc, size_t pc_bytes, const char *entry) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  axh_status s = axh_validate_request(plan, workgroups, n_inputs, n_outputs, pc_bytes,
                                      ctx->core->max_wg);
  if (s != AXH_OK) return s;
  axh_kernel *k = nullptr;
  s = axh_prepare_kernel(ctx, code_object, co_bytes, plan, plan->push_constant_total_bytes, entry,
                         &k);
  if (s != AXH_OK) return s;
  s = axh_dispatch_handle(ctx, k, workgroups, inputs, input_sizes, n_inputs, output_sizes,
                          n_outputs, outputs, pc, pc_bytes);
  const std::string msg = t_last_error;
  axh_kernel_release(k);
  t_last_error = msg;
  return s;
}

axh_status axh_buffer_alloc(axh_context *ctx, size_t bytes, void **device_ptr) {
  if (!ctx || !device_ptr) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  *device_ptr = nullptr;
  hipSetDevice(ctx->core->device);
  hipError_t e = hipMalloc(device_ptr, bytes ? bytes : 4);
  if (e != hipSuccess)
    return fail(AXH_ERR_BUFFER_ALLOCATION,
                "allocation of " + std::to_string(bytes) + " bytes failed: " + hip_msg("hipMalloc", e));
  return ok();
}

axh_status axh_buffer_free(axh_context *ctx, void *device_ptr) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  if (!device_ptr) return ok();
  hipSetDevice(ctx->core->device);
  hipError_t e = hipFree(device_ptr);
  if (e != hipSuccess) return fail(AXH_ERR_INVALID_ARGUMENT, hip_msg("hipFree", e));
  return ok();
}

axh_status axh_upload(axh_context *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (bytes == 0) return ok();
  hipSetDevice(ctx->core->device);
  axh_status s = staged_upload(*ctx->core, dst, src, bytes, 0);
  return s == AXH_OK ? ok() : s;
}

axh_status axh_download(axh_context *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (bytes == 0) return ok();
  hipSetDevice(ctx->core->device);
  axh_status s = staged_download(*ctx->core, dst, src, bytes, 0);
  return s == AXH_OK ? ok() : s;
}

axh_status axh_copy_device(axh_context *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (bytes == 0) return ok();
  hipSetDevice(ctx->core->device);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->core->stream);
  if (e != hipSuccess) return fail(AXH_ERR_STAGING_COPY, hip_msg("hipMemcpyAsync", e));
  axh_status s = wait_stream(*ctx->core, ctx->core->stream);
  return s == AXH_OK ? ok() : s;
}

axh_status axh_launch(axh_context *ctx, axh_kernel *k, const uint32_t workgroups[3],
                      void *const *bufs, size_t n_buffers, const void *pc, size_t pc_bytes,
                      void *stream) {
  if (!ctx || !k || !workgroups) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  if (n_buffers != k->access.size())
    return fail(AXH_ERR_BINDING_COUNT_MISMATCH, "binding count mismatch: expected " +
                                                    std::to_string(k->access.size()) + ", got " +
                                                    std::to_string(n_buffers));
  if (pc_bytes != k->pc_bytes)
    return fail(AXH_ERR_PUSH_CONSTANT_SIZE_MISMATCH,
                "push constant size mismatch: expected " + std::to_string(k->pc_bytes) +
                    " bytes, got " + std::to_string(pc_bytes));
  for (int a = 0; a < 3; ++a)
    if (workgroups[a] > ctx->core->max_wg[a])
      return fail(AXH_ERR_WORKGROUP_COUNT_EXCEEDS_LIMIT, "workgroup count exceeds device limit");
  hipSetDevice(ctx->core->device);
  axh_status s = launch_raw(k, workgroups, bufs, n_buffers, pc, pc_bytes, 0, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

axh_status axh_device_synchronize(axh_context *ctx) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  hipSetDevice(ctx->core->device);
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipDeviceSynchronize", e));
  return ok();
}

axh_status axh_event_create(axh_context *ctx, axh_event **out) {
  if (!ctx || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  hipSetDevice(ctx->core->device);
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventCreate", e));
  *out = reinterpret_cast<axh_event *>(ev);
  return ok();
}

axh_status axh_event_record(axh_context *ctx, axh_event *ev, void *stream) {
  if (!ctx || !ev) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  hipError_t e = hipEventRecord(reinterpret_cast<hipEvent_t>(ev), pick_stream(ctx, stream));
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventRecord", e));
  return ok();
}

axh_status axh_event_synchronize(axh_context *ctx, axh_event *ev) {
  if (!ctx || !ev) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  hipError_t e = hipEventSynchronize(reinterpret_cast<hipEvent_t>(ev));
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventSynchronize", e));
  return ok();
}

axh_status axh_event_elapsed_ms(axh_event *start, axh_event *end, float *ms) {
  if (!start || !end || !ms) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  hipError_t e = hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                     reinterpret_cast<hipEvent_t>(end));
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipEventElapsedTime", e));
  return ok();
}

void axh_event_destroy(axh_event *ev) {
  if (ev) hipEventDestroy(reinterpret_cast<hipEvent_t>(ev));
}

// ---- graph capture ----------------------------------------------------------
// A captured sequence of launches on the context stream, replayed as one
// hipGraphExec (no host work per kernel).  Only kernel launches are captured:
// the operations of this library record no memset or copy nodes.
struct axh_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  uint64_t n_nodes = 0;
  // Holds a split-K launch bound to the context stream's workspace: replays
  // on another stream could overlap calls that share that workspace.
  bool uses_workspace = false;
  hipStream_t home = nullptr;
};

axh_status axh_capture_begin(axh_context *ctx) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  hipSetDevice(ctx->core->device);
  ctx->capture_uses_workspace = false;
  hipError_t e = hipStreamBeginCapture(ctx->core->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return fail(AXH_ERR_COMMAND_RECORD, hip_msg("hipStreamBeginCapture", e));
  return ok();
}

axh_status axh_capture_end(axh_context *ctx, axh_graph **out) {
  if (!ctx || !out) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  hipSetDevice(ctx->core->device);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->core->stream, &g);
  if (e != hipSuccess || !g)
    return fail(AXH_ERR_COMMAND_RECORD, hip_msg("hipStreamEndCapture", e));
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g);
    return fail(AXH_ERR_COMMAND_RECORD, hip_msg("hipGraphInstantiate", e));
  }
  size_t n = 0;
  hipGraphGetNodes(g, nullptr, &n);
  auto *G = new axh_graph;
  G->graph = g;
  G->exec = exec;
  G->n_nodes = n;
  G->uses_workspace = ctx->capture_uses_workspace.exchange(false);
  G->home = ctx->core->stream;
  *out = G;
  return ok();
}

axh_status axh_graph_launch(axh_context *ctx, axh_graph *g, void *stream) {
  if (!ctx || !g) return fail(AXH_ERR_INVALID_ARGUMENT, "NULL argument");
  const hipStream_t st = pick_stream(ctx, stream);
  if (g->uses_workspace && st != g->home)
    return fail(AXH_ERR_INVALID_ARGUMENT,
                "this graph holds a split-K matvec bound to the context stream's workspace; "
                "replay it on the context stream (NULL)");
  hipSetDevice(ctx->core->device);
  hipError_t e = hipGraphLaunch(g->exec, st);
  if (e != hipSuccess) return fail(AXH_ERR_QUEUE_SUBMIT, hip_msg("hipGraphLaunch", e));
  return ok();
}

uint64_t axh_graph_node_count(const axh_graph *g) { return g ? g->n_nodes : 0; }

void axh_graph_destroy(axh_graph *g) {
  if (!g) return;
  if (g->exec) hipGraphExecDestroy(g->exec);
  if (g->graph) hipGraphDestroy(g->graph);
  delete g;
}

axh_status axh_synchronize(axh_context *ctx, void *stream) {
  if (!ctx) return fail(AXH_ERR_INVALID_ARGUMENT, "ctx is NULL");
  hipSetDevice(ctx->core->device);
  axh_status s = wait_stream(*ctx->core, pick_stream(ctx, stream));
  return s == AXH_OK ? ok() : s;
}

} // extern "C"
