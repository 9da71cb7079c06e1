// libsile_hip runtime: device selection, HBM memory, streams/events, code
// object loading and kernel launch behind the C ABI of include/sile_hip.h.
//
// The library carries its gfx950 code objects inside its own image (the
// build assembles them in with .incbin) and loads them with hipModuleLoadData
// on first use of a device; kernels are launched with hipModuleLaunchKernel.
// This replaces the reference CPU backend's per-launch `cc` compile and
// dlopen (crates/sile-backend/src/cpu/mod.rs:48-134): compilation happens
// once, at library build time.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "runtime_internal.h"

// ---- embedded code objects -------------------------------------------------
// SILE_CO_DIR is the build directory holding <name>.hsaco (raw ELF for gfx950).
#ifndef SILE_CO_DIR
#error "SILE_CO_DIR must name the directory of the built code objects"
#endif

#define SILE_EMBED(sym, file)                                           \
  __asm__(".section .rodata." #sym ",\"a\",@progbits\n"                 \
          ".p2align 12\n"                                               \
          ".global " #sym "_begin\n" #sym "_begin:\n"                   \
          ".incbin \"" SILE_CO_DIR "/" file "\"\n"                      \
          ".global " #sym "_end\n" #sym "_end:\n"                       \
          ".previous\n");                                               \
  extern "C" const unsigned char sym##_begin[];                         \
  extern "C" const unsigned char sym##_end[];

SILE_EMBED(sile_co_dsl, "dsl.hsaco")
SILE_EMBED(sile_co_softmax, "softmax.hsaco")
SILE_EMBED(sile_co_gemm, "gemm.hsaco")
SILE_EMBED(sile_co_attention, "attention.hsaco")
SILE_EMBED(sile_co_flash_attn, "flash_attn.hsaco")

namespace sile_rt {
namespace {

struct Image {
  const unsigned char* begin;
  const unsigned char* end;
  const char* name;
};

const Image kImages[static_cast<int>(Module::kCount)] = {
    {sile_co_dsl_begin, sile_co_dsl_end, "dsl"},
    {sile_co_softmax_begin, sile_co_softmax_end, "softmax"},
    {sile_co_gemm_begin, sile_co_gemm_end, "gemm"},
    {sile_co_attention_begin, sile_co_attention_end, "attention"},
    {sile_co_flash_attn_begin, sile_co_flash_attn_end, "flash_attn"},
};

struct DeviceState {
  hipModule_t modules[static_cast<int>(Module::kCount)] = {};
  std::map<std::string, hipFunction_t> functions;
};

std::mutex g_mu;
std::map<int, DeviceState> g_devices;
thread_local std::string t_last_error;

}  // namespace

int fail(int status, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  t_last_error = buf;
  return status;
}

int ok() {
  t_last_error.clear();
  return SILE_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(SILE_ERR_RUNTIME, "%s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
}

static int load_device_locked(int dev, DeviceState** out) {
  auto it = g_devices.find(dev);
  if (it != g_devices.end()) {
    *out = &it->second;
    return SILE_OK;
  }
  DeviceState st;
  for (int i = 0; i < static_cast<int>(Module::kCount); ++i) {
    hipError_t e = hipModuleLoadData(&st.modules[i], kImages[i].begin);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipModuleUnload(st.modules[j]);
      return fail(SILE_ERR_COMPILE, "hipModuleLoadData(%s code object, %zu bytes) on device %d: %s",
                  kImages[i].name, (size_t)(kImages[i].end - kImages[i].begin), dev,
                  hipGetErrorString(e));
    }
  }
  auto res = g_devices.emplace(dev, std::move(st));
  *out = &res.first->second;
  return SILE_OK;
}

int ensure_device() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "no HIP device visible");
  int dev = 0;
  SILE_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* st = nullptr;
  return load_device_locked(dev, &st);
}

int get_function(Module m, const char* name, hipFunction_t* out) {
  int dev = 0;
  SILE_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState* st = nullptr;
  int rc = load_device_locked(dev, &st);
  if (rc != SILE_OK) return rc;
  auto it = st->functions.find(name);
  if (it != st->functions.end()) {
    *out = it->second;
    return SILE_OK;
  }
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, st->modules[static_cast<int>(m)], name);
  if (e != hipSuccess)
    return fail(SILE_ERR_COMPILE, "kernel %s not found in the %s code object: %s", name,
                kImages[static_cast<int>(m)].name, hipGetErrorString(e));
  st->functions.emplace(name, f);
  *out = f;
  return SILE_OK;
}

int resident_blocks(Module m, const char* name, int block_threads, int64_t* out) {
  hipFunction_t f = nullptr;
  int rc = get_function(m, name, &f);
  if (rc != SILE_OK) return rc;
  int dev = 0, cus = 0, per_cu = 0;
  SILE_HIP_CHECK(hipGetDevice(&dev));
  SILE_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  SILE_HIP_CHECK(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, block_threads, 0));
  *out = (int64_t)cus * (per_cu > 0 ? per_cu : 1);
  return SILE_OK;
}

namespace {
constexpr int kScratchDevices = 64;
struct DeviceScratch {
  std::mutex mu;
  void* p = nullptr;
  size_t cap = 0;
  hipEvent_t last = nullptr;   // recorded after the last user's kernels
  bool used = false;
};
DeviceScratch g_scratch[kScratchDevices][kScratchSlots];
thread_local int t_scratch_dev[kScratchSlots] = {-1, -1};  // device whose slot lock this thread holds
}  // namespace

int scratch_acquire(size_t bytes, hipStream_t s, void** out, int slot) {
  int dev = 0;
  SILE_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kScratchDevices)
    return fail(SILE_ERR_INVALID_DEVICE, "device %d beyond the %d the scratch covers", dev,
                kScratchDevices);
  if (slot < 0 || slot >= kScratchSlots) return fail(SILE_ERR_SHAPE, "scratch slot %d", slot);
  DeviceScratch& d = g_scratch[dev][slot];
  d.mu.lock();
  auto bail = [&](hipError_t e, const char* what) {
    d.mu.unlock();
    return hip_fail(e, what);
  };
  hipError_t e = hipSuccess;
  if (!d.last && (e = hipEventCreateWithFlags(&d.last, hipEventDisableTiming)) != hipSuccess)
    return bail(e, "hipEventCreateWithFlags");
  if (d.cap < bytes) {
    if (d.p) {
      // the previous buffer may still be in use on another stream
      if (d.used && (e = hipEventSynchronize(d.last)) != hipSuccess)
        return bail(e, "hipEventSynchronize");
      (void)hipFree(d.p);
      d.p = nullptr;
      d.cap = 0;
    }
    if ((e = hipMalloc(&d.p, bytes)) != hipSuccess) {
      d.p = nullptr;
      return bail(e, "hipMalloc(scratch)");
    }
    d.cap = bytes;
  }
  if (d.used && (e = hipStreamWaitEvent(s, d.last, 0)) != hipSuccess)
    return bail(e, "hipStreamWaitEvent");
  t_scratch_dev[slot] = dev;
  *out = d.p;
  return SILE_OK;
}

void scratch_release(hipStream_t s, int slot) {
  if (slot < 0 || slot >= kScratchSlots) return;
  const int dev = t_scratch_dev[slot];
  if (dev < 0) return;
  DeviceScratch& d = g_scratch[dev][slot];
  if (hipEventRecord(d.last, s) == hipSuccess)
    d.used = true;
  else
    (void)hipStreamSynchronize(s);   // this call's kernels (and those s waited for) are done
  t_scratch_dev[slot] = -1;
  d.mu.unlock();
}

int launch(Module m, const char* name, dim3 grid, dim3 block, void** params, hipStream_t stream,
           size_t dynamic_lds) {
  hipFunction_t f = nullptr;
  int rc = get_function(m, name, &f);
  if (rc != SILE_OK) return rc;
  hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                       (unsigned)dynamic_lds, stream, params, nullptr);
  if (e != hipSuccess) return hip_fail(e, name);
  return SILE_OK;
}

}  // namespace sile_rt

using namespace sile_rt;

extern "C" {

const char* sile_hip_last_error(void) { return t_last_error.c_str(); }

const char* sile_hip_version(void) { return "sile_hip 0.1 (gfx950)"; }

int sile_hip_device_count(int* count) {
  if (!count) return fail(SILE_ERR_SHAPE, "count is NULL");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return ok();
}

int sile_hip_init(int ordinal) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "no HIP device visible");
  if (ordinal < 0 || ordinal >= count)
    return fail(SILE_ERR_INVALID_DEVICE, "device ordinal %d out of range [0, %d)", ordinal, count);
  SILE_HIP_CHECK(hipSetDevice(ordinal));
  int rc = ensure_device();
  if (rc != SILE_OK) return rc;
  // set-up of the no-allocation launch: this device's address of its tables
  void* scratch = nullptr;
  rc = noalloc_scratch(&scratch, nullptr);
  if (rc != SILE_OK) return rc;
  return ok();
}

int sile_hip_device_info(int ordinal, sile_hip_device_props* out) {
  if (!out) return fail(SILE_ERR_SHAPE, "out is NULL");
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "no HIP device visible");
  if (ordinal < 0 || ordinal >= count)
    return fail(SILE_ERR_INVALID_DEVICE, "device ordinal %d out of range [0, %d)", ordinal, count);
  hipDeviceProp_t p;
  SILE_HIP_CHECK(hipGetDeviceProperties(&p, ordinal));
  memset(out, 0, sizeof *out);
  snprintf(out->name, sizeof out->name, "%s", p.name);
  snprintf(out->gcn_arch, sizeof out->gcn_arch, "%s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->clock_khz = p.clockRate;
  out->memory_clock_khz = p.memoryClockRate;
  out->memory_bus_width = p.memoryBusWidth;
  out->total_global_mem = (int64_t)p.totalGlobalMem;
  out->l2_cache_bytes = p.l2CacheSize;
  out->lds_per_block = (int64_t)p.sharedMemPerBlock;
  return ok();
}

int sile_hip_device_synchronize(void) {
  SILE_HIP_CHECK(hipDeviceSynchronize());
  return ok();
}

int sile_hip_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(SILE_ERR_SHAPE, "ptr is NULL");
  *ptr = nullptr;
  if (bytes == 0) return ok();
  SILE_HIP_CHECK(hipMalloc(ptr, bytes));
  return ok();
}

int sile_hip_free(void* ptr) {
  if (ptr) SILE_HIP_CHECK(hipFree(ptr));
  return ok();
}

int sile_hip_memcpy_htod(void* dst, const void* src, size_t bytes) {
  if (bytes) SILE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return ok();
}

int sile_hip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  if (bytes) SILE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return ok();
}

int sile_hip_memcpy_dtod(void* dst, const void* src, size_t bytes) {
  if (bytes) SILE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return ok();
}

int sile_hip_memset(void* dst, int value, size_t bytes) {
  if (bytes) SILE_HIP_CHECK(hipMemset(dst, value, bytes));
  return ok();
}

int sile_hip_stream_create(sile_hip_stream* out) {
  if (!out) return fail(SILE_ERR_SHAPE, "out is NULL");
  hipStream_t s = nullptr;
  SILE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = s;
  return ok();
}

int sile_hip_stream_destroy(sile_hip_stream stream) {
  if (stream) SILE_HIP_CHECK(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return ok();
}

int sile_hip_stream_synchronize(sile_hip_stream stream) {
  SILE_HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return ok();
}

int sile_hip_graph_begin(sile_hip_stream stream) {
  if (!stream) return fail(SILE_ERR_SHAPE, "the null stream cannot be captured");
  SILE_HIP_CHECK(hipStreamBeginCapture(static_cast<hipStream_t>(stream),
                                       hipStreamCaptureModeThreadLocal));
  return ok();
}

int sile_hip_graph_end(sile_hip_stream stream, sile_hip_graph* out) {
  if (!stream || !out) return fail(SILE_ERR_SHAPE, "NULL stream or out");
  hipGraph_t g = nullptr;
  SILE_HIP_CHECK(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *out = exec;
  return ok();
}

int sile_hip_graph_launch(sile_hip_graph graph, sile_hip_stream stream) {
  if (!graph) return fail(SILE_ERR_SHAPE, "graph is NULL");
  SILE_HIP_CHECK(hipGraphLaunch(static_cast<hipGraphExec_t>(graph),
                                static_cast<hipStream_t>(stream)));
  return ok();
}

int sile_hip_graph_destroy(sile_hip_graph graph) {
  if (graph) SILE_HIP_CHECK(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
  return ok();
}

int sile_hip_event_create(sile_hip_event* out) {
  if (!out) return fail(SILE_ERR_SHAPE, "out is NULL");
  hipEvent_t e = nullptr;
  SILE_HIP_CHECK(hipEventCreate(&e));
  *out = e;
  return ok();
}

int sile_hip_event_destroy(sile_hip_event event) {
  if (event) SILE_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return ok();
}

int sile_hip_event_record(sile_hip_event event, sile_hip_stream stream) {
  SILE_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return ok();
}

int sile_hip_event_synchronize(sile_hip_event event) {
  SILE_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return ok();
}

int sile_hip_event_elapsed_ms(float* ms, sile_hip_event start, sile_hip_event stop) {
  if (!ms) return fail(SILE_ERR_SHAPE, "ms is NULL");
  SILE_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                     static_cast<hipEvent_t>(stop)));
  return ok();
}

int sile_hip_module_load(const void* image, size_t bytes, sile_hip_module* out) {
  if (!image || !out || bytes < 4) return fail(SILE_ERR_COMPILE, "empty code object image");
  int rc = ensure_device();
  if (rc != SILE_OK) return rc;
  hipModule_t m = nullptr;
  hipError_t e = hipModuleLoadData(&m, image);
  if (e != hipSuccess)
    return fail(SILE_ERR_COMPILE, "hipModuleLoadData(%zu bytes): %s", bytes, hipGetErrorString(e));
  *out = m;
  return ok();
}

int sile_hip_module_unload(sile_hip_module module) {
  if (module) SILE_HIP_CHECK(hipModuleUnload(static_cast<hipModule_t>(module)));
  return ok();
}

int sile_hip_module_get(sile_hip_module module, const char* name, sile_hip_function* out) {
  if (!module || !name || !out) return fail(SILE_ERR_COMPILE, "module, name or out is NULL");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name);
  if (e != hipSuccess)
    return fail(SILE_ERR_COMPILE, "symbol %s not found: %s", name, hipGetErrorString(e));
  *out = f;
  return ok();
}

}  // extern "C"

namespace {

// Device buffers for the launch tables, kept per device and reused: a launch
// takes one, and returns it once the kernel has finished, so the synchronous
// launches neither allocate nor free device memory after the first calls
// (hipFree would also wait for the whole device, other streams included).
constexpr int kTablePoolDevices = 64;
struct TablePool {
  std::mutex mu;
  std::vector<std::pair<void*, size_t>> free_list;
};
TablePool g_table_pools[kTablePoolDevices];

int table_acquire(size_t bytes, int* dev_out, void** out, size_t* cap_out) {
  int dev = 0;
  SILE_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kTablePoolDevices)
    return fail(SILE_ERR_INVALID_DEVICE, "device %d beyond the %d the table pool covers", dev,
                kTablePoolDevices);
  *dev_out = dev;
  {
    std::lock_guard<std::mutex> lk(g_table_pools[dev].mu);
    auto& fl = g_table_pools[dev].free_list;
    for (size_t i = 0; i < fl.size(); ++i)
      if (fl[i].second >= bytes) {
        *out = fl[i].first;
        *cap_out = fl[i].second;
        fl.erase(fl.begin() + (long)i);
        return ok();
      }
  }
  const size_t cap = bytes < 4096 ? 4096 : bytes;
  SILE_HIP_CHECK(hipMalloc(out, cap));
  *cap_out = cap;
  return ok();
}

void table_release(int dev, void* p, size_t cap) {
  std::lock_guard<std::mutex> lk(g_table_pools[dev].mu);
  g_table_pools[dev].free_list.push_back({p, cap});
}

// Uploads the buffer-pointer and shape tables, launches `fn` over `workgroups`
// workgroups of `threads` threads with (buffers, programs, shapes, num_shapes)
// and waits for it.
int launch_with_tables(hipFunction_t fn, void* const* buffers, int64_t num_buffers,
                       const int64_t* shapes, int64_t num_shapes, int64_t programs,
                       int64_t workgroups, uint32_t threads, hipStream_t s) {
  // Device copies of the pointer and shape tables, as the Metal runtime binds a
  // shapes buffer after the args (crates/sile-backend/src/metal/mod.rs:131-144).
  const size_t buf_bytes = (size_t)num_buffers * sizeof(void*);
  const size_t shp_bytes = (size_t)num_shapes * sizeof(int64_t);
  void* table = nullptr;
  size_t table_cap = 0;
  int dev = 0;
  int rc = table_acquire(buf_bytes + shp_bytes + 16, &dev, &table, &table_cap);
  if (rc != SILE_OK) return rc;
  std::vector<unsigned char> host(buf_bytes + shp_bytes + 16);
  if (buf_bytes) memcpy(host.data(), buffers, buf_bytes);
  if (shp_bytes) memcpy(host.data() + buf_bytes, shapes, shp_bytes);
  hipError_t e = hipMemcpyAsync(table, host.data(), buf_bytes + shp_bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) {
    void* dev_buffers = table;
    void* dev_shapes = static_cast<unsigned char*>(table) + buf_bytes;
    int64_t np = programs, ns = num_shapes;
    void* params[] = {&dev_buffers, &np, &dev_shapes, &ns};
    e = hipModuleLaunchKernel(fn, (unsigned)workgroups, 1, 1, threads, 1, 1, 0, s, params, nullptr);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) {
    // the table may still be in use by a failed or unfinished launch: not reused
    return hip_fail(e, "kernel launch");
  }
  table_release(dev, table, table_cap);
  return ok();
}

int check_launch_args(sile_hip_function fn, void* const* buffers, int64_t num_buffers,
                      const int64_t* shapes, int64_t num_shapes, const uint32_t grid[3],
                      int64_t* programs) {
  if (!fn) return fail(SILE_ERR_COMPILE, "function is NULL");
  if (!grid) return fail(SILE_ERR_SHAPE, "grid not set");
  if (num_buffers < 0 || num_shapes < 0 || (num_buffers && !buffers) || (num_shapes && !shapes))
    return fail(SILE_ERR_SHAPE, "buffers/shapes arrays do not match their counts");
  *programs = (int64_t)grid[0] * grid[1] * grid[2];
  if (*programs > 0x7fffffffLL)
    return fail(SILE_ERR_SHAPE, "too many programs (%lld)", (long long)*programs);
  return ok();
}

}  // namespace

extern "C" {

int sile_hip_launch_tiles(sile_hip_function fn, void* const* buffers, int64_t num_buffers,
                          const int64_t* shapes, int64_t num_shapes, const uint32_t grid[3],
                          uint32_t threads_per_program, sile_hip_stream stream) {
  int64_t programs = 0;
  int rc = check_launch_args(fn, buffers, num_buffers, shapes, num_shapes, grid, &programs);
  if (rc != SILE_OK) return rc;
  if (threads_per_program == 0 || threads_per_program > 1024)
    return fail(SILE_ERR_SHAPE, "threads_per_program %u not in [1, 1024]", threads_per_program);
  if (programs == 0) return ok();
  return launch_with_tables(static_cast<hipFunction_t>(fn), buffers, num_buffers, shapes,
                            num_shapes, programs, programs, threads_per_program,
                            static_cast<hipStream_t>(stream));
}

int sile_hip_launch_llir(sile_hip_function fn, void* const* buffers, int64_t num_buffers,
                         const int64_t* shapes, int64_t num_shapes, const uint32_t grid[3],
                         sile_hip_stream stream) {
  int64_t programs = 0;
  int rc = check_launch_args(fn, buffers, num_buffers, shapes, num_shapes, grid, &programs);
  if (rc != SILE_OK) return rc;
  if (programs == 0) return ok();
  // a generated kernel takes one program per lane (64 lanes a workgroup) or,
  // when its loops are spread over a workgroup, one program per workgroup;
  // the generator sets the kernel's workgroup size to tell them apart
  int max_threads = 64;
  SILE_HIP_CHECK(hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK,
                                     static_cast<hipFunction_t>(fn)));
  if (max_threads > 64) {
    if (programs > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many programs");
    return launch_with_tables(static_cast<hipFunction_t>(fn), buffers, num_buffers, shapes,
                              num_shapes, programs, programs, max_threads,
                              static_cast<hipStream_t>(stream));
  }
  return launch_with_tables(static_cast<hipFunction_t>(fn), buffers, num_buffers, shapes,
                            num_shapes, programs, (programs + 63) / 64, 64,
                            static_cast<hipStream_t>(stream));
}

}  // extern "C"
