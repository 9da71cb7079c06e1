// sile_hip_launch_tiles_noalloc: the generic tile launch for callers that
// cannot allocate device memory (serving loops or harnesses that forbid
// hipMalloc).  sile_hip_launch_tiles copies the buffer-pointer
// and shape tables into a device buffer from a per-device pool, which it
// allocates (hipMalloc) whenever no pooled buffer is free or large enough;
// this variant copies them into `scratch`, a fixed device array of this
// library that lives until the process ends, and calls no allocating routine.
//
// Compiled by hipcc (host and device), so that `scratch` is a device symbol of
// this file: each device holds its own copy at its own address, which
// hipGetSymbolAddress returns once per device (at sile_hip_init, or at the
// first call on a device).  Host code uses only that address; the name
// `scratch` on the host is a stand-in, not a device address.
#include <hip/hip_runtime.h>

#include <cstring>
#include <mutex>

#include "runtime_internal.h"

// Room for the tables of one launch: 8-byte buffer pointers followed by the
// 8-byte shape values, at most kNoallocTableEntries entries together.
constexpr size_t kNoallocScratchBytes = 4096;
constexpr int64_t kNoallocTableEntries = kNoallocScratchBytes / 8;

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device
// Held by a call from the table copy until its launch has completed, so calls
// from several host threads on one device take the shared array in turn.
std::mutex g_call_mu[kMaxDevices];

}  // namespace

namespace sile_rt {

// The current device's address of `scratch`, looked up once per device;
// *dev_out is the current device.
int noalloc_scratch(void** out, int* dev_out) {
  int dev = 0;
  SILE_HIP_CHECK(hipGetDevice(&dev));
  if (dev_out) *dev_out = dev;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(SILE_ERR_INVALID_DEVICE, "device %d beyond the %d the scratch table covers", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SILE_OK;
}

}  // namespace sile_rt

using namespace sile_rt;

extern "C" int sile_hip_launch_tiles_noalloc(sile_hip_function fn, void* const* buffers,
                                             int64_t num_buffers, const int64_t* shapes,
                                             int64_t num_shapes, const uint32_t grid[3],
                                             uint32_t threads_per_program,
                                             sile_hip_stream stream) {
  if (!fn) return fail(SILE_ERR_COMPILE, "function is NULL");
  if (!grid) return fail(SILE_ERR_SHAPE, "grid not set");
  if (num_buffers < 0 || num_shapes < 0 || (num_buffers && !buffers) || (num_shapes && !shapes))
    return fail(SILE_ERR_SHAPE, "buffers/shapes arrays do not match their counts");
  if (num_buffers + num_shapes > kNoallocTableEntries)
    return fail(SILE_ERR_SHAPE,
                "%lld buffers + %lld shape values exceed the %lld table entries (%zu bytes) of "
                "the no-allocation launch",
                (long long)num_buffers, (long long)num_shapes, (long long)kNoallocTableEntries,
                kNoallocScratchBytes);
  if (threads_per_program == 0 || threads_per_program > 1024)
    return fail(SILE_ERR_SHAPE, "threads_per_program %u not in [1, 1024]", threads_per_program);
  const int64_t programs = (int64_t)grid[0] * grid[1] * grid[2];
  if (programs > 0x7fffffffLL)
    return fail(SILE_ERR_SHAPE, "too many programs (%lld)", (long long)programs);
  if (programs == 0) return ok();
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The call waits for its launch (a capturing stream cannot be waited on) and
  // copies its tables from the stack (a captured copy would read them again
  // after the call returned): both rule out graph capture.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  SILE_HIP_CHECK(hipStreamIsCapturing(s, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND,
                "the no-allocation launch is synchronous and cannot run on a capturing stream");
  void* table = nullptr;
  int dev = 0;
  int rc = noalloc_scratch(&table, &dev);
  if (rc != SILE_OK) return rc;
  std::lock_guard<std::mutex> lk(g_call_mu[dev]);
  // host image of the tables on the stack (no heap allocation either)
  unsigned char host[kNoallocScratchBytes];
  const size_t buf_bytes = (size_t)num_buffers * sizeof(void*);
  const size_t shp_bytes = (size_t)num_shapes * sizeof(int64_t);
  if (buf_bytes) memcpy(host, buffers, buf_bytes);
  if (shp_bytes) memcpy(host + buf_bytes, shapes, shp_bytes);
  if (buf_bytes + shp_bytes)
    SILE_HIP_CHECK(hipMemcpyAsync(table, host, buf_bytes + shp_bytes, hipMemcpyHostToDevice, s));
  void* dev_buffers = table;
  void* dev_shapes = static_cast<unsigned char*>(table) + buf_bytes;
  int64_t np = programs, ns = num_shapes;
  void* params[] = {&dev_buffers, &np, &dev_shapes, &ns};
  SILE_HIP_CHECK(hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), (unsigned)programs, 1, 1,
                                       threads_per_program, 1, 1, 0, s, params, nullptr));
  // synchronous, like sile_hip_launch_tiles: the host image on the stack and
  // the shared tables are done with when this returns
  SILE_HIP_CHECK(hipStreamSynchronize(s));
  return ok();
}
