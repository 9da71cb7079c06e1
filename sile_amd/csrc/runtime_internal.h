// Internal interface between the runtime (runtime.cpp) and the op entry
// points (ops.cpp) of libsile_hip.so.  Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/sile_hip.h"

namespace sile_rt {

// Records `msg` as this thread's last error and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the last error and returns SILE_OK.
int ok();
// Maps a HIP error to SILE_ERR_RUNTIME with the call site in the message.
int hip_fail(hipError_t e, const char* what);

#define SILE_HIP_CHECK(expr)                                     \
  do {                                                           \
    hipError_t _e = (expr);                                      \
    if (_e != hipSuccess) return ::sile_rt::hip_fail(_e, #expr); \
  } while (0)

// The gfx950 code objects built into the library.
enum class Module : int {
  kDsl = 0,
  kSoftmax = 1,
  kGemm = 2,
  kAttention = 3,
  kFlashAttn = 4,
  kCount = 5
};

// Makes sure the current device is initialised and its code objects are
// loaded; returns a status.
int ensure_device();
// Looks up `name` in the given embedded module on the current device.
int get_function(Module m, const char* name, hipFunction_t* out);
// Number of workgroups of `block_threads` threads of kernel `name` that fit on
// the whole current device at once (CUs x resident workgroups per CU).
int resident_blocks(Module m, const char* name, int block_threads, int64_t* out);
// The current device's address of the no-allocation launch's table array
// (launch_noalloc.hip); looked up once per device.
int noalloc_scratch(void** out, int* dev_out);
// The matmul DSL kernel with the sile_kernel_<name> tile semantics
// (buffers a, b, c; shapes of a, b, c: 6 values), each cell's chain seeded
// from `seed` (an accumulator source of shape seed_shape[2], the same tile of
// it as of c) or, when seed is NULL, from seed_value.  Synchronous.
int kernel_matmul_seeded(void* const* buffers, int64_t num_threadgroups, int64_t threads_per_group,
                         const int64_t* shapes, int64_t bm, int64_t bn, int64_t bk,
                         const float* seed, const int64_t* seed_shape, float seed_value,
                         hipStream_t s);
// Device scratch shared by the calls on one device, in two slots: slot 0 the
// split-K GEMM's fp32 partials and the transposed form's planes, slot 1 a
// row-major B transposed for the column-major kernels (each at most
// 256 MiB).  scratch_acquire makes stream s wait for the kernels of the
// slot's previous user (an event, so calls on different streams are ordered
// on the GPU, not on the host), and returns at least `bytes` of it; the
// caller launches its kernels on s and then calls scratch_release, which
// records the event on s.  The slot's lock is held in between; a caller
// holding both takes slot 1 first.  The memory is allocated on first use and
// grows when a call needs more.
constexpr int kScratchSlots = 2;
int scratch_acquire(size_t bytes, hipStream_t s, void** out, int slot = 0);
void scratch_release(hipStream_t s, int slot = 0);
// hipModuleLaunchKernel with kernelParams.
int launch(Module m, const char* name, dim3 grid, dim3 block, void** params, hipStream_t stream,
           size_t dynamic_lds = 0);

}  // namespace sile_rt
