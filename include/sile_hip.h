/*
 * sile_hip.h -- C ABI of libsile_hip.so, the MI355X (gfx950) execution path
 * for sile's tile kernels.
 *
 * Plain C: pointers, sizes and status codes only.  Every entry point returns
 * an int status (SILE_OK = 0); on failure sile_hip_last_error() gives the
 * message.  This is the surface a Rust `HipBackend` in crates/sile-backend
 * binds through FFI, beside the CPU and Metal runtimes
 * (crates/sile-backend/src/cpu/mod.rs:14-145, crates/sile-backend/src/metal/mod.rs:11-172).
 *
 * Device pointers are HBM addresses from sile_hip_malloc.  Streams are HIP
 * streams (NULL = the device's default stream).  The sile_hip_kernel_* entry
 * points keep the reference's apply() contract and return after the work has
 * completed; the op entry points (sile_hip_gemm, sile_hip_softmax_rows,
 * sile_hip_reduce_rows, sile_hip_flash_attn_fwd) only enqueue on the stream.
 */
#ifndef SILE_HIP_H
#define SILE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1..5 map 1:1 onto sile_core::Error
 * (crates/sile-core/src/error.rs:1-13); SILE_ERR_RUNTIME is a HIP runtime
 * failure after validation (a Rust binding reports it as Error::Compile with
 * the message, the variant the reference uses for backend failures,
 * crates/sile-backend/src/cpu/mod.rs:86-102). */
enum {
  SILE_OK = 0,
  SILE_ERR_INVALID_DEVICE = 1,      /* Error::InvalidDevice: bad ordinal / SILE_DEVICE value */
  SILE_ERR_UNSUPPORTED_BACKEND = 2, /* Error::UnsupportedBackend: no GPU, unsupported dtype/layout */
  SILE_ERR_COMPILE = 3,             /* Error::Compile: code object load or symbol lookup failed */
  SILE_ERR_IO = 4,                  /* Error::Io */
  SILE_ERR_SHAPE = 5,               /* Error::Shape: bad or non-divisible shape, grid not set */
  SILE_ERR_RUNTIME = 6              /* HIP runtime error during copy / launch / sync */
};

/* Element types.  The reference knows only f32 (crates/sile-hir/src/types.rs:11-14,
 * crates/sile-core/src/kernel.rs:8-14); the 16-bit and fp8 types are additive. */
typedef enum {
  SILE_F32 = 0,
  SILE_F16 = 1,
  SILE_BF16 = 2,
  SILE_F8E4M3 = 3 /* OCP e4m3fn: finite, max 448 */
} sile_dtype;

/* Matrix layouts of sile_hip_gemm operands. */
typedef enum {
  SILE_ROW_MAJOR = 0, /* element (i, j) at p[i * ld + j] */
  SILE_COL_MAJOR = 1  /* element (i, j) at p[j * ld + i] */
} sile_layout;

/* Row reduce ops: TileIrOp::ReduceMax / ReduceSum (crates/sile-tile-ir/src/ir.rs:128-262). */
typedef enum { SILE_REDUCE_MAX = 0, SILE_REDUCE_SUM = 1 } sile_reduce_op;

typedef void *sile_hip_stream;   /* hipStream_t */
typedef void *sile_hip_event;    /* hipEvent_t */
typedef void *sile_hip_module;   /* hipModule_t */
typedef void *sile_hip_function; /* hipFunction_t */
typedef void *sile_hip_graph;    /* hipGraphExec_t */

typedef struct {
  char name[256];
  char gcn_arch[64];       /* e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t clock_khz;       /* peak engine clock */
  int32_t memory_clock_khz;
  int32_t memory_bus_width;
  int64_t total_global_mem;
  int64_t l2_cache_bytes;
  int64_t lds_per_block;
} sile_hip_device_props;

/* ---- device ------------------------------------------------------------ */

/* Selects device `ordinal` for this thread and loads the gfx950 code objects
 * on it (hipModuleLoadData).  Replaces Device::default()/create_stream for the
 * HIP arm (crates/sile-core/src/device.rs:15-50): no GPU -> UNSUPPORTED_BACKEND,
 * bad ordinal -> INVALID_DEVICE, code object rejected -> COMPILE. */
int sile_hip_init(int ordinal);
int sile_hip_device_count(int *count);
int sile_hip_device_info(int ordinal, sile_hip_device_props *out);
int sile_hip_device_synchronize(void);
/* Message of the last failed call on this thread ("" if none). */
const char *sile_hip_last_error(void);
/* Library version string. */
const char *sile_hip_version(void);

/* ---- HBM memory (the reference only has host Vec<f32> tensors,
 *      crates/sile/src/tensor.rs:27-132; these make them device-resident) -- */
int sile_hip_malloc(void **ptr, size_t bytes);
int sile_hip_free(void *ptr);
int sile_hip_memcpy_htod(void *dst, const void *src, size_t bytes);
int sile_hip_memcpy_dtoh(void *dst, const void *src, size_t bytes);
int sile_hip_memcpy_dtod(void *dst, const void *src, size_t bytes);
int sile_hip_memset(void *dst, int value, size_t bytes);

/* ---- streams and events (Stream is a device tag with a no-op synchronize in
 *      the reference, crates/sile-core/src/stream.rs:3-20) ----------------- */
int sile_hip_stream_create(sile_hip_stream *out);
int sile_hip_stream_destroy(sile_hip_stream stream);
int sile_hip_stream_synchronize(sile_hip_stream stream);
int sile_hip_event_create(sile_hip_event *out);
int sile_hip_event_destroy(sile_hip_event event);
int sile_hip_event_record(sile_hip_event event, sile_hip_stream stream);
int sile_hip_event_synchronize(sile_hip_event event);
int sile_hip_event_elapsed_ms(float *ms, sile_hip_event start, sile_hip_event stop);

/* ---- graphs (no counterpart in the reference, whose launches are host
 *      calls; for callers that replay a fixed sequence of op calls) ---------
 * sile_hip_graph_begin starts capturing `stream` (not the null stream;
 * thread-local mode); op calls on it are then recorded, not run.
 * sile_hip_graph_end stops the capture and instantiates what was recorded.
 * The op entry points record plain kernel launches (sile_hip_gemm leaves out
 * its scratch-using forms under capture); the synchronous calls
 * (sile_hip_launch_tiles and the sile_hip_kernel_* DSL kernels) cannot be
 * captured and fail on a capturing stream. */
int sile_hip_graph_begin(sile_hip_stream stream);
int sile_hip_graph_end(sile_hip_stream stream, sile_hip_graph *out);
int sile_hip_graph_launch(sile_hip_graph graph, sile_hip_stream stream);
int sile_hip_graph_destroy(sile_hip_graph graph);

/* ---- code objects and the generic tile launch --------------------------- */

/* Loads a gfx950 code object (ELF) image: hipModuleLoadData.  Replaces the
 * compile + dlopen step of CpuBackend::execute_compiled_source
 * (crates/sile-backend/src/cpu/mod.rs:56-102); failure -> SILE_ERR_COMPILE. */
int sile_hip_module_load(const void *image, size_t bytes, sile_hip_module *out);
int sile_hip_module_unload(sile_hip_module module);
/* hipModuleGetFunction; a missing symbol -> SILE_ERR_COMPILE (the reference's
 * missing dlsym, crates/sile-backend/src/cpu/mod.rs:96-102). */
int sile_hip_module_get(sile_hip_module module, const char *name, sile_hip_function *out);

/* Launches `fn` with sile's kernel-wrapper convention
 * (crates/sile-backend/src/cpu/codegen.rs:433-555, called as in
 * crates/sile-backend/src/cpu/mod.rs:104-128): one workgroup of
 * `threads_per_program` threads per program, grid[0]*grid[1]*grid[2]
 * programs.  The kernel receives (void **buffers, int64_t num_programs,
 * const int64_t *shapes, int64_t num_shapes) where `buffers` and `shapes` are
 * device copies of the host arrays given here (buffers in kernel-param order,
 * shapes = every arg's dims concatenated).  The kernel applies the
 * `pid < total_tiles` guard itself.  Synchronous, like apply().  The device
 * copies of the tables go into buffers of a per-device pool that the library
 * allocates on demand and reuses (never freed before the process ends). */
int sile_hip_launch_tiles(sile_hip_function fn, void *const *buffers, int64_t num_buffers,
                          const int64_t *shapes, int64_t num_shapes, const uint32_t grid[3],
                          uint32_t threads_per_program, sile_hip_stream stream);

/* sile_hip_launch_tiles without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (serving loops
 * or harnesses that forbid hipMalloc).  Same
 * arguments, semantics and synchronous return as sile_hip_launch_tiles, but
 * the device copies of the buffer and shape tables go into a fixed 4 KiB
 * array of the library (one per device, held until the process ends) rather
 * than into a pooled buffer that sile_hip_launch_tiles allocates when its
 * per-device pool has none free: num_buffers + num_shapes
 * may not exceed 512 (SILE_ERR_SHAPE beyond).  Calls on one device share
 * that array: a call holds it (a per-device lock) from its table copy until
 * its launch has completed, so calls from several host threads run one
 * after another.  The call waits for its launch, so a stream being captured
 * into a graph is refused (SILE_ERR_UNSUPPORTED_BACKEND). */
int sile_hip_launch_tiles_noalloc(sile_hip_function fn, void *const *buffers,
                                  int64_t num_buffers, const int64_t *shapes, int64_t num_shapes,
                                  const uint32_t grid[3], uint32_t threads_per_program,
                                  sile_hip_stream stream);

/* ---- generic code generation for LLIR (sile_llvm_ir::Function) ----
 * `llir_text` is a function in the reference's printed LLIR form
 * (format_llvm_ir, crates/sile-llvm-ir/src/print.rs:6-57).  It is translated
 * to HIP C++ following the CPU backend's C codegen
 * (crates/sile-backend/src/cpu/codegen.rs, crates/sile-backend/src/emit.rs:112-177):
 * a per-program body sile_llvm_ir_<name> and a wrapper sile_kernel_<name>
 * with the (buffers, num_programs, shapes, num_shapes) ABI that derives the
 * tile count and pid -> (gid0, gid1) decode as the CPU wrapper does
 * (crates/sile-backend/src/cpu/codegen.rs:409-555).  The tile plan is given
 * by the caller: the output parameter's index and the tile's rows and cols,
 * the result of crates/sile-backend/src/emit.rs:241-296 infer_tile_plan;
 * plan_output_param < 0 selects the CPU wrapper's fallbacks.  This is the
 * codegen half of CodegenTarget / BackendArtifact
 * (crates/sile-backend/src/lib.rs:11-26) for a HIP target.  The buffer
 * parameters are emitted restrict-qualified: as for the DSL's tensors (`&T`
 * inputs, `&mut T` outputs, crates/sile-core/src/kernel.rs:8-14), a buffer a
 * kernel writes must not overlap any other buffer argument of the launch. */

/* Writes the generated HIP source (NUL-terminated) into out[out_capacity];
 * *out_len receives its length.  Parse errors -> SILE_ERR_COMPILE.  Needs no
 * GPU. */
int sile_hip_llir_to_hip(const char *llir_text, int64_t plan_output_param, int64_t plan_rows,
                         int64_t plan_cols, char *out, size_t out_capacity, size_t *out_len);
/* Translates and compiles for gfx950 with hiprtc (as the CPU backend runs cc
 * on every launch, crates/sile-backend/src/cpu/mod.rs:48-134).  *code_out is a
 * malloc'd code object of *code_bytes bytes for sile_hip_module_load (free it
 * with sile_hip_llir_free_code); kernel_name receives "sile_kernel_<name>".
 * Compiler errors -> SILE_ERR_COMPILE with the log and the source.  Needs no
 * GPU. */
int sile_hip_llir_compile(const char *llir_text, int64_t plan_output_param, int64_t plan_rows,
                          int64_t plan_cols, void **code_out, size_t *code_bytes,
                          char *kernel_name, size_t name_capacity);
void sile_hip_llir_free_code(void *code);
/* Launches a generated sile_kernel_<name>: grid[0]*grid[1]*grid[2] programs.
 * A function with a counted loop of at least 256 iterations that lanes can
 * split (sums, max folds, stores one element per iteration) runs one program
 * per workgroup of 1024 lanes with those loops spread over the lanes, as the
 * Metal template runs one program per threadgroup
 * (crates/sile-backend/src/metal/mod.rs:146-154); any other function runs
 * one program per lane, 64 per workgroup (the CPU backend runs one program
 * per thread, crates/sile-backend/src/cpu/codegen.rs:517-551).  The kernel's
 * workgroup size tells the launch which.  Arguments as
 * sile_hip_launch_tiles.  Synchronous. */
int sile_hip_launch_llir(sile_hip_function fn, void *const *buffers, int64_t num_buffers,
                         const int64_t *shapes, int64_t num_shapes, const uint32_t grid[3],
                         sile_hip_stream stream);

/* ---- the DSL kernels on the hot path, with the sile_kernel_<name> ABI ----
 * Same arguments as the generated `void sile_kernel_<name>(void **buffers,
 * int64_t num_threadgroups, int64_t threads_per_group, const int64_t *shapes,
 * int64_t num_shapes)` (crates/sile-backend/src/cpu/codegen.rs:448-454), plus
 * the kernel's const generics, plus a stream.  `buffers` holds DEVICE
 * pointers; `shapes` is a HOST array.  num_threadgroups = grid.x*grid.y*grid.z;
 * threads_per_group must be 1 (LLVM-IR mode, crates/sile-backend/src/cpu/mod.rs:109-120).
 * Each program runs as one workgroup; programs with pid >= total_tiles do
 * nothing.  Synchronous. */

/* matmul<BM,BN,BK> of crates/sile/tests/backend_matmul.rs:3-19:
 * buffers {a, b, c} f32; shapes = shape(a) ++ shape(b) ++ shape(c) (6 values).
 * Bit-identical to the CPU backend (canonical matmul order,
 * crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:24-444). */
int sile_hip_kernel_matmul(void *const *buffers, int64_t num_threadgroups,
                           int64_t threads_per_group, const int64_t *shapes, int64_t num_shapes,
                           int64_t bm, int64_t bn, int64_t bk, sile_hip_stream stream);

/* softmax<BM,BN> of crates/sile/tests/backend_softmax.rs:3-15:
 * buffers {x, y} f32; shapes = shape(x) ++ shape(y) (4 values). */
int sile_hip_kernel_softmax(void *const *buffers, int64_t num_threadgroups,
                            int64_t threads_per_group, const int64_t *shapes, int64_t num_shapes,
                            int64_t bm, int64_t bn, sile_hip_stream stream);

/* parallel_reduce<TILE> of crates/sile/examples/parallel_reduce.rs:3-9
 * (test crates/sile/tests/backend_parallel_reduce.rs:3-9): buffers {a, out} f32;
 * shapes = shape(a) ++ shape(out) (2 values).  out[0] += tile sums atomically.
 * `partials` (device, may be NULL) receives each program's tile sum. */
int sile_hip_kernel_parallel_reduce(void *const *buffers, int64_t num_threadgroups,
                                    int64_t threads_per_group, const int64_t *shapes,
                                    int64_t num_shapes, int64_t tile, float *partials,
                                    sile_hip_stream stream);

/* ---- op entry points (asynchronous on `stream`) ------------------------- */

/* C[M,N] = (scale_a * scale_b) * A . B, fp32 accumulation; the tile op MmaF of
 * the canonical matmul (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:24-444,
 * crates/sile-tile-ir/src/ir.rs:128-262).  k runs over K' = (K / bk) * bk
 * (bk <= 0: K' = K), the reference's K truncation.
 * Supported:
 *   f32  x f32  -> f32 : any shape/layout of B, A row-major; exact canonical order
 *                        (bit-identical to the CPU backend).
 *   bf16 x bf16 -> bf16|f32, f16 x f16 -> f16|f32, f8e4m3 x f8e4m3 -> bf16|f32:
 *                        A row-major, B column-major ([N, K]) or row-major
 *                        ([K, N], the canonical matmul's own layout,
 *                        canonical_matmul.rs:55-57), any M, N, K', A and a
 *                        column-major B (and their leading dimensions)
 *                        16-byte aligned.  A row-major 16-bit B runs the LDS
 *                        kernels with transposed fragment reads when N is a
 *                        multiple of 8, B's rows are 16-byte aligned and the
 *                        shape takes the direct form below; any other
 *                        row-major B (and every fp8 one) is first written
 *                        column-major into a second device scratch buffer
 *                        (at most 256 MiB; not under graph capture).  MFMA
 *                        path (N a multiple of 4, C's rows 16-byte aligned
 *                        and N >= 128, any M: 256 x 256 or 128 x 128 tiles
 *                        through LDS,
 *                        the size chosen by shape; when C cannot take the
 *                        tiles' stores but M is a multiple of 4 and at least
 *                        one tile, the same kernels compute C^T into fp32
 *                        scratch and a second kernel writes C; other shapes:
 *                        64 x 64 tiles).
 * When the tiles are fewer than the device's CUs and K' is long, K' may be
 * split into ranges computed side by side: their fp32 partial C planes go
 * to a device scratch buffer shared by all calls on the device (allocated on
 * the first such call, grown when a call needs more, at most
 * 4 * (CUs * 65536) bytes for the split chosen by shape and 256 MiB for
 * any form; calls on different streams are ordered on the GPU by an event)
 * and a second kernel adds them in range order.  The result
 * does not depend on the stream or on earlier calls (outside graph capture,
 * below).  The transposed form
 * (above) keeps all of C^T there, up to 256 MiB (larger: 64 x 64 tiles).
 * On a stream that is being captured into a graph neither form is used (no
 * split; the 64 x 64 kernel instead of the transposed form), so a captured
 * call is plain kernel launches.
 * M = 0 or N = 0: nothing is written.  K' = 0 (K below one bk): C = +0.0 for
 * any M, N and supported types, as the canonical matmul's sums start at 0.0f
 * and add no term (canonical_matmul.rs:58-73).
 * Anything else -> SILE_ERR_UNSUPPORTED_BACKEND or SILE_ERR_SHAPE. */
int sile_hip_gemm(sile_dtype a_type, sile_dtype b_type, sile_dtype c_type, int64_t m, int64_t n,
                  int64_t k, const void *a, int64_t lda, sile_layout a_layout, const void *b,
                  int64_t ldb, sile_layout b_layout, void *c, int64_t ldc, float scale_a,
                  float scale_b, int64_t bk, sile_hip_stream stream);

/* sile_hip_gemm with the tile size and the K split chosen by the caller
 * instead of by shape.  No counterpart in the reference; for tests that must
 * reach each kernel and for tuning.  tile: 0 (by shape), 256 or 128; a
 * forced size the shape cannot take (N below it, M below 256 for 256, N not
 * a multiple of 4, C's rows not 16-byte aligned) -> SILE_ERR_SHAPE.  splits:
 * 0 (by shape) or 1 .. 64 ranges of K' (fewer when K' has fewer whole
 * k-steps); a split needs splits * M * N * 4 bytes of the device scratch,
 * and a forced split beyond 256 MiB of it -> SILE_ERR_SHAPE. */
int sile_hip_gemm_tiled(sile_dtype a_type, sile_dtype b_type, sile_dtype c_type, int64_t m,
                        int64_t n, int64_t k, const void *a, int64_t lda, sile_layout a_layout,
                        const void *b, int64_t ldb, sile_layout b_layout, void *c, int64_t ldc,
                        float scale_a, float scale_b, int64_t bk, int32_t tile, int32_t splits,
                        sile_hip_stream stream);

/* fp32 tile MMA with a seeded accumulator, in the reference's exact order:
 * C[r][c] = the chain s = s + A[r][k] * B[k][c] over k < K' (K' = (K / bk) * bk,
 * bk <= 0: K), the product and the sum rounded separately, starting from
 * s = acc[r * ld_acc + c] (acc != NULL; acc may be C itself, for C += A.B) or
 * from s = acc_value.  This is MmaF lowered with an accumulator that is a
 * loaded tile or a constant splat (crates/sile-tile-ir/src/passes/lowering/tile_compute/mma.rs:25-260,
 * 262-739, seeds at :213-229 and :483-558; plan crates/sile-tile-ir/src/passes/lowering/block.rs:294-377);
 * acc_value = 0.0f with acc = NULL is the canonical matmul.  A row-major
 * [M, K]; B row-major [K, N] or column-major.  Bit-identical to the CPU
 * backend. */
int sile_hip_mma_f32(int64_t m, int64_t n, int64_t k, const float *a, int64_t lda, const float *b,
                     int64_t ldb, sile_layout b_layout, const float *acc, int64_t ld_acc,
                     float acc_value, float *c, int64_t ldc, int64_t bk, sile_hip_stream stream);

/* fp32 matrix-vector product in the order of the matvec DSL kernel
 * (crates/sile/examples/mlp.rs:26-44): out[r] = ((seed + p_0) + p_1) + ...
 * over the tiles t < k / bk of row r, p_t = x[r][t bk] y[t bk] + ... summed in
 * order from the tile's first element (the fused map + reduce,
 * crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:189-293),
 * every product and sum rounded on its own.  x row-major [m, >= k] with row
 * pitch ldx, y [>= (k / bk) bk], out [m]; seed is the accumulator's splat
 * value (0.0f in the example).  Bit-identical to the CPU backend.  The
 * router's matvec route calls it. */
int sile_hip_matvec_f32(int64_t m, int64_t k, int64_t bk, const float *x, int64_t ldx,
                        const float *y, float seed, float *out, sile_hip_stream stream);

/* Row softmax of a [rows, cols] matrix: y = exp(x - max) / sum(exp(x - max))
 * per row with fp32 max/exp/sum (the softmax DSL kernel with BN = cols,
 * crates/sile/tests/backend_softmax.rs:3-15).  in/out dtypes: f16->f16,
 * bf16->bf16, f32->f32, f16->f32. */
int sile_hip_softmax_rows(sile_dtype in_type, sile_dtype out_type, int64_t rows, int64_t cols,
                          const void *x, int64_t ldx, void *y, int64_t ldy,
                          sile_hip_stream stream);

/* out[r] = max_c x[r][c] or sum_c x[r][c] in fp32 (ReduceMax/ReduceSum along
 * axis 1, crates/sile-tile-ir/src/passes/lowering/tile_compute/reduce.rs:10-112).
 * in: f32, f16, bf16.  `out` is fp32 [rows].  The max is the reference's
 * fold acc = x0; acc = x > acc ? x : acc bit for bit: a NaN in column 0
 * gives NaN, NaNs elsewhere never enter, and of a +0 / -0 tie the first in
 * row order is kept (cols < 2^31).  The sum is a tree, within fp32 rounding
 * of the reference's order (sile_hip_reduce_rows_fused_sum keeps that order
 * bit for bit). */
int sile_hip_reduce_rows(sile_reduce_op op, sile_dtype in_type, int64_t rows, int64_t cols,
                         const void *x, int64_t ldx, float *out, sile_hip_stream stream);

/* y[r][0, row_bytes) = x[r][0, row_bytes) for r < rows, rows at byte pitches
 * ldx_bytes / ldy_bytes: the HBM move of a tile store
 * (crates/sile-tile-ir/src/passes/lowering/tile_memory.rs:114-162) with no
 * arithmetic, in the row softmax's access pattern (one wave per row,
 * non-temporal 16-byte accesses when rows and pitches are multiples of 16
 * bytes); the read + write rate it reaches bounds the row softmax's. */
int sile_hip_copy_rows(int64_t rows, int64_t row_bytes, const void *x, int64_t ldx_bytes,
                       void *y, int64_t ldy_bytes, sile_hip_stream stream);

/* y[r][c] = value (rounded to nearest even for f16 / bf16) for r < rows,
 * c < cols, rows at pitch ldy elements: the store of a splat tile, DSL
 * `y.store(sile::constant(value, [BM, BN]))` (Splat,
 * crates/sile-tile-ir/src/lower.rs:509-524, stored by
 * crates/sile-tile-ir/src/passes/lowering/tile_memory.rs:114-162).  type:
 * f32, f16, bf16.  Write-only: contiguous 16-byte aligned rows are written in
 * the copy's shape (non-temporal 16-byte stores), the rate that bounds the
 * write half of the row softmax. */
int sile_hip_fill_rows(sile_dtype type, int64_t rows, int64_t cols, float value, void *y,
                       int64_t ldy, sile_hip_stream stream);

/* fp32 row sums in the order of the reference's fused load + reduce: the
 * CPU backend's sum of a tile it reads straight from a buffer
 * (crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:31-177,
 * 1142-1256), bit-identical to it.  4-element windows ((v0+v1)+v2)+v3 in
 * order; for cols > 16 a step-4 loop from 0.0f while idx < cols, whose last
 * window for cols % 4 != 0 reads the buffer's next elements past the row,
 * then a scalar tail from 4*(cols/4).  x_len (>= (rows-1)*ldx + cols) is the
 * number of elements of the buffer from x on; window elements past it are
 * taken as 0.0f, where the reference reads past its buffer.  The router's
 * row-sum route runs on this entry point. */
int sile_hip_reduce_rows_fused_sum(int64_t rows, int64_t cols, const float *x, int64_t ldx,
                                   int64_t x_len, float *out, sile_hip_stream stream);

/* fp32 attention with K given transposed, the attention program of sile's
 * DSL: per query row, over keys 0 .. n_k - 1 in order, s = (q . kt[:, j]) *
 * scale, an online softmax whose running max starts at m0 and is updated as
 * m_new = m >= rowmax ? m : rowmax, o = (sum_j p_j v[j]) / l.  No single
 * counterpart in the reference: it composes the ops the DSL program uses
 * (mma, tile_compute/mma.rs:25-739; max_tile, crates/sile-tile-ir/src/lower.rs:619-641;
 * reduce_max / reduce_sum, tile_compute/reduce.rs:10-112; exp, broadcast and
 * the pointwise maps, tile_expr.rs:646-813) and is the kernel the Tile IR
 * router sends that program to.  q [n_q, ldq], kt [head_dim, ldkt] (key j,
 * dim t at kt[t * ldkt + j]), v [n_k, ldv], o [n_q, ldo]; head_dim <= 128;
 * results within fp32 rounding of the program (sums in another order; exp
 * is the device's). */
int sile_hip_attention_f32_kt(int64_t n_q, int64_t n_k, int64_t head_dim, const float *q,
                              int64_t ldq, const float *kt, int64_t ldkt, const float *v,
                              int64_t ldv, float *o, int64_t ldo, float scale, float m0,
                              sile_hip_stream stream);

/* Flash-attention forward, O = softmax(Q K^T * scale [+ causal mask]) V with
 * fp32 online-softmax state.  Q, K, V, O are [B, H, S, D] contiguous, f16 or
 * bf16, any S.  D a multiple of 16 up to 256 with 16-byte aligned operands
 * runs on the matrix cores; other D up to 256 (or unaligned operands) on a
 * VALU kernel of one wave per query row.  No reference counterpart: sile's DSL
 * cannot express attention (no mask/iota/transpose); built from the Tile IR
 * ops MmaF, ReduceMax, Exp, ReduceSum (crates/sile-tile-ir/src/ir.rs:128-262). */
int sile_hip_flash_attn_fwd(sile_dtype dtype, int64_t batch, int64_t heads, int64_t seq_len,
                            int64_t head_dim, const void *q, const void *k, const void *v,
                            void *o, float scale, int causal, sile_hip_stream stream);

/* ---- pattern router: Tile IR -> hand-written kernels ---------------------
 * Generalises the reference's canonical-matmul detector
 * (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:446-666) to
 * the other tile patterns of the hot path.  The input is a kernel in the
 * printed Tile IR form (format_tile_ir, crates/sile-tile-ir/src/print.rs:5-354)
 * after or before the default Tile IR passes
 * (crates/sile-tile-ir/src/passes/mod.rs:31-42), which
 * crates/sile/src/compiler.rs compile_kernel_to_llvm_ir returns beside the
 * LLIR.  A HipBackend calls the router first and lowers to LLIR
 * (sile_hip_llir_compile) only on SILE_ROUTE_NONE. */
typedef enum {
  SILE_ROUTE_NONE = 0,          /* no hand-written kernel: use the LLIR code generation */
  SILE_ROUTE_MATMUL = 1,        /* canonical matmul, or the tile MMA loop from a splat or a
                                   loaded accumulator -> the matmul tile kernel (bit-identical) */
  SILE_ROUTE_SOFTMAX_ROWS = 2,  /* softmax chain, one tile per row band -> sile_hip_softmax_rows */
  SILE_ROUTE_SOFTMAX_TILES = 3, /* softmax chain, other tilings -> sile_hip_kernel_softmax */
  SILE_ROUTE_REDUCE_ROWS = 4,   /* load + reduce(axis 1) + store -> sile_hip_reduce_rows */
  SILE_ROUTE_ATOMIC_REDUCE = 5, /* load + sum + extract + atomic add -> sile_hip_kernel_parallel_reduce */
  SILE_ROUTE_ATTENTION = 6,     /* the DSL's online-softmax attention loop (K transposed)
                                   -> sile_hip_attention_f32_kt */
  SILE_ROUTE_MATVEC = 7         /* the matvec loop (acc + reduce_sum(x tile * broadcast(y tile)))
                                   -> sile_hip_matvec_f32 */
} sile_route_kind;

typedef struct {
  int32_t kind;              /* sile_route_kind */
  int32_t reduce_op;         /* SILE_ROUTE_REDUCE_ROWS: sile_reduce_op */
  int32_t buffer[4];         /* kernel-parameter index of each operand: inputs, then output,
                                then (matmul) the buffer the accumulator tile is loaded from */
  int32_t shape_offset[4];   /* offset of each operand's dims in `shapes` */
  int32_t rank[4];           /* rank of each operand (0: unused) */
  int32_t num_buffers;       /* buffer parameters of the kernel */
  int32_t seed_from_tile;    /* SILE_ROUTE_MATMUL: 1 = accumulator loaded from operand 3 */
  float seed_value;          /* SILE_ROUTE_MATMUL / MATVEC: the accumulator's splat value
                                (matmul: when seed_from_tile is 0) */
  float attn_scale;          /* SILE_ROUTE_ATTENTION: the score scale (1 without one) */
  float attn_m0;             /* SILE_ROUTE_ATTENTION: the running max's initial value */
  int64_t num_shapes;        /* shape values the route was made with */
  int64_t operand_shapes[8]; /* the operands' dims the route was made for */
  int64_t num_threadgroups;  /* the grid the route was made for */
  int64_t tile_m, tile_n, tile_k; /* BM, BN, BK (TILE in tile_n for the atomic reduce;
                                      BM, BN, D for attention; BM, -, BK for matvec) */
  int64_t rows, cols;        /* extents handed to the row kernels; attention: queries, keys;
                                matvec: rows, K */
  char reason[512];          /* SILE_ROUTE_NONE: why each detector declined */
} sile_hip_route;

/* Parses `tile_ir_text` and picks the kernel for a launch of num_threadgroups
 * programs over buffers of the given shapes (every buffer parameter's dims,
 * concatenated in parameter order, as for sile_kernel_<name>).  A pattern is
 * routed only where the kernel writes exactly the tiles that the CPU
 * backend's wrapper writes (crates/sile-backend/src/cpu/codegen.rs:409-555).
 * Malformed text -> SILE_ERR_COMPILE; a kernel without a route is SILE_OK
 * with kind SILE_ROUTE_NONE.  Needs no GPU. */
int sile_hip_tile_ir_route(const char *tile_ir_text, const int64_t *shapes, int64_t num_shapes,
                           int64_t num_threadgroups, sile_hip_route *out);
/* Runs a route on device buffers (kernel parameter order) with the shapes and
 * grid it was made for.  Synchronous, like the sile_kernel_<name> launches. */
int sile_hip_tile_ir_launch(const sile_hip_route *route, void *const *buffers,
                            int64_t num_buffers, const int64_t *shapes, int64_t num_shapes,
                            int64_t num_threadgroups, sile_hip_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* SILE_HIP_H */
