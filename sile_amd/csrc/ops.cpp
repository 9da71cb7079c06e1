// Op entry points of libsile_hip: argument validation on the host, then one
// launch of the matching gfx950 kernel.  Every shape the kernels index with is
// checked here first, so a launch never addresses memory outside the buffers
// the caller described.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "runtime_internal.h"

using namespace sile_rt;

namespace {

// The exact-order fp32 GEMM: the largest tile (128, 64 or 32) that still gives
// about 1024 workgroups (4 per CU), or 32.
int launch_f32_exact(bool b_col_major, const void* a, const void* b, void* c, int64_t m,
                     int64_t n, int64_t kp, int64_t lda, int64_t ldb, int64_t ldc,
                     const float* seed, int64_t ld_seed, float seed_value, hipStream_t s);

// Kernel argument blocks; layouts match the structs in kernels/*.hip.
struct MatmulTileArgs {
  int64_t lda, ldb, ldc, bm, bn, bk, tiles_n, total;
  const float* seed;
  int64_t ld_seed;
  float seed_value;
};
struct SoftmaxTileArgs {
  int64_t ldx, ldy, bm, bn, tiles_n, total;
};
struct ReduceTileArgs {
  int64_t tile, total, len;
};
struct GemmArgs {
  int64_t lda, ldb, ldc;
  int32_t tiles_m, tiles_n, k_steps;
  float alpha;
  int32_t m, n;
  int32_t k_rem;  // elements of the last half k-step inside K'
  int32_t split_steps;  // half k-steps per k-range (even, or k_steps unsplit)
  int64_t c_split;      // elements between the fp32 C planes of the k-ranges
  int64_t b_rows;       // B row-major: rows of B's buffer
};

// Tile size and K split of the LDS GEMM kernels: the pair that minimises a
// time model fitted to measurements on MI355X (forced tile sizes and split
// counts over bf16 shapes from 1024^3 to 256 x 8192 x 8192):
//   a tile over k elements of K' takes k * t(w) + 6 us (4.7 us for 128 x
//   128), where t depends on the tile size and on how many workgroups w run
//   at once (the clock drops as more CUs draw power; two 128 x 128
//   workgroups share a CU); half that for fp8; workgroups
//   beyond what the device holds at once run in further rounds;
//   a split of K' into S ranges (at least 8 whole k-steps each, all ranges
//   resident at once) adds the burst of fp32 planes the workgroups write as
//   they finish, the second launch reading them and writing C (both at
//   5.2 TB/s), and 4 us of launch and ordering; it is taken only for a
//   modelled gain above 5 %.
// Largest fp32 planes a GEMM keeps in the device scratch: the transposed
// form's and a forced split's are checked against it; the split the planner
// chooses stays below 4 * CUs * 65536 bytes (64 MiB) by construction.
constexpr int64_t kScratchPlanesMax = 256ll << 20;

struct GemmPlan {
  int tile;        // 256 or 128
  int64_t splits;  // k-ranges (1: K' not split)
};

// seconds per element of K' for one tile, with w workgroups of that size
// running at once on `cus` CUs (fitted: 256 x 256 16 ns up to cus / 2
// workgroups, 21.8 ns at cus; 128 x 128 7.2 ns up to cus / 2, 7.8 ns at cus,
// 13.3 ns at 2 cus, two sharing each CU)
double tile_time_per_k(int tile, int64_t w, int cus) {
  const double half = cus / 2.0;
  const double f = std::min(1.0, std::max(0.0, ((double)w - half) / half));
  if (tile == 256) return 16e-9 + 5.8e-9 * f;
  if (w <= cus) return 7.2e-9 + 0.6e-9 * f;
  return 7.8e-9 + 5.5e-9 * std::min(1.0, (double)(w - cus) / cus);
}

GemmPlan gemm_plan(int64_t m, int64_t n, int64_t kp, int64_t half_steps, int64_t cb, bool fp8,
                   int only_tile) {
  GemmPlan best{only_tile ? only_tile : m >= 256 && n >= 256 ? 256 : 128, 1};
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return best;
  double best_t = 1e30, best_unsplit_t = 1e30;
  GemmPlan best_unsplit = best;
  for (int tile : {256, 128}) {
    if ((tile == 256 && m < tile) || n < tile || (only_tile && tile != only_tile)) continue;
    const int64_t tiles = ((m + tile - 1) / tile) * ((n + tile - 1) / tile);
    const int64_t slots = (int64_t)cus * (tile == 256 ? 1 : 2);
    const int64_t max_splits = std::min<int64_t>(slots / tiles, half_steps / 16);
    for (int64_t sp = 1; sp == 1 || sp <= max_splits; ++sp) {
      // full rounds of `slots` workgroups, then the rest
      const int64_t w = tiles * sp, full = w / slots, rest = w % slots;
      const double per_k = (double)full * tile_time_per_k(tile, slots, cus) +
                           (rest ? tile_time_per_k(tile, rest, cus) : 0.0);
      double t = per_k * (double)((kp + sp - 1) / sp) * (fp8 ? 0.5 : 1.0) +
                 (tile == 256 ? 6e-6 : 4.7e-6);
      if (sp > 1) {
        const double planes = 4.0 * (double)sp * (double)m * (double)n;
        t += (2 * planes + (double)(cb * m * n)) / 5.2e12 + 4e-6;
      }
      if (sp == 1 && t < best_unsplit_t) {
        best_unsplit_t = t;
        best_unsplit = {tile, 1};
      }
      if (t < best_t) {
        best_t = t;
        best = {tile, sp};
      }
    }
  }
  return best.splits > 1 && !(best_t < 0.95 * best_unsplit_t) ? best_unsplit : best;
}

// fp32 -> 16-bit element bits, round to nearest even (NaN stays a quiet NaN),
// for fill values converted on the host.
uint32_t bf16_bits_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (x >> 16) | 0x40u;
  return (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
}
uint32_t f16_bits_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;
  if (ax >= 0x477ff000u) return sign | 0x7c00u;  // |f| >= 65520 rounds to inf
  if (ax < 0x38800000u) {                        // below 2^-14: subnormal (exact scaling)
    float v;
    memcpy(&v, &ax, 4);
    return sign | (uint32_t)nearbyintf(v * 16777216.0f);
  }
  uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return sign | h;
}

const char* dtype_name(int t) {
  switch (t) {
    case SILE_F32: return "f32";
    case SILE_F16: return "f16";
    case SILE_BF16: return "bf16";
    case SILE_F8E4M3: return "f8e4m3";
    default: return "?";
  }
}

size_t dtype_bytes(int t) {
  switch (t) {
    case SILE_F32: return 4;
    case SILE_F16:
    case SILE_BF16: return 2;
    case SILE_F8E4M3: return 1;
    default: return 0;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Programs that execute a body: min(num_threadgroups * threads_per_group, total),
// since programs with pid >= total_tiles are skipped by the wrapper guard
// (crates/sile-backend/src/cpu/codegen.rs:517-531).
int programs_to_run(int64_t num_threadgroups, int64_t threads_per_group, int64_t total,
                    int64_t* out) {
  if (num_threadgroups < 0 || threads_per_group < 1)
    return fail(SILE_ERR_SHAPE, "num_threadgroups %lld / threads_per_group %lld invalid",
                (long long)num_threadgroups, (long long)threads_per_group);
  const int64_t launched = num_threadgroups * threads_per_group;
  *out = std::max<int64_t>(0, std::min(launched, total));
  if (*out > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many programs");
  return SILE_OK;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// DSL kernels (sile_kernel_<name> ABI)
// ---------------------------------------------------------------------------

int sile_hip_kernel_matmul(void* const* buffers, int64_t num_threadgroups,
                           int64_t threads_per_group, const int64_t* shapes, int64_t num_shapes,
                           int64_t bm, int64_t bn, int64_t bk, sile_hip_stream stream) {
  if (!buffers || !shapes || num_shapes != 6)
    return fail(SILE_ERR_SHAPE, "matmul expects 3 buffers and 6 shape values (got %lld)",
                (long long)num_shapes);
  return kernel_matmul_seeded(buffers, num_threadgroups, threads_per_group, shapes, bm, bn, bk,
                              nullptr, nullptr, 0.0f, static_cast<hipStream_t>(stream));
}

}  // extern "C"

namespace sile_rt {

int kernel_matmul_seeded(void* const* buffers, int64_t num_threadgroups, int64_t threads_per_group,
                         const int64_t* shapes, int64_t bm, int64_t bn, int64_t bk,
                         const float* seed, const int64_t* seed_shape, float seed_value,
                         hipStream_t s) {
  if (!buffers || !shapes) return fail(SILE_ERR_SHAPE, "NULL buffers / shapes");
  if (bm <= 0 || bn <= 0 || bk <= 0) return fail(SILE_ERR_SHAPE, "BM, BN, BK must be positive");
  const int64_t a0 = shapes[0], a1 = shapes[1], b0 = shapes[2], b1 = shapes[3], c0 = shapes[4],
                c1 = shapes[5];
  if (a0 < 0 || a1 < 0 || b0 < 0 || b1 < 0 || c0 < 0 || c1 < 0)
    return fail(SILE_ERR_SHAPE, "negative extent");
  if (seed && (!seed_shape || seed_shape[0] < 0 || seed_shape[1] < 0))
    return fail(SILE_ERR_SHAPE, "accumulator tile source without a valid shape");
  MatmulTileArgs t{a1, b1, c1, bm, bn, bk, c1 / bn, 0, seed, seed ? seed_shape[1] : 0, seed_value};
  t.total = (c0 / bm) * t.tiles_n;
  int64_t run = 0;
  int rc = programs_to_run(num_threadgroups, threads_per_group, t.total, &run);
  if (rc != SILE_OK) return rc;
  if (run == 0) return ok();
  // Extents the programs touch: rows of a/c up to the last program's row tile,
  // columns of b/c up to the last column tile any program reaches.
  const int64_t kp = (a1 / bk) * bk;
  const int64_t rows_needed = ((run - 1) / t.tiles_n + 1) * bm;
  const int64_t cols_needed = std::min<int64_t>(run, t.tiles_n) * bn;
  if (a0 < rows_needed || b0 < kp || b1 < cols_needed || c0 < rows_needed || c1 < cols_needed)
    return fail(SILE_ERR_SHAPE,
                "matmul shapes a[%lld,%lld] b[%lld,%lld] c[%lld,%lld] do not cover the tiles of "
                "%lld programs (BM=%lld BN=%lld BK=%lld)",
                (long long)a0, (long long)a1, (long long)b0, (long long)b1, (long long)c0,
                (long long)c1, (long long)run, (long long)bm, (long long)bn, (long long)bk);
  if (seed && (seed_shape[0] < rows_needed || seed_shape[1] < cols_needed))
    return fail(SILE_ERR_SHAPE,
                "accumulator source [%lld,%lld] does not cover the tiles of %lld programs",
                (long long)seed_shape[0], (long long)seed_shape[1], (long long)run);
  const void* a = buffers[0];
  const void* b = buffers[1];
  void* c = buffers[2];
  if (run == t.total && (c0 / bm) * bm <= 65535LL * 32) {
    // every tile runs: the tiles form the rectangle [0, M') x [0, N') of C,
    // computed by the register-tiled kernel in the same per-cell order
    rc = launch_f32_exact(false, a, b, c, (c0 / bm) * bm, t.tiles_n * bn, kp, a1, b1, c1, seed,
                          t.ld_seed, seed_value, s);
    if (rc != SILE_OK) return rc;
    SILE_HIP_CHECK(hipStreamSynchronize(s));
    return ok();
  }
  void* params[] = {&a, &b, &c, &t};
  rc = launch(Module::kDsl, "sile_dsl_matmul_f32", dim3((unsigned)run), dim3(256), params, s);
  if (rc != SILE_OK) return rc;
  SILE_HIP_CHECK(hipStreamSynchronize(s));
  return ok();
}

}  // namespace sile_rt

extern "C" {

int sile_hip_kernel_softmax(void* const* buffers, int64_t num_threadgroups,
                            int64_t threads_per_group, const int64_t* shapes, int64_t num_shapes,
                            int64_t bm, int64_t bn, sile_hip_stream stream) {
  if (!buffers || !shapes || num_shapes != 4)
    return fail(SILE_ERR_SHAPE, "softmax expects 2 buffers and 4 shape values (got %lld)",
                (long long)num_shapes);
  if (bm <= 0 || bn <= 0) return fail(SILE_ERR_SHAPE, "BM, BN must be positive");
  const int64_t x0 = shapes[0], x1 = shapes[1], y0 = shapes[2], y1 = shapes[3];
  if (x0 < 0 || x1 < 0 || y0 < 0 || y1 < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  SoftmaxTileArgs t{x1, y1, bm, bn, y1 / bn, 0};
  t.total = (y0 / bm) * t.tiles_n;
  int64_t run = 0;
  int rc = programs_to_run(num_threadgroups, threads_per_group, t.total, &run);
  if (rc != SILE_OK) return rc;
  if (run == 0) return ok();
  const int64_t rows_needed = ((run - 1) / t.tiles_n + 1) * bm;
  const int64_t cols_needed = std::min<int64_t>(run, t.tiles_n) * bn;
  if (x0 < rows_needed || x1 < cols_needed || y0 < rows_needed || y1 < cols_needed)
    return fail(SILE_ERR_SHAPE,
                "softmax shapes x[%lld,%lld] y[%lld,%lld] do not cover the tiles of %lld "
                "programs (BM=%lld BN=%lld)",
                (long long)x0, (long long)x1, (long long)y0, (long long)y1, (long long)run,
                (long long)bm, (long long)bn);
  const void* x = buffers[0];
  void* y = buffers[1];
  void* params[] = {&x, &y, &t};
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = launch(Module::kDsl, "sile_dsl_softmax_f32", dim3((unsigned)run), dim3(256), params, s);
  if (rc != SILE_OK) return rc;
  SILE_HIP_CHECK(hipStreamSynchronize(s));
  return ok();
}

int sile_hip_kernel_parallel_reduce(void* const* buffers, int64_t num_threadgroups,
                                    int64_t threads_per_group, const int64_t* shapes,
                                    int64_t num_shapes, int64_t tile, float* partials,
                                    sile_hip_stream stream) {
  if (!buffers || !shapes || num_shapes != 2)
    return fail(SILE_ERR_SHAPE, "parallel_reduce expects 2 buffers and 2 shape values (got %lld)",
                (long long)num_shapes);
  if (tile <= 0) return fail(SILE_ERR_SHAPE, "TILE must be positive");
  const int64_t len = shapes[0], out_len = shapes[1];
  if (len < 0 || out_len < 1) return fail(SILE_ERR_SHAPE, "out must hold at least one element");
  // No tile store to infer a plan from: total = shape(first buffer)[0]
  // (crates/sile-backend/src/cpu/codegen.rs:479-503).
  ReduceTileArgs t{tile, len, len};
  int64_t run = 0;
  int rc = programs_to_run(num_threadgroups, threads_per_group, t.total, &run);
  if (rc != SILE_OK) return rc;
  if (run == 0) return ok();
  if (run > len / tile)
    return fail(SILE_ERR_SHAPE, "%lld programs of TILE=%lld read past a[%lld]", (long long)run,
                (long long)tile, (long long)len);
  const void* a = buffers[0];
  void* out = buffers[1];
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (tile > 16 && tile % 4 == 0 && aligned16(a)) {
    // whole windows only: 4 programs per workgroup, window sums in parallel
    void* params[] = {&a, &out, &partials, &run, &tile};
    rc = launch(Module::kDsl, "sile_dsl_parallel_reduce_f32_tiled", dim3((unsigned)((run + 3) / 4)),
                dim3(256), params, s);
  } else if (tile > 16) {
    // any other TILE past 16: the same windows with element loads
    int64_t len_ = len;
    void* params[] = {&a, &out, &partials, &run, &tile, &len_};
    rc = launch(Module::kDsl, "sile_dsl_parallel_reduce_f32_tiled_any",
                dim3((unsigned)((run + 3) / 4)), dim3(256), params, s);
  } else {
    void* params[] = {&a, &out, &partials, &t};
    rc = launch(Module::kDsl, "sile_dsl_parallel_reduce_f32", dim3((unsigned)run), dim3(64),
                params, s);
  }
  if (rc != SILE_OK) return rc;
  SILE_HIP_CHECK(hipStreamSynchronize(s));
  return ok();
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------

}  // extern "C"

namespace {

// sile_hip_gemm with an optional forced tile size (0: by shape) and K split
// (0: by shape)
int gemm_impl(sile_dtype a_type, sile_dtype b_type, sile_dtype c_type, int64_t m, int64_t n,
              int64_t k, const void* a, int64_t lda, sile_layout a_layout, const void* b,
              int64_t ldb, sile_layout b_layout, void* c, int64_t ldc, float scale_a,
              float scale_b, int64_t bk, int tile_req, int splits_req, sile_hip_stream stream) {
  if (m < 0 || n < 0 || k < 0) return fail(SILE_ERR_SHAPE, "negative GEMM extent");
  const int64_t kp = bk > 0 ? (k / bk) * bk : k;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (m == 0 || n == 0) return ok();
  if (!a || !b || !c) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (a_layout != SILE_ROW_MAJOR)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "A must be row-major");

  if (a_type == SILE_F32 && b_type == SILE_F32 && c_type == SILE_F32) {
    const bool bcol = b_layout == SILE_COL_MAJOR;
    if (lda < k || ldc < n || (bcol ? ldb < k : ldb < n))
      return fail(SILE_ERR_SHAPE, "leading dimension smaller than the matrix extent");
    if (m > 65535LL * 32) return fail(SILE_ERR_SHAPE, "f32 GEMM too large");
    int rc = launch_f32_exact(bcol, a, b, c, m, n, kp, lda, ldb, ldc, nullptr, 0, 0.0f, s);
    return rc == SILE_OK ? ok() : rc;
  }

  const char* name = nullptr;
  int64_t kstep = 32;  // elements per half k-step (64 bytes of a row): 32 16-bit, 64 fp8
  if (a_type == SILE_BF16 && b_type == SILE_BF16) {
    name = c_type == SILE_BF16 ? "sile_gemm_nt_bf16_bf16"
           : c_type == SILE_F32 ? "sile_gemm_nt_bf16_f32" : nullptr;
  } else if (a_type == SILE_F16 && b_type == SILE_F16) {
    name = c_type == SILE_F16 ? "sile_gemm_nt_f16_f16"
           : c_type == SILE_F32 ? "sile_gemm_nt_f16_f32" : nullptr;
  } else if (a_type == SILE_F8E4M3 && b_type == SILE_F8E4M3) {
    name = c_type == SILE_BF16 ? "sile_gemm_nt_fp8_bf16"
           : c_type == SILE_F32 ? "sile_gemm_nt_fp8_f32" : nullptr;
    kstep = 64;
  }
  if (!name)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "GEMM %s x %s -> %s not supported",
                dtype_name(a_type), dtype_name(b_type), dtype_name(c_type));
  if (b_layout != SILE_COL_MAJOR && b_layout != SILE_ROW_MAJOR)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "unknown B layout %d", (int)b_layout);
  const bool b_row = b_layout == SILE_ROW_MAJOR;
  if (kp == 0) {
    // no k term: C = 0 (+0.0 in every output type), any M, N
    const int64_t cb16 = (int64_t)dtype_bytes(c_type) / 2;
    if (ldc < n) return fail(SILE_ERR_SHAPE, "leading dimension smaller than the matrix extent");
    int64_t ldc16 = ldc * cb16, n16 = n * cb16, rows = m;
    void* zp[] = {&c, &ldc16, &n16, &rows};
    int rc = launch(Module::kGemm, "sile_gemm_zero_c", dim3((unsigned)std::min<int64_t>(m, 4096)),
                    dim3(256), zp, s);
    return rc == SILE_OK ? ok() : rc;
  }
  const size_t eb = dtype_bytes(a_type), cb = dtype_bytes(c_type);
  if (lda < k || (b_row ? ldb < n : ldb < k) || ldc < n)
    return fail(SILE_ERR_SHAPE, "leading dimension too small");
  const bool fp8 = kstep == 64;
  if ((lda * eb) % 16 || !aligned16(a) || (!b_row && ((ldb * eb) % 16 || !aligned16(b))))
    return fail(SILE_ERR_SHAPE, "A, B and their leading dimensions must be 16-byte aligned");
  // the LDS kernels need N >= the tile edge (128 x 128 tiles take any M,
  // 256 x 256 tiles M >= 256)
  const int64_t min_tile = tile_req ? tile_req : 128;
  const bool lds_ok = (min_tile == 128 || m >= min_tile) && n >= min_tile && n % 4 == 0 &&
                      (ldc * cb) % 16 == 0 && aligned16(c);
  if (tile_req && !lds_ok)
    return fail(SILE_ERR_SHAPE,
                "%d x %d tiles need %sN >= %d, N a multiple of 4 and C's rows 16-byte aligned",
                tile_req, tile_req, tile_req == 256 ? "M, " : "", tile_req);
  // The transposed form runs C^T = B . A^T (A and B swapped) into fp32
  // planes of C^T and writes them back transposed, for the shapes the direct
  // form cannot take (N below one tile, N not a multiple of 4, C's rows not
  // 16-byte aligned) whose M can be the column extent: a multiple of 4 and
  // at least one tile.
  // Its fp32 planes (all of C^T) are kept to kScratchPlanesMax bytes.  The
  // forms that use the device scratch (this one and the K split) are left
  // out while the stream is being captured into a graph: the scratch is
  // ordered by events recorded at call time, which a graph's replays would
  // not follow.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const bool capturing =
      hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
  if (capturing && splits_req > 1)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "a K split needs the device scratch, which stream "
                                              "capture cannot order");
  // Row-major B ([K, N], N contiguous): the LDS kernels read its tiles
  // transposed (16-bit operands; N a multiple of 8, so every tile's columns
  // start on a 16-byte boundary; B's rows 0 .. K as one buffer resource).
  // Other row-major shapes and fp8 write B column-major into the device
  // scratch first (slot 1) and take the column-major path below.
  if (b_row && !(eb == 2 && lds_ok && n % 8 == 0 && (ldb * eb) % 16 == 0 && aligned16(b) &&
                 (double)k * (double)ldb * (double)eb <= 2147483647.0)) {
    if (capturing)
      return fail(SILE_ERR_UNSUPPORTED_BACKEND, "row-major B of this shape needs the device "
                                                "scratch, which stream capture cannot order");
    const int64_t per16 = 16 / (int64_t)eb;
    const int64_t ldt = (kp + per16 - 1) / per16 * per16;   // 16-byte aligned rows of B^T
    if ((double)n * (double)ldt * (double)eb > (double)kScratchPlanesMax)
      return fail(SILE_ERR_SHAPE, "row-major B of %lld x %lld exceeds the %lld MiB of scratch a "
                  "GEMM may use", (long long)kp, (long long)n, (long long)(kScratchPlanesMax >> 20));
    void* bt = nullptr;
    int rc = scratch_acquire((size_t)(n * ldt) * eb, s, &bt, 1);
    if (rc != SILE_OK) return rc;
    int64_t rows = kp, cols = n, ldi = ldb, ldo = ldt;
    int vec = (ldb * (int64_t)eb) % 16 == 0 && aligned16(b) ? 1 : 0;   // B^T rows are aligned
    void* tp[] = {(void*)&b, &ldi, &bt, &ldo, &rows, &cols, &vec};
    const int64_t tcols = 128 / (int64_t)eb;   // a tile: 128 rows of 128 bytes
    if ((kp + 127) / 128 > 65535) {
      rc = fail(SILE_ERR_SHAPE, "K too large for the transpose");
    } else {
      rc = launch(Module::kGemm, eb == 1 ? "sile_transpose_e1" : "sile_transpose_e2",
                  dim3((unsigned)((n + tcols - 1) / tcols), (unsigned)((kp + 127) / 128)),
                  dim3(256), tp, s);
    }
    if (rc == SILE_OK)
      rc = gemm_impl(a_type, b_type, c_type, m, n, kp, a, lda, a_layout, bt, ldt, SILE_COL_MAJOR,
                     c, ldc, scale_a, scale_b, 0, tile_req, splits_req, stream);
    scratch_release(s, 1);
    return rc;
  }
  const bool transposed = !b_row && !lds_ok && !capturing && m % 4 == 0 && m >= 128 &&
                          m * n * 4 <= kScratchPlanesMax;
  if (!lds_ok && !transposed) {
    // the any-shape kernel, 64 x 64 tiles with fragments loaded straight
    // from the operands
    const int64_t gx = (n + 63) / 64, gy = (m + 63) / 64;
    if (gx > 0x7fffffffLL || gy > 65535) return fail(SILE_ERR_SHAPE, "GEMM too large");
    char sname[64];
    snprintf(sname, sizeof sname, "sile_gemm_small_%s", name + strlen("sile_gemm_nt_"));
    struct {
      int64_t lda, ldb, ldc, m, n, kp;
      float alpha;
    } sg{lda, ldb, ldc, m, n, kp, scale_a * scale_b};
    void* sp[] = {&a, &b, &c, &sg};
    int rc = launch(Module::kGemm, sname, dim3((unsigned)gx, (unsigned)gy), dim3(256), sp, s);
    return rc == SILE_OK ? ok() : rc;
  }
  // the LDS kernels: 256 x 256 or 128 x 128 tiles over the
  // form that runs, (ra: [rm, K], rb: [rn, K]) -> [rm, rn]; any K' (the kernel
  // zeroes the elements of its last half k-step past K')
  const void* ra = transposed ? b : a;
  const void* rb = transposed ? a : b;
  const int64_t rlda = transposed ? ldb : lda, rldb = transposed ? lda : ldb;
  const int64_t rm = transposed ? n : m, rn = transposed ? m : n;
  // a tile's panel of A or B is one buffer resource: 32-bit byte range
  if (256 * std::max(lda, b_row ? 0 : ldb) * (int64_t)eb > 0x7fffffffLL)
    return fail(SILE_ERR_SHAPE, "leading dimension too large for a 256-row panel (%lld, %lld)",
                (long long)lda, (long long)ldb);
  if (m > 0x7fffffffLL || n > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "GEMM too large");
  const int64_t half_steps = (kp + kstep - 1) / kstep;
  if (half_steps > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "GEMM K too large");
  GemmPlan plan = gemm_plan(rm, rn, kp, half_steps, (int64_t)cb, fp8, tile_req);
  if (splits_req) plan.splits = splits_req;
  if (splits_req > 1 && (double)splits_req * (double)rm * (double)rn * 4.0 > (double)kScratchPlanesMax)
    return fail(SILE_ERR_SHAPE,
                "%d k-ranges of %lld x %lld fp32 planes exceed the %lld MiB of device scratch a "
                "GEMM may use", splits_req, (long long)rm, (long long)rn,
                (long long)(kScratchPlanesMax >> 20));
  if (capturing) plan.splits = 1;
  if (transposed) plan.splits = std::max<int64_t>(1, std::min(plan.splits, kScratchPlanesMax / (rm * rn * 4)));
  const int64_t tiles_m = (rm + plan.tile - 1) / plan.tile;
  const int64_t tiles_n = (rn + plan.tile - 1) / plan.tile;
  if (tiles_m * tiles_n > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "GEMM too large");
  GemmArgs g{rlda, rldb, ldc, (int32_t)tiles_m, (int32_t)tiles_n, (int32_t)half_steps,
             scale_a * scale_b, (int32_t)rm, (int32_t)rn,
             (int32_t)(kp - (half_steps - 1) * kstep), (int32_t)half_steps, 0, k};
  const unsigned tiles = (unsigned)(tiles_m * tiles_n);
  const char* tname = b_row ? (plan.tile == 256 ? "sile_gemm_nn_" : "sile_gemm_nn128_")
                            : (plan.tile == 256 ? "sile_gemm_nt_" : "sile_gemm_nt128_");
  const char* ab = a_type == SILE_BF16 ? "bf16" : a_type == SILE_F16 ? "f16" : "fp8";
  char kname[64];
  int64_t splits = plan.splits;
  if (splits >= 2) {
    // whole k-steps per range; the last range takes what is left of K'
    int64_t per = (half_steps + splits - 1) / splits;
    per += per & 1;
    splits = (half_steps + per - 1) / per;
    g.split_steps = (int32_t)per;
  }
  if (splits < 2 && !transposed) {
    snprintf(kname, sizeof kname, "%s%s", tname, name + strlen("sile_gemm_nt_"));
    void* params[] = {&ra, &rb, &c, &g};
    int rc = launch(Module::kGemm, kname, dim3(tiles), dim3(256), params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  // fp32 planes in the device scratch (one per k-range; rows of rn, a
  // multiple of 4), then their sum in k-range order, scaled, converted and,
  // for the transposed form, transposed
  void* ws = nullptr;
  int rc = scratch_acquire((size_t)(splits * rm * rn) * sizeof(float), s, &ws);
  if (rc != SILE_OK) return rc;
  snprintf(kname, sizeof kname, "%s%s_f32", tname, ab);
  const float alpha = g.alpha;
  g.alpha = 1.0f;
  g.ldc = rn;
  g.c_split = rm * rn;
  void* params[] = {&ra, &rb, &ws, &g};
  rc = launch(Module::kGemm, kname, dim3(tiles, (unsigned)splits), dim3(256), params, s);
  if (rc == SILE_OK) {
    const char* out = c_type == SILE_BF16 ? "bf16" : c_type == SILE_F16 ? "f16" : "f32";
    char rname[64];
    int64_t plane = rm * rn, ldc_ = ldc, m_ = m, n_ = n, pitch = rn;
    int sp = (int)splits;
    float al = alpha;
    if (transposed) {
      snprintf(rname, sizeof rname, "sile_gemm_splitk_reduce_t_%s", out);
      void* rp[] = {&ws, &c, &ldc_, &m_, &n_, &plane, &pitch, &sp, &al};
      rc = launch(Module::kGemm, rname, dim3((unsigned)((m + 31) / 32), (unsigned)((n + 63) / 64)),
                  dim3(256), rp, s);
    } else {
      snprintf(rname, sizeof rname, "sile_gemm_splitk_reduce_%s", out);
      void* rp[] = {&ws, &c, &ldc_, &m_, &n_, &plane, &sp, &al};
      rc = launch(Module::kGemm, rname,
                  dim3((unsigned)((n / 4 + 255) / 256), (unsigned)std::min<int64_t>(m, 65535)),
                  dim3(256), rp, s);
    }
  }
  scratch_release(s);
  return rc == SILE_OK ? ok() : rc;
}

}  // namespace

extern "C" {

int sile_hip_gemm(sile_dtype a_type, sile_dtype b_type, sile_dtype c_type, int64_t m, int64_t n,
                  int64_t k, const void* a, int64_t lda, sile_layout a_layout, const void* b,
                  int64_t ldb, sile_layout b_layout, void* c, int64_t ldc, float scale_a,
                  float scale_b, int64_t bk, sile_hip_stream stream) {
  return gemm_impl(a_type, b_type, c_type, m, n, k, a, lda, a_layout, b, ldb, b_layout, c, ldc,
                   scale_a, scale_b, bk, 0, 0, stream);
}

int sile_hip_gemm_tiled(sile_dtype a_type, sile_dtype b_type, sile_dtype c_type, int64_t m,
                        int64_t n, int64_t k, const void* a, int64_t lda, sile_layout a_layout,
                        const void* b, int64_t ldb, sile_layout b_layout, void* c, int64_t ldc,
                        float scale_a, float scale_b, int64_t bk, int32_t tile, int32_t splits,
                        sile_hip_stream stream) {
  if (tile != 0 && tile != 128 && tile != 256)
    return fail(SILE_ERR_SHAPE, "tile must be 0 (by shape), 128 or 256 (got %d)", tile);
  if (splits < 0 || splits > 64)
    return fail(SILE_ERR_SHAPE, "splits must be 0 (by shape) or 1 .. 64 (got %d)", splits);
  return gemm_impl(a_type, b_type, c_type, m, n, k, a, lda, a_layout, b, ldb, b_layout, c, ldc,
                   scale_a, scale_b, bk, tile, splits, stream);
}

int sile_hip_mma_f32(int64_t m, int64_t n, int64_t k, const float* a, int64_t lda,
                     const float* b, int64_t ldb, sile_layout b_layout, const float* acc,
                     int64_t ld_acc, float acc_value, float* c, int64_t ldc, int64_t bk,
                     sile_hip_stream stream) {
  if (m < 0 || n < 0 || k < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (m == 0 || n == 0) return ok();
  if (!a || !b || !c) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (b_layout != SILE_ROW_MAJOR && b_layout != SILE_COL_MAJOR)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "unknown layout of B");
  const bool bcol = b_layout == SILE_COL_MAJOR;
  const int64_t kp = bk > 0 ? (k / bk) * bk : k;
  if (lda < k || ldc < n || (bcol ? ldb < k : ldb < n) || (acc && ld_acc < n))
    return fail(SILE_ERR_SHAPE, "leading dimension smaller than the matrix extent");
  if (m > 65535LL * 32) return fail(SILE_ERR_SHAPE, "f32 MMA too large");
  int rc = launch_f32_exact(bcol, a, b, c, m, n, kp, lda, ldb, ldc, acc, ld_acc, acc_value,
                            static_cast<hipStream_t>(stream));
  return rc == SILE_OK ? ok() : rc;
}

int sile_hip_matvec_f32(int64_t m, int64_t k, int64_t bk, const float* x, int64_t ldx,
                        const float* y, float seed, float* out, sile_hip_stream stream) {
  if (m < 0 || k < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (bk <= 0) return fail(SILE_ERR_SHAPE, "matvec tile BK must be positive (got %lld)", (long long)bk);
  if (m == 0) return ok();
  if (!x || !y || !out) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldx < k) return fail(SILE_ERR_SHAPE, "leading dimension smaller than K");
  const int64_t blocks = (m + 3) / 4;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
  struct {
    int64_t m, ldx, tiles, bk;
    float seed;
  } args{m, ldx, k / bk, bk, seed};
  // 16-byte loads when every tile of every row starts on a 16-byte boundary;
  // tiles of 1 .. 16 such chunks: coalesced spans with the chain carried
  // across lanes, else a lane per tile
  const bool vec4 = bk % 4 == 0 && ldx % 4 == 0 && aligned16(x) && aligned16(y);
  // (BK 4 and 8: 8 rows a wave, so that one in-order add serves 8 rows)
  char name[40];
  int64_t rows_per_block = 4;
  if (vec4 && (bk == 4 || bk == 8)) {
    snprintf(name, sizeof name, "sile_dsl_matvec_f32_l%d_r8", (int)(bk / 4));
    rows_per_block = 32;
  } else if (vec4 && (bk == 16 || bk == 32 || bk == 64)) {
    snprintf(name, sizeof name, "sile_dsl_matvec_f32_l%d", (int)(bk / 4));
  } else {
    snprintf(name, sizeof name, "%s", vec4 ? "sile_dsl_matvec_f32_v4" : "sile_dsl_matvec_f32");
  }
  void* params[] = {(void*)&x, (void*)&y, &out, &args};
  int rc = launch(Module::kDsl, name, dim3((unsigned)((m + rows_per_block - 1) / rows_per_block)),
                  dim3(256), params, static_cast<hipStream_t>(stream));
  return rc == SILE_OK ? ok() : rc;
}

// ---------------------------------------------------------------------------
// Row softmax / row reduce
// ---------------------------------------------------------------------------

int sile_hip_softmax_rows(sile_dtype in_type, sile_dtype out_type, int64_t rows, int64_t cols,
                          const void* x, int64_t ldx, void* y, int64_t ldy,
                          sile_hip_stream stream) {
  const char* tag = nullptr;
  if (in_type == SILE_F16 && out_type == SILE_F16) tag = "f16_f16";
  else if (in_type == SILE_BF16 && out_type == SILE_BF16) tag = "bf16_bf16";
  else if (in_type == SILE_F32 && out_type == SILE_F32) tag = "f32_f32";
  else if (in_type == SILE_F16 && out_type == SILE_F32) tag = "f16_f32";
  if (!tag)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "softmax %s -> %s not supported",
                dtype_name(in_type), dtype_name(out_type));
  if (rows < 0 || cols < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (rows == 0) return ok();
  if (cols == 0) return fail(SILE_ERR_SHAPE, "softmax over an empty row");
  if (!x || !y) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldx < cols || ldy < cols) return fail(SILE_ERR_SHAPE, "leading dimension smaller than cols");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
  // register-resident kernels: a row of chunks * 64 lanes * E elements, E = 4
  // for fp32 -> fp32 (one 16-byte access per lane and chunk), 8 otherwise
  const bool f32_rows = in_type == SILE_F32 && out_type == SILE_F32;
  const int64_t elems = f32_rows ? 4 : 8;
  const int64_t ib = dtype_bytes(in_type), ob = dtype_bytes(out_type);
  const bool vec_ok = (ldx * ib) % 16 == 0 && (ldy * ob) % 16 == 0 && aligned16(x) && aligned16(y);
  int chunks = 0;
  if (vec_ok) {
    for (int c : {1, 2, 4, 8, 16, 32})
      if (cols == (int64_t)c * 64 * elems && (c < 32 || f32_rows)) chunks = c;
  }
  char name[64];
  int rc;
  // rows of 256 / 512 / 1024 threads x 2 chunks: one row per workgroup
  int block_threads = 0;
  if (vec_ok) {
    for (int t : {256, 512, 1024})
      if (cols == (int64_t)t * 2 * elems) block_threads = t;
  }
  if (block_threads) {
    if (rows > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
    snprintf(name, sizeof name, "sile_softmax_rows_%s_b%d", tag, block_threads);
    void* params[] = {&x, &y, &rows, &ldx, &ldy};
    rc = launch(Module::kSoftmax, name, dim3((unsigned)rows), dim3(block_threads), params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  // rows of up to 32 chunks: kL lanes per row (the smallest of 4, 8, 16, 32
  // that covers it), several rows per wave
  if (vec_ok && cols <= 32 * elems) {
    int lanes = 4;
    while ((int64_t)lanes * elems < cols) lanes *= 2;
    const int64_t per_block = 256 / lanes;
    if ((rows + per_block - 1) / per_block > 0x7fffffffLL)
      return fail(SILE_ERR_SHAPE, "too many rows");
    snprintf(name, sizeof name, "sile_softmax_rows_%s_n%d", tag, lanes);
    void* params[] = {&x, &y, &rows, &cols, &ldx, &ldy};
    rc = launch(Module::kSoftmax, name, dim3((unsigned)((rows + per_block - 1) / per_block)),
                dim3(256), params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  // other widths up to 8192 (16-bit) / 8192 (fp32): one pass with a masked
  // last chunk, the smallest power-of-two chunk count that covers the row
  int masked = 0;
  if (!chunks && vec_ok) {
    for (int c : {1, 2, 4, 8, 16, 32})
      if (!masked && cols <= (int64_t)c * 64 * elems && (c < 32 || f32_rows)) masked = c;
  }
  // wider rows: one row per 1024-thread workgroup, in registers up to
  // 1024 * 8 chunks, in two passes beyond
  if (!chunks && !masked && vec_ok) {
    if (rows > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
    int wide = 0;
    for (int c : {2, 4, 8})
      if (!wide && cols <= (int64_t)c * 1024 * elems) wide = c;
    if (wide)
      snprintf(name, sizeof name, "sile_softmax_rows_%s_w%d", tag, wide);
    else
      snprintf(name, sizeof name, "sile_softmax_rows_%s_wide", tag);
    void* params[] = {&x, &y, &rows, &cols, &ldx, &ldy};
    rc = launch(Module::kSoftmax, name, dim3((unsigned)rows), dim3(1024), params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  if (masked) {
    snprintf(name, sizeof name, "sile_softmax_rows_%s_m%d", tag, masked);
    void* params[] = {&x, &y, &rows, &cols, &ldx, &ldy};
    rc = launch(Module::kSoftmax, name, dim3((unsigned)blocks), dim3(256), params, s);
  } else if (chunks) {
    snprintf(name, sizeof name, "sile_softmax_rows_%s_c%d", tag, chunks);
    void* params[] = {&x, &y, &rows, &ldx, &ldy};
    rc = launch(Module::kSoftmax, name, dim3((unsigned)blocks), dim3(256), params, s);
  } else {
    snprintf(name, sizeof name, "sile_softmax_rows_%s_any", tag);
    void* params[] = {&x, &y, &rows, &cols, &ldx, &ldy};
    rc = launch(Module::kSoftmax, name, dim3((unsigned)blocks), dim3(256), params, s);
  }
  return rc == SILE_OK ? ok() : rc;
}

int sile_hip_reduce_rows(sile_reduce_op op, sile_dtype in_type, int64_t rows, int64_t cols,
                         const void* x, int64_t ldx, float* out, sile_hip_stream stream) {
  const char* name = in_type == SILE_F32    ? "sile_reduce_rows_f32"
                     : in_type == SILE_F16  ? "sile_reduce_rows_f16"
                     : in_type == SILE_BF16 ? "sile_reduce_rows_bf16"
                                            : nullptr;
  if (!name)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "reduce over %s not supported", dtype_name(in_type));
  if (op != SILE_REDUCE_MAX && op != SILE_REDUCE_SUM)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "unknown reduce op %d", (int)op);
  if (rows < 0 || cols < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (rows == 0) return ok();
  if (cols == 0) return fail(SILE_ERR_SHAPE, "reduce over an empty row");
  if (!x || !out) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldx < cols) return fail(SILE_ERR_SHAPE, "leading dimension smaller than cols");
  // the max kernels carry the column of each partial maximum in 32 bits
  if (op == SILE_REDUCE_MAX && cols > 0x7fffffffLL)
    return fail(SILE_ERR_SHAPE, "row max over more than 2^31 - 1 columns");
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
  int iop = (int)op;
  // The 128-bit paths need every row start 16-byte aligned; otherwise the
  // wave-per-row kernel runs its scalar loop only.
  int vec = aligned16(x) && (ldx * (int64_t)dtype_bytes(in_type)) % 16 == 0 ? 1 : 0;
  const int64_t elems = in_type == SILE_F32 ? 4 : 8;   // per 16-byte chunk
  char kname[64];
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec && cols <= 32 * elems) {
    // up to 32 chunks: kL lanes per row, several rows per wave
    int lanes = 4;
    while ((int64_t)lanes * elems < cols) lanes *= 2;
    const int64_t per_block = 256 / lanes;
    snprintf(kname, sizeof kname, "%s_n%d", name, lanes);
    void* params[] = {&iop, &x, &out, &rows, &cols, &ldx};
    int rc = launch(Module::kSoftmax, kname, dim3((unsigned)((rows + per_block - 1) / per_block)),
                    dim3(256), params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  for (int t : {256, 512}) {
    if (vec && cols == (int64_t)t * 2 * elems) {
      // rows of 2 chunks per thread of a 256 / 512-thread workgroup (the
      // 1024-thread shape read 16384-wide f16 rows at 4.5 TB/s)
      if (rows > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
      snprintf(kname, sizeof kname, "%s_b%d", name, t);
      void* params[] = {&iop, &x, &out, &rows, &ldx};
      int rc = launch(Module::kSoftmax, kname, dim3((unsigned)rows), dim3(t), params, s);
      return rc == SILE_OK ? ok() : rc;
    }
  }
  if (vec && cols >= 16384 && rows <= 4096) {
    // few wide rows: a 1024-thread workgroup per row
    snprintf(kname, sizeof kname, "%s_block", name);
    void* params[] = {&iop, &x, &out, &rows, &cols, &ldx};
    int rc = launch(Module::kSoftmax, kname, dim3((unsigned)rows), dim3(1024), params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  void* params[] = {&iop, &vec, &x, &out, &rows, &cols, &ldx};
  int rc = launch(Module::kSoftmax, name, dim3((unsigned)blocks), dim3(256), params, s);
  return rc == SILE_OK ? ok() : rc;
}

int sile_hip_fill_rows(sile_dtype type, int64_t rows, int64_t cols, float value, void* y,
                       int64_t ldy, sile_hip_stream stream) {
  if (type != SILE_F32 && type != SILE_F16 && type != SILE_BF16)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "fill of %s not supported", dtype_name(type));
  if (rows < 0 || cols < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (rows == 0 || cols == 0) return ok();
  if (!y) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldy < cols) return fail(SILE_ERR_SHAPE, "leading dimension smaller than cols");
  const int eb = (int)dtype_bytes(type);
  uint32_t bits = 0;
  if (type == SILE_F32) {
    memcpy(&bits, &value, 4);
  } else {
    bits = type == SILE_BF16 ? bf16_bits_rne(value) : f16_bits_rne(value);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ldy == cols && (cols * eb) % 16 == 0 && aligned16(y)) {
    int64_t chunks = rows * cols * eb / 16;
    const int64_t groups = (chunks + 1023) / 1024;
    if (groups > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "fill too large");
    uint32_t word = eb == 4 ? bits : bits | (bits << 16);
    void* params[] = {&y, &chunks, &word};
    int rc = launch(Module::kSoftmax, "sile_fill_flat_b128", dim3((unsigned)groups), dim3(512),
                    params, s);
    return rc == SILE_OK ? ok() : rc;
  }
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
  void* params[] = {&y, &rows, &cols, &ldy, &bits, (void*)&eb};
  int rc = launch(Module::kSoftmax, "sile_fill_rows_elem", dim3((unsigned)blocks), dim3(256),
                  params, s);
  return rc == SILE_OK ? ok() : rc;
}

int sile_hip_copy_rows(int64_t rows, int64_t row_bytes, const void* x, int64_t ldx_bytes,
                       void* y, int64_t ldy_bytes, sile_hip_stream stream) {
  if (rows < 0 || row_bytes < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (rows == 0 || row_bytes == 0) return ok();
  if (!x || !y) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldx_bytes < row_bytes || ldy_bytes < row_bytes)
    return fail(SILE_ERR_SHAPE, "pitch smaller than the row");
  const bool vec = row_bytes % 16 == 0 && ldx_bytes % 16 == 0 && ldy_bytes % 16 == 0 &&
                   aligned16(x) && aligned16(y);
  if (vec && ldx_bytes == row_bytes && ldy_bytes == row_bytes) {
    // contiguous rows: one flat run of 16-byte chunks, 16 KiB per workgroup
    int64_t chunks = rows * (row_bytes / 16);
    const int64_t groups = (chunks + 1023) / 1024;
    if (groups > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "copy too large");
    void* params[] = {(void*)&x, &y, &chunks};
    int rc = launch(Module::kSoftmax, "sile_copy_flat_b128", dim3((unsigned)groups), dim3(512),
                    params, static_cast<hipStream_t>(stream));
    return rc == SILE_OK ? ok() : rc;
  }
  // 16-byte path: one workgroup of 512 threads per 16 KiB segment of a row
  // (grid rows x segments); byte path: one wave per row
  const int64_t segs = vec ? (row_bytes + 16383) / 16384 : 1;
  const int64_t blocks = vec ? rows : (rows + 3) / 4;
  if (blocks > 0x7fffffffLL || segs > 65535) return fail(SILE_ERR_SHAPE, "too many rows");
  void* params[] = {(void*)&x, &y, &rows, &row_bytes, &ldx_bytes, &ldy_bytes};
  int rc = launch(Module::kSoftmax, vec ? "sile_copy_rows_b128" : "sile_copy_rows_b8",
                  dim3((unsigned)blocks, (unsigned)segs), dim3(vec ? 512 : 256), params,
                  static_cast<hipStream_t>(stream));
  return rc == SILE_OK ? ok() : rc;
}

int sile_hip_reduce_rows_fused_sum(int64_t rows, int64_t cols, const float* x, int64_t ldx,
                                   int64_t x_len, float* out, sile_hip_stream stream) {
  if (rows < 0 || cols < 0) return fail(SILE_ERR_SHAPE, "negative extent");
  if (rows == 0) return ok();
  if (cols == 0) return fail(SILE_ERR_SHAPE, "reduce over an empty row");
  if (!x || !out) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldx < cols) return fail(SILE_ERR_SHAPE, "leading dimension smaller than cols");
  if (x_len < (rows - 1) * ldx + cols)
    return fail(SILE_ERR_SHAPE, "x_len %lld does not cover %lld rows of %lld at pitch %lld",
                (long long)x_len, (long long)rows, (long long)cols, (long long)ldx);
  if (cols > 16 && cols % 4 == 0 && ldx % 4 == 0 && aligned16(x)) {
    // no window past a row: window sums in parallel, one chain per row (4 rows per workgroup)
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
    void* params[] = {(void*)&x, &out, &rows, &cols, &ldx};
    int rc = launch(Module::kSoftmax, "sile_reduce_rows_fused_sum_f32_tiled",
                    dim3((unsigned)blocks), dim3(256), params, static_cast<hipStream_t>(stream));
    return rc == SILE_OK ? ok() : rc;
  }
  if (cols > 16) {
    // any pitch / alignment / width: element loads, windows past a row read
    // the buffer's next elements (zero past x_len), then the scalar tail
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
    void* params[] = {(void*)&x, &out, &rows, &cols, &ldx, &x_len};
    int rc = launch(Module::kSoftmax, "sile_reduce_rows_fused_sum_f32_tiled_any",
                    dim3((unsigned)blocks), dim3(256), params, static_cast<hipStream_t>(stream));
    return rc == SILE_OK ? ok() : rc;
  }
  const int64_t blocks = (rows + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "too many rows");
  void* params[] = {(void*)&x, &out, &rows, &cols, &ldx, &x_len};
  int rc = launch(Module::kSoftmax, "sile_reduce_rows_fused_sum_f32", dim3((unsigned)blocks),
                  dim3(256), params, static_cast<hipStream_t>(stream));
  return rc == SILE_OK ? ok() : rc;
}

// ---------------------------------------------------------------------------
// Attention
// ---------------------------------------------------------------------------

int sile_hip_attention_f32_kt(int64_t n_q, int64_t n_k, int64_t head_dim, const float* q,
                              int64_t ldq, const float* kt, int64_t ldkt, const float* v,
                              int64_t ldv, float* o, int64_t ldo, float scale, float m0,
                              sile_hip_stream stream) {
  if (n_q < 0 || n_k < 0 || head_dim <= 0) return fail(SILE_ERR_SHAPE, "invalid attention shape");
  if (head_dim > 128)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "fp32 attention: head_dim > 128 not supported");
  if (n_q == 0) return ok();
  if (!q || !kt || !v || !o) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (ldq < head_dim || ldkt < n_k || ldv < head_dim || ldo < head_dim)
    return fail(SILE_ERR_SHAPE, "leading dimension smaller than the matrix extent");
  const int64_t blocks = (n_q + 63) / 64;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "attention too large");
  const int dp = (int)((head_dim + 15) / 16 * 16);
  char name[64];
  snprintf(name, sizeof name, "sile_attn_f32_kt_d%d", dp);
  int d = (int)head_dim;
  void* params[] = {(void*)&q, &ldq, (void*)&kt, &ldkt, (void*)&v, &ldv, &o, &ldo,
                    &n_q, &n_k, &d, &scale, &m0};
  int rc = launch(Module::kAttention, name, dim3((unsigned)blocks), dim3(256), params,
                  static_cast<hipStream_t>(stream));
  return rc == SILE_OK ? ok() : rc;
}

int sile_hip_flash_attn_fwd(sile_dtype dtype, int64_t batch, int64_t heads, int64_t seq_len,
                            int64_t head_dim, const void* q, const void* k, const void* v,
                            void* o, float scale, int causal, sile_hip_stream stream) {
  if (dtype != SILE_F16 && dtype != SILE_BF16)
    return fail(SILE_ERR_UNSUPPORTED_BACKEND, "attention over %s not supported", dtype_name(dtype));
  if (batch < 0 || heads < 0 || seq_len < 0 || head_dim <= 0)
    return fail(SILE_ERR_SHAPE, "invalid attention shape");
  if (batch == 0 || heads == 0 || seq_len == 0) return ok();
  if (!q || !k || !v || !o) return fail(SILE_ERR_SHAPE, "NULL operand");
  if (head_dim > 256) return fail(SILE_ERR_UNSUPPORTED_BACKEND, "head_dim > 256 not supported");
  hipStream_t s = static_cast<hipStream_t>(stream);
  int64_t bh = batch * heads;
  if (bh > 0x7fffffffLL / std::max<int64_t>(seq_len, 1))
    return fail(SILE_ERR_SHAPE, "attention too large");
  // one head's K or V is one buffer resource (32-bit byte range)
  if (seq_len * head_dim * 2 > 0x7fffffffLL)
    return fail(SILE_ERR_SHAPE, "sequence too long for one head (S=%lld)", (long long)seq_len);

  // MFMA flash kernel, 16-byte aligned operands, any S: the pipelined kernel
  // (32-query waves, key blocks through LDS-DMA; causal query blocks taken
  // in balanced pairs; keys and queries past S masked), one instantiation
  // per head dimension (a multiple of 16 up to 256): 8 waves up to 128
  // (32-key blocks, or 64-key blocks over 128-byte rows up to 64), 4 waves
  // past 128.
  const bool aligned = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
  if (head_dim % 16 == 0 && head_dim >= 16 && head_dim <= 256 && aligned) {
    const char* dt = dtype == SILE_F16 ? "f16" : "bf16";
    const int waves = head_dim <= 128 ? 8 : 4;
    char suffix[32];
    if (head_dim == 128)
      snprintf(suffix, sizeof suffix, "v2w8");
    else
      snprintf(suffix, sizeof suffix, "v2w%d_d%d", waves, (int)head_dim);
    const int64_t bq = 32 * waves;
    const bool pair = causal;
    const int64_t q_blocks = (seq_len + bq - 1) / bq;
    if (q_blocks > 0x7fffffffLL / std::max<int64_t>(bh, 1))
      return fail(SILE_ERR_SHAPE, "attention too large");
    struct {
      int64_t seq;
      int32_t bh, q_blocks;
      float scale_log2;
      int32_t causal, xcd_map, pair;
    } fa{seq_len, (int32_t)bh, (int32_t)q_blocks, scale * 1.4426950408889634f,
         causal ? 1 : 0, (bh % 8 == 0) ? 1 : 0, pair ? 1 : 0};
    const int64_t units = pair ? (q_blocks + 1) / 2 : q_blocks;
    const int64_t blocks = bh * units;
    char name[64];
    snprintf(name, sizeof name, "sile_flash_attn_fwd_%s_%s", dt, suffix);
    const unsigned threads = 64 * waves;
    void* params[] = {(void*)&q, (void*)&k, (void*)&v, &o, &fa};
    int rc = launch(Module::kFlashAttn, name, dim3((unsigned)blocks), dim3(threads), params, s);
    return rc == SILE_OK ? ok() : rc;
  }

  const int64_t rows = bh * seq_len;
  const int64_t blocks = (rows + 3) / 4;
  if (blocks > 0x7fffffffLL) return fail(SILE_ERR_SHAPE, "attention too large");
  const char* name = dtype == SILE_F16 ? "sile_attn_fwd_rowwise_f16" : "sile_attn_fwd_rowwise_bf16";
  void* params[] = {(void*)&q, (void*)&k, (void*)&v, &o, &bh, &seq_len, &head_dim, &scale, &causal};
  int rc = launch(Module::kAttention, name, dim3((unsigned)blocks), dim3(256), params, s);
  return rc == SILE_OK ? ok() : rc;
}

}  // extern "C"

namespace {
int launch_f32_exact(bool b_col_major, const void* a, const void* b, void* c, int64_t m,
                     int64_t n, int64_t kp, int64_t lda, int64_t ldb, int64_t ldc,
                     const float* seed, int64_t ld_seed, float seed_value, hipStream_t s) {
  int tile = 32;
  for (int t : {128, 64})
    if (tile == 32 && ((m + t - 1) / t) * ((n + t - 1) / t) >= 1024 && (m + t - 1) / t <= 65535)
      tile = t;
  const int64_t gx = (n + tile - 1) / tile, gy = (m + tile - 1) / tile;
  if (gx > 0x7fffffffLL || gy > 65535) return fail(SILE_ERR_SHAPE, "f32 GEMM too large");
  char name[64];
  snprintf(name, sizeof name, "sile_gemm_f32_exact_%s_t%d", b_col_major ? "nt" : "nn", tile);
  void* params[] = {(void*)&a, (void*)&b, &c,    &m,      &n,        &kp,
                    &lda,      &ldb,      &ldc,  &seed, &ld_seed, &seed_value};
  return launch(Module::kGemm, name, dim3((unsigned)gx, (unsigned)gy), dim3(256), params, s);
}
}  // namespace
