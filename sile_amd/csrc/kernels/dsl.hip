// gfx950 kernels for sile's DSL example kernels, run with the reference's
// program semantics: one workgroup per program, program ids decoded from the
// workgroup index exactly as the generated CPU wrapper decodes its OpenMP
// loop index (crates/sile-backend/src/cpu/codegen.rs:517-551):
//   pid < total_tiles, gid0 = pid / tiles_n, gid1 = pid % tiles_n.
// Element type is f32 only, as in the reference (crates/sile-hir/src/types.rs:11-14).
#include "common.h"

using namespace sile;

struct MatmulTileArgs {
  int64_t lda, ldb, ldc;  // shape(a)[1], shape(b)[1], shape(c)[1]
  int64_t bm, bn, bk;     // const generics of the DSL kernel
  int64_t tiles_n;        // shape(c)[1] / BN
  int64_t total;          // (shape(c)[0] / BM) * tiles_n
  const float* seed;      // accumulator tile source (row stride ld_seed), or NULL
  int64_t ld_seed;
  float seed_value;       // the accumulator's splat value when seed is NULL
};

// Matmul program (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:24-444
// and the tile MMA lowering, crates/sile-tile-ir/src/passes/lowering/tile_compute/mma.rs:25-739):
// every cell sums a[.]*b[.] in increasing k with a separate rounding for the
// product and for the add, over k < (lda / BK) * BK, starting from the
// accumulator's seed: 0.0f for the canonical matmul, the splat value, or the
// cell of a loaded accumulator tile (which may be c's own tile).  Threads own
// cells; each cell keeps the reference's sequential order, so results are
// bit-identical to the CPU backend's.
extern "C" __global__ __launch_bounds__(256) void sile_dsl_matmul_f32(const float* __restrict__ a,
                                                                       const float* __restrict__ b,
                                                                       float* c,
                                                                       MatmulTileArgs args) {
#pragma clang fp contract(off)
  const int64_t pid = blockIdx.x;
  if (pid >= args.total) return;
  const int64_t gid0 = pid / args.tiles_n, gid1 = pid % args.tiles_n;
  const int64_t kp = (args.lda / args.bk) * args.bk;
  const int64_t row0 = gid0 * args.bm, col0 = gid1 * args.bn;
  const int64_t cells = args.bm * args.bn;
  for (int64_t cell = threadIdx.x; cell < cells; cell += blockDim.x) {
    const int64_t r = cell / args.bn, cc = cell % args.bn;
    const float* ap = a + row0 * args.lda + r * args.lda;
    const float* bp = b + col0 + cc;
    float s = args.seed ? args.seed[row0 * args.ld_seed + col0 + r * args.ld_seed + cc]
                        : args.seed_value;
    for (int64_t k = 0; k < kp; ++k) {
      float p = ap[k] * bp[0];
      s = s + p;
      bp += args.ldb;
    }
    c[row0 * args.ldc + col0 + r * args.ldc + cc] = s;
  }
}

struct SoftmaxTileArgs {
  int64_t ldx, ldy;  // shape(x)[1], shape(y)[1]
  int64_t bm, bn;
  int64_t tiles_n, total;
};

// Softmax DSL program (crates/sile/tests/backend_softmax.rs:3-15): for each of
// the BM rows of the [BM, BN] tile at (gid0, gid1): m = row max, e = exp(x - m),
// s = sum(e), y = e / s (IEEE division, as the reference's Div,
// crates/sile-tile-ir/src/passes/lowering/tile_expr.rs:646-813).  One wave per
// row; the max is order-independent, the sum is a wave tree (the reference
// sums left to right; the results agree within fp32 rounding of the sum, not
// bit for bit, and exp is the device's v_exp_f32, not the host's expf).
extern "C" __global__ __launch_bounds__(256) void sile_dsl_softmax_f32(const float* __restrict__ x,
                                                                        float* __restrict__ y,
                                                                        SoftmaxTileArgs args) {
  const int64_t pid = blockIdx.x;
  if (pid >= args.total) return;
  const int64_t gid0 = pid / args.tiles_n, gid1 = pid % args.tiles_n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  for (int64_t r = wave; r < args.bm; r += nwaves) {
    const float* xr = x + (gid0 * args.bm) * args.ldx + gid1 * args.bn + r * args.ldx;
    float* yr = y + (gid0 * args.bm) * args.ldy + gid1 * args.bn + r * args.ldy;
    float m = -__builtin_inff();
    for (int64_t c = lane; c < args.bn; c += 64) m = fmax_ordered(m, xr[c]);
    m = wave_max(m);
    float s = 0.0f;
    for (int64_t c = lane; c < args.bn; c += 64) s += exp2_fast((xr[c] - m) * kLog2e);
    s = wave_sum(s);
    for (int64_t c = lane; c < args.bn; c += 64) yr[c] = exp2_fast((xr[c] - m) * kLog2e) / s;
  }
}

struct ReduceTileArgs {
  int64_t tile;   // TILE const generic
  int64_t total;  // shape(a)[0] (wrapper fallback: no tile store to infer from)
  int64_t len;    // elements of a
};

// parallel_reduce program (crates/sile/examples/parallel_reduce.rs:3-9): the
// tile a[pid*TILE, pid*TILE+TILE) is summed in the fused load+reduce vec4
// order (crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:80-113,
// 1182-1256): window sums ((v0+v1)+v2)+v3 added in window order, then the
// scalar tail from 4*(TILE/4) in order.
//  * TILE <= 16: TILE/4 windows, the accumulator starts at window 0;
//  * TILE > 16: the loop runs while idx < TILE (step 4,
//    crates/sile-tile-ir/src/passes/lowering/core/emit/tile_loops/single_axis.rs:180-260)
//    from 0.0f: ceil(TILE/4) windows, the last of which, for TILE % 4 != 0,
//    reads the first elements of the next tile and is followed by the tail,
//    which adds its in-tile elements again.  Window elements past the end of
//    a (the last program) are taken as 0.0f; the reference reads past the
//    buffer there.
// Lanes form the window sums in parallel; lane 0 folds them in order, so the
// per-program partial is bit-identical to the CPU backend's.  Programs then
// add their partial to out[0] atomically; the order across programs is
// unspecified there as here.
// TILE > 16 with TILE % 4 == 0 and a 16-byte aligned: no window runs past a
// tile and there is no tail, so kFsRows programs share a workgroup and their
// tile sums come from fused_sum_rows_tiled (the same windows, added in the
// same order: bit-identical partials), then go to out[0] atomically.
extern "C" __global__ __launch_bounds__(256) void sile_dsl_parallel_reduce_f32_tiled(
    const float* __restrict__ a, float* __restrict__ out, float* __restrict__ partials,
    int64_t programs, int64_t tile) {
  __shared__ __attribute__((aligned(16))) float w[kFsLds];
  const int64_t pid0 = (int64_t)blockIdx.x * kFsRows;
  const int nprog = (int)min((int64_t)kFsRows, programs - pid0);
  const float acc = fused_sum_rows_tiled<false>(a, tile, tile, 0, pid0, nprog, w);
  if ((int)threadIdx.x < nprog) {
    if (partials) partials[pid0 + threadIdx.x] = acc;
    atomicAdd(out, acc);
  }
}

// TILE > 16 otherwise (a ragged last window, read past the tile as the
// reference does, then the scalar tail; elements past len taken as 0.0f):
// the same windows and order through fused_sum_rows_tiled<true>.
extern "C" __global__ __launch_bounds__(256) void sile_dsl_parallel_reduce_f32_tiled_any(
    const float* __restrict__ a, float* __restrict__ out, float* __restrict__ partials,
    int64_t programs, int64_t tile, int64_t len) {
  __shared__ __attribute__((aligned(16))) float w[kFsLds];
  const int64_t pid0 = (int64_t)blockIdx.x * kFsRows;
  const int nprog = (int)min((int64_t)kFsRows, programs - pid0);
  const float acc = fused_sum_rows_tiled<true>(a, tile, tile, len, pid0, nprog, w);
  if ((int)threadIdx.x < nprog) {
    if (partials) partials[pid0 + threadIdx.x] = acc;
    atomicAdd(out, acc);
  }
}

extern "C" __global__ __launch_bounds__(64) void sile_dsl_parallel_reduce_f32(
    const float* __restrict__ a, float* __restrict__ out, float* __restrict__ partials,
    ReduceTileArgs args) {
#pragma clang fp contract(off)
  __shared__ float window_sums[64];
  const int64_t pid = blockIdx.x;
  if (pid >= args.total) return;
  const int lane = threadIdx.x;
  const float* t = a + pid * args.tile;
  const int64_t avail = args.len - pid * args.tile;  // elements of a from t on
  const int64_t chunks = args.tile / 4;
  const bool unrolled = args.tile <= 16;
  const int64_t windows = unrolled ? chunks : (args.tile + 3) / 4;
  float acc = 0.0f;
  int64_t first = 0;
  if (unrolled && chunks > 0) {
    acc = ((t[0] + t[1]) + t[2]) + t[3];
    first = 1;
  }
  for (int64_t base = first; base < windows; base += 64) {
    const int64_t wi = base + lane;
    if (wi < windows) {
      const int64_t e = 4 * wi;
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = e + j < avail ? t[e + j] : 0.0f;
      window_sums[lane] = ((v[0] + v[1]) + v[2]) + v[3];
    }
    __syncthreads();
    if (lane == 0) {
      const int64_t n = (windows - base) < 64 ? (windows - base) : 64;
      for (int64_t i = 0; i < n; ++i) acc = acc + window_sums[i];
    }
    __syncthreads();
  }
  if (lane == 0) {
    if (args.tile < 4) {
      // extent < 4 takes the plain sequential fold from element 0 (reduce.rs:32-112)
      acc = t[0];
      for (int64_t i = 1; i < args.tile; ++i) acc = acc + t[i];
    } else {
      for (int64_t i = chunks * 4; i < args.tile; ++i) acc = acc + t[i];
    }
    if (partials) partials[pid] = acc;
    atomicAdd(out, acc);
  }
}

// vec_add of crates/sile/tests/backend_vec_add.rs:3-9 (outside the hot path),
// written against the generic tile-launch convention of sile_hip_launch_tiles:
// (buffers, num_programs, shapes, num_shapes) with buffers = {a, b, c} and
// shapes = shape(a) ++ shape(b) ++ shape(c).  The output is rank 1, so
// total_tiles = shape(c)[0] and gid0 = pid (crates/sile-backend/src/cpu/codegen.rs:409-431,
// 517-531); the [4] tile of program pid starts at pid * 4 (rank-1 addressing,
// crates/sile-tile-ir/src/passes/lowering/tile_memory.rs:175-188).  Elements past
// shape(c)[0] are skipped (the CPU backend has no such guard).
extern "C" __global__ __launch_bounds__(64) void sile_tiles_vec_add4(void** buffers,
                                                                     int64_t num_programs,
                                                                     const int64_t* shapes,
                                                                     int64_t num_shapes) {
  const int64_t pid = blockIdx.x;
  if (num_shapes < 3 || pid >= num_programs) return;
  const int64_t total = shapes[2];
  if (pid >= total) return;
  const float* a = static_cast<const float*>(buffers[0]);
  const float* b = static_cast<const float*>(buffers[1]);
  float* c = static_cast<float*>(buffers[2]);
  const int64_t i = pid * 4 + threadIdx.x;
  if (threadIdx.x < 4 && i < shapes[0] && i < shapes[1] && i < shapes[2]) c[i] = a[i] + b[i];
}
