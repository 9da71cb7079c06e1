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

struct MatvecArgs {
  int64_t m;      // rows of the output (programs x BM)
  int64_t ldx;    // row pitch of x in elements (shape(x)[1])
  int64_t tiles;  // whole BK tiles of K: shape(x)[1] / BK
  int64_t bk;
  float seed;     // the accumulator's splat value
};

// Matvec program (crates/sile/examples/mlp.rs:26-44):
//   out[r] = ((seed + p_0) + p_1) + ... + p_{tiles-1},
//   p_t = x[r][t BK] y[t BK] + x[r][t BK + 1] y[t BK + 1] + ... in order,
// every product and every sum rounded on its own (the fused map + reduce,
// crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:189-293,
// then the carried add).  One wave per row, four rows per workgroup: lane l
// computes the partials of tiles l, l + 64, ... of its row, and the wave adds
// them to the accumulator in tile order (lane 0 first, through readlane), so
// the result is the reference's, bit for bit.  kVec4: x rows, y and BK allow
// 16-byte loads.
template <bool kVec4>
__device__ __forceinline__ void matvec_rows(const float* __restrict__ x, const float* __restrict__ y,
                                            float* __restrict__ out, const MatvecArgs& a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.m) return;   // the whole wave
  const float* xr = x + row * a.ldx;
  float acc = a.seed;
  for (int64_t base = 0; base < a.tiles; base += 64) {
    const int64_t t = base + lane;
    float p = 0.0f;
    if (t < a.tiles) {
      const float* xt = xr + t * a.bk;
      const float* yt = y + t * a.bk;
      if constexpr (kVec4) {
        f32x4 xv = *reinterpret_cast<const f32x4*>(xt);
        f32x4 yv = *reinterpret_cast<const f32x4*>(yt);
        p = xv[0] * yv[0];
        p = p + xv[1] * yv[1];
        p = p + xv[2] * yv[2];
        p = p + xv[3] * yv[3];
        for (int64_t i = 4; i < a.bk; i += 4) {
          xv = *reinterpret_cast<const f32x4*>(xt + i);
          yv = *reinterpret_cast<const f32x4*>(yt + i);
          p = p + xv[0] * yv[0];
          p = p + xv[1] * yv[1];
          p = p + xv[2] * yv[2];
          p = p + xv[3] * yv[3];
        }
      } else {
        p = xt[0] * yt[0];
        for (int64_t i = 1; i < a.bk; ++i) p = p + xt[i] * yt[i];
      }
    }
    const int n = (int)min<int64_t>(64, a.tiles - base);
    for (int i = 0; i < n; ++i)
      acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), i));
  }
  if (lane == 0) out[row] = acc;
}

// BK = 4 L with L = 1, 2, 4, 8 or 16 lanes a tile, x rows, y and BK allowing
// 16-byte loads: the wave reads the row 256 elements at a time with one
// 16-byte load per lane (coalesced; four such spans in flight), lane j holding
// elements 4 j .. 4 j + 3 of a span, so tile g of a span lives on lanes
// g L .. g L + L - 1 of one 16-lane DPP row.  Its sequential sum is carried
// from lane to lane in L steps (a DPP shift by one lane), each lane adding its
// four products in order, so the tile's partial, on its last lane, is the
// reference's chain; the partials are then added to the accumulator in tile
// order as above.
template <int kL>
__device__ __forceinline__ void matvec_rows_chain(const float* __restrict__ x,
                                                  const float* __restrict__ y,
                                                  float* __restrict__ out, const MatvecArgs& a) {
#pragma clang fp contract(off)
  constexpr int kU = 4;              // spans in flight
  const int lane = threadIdx.x & 63, s = lane % kL;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.m) return;   // the whole wave
  const float* xr = x + row * a.ldx;
  const int64_t n = a.tiles * 4 * kL;   // elements of the whole tiles
  float acc = a.seed;
  for (int64_t base = 0; base < n; base += 256 * kU) {
    f32x4 xv[kU], yv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t e = base + 256 * u + 4 * lane;
      xv[u] = yv[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (e < n) {
        xv[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(xr + e));
        yv[u] = *reinterpret_cast<const f32x4*>(y + e);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t b = base + 256 * u;
      if (b >= n) break;
      const float p0 = xv[u][0] * yv[u][0], p1 = xv[u][1] * yv[u][1];
      const float p2 = xv[u][2] * yv[u][2], p3 = xv[u][3] * yv[u][3];
      float p = 0.0f, carry = 0.0f;
#pragma unroll
      for (int step = 0; step < kL; ++step) {
        float c = step == 0 ? p0 : carry + p0;
        c = c + p1;
        c = c + p2;
        c = c + p3;
        p = s == step ? c : p;
        if (step + 1 < kL) carry = dpp<0x111>(p);   // row_shr:1
      }
      const int g_n = (int)min<int64_t>(64 / kL, (n - b) / (4 * kL));
      for (int g = 0; g < g_n; ++g)
        acc = acc + __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), g * kL + kL - 1));
    }
  }
  if (lane == 0) out[row] = acc;
}

// The same with kR rows per wave (the wave's rows read in turn, y once for
// them all): each tile partial goes to LDS, and lane r < kR adds row r's
// partials to its accumulator in tile order, so one add advances kR rows.
template <int kL, int kR, int kU>
__device__ __forceinline__ void matvec_rows_multi(const float* __restrict__ x,
                                                  const float* __restrict__ y,
                                                  float* __restrict__ out, const MatvecArgs& a) {
#pragma clang fp contract(off)
  constexpr int kG = 64 / kL;        // tiles per span
  __shared__ float part[4][kR][kG];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, s = lane % kL;
  const int64_t row0 = ((int64_t)blockIdx.x * 4 + wave) * kR;
  if (row0 >= a.m) return;   // the whole wave
  const int64_t n = a.tiles * 4 * kL;   // elements of the whole tiles
  float acc = a.seed;                   // lane r < kR: row row0 + r
  for (int64_t base = 0; base < n; base += 256 * kU) {
    f32x4 yv[kU], xv[kU][kR];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t e = base + 256 * u + 4 * lane;
      yv[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (e < n) yv[u] = *reinterpret_cast<const f32x4*>(y + e);
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        xv[u][r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (e < n && row0 + r < a.m)
          xv[u][r] = __builtin_nontemporal_load(
              reinterpret_cast<const f32x4*>(x + (row0 + r) * a.ldx + e));
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t b = base + 256 * u;
      if (b >= n) break;
#pragma unroll
      for (int r = 0; r < kR; ++r) {
        const float p0 = xv[u][r][0] * yv[u][0], p1 = xv[u][r][1] * yv[u][1];
        const float p2 = xv[u][r][2] * yv[u][2], p3 = xv[u][r][3] * yv[u][3];
        float p = 0.0f, carry = 0.0f;
#pragma unroll
        for (int step = 0; step < kL; ++step) {
          float c = step == 0 ? p0 : carry + p0;
          c = c + p1;
          c = c + p2;
          c = c + p3;
          p = s == step ? c : p;
          if (step + 1 < kL) carry = dpp<0x111>(p);   // row_shr:1
        }
        if (s == kL - 1) part[wave][r][lane / kL] = p;
      }
      __builtin_amdgcn_wave_barrier();
      const int g_n = (int)min<int64_t>(kG, (n - b) / (4 * kL));
      if (lane < kR)
        for (int g = 0; g < g_n; ++g) acc = acc + part[wave][lane][g];
      __builtin_amdgcn_wave_barrier();
    }
  }
  if (lane < kR && row0 + lane < a.m) out[row0 + lane] = acc;
}

#define SILE_MATVEC_MULTI(L, R, U)                                                             \
  extern "C" __global__ __launch_bounds__(256) void sile_dsl_matvec_f32_l##L##_r##R(           \
      const float* x, const float* y, float* out, MatvecArgs a) {                              \
    matvec_rows_multi<L, R, U>(x, y, out, a);                                                  \
  }
// BK = 4 and 8 (16 or 32 tiles a span): 8 rows a wave, 4.73 and 4.84 TB/s
// at 8192^2 against 2.08 and 3.70 with a row a wave; from BK = 16 on the
// row-a-wave kernels are faster (4.82 TB/s at 16 against 4.64 with 8 rows)
SILE_MATVEC_MULTI(1, 8, 2)
SILE_MATVEC_MULTI(2, 8, 2)

#define SILE_MATVEC_CHAIN(L)                                                                   \
  extern "C" __global__ __launch_bounds__(256) void sile_dsl_matvec_f32_l##L(                 \
      const float* x, const float* y, float* out, MatvecArgs a) {                              \
    matvec_rows_chain<L>(x, y, out, a);                                                        \
  }
SILE_MATVEC_CHAIN(1)
SILE_MATVEC_CHAIN(2)
SILE_MATVEC_CHAIN(4)
SILE_MATVEC_CHAIN(8)
SILE_MATVEC_CHAIN(16)

extern "C" __global__ __launch_bounds__(256) void sile_dsl_matvec_f32(const float* x,
                                                                       const float* y, float* out,
                                                                       MatvecArgs a) {
  matvec_rows<false>(x, y, out, a);
}
extern "C" __global__ __launch_bounds__(256) void sile_dsl_matvec_f32_v4(const float* x,
                                                                          const float* y,
                                                                          float* out,
                                                                          MatvecArgs a) {
  matvec_rows<true>(x, y, out, a);
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
