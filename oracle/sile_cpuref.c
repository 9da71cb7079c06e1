/*
 * sile_cpuref.c -- CPU oracle for the sile tile-kernel hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP path is
 * compared against; it is never part of the product.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the
 * library built from it (oracle/_build/libsile_cpuref.so).
 *
 * What it restates: the arithmetic and indexing semantics that sile's CPU
 * backend gives the DSL kernels on the hot path (GEMM, row softmax, row
 * reduce, parallel reduce with atomic add), derived from the reference
 * sources cited on each function.  The reference is Rust and cannot be built
 * in this image (no rustc/cargo), so it is restated, not linked.
 *
 * It is compiled the way the reference compiles the C it generates
 * (crates/sile-backend/src/cpu/mod.rs:83: `cc -shared -fPIC -O2 -fopenmp
 * -lm`, no -march) plus an explicit -ffp-contract=off, so that `s = s + a*b`
 * keeps its two roundings (no FMA contraction).
 *
 * Pinning status (checked by tests/test_oracle.py against the reference's own
 * literal fixtures in tests/golden/, closed forms and float64 brute force):
 *   cpuref_kernel_matmul          pinned (reference fixture + exact integer GEMMs + order check)
 *   cpuref_kernel_softmax         pinned (reference fixture row sums, closed forms, fp64)
 *   cpuref_kernel_parallel_reduce pinned (reference fixture, closed form n(n+1)/2; TILE = 18
 *                                 ones give 22 per program, 20 for the last)
 *   cpuref_gemm_nt                pinned (equals cpuref_kernel_matmul on transposed B; fp64)
 *   cpuref_mma_f32                pinned (seed 0 equals cpuref_kernel_matmul; exact integer
 *                                 seeds + products; a 2^24 order probe that fails for a seed
 *                                 added last; signed-zero seeds with K' = 0)
 *   cpuref_softmax_rows           pinned (same program body as cpuref_kernel_softmax)
 *   cpuref_reduce_rows            pinned (max exact vs numpy on finite rows, and the fold's
 *                                 NaN / -inf / signed-zero cases by closed forms; sequential
 *                                 sum vs a left fold; the vec4 loop's windows, tail and
 *                                 over-read by closed forms over ones and order probes)
 *   cpuref_attention_causal       pinned by closed forms and fp64 brute force only; the
 *                                 reference has no attention kernel (no mask/iota/transpose
 *                                 in its DSL), so there is no reference vector for it.
 *   cpuref_dsl_attention_f32      pinned by fp64 brute force (any initial max below the
 *                                 scores), key truncation to whole BN blocks, the initial
 *                                 max's underflow closed form (m0 above every score: 0 / 0),
 *                                 and agreement with cpuref_attention_fwd (non-causal)
 *   cpuref_dsl_matvec_f32         pinned by exact integer-valued rows, fp64 brute force, order
 *                                 probes inside a tile ([2^24, 1, 1] gives 2^24, a tree gives
 *                                 2^24 + 2) and across tiles (partials 2^24, 1, 1 in order),
 *                                 K truncation to whole BK tiles, the seed, and -0.0 products
 *                                 (+0.0 once added to the +0.0 seed)
 *   cpuref_e4m3_encode/decode     pinned (OCP e4m3fn table: 448 max, 2^-9 min subnormal,
 *                                 exhaustive decode/encode round trip of all 254 finite codes)
 *   cpuref_bf16_from_f32          pinned (RNE vs exhaustive cases and numpy bit tricks)
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Launch-wrapper semantics.                                                 */
/* ------------------------------------------------------------------------ */

/* Number of programs that execute a body: crates/sile-backend/src/cpu/codegen.rs:409-431
 * (emit_tile_count_logic).  Rank 1: shapes[off]; rank >= 2:
 * (shape0 / rows) * (shape1 / cols) with truncating integer division. */
int64_t cpuref_total_tiles(int64_t out_rank, const int64_t *out_shape, int64_t rows,
                           int64_t cols) {
  if (out_rank <= 1) return out_shape[0];
  int64_t tiles_n = out_shape[1] / cols;
  return (out_shape[0] / rows) * tiles_n;
}

/* ------------------------------------------------------------------------ */
/* a1: canonical matmul.                                                     */
/* ------------------------------------------------------------------------ */

/* One program of the canonical matmul loop nest,
 * crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:38-422:
 *   lda = shape(a)[1], ldb = shape(b)[1], ldc = shape(c)[1]
 *   Kp  = (lda / BK) * BK                       (:58-73, K truncation)
 *   for r < BM, c < BN:
 *     s = 0.0f; ai = (gid0*BM)*lda + r*lda; bi = gid1*BN + c
 *     for k < Kp: s = s + (a[ai] * b[bi]); ai += 1; bi += ldb   (:226-370)
 *     c[(gid0*BM)*ldc + gid1*BN + r*ldc + c] = s                (:372-422)
 */
static void matmul_program(const float *a, const float *b, float *c, const int64_t *shapes,
                           int64_t bm, int64_t bn, int64_t bk, int64_t gid0, int64_t gid1) {
  const int64_t lda = shapes[1], ldb = shapes[3], ldc = shapes[5];
  const int64_t kp = (lda / bk) * bk;
  const int64_t row0 = gid0 * bm, col0 = gid1 * bn;
  const int64_t a_tile_base = row0 * lda;
  const int64_t c_tile_base = row0 * ldc + col0;
  for (int64_t r = 0; r < bm; ++r) {
    for (int64_t cc = 0; cc < bn; ++cc) {
      float s = 0.0f;
      int64_t ai = a_tile_base + r * lda;
      int64_t bi = col0 + cc;
      for (int64_t k = 0; k < kp; ++k) {
        float p = a[ai] * b[bi];
        s = s + p;
        ai += 1;
        bi += ldb;
      }
      c[c_tile_base + r * ldc + cc] = s;
    }
  }
}

/* sile_kernel_matmul wrapper for the DSL kernel of
 * crates/sile/tests/backend_matmul.rs:3-19, generated by
 * crates/sile-backend/src/cpu/codegen.rs:433-555:
 *   buffers = {a, b, c}; shapes = shape(a) ++ shape(b) ++ shape(c)
 *   tiles_n = shape(c)[1] / BN; total = (shape(c)[0] / BM) * tiles_n
 *   omp parallel for schedule(static) over pid in [0, num_threadgroups):
 *     if pid < total: gid0 = pid / tiles_n, gid1 = pid % tiles_n
 * threads_per_group is 1 in LLVM-IR mode (crates/sile-backend/src/cpu/mod.rs:109-120). */
void cpuref_kernel_matmul(void **buffers, int64_t num_threadgroups, int64_t threads_per_group,
                          const int64_t *shapes, int64_t num_shapes, int64_t bm, int64_t bn,
                          int64_t bk) {
  (void)num_shapes;
  const float *a = (const float *)buffers[0];
  const float *b = (const float *)buffers[1];
  float *c = (float *)buffers[2];
  const int64_t tiles_n = shapes[5] / bn;
  const int64_t total = (shapes[4] / bm) * tiles_n;
#pragma omp parallel for schedule(static)
  for (int64_t tg = 0; tg < num_threadgroups; ++tg) {
    int64_t base = tg * threads_per_group;
    for (int64_t t = 0; t < threads_per_group; ++t) {
      int64_t pid = base + t;
      if (pid < total) matmul_program(a, b, c, shapes, bm, bn, bk, pid / tiles_n, pid % tiles_n);
    }
  }
}

/* GEMM with B stored column-major ([N, K] row-major, "B^T"), the layout of the
 * bf16 / fp8 configurations.  Same per-cell arithmetic as matmul_program
 * (canonical_matmul.rs:226-370): s starts at 0.0f and accumulates a*b in
 * increasing k with two roundings per step; K is truncated to (K/bk)*bk.
 * Inputs are the fp32 (de)quantised values.  Only row tiles whose index t
 * satisfies t % row_tile_step == 0 (tiles of bm rows) are computed, so a
 * deterministic sample of a large GEMM can be timed; row_tile_step = 1
 * computes everything.  Rows that are not computed are left untouched. */
void cpuref_gemm_nt(const float *a, const float *bt, float *c, int64_t m, int64_t n, int64_t k,
                    int64_t lda, int64_t ldb, int64_t ldc, int64_t bk, int64_t bm,
                    int64_t row_tile_step) {
  const int64_t kp = bk > 0 ? (k / bk) * bk : k;
  const int64_t row_tiles = m / bm;
  const int64_t sampled_tiles = (row_tiles + row_tile_step - 1) / row_tile_step;
  const int64_t sampled_rows = sampled_tiles * bm;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < sampled_rows; ++i) {
    const int64_t row = (i / bm) * row_tile_step * bm + (i % bm);
    const float *ar = a + row * lda;
    for (int64_t col = 0; col < n; ++col) {
      const float *br = bt + col * ldb;
      float s = 0.0f;
      for (int64_t kk = 0; kk < kp; ++kk) {
        float p = ar[kk] * br[kk];
        s = s + p;
      }
      c[row * ldc + col] = s;
    }
  }
}

/* Tile MMA with a seeded accumulator (a2):
 * crates/sile-tile-ir/src/passes/lowering/tile_compute/mma.rs.  Per k-step
 * (one MmaF of a tile_k-deep slice) every cell runs sum = acc[r][c];
 * sum = sum + (a[r][k] * b[k][c]) for k < tile_k; acc[r][c] = sum (the
 * unfused form :25-260, init :213-229; the fused form :262-739 reads the same
 * values straight from the buffers, :483-558 seeding the first k-step of a
 * LoopCarriedSplat from its constant).  Over the k loop of a kernel the
 * accumulator therefore carries one sequential chain per cell, from its seed
 * (a loaded tile, or the splat value) through every product in increasing k,
 * two roundings per step.  This function computes that chain over k < K'
 * ((K / bk) * bk, bk <= 0: K) for a whole [M, N] result:
 *   C[r][c] = fold(acc ? acc[r * ld_acc + c] : acc_value, A[r][k] * B[k][c])
 * with B row-major [K, N] (b_col_major = 0, the reference's layout) or
 * column-major (stored [N, K]).  acc may alias c. */
void cpuref_mma_f32(const float *a, const float *b, const float *acc, float *c, int64_t m,
                    int64_t n, int64_t k, int64_t lda, int64_t ldb, int b_col_major,
                    int64_t ld_acc, float acc_value, int64_t ldc, int64_t bk) {
  const int64_t kp = bk > 0 ? (k / bk) * bk : k;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < m; ++r) {
    for (int64_t cc = 0; cc < n; ++cc) {
      float s = acc ? acc[r * ld_acc + cc] : acc_value;
      for (int64_t kk = 0; kk < kp; ++kk) {
        const float bv = b_col_major ? b[cc * ldb + kk] : b[kk * ldb + cc];
        float p = a[r * lda + kk] * bv;
        s = s + p;
      }
      c[r * ldc + cc] = s;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* a4 / a5: reductions.                                                      */
/* ------------------------------------------------------------------------ */

/* reduce_combine, crates/sile-tile-ir/src/passes/lowering/tile_compute/reduce.rs:10-30:
 * max: acc = (next > acc) ? next : acc   (ordered compare: a NaN `next` never wins)
 * sum: acc = acc + next */
static inline float combine_max(float acc, float next) { return (next > acc) ? next : acc; }

/* Unfused row reduce, reduce.rs:32-112 and the loop form at :116-572:
 * acc = x[r][0]; for c = 1..cols-1: acc = combine(acc, x[r][c]). */
static float reduce_row_seq(const float *row, int64_t cols, int is_max) {
  float acc = row[0];
  for (int64_t c = 1; c < cols; ++c) acc = is_max ? combine_max(acc, row[c]) : acc + row[c];
  return acc;
}

/* llir_vec_reduce_add, crates/sile-backend/src/cpu/codegen.rs:71-86:
 * v0 + v1 + v2 + v3 evaluated left to right. */
static inline float vec4_sum(const float *p) { return ((p[0] + p[1]) + p[2]) + p[3]; }

/* Fused load + sum along axis 1 with extent >= 4,
 * crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:
 *  - extent <= 16 (unrolled, :80-113 with emit_vec_sum_reduce :1142-1172):
 *      acc = vec4_sum(row + 0); acc = acc + vec4_sum(row + 4i) for i < extent/4;
 *  - extent  > 16 (loop, emit_vec_reduce_loop :1182-1256, which steps
 *    lower_reduce_extent_loop_step of
 *    crates/sile-tile-ir/src/passes/lowering/core/emit/tile_loops/single_axis.rs:180-260):
 *      acc = 0.0f; for (idx = 0; idx < extent; idx += 4) acc = acc + vec4_sum(row + idx);
 *    the loop runs while idx < extent, so for extent % 4 != 0 its last
 *    window starts at 4*(extent/4) and reads 4 - extent%4 elements past the
 *    tile row (the next elements of the buffer);
 *  then, in both forms, the scalar tail acc = acc + row[c] for
 *  c = 4*(extent/4) .. extent-1 (:1226-1251), which adds the elements of a
 *  partial last window a second time in the loop form.
 * The threshold is REDUCE_UNROLL_THRESHOLD = 16 (single_axis.rs:8).
 * `avail` is the number of buffer elements from `row` to the end of the
 * buffer: a window element at offset >= avail lies past the buffer (the
 * reference reads whatever memory follows there) and is taken as 0.0f here. */
static float fused_row_sum_vec4(const float *row, int64_t cols, int64_t avail) {
  const int64_t chunks = cols / 4;
  float acc;
  if (cols <= 16) {
    acc = vec4_sum(row);
    for (int64_t i = 1; i < chunks; ++i) acc = acc + vec4_sum(row + 4 * i);
  } else {
    acc = 0.0f;
    for (int64_t idx = 0; idx < cols; idx += 4) {
      if (idx + 4 <= avail) {
        acc = acc + vec4_sum(row + idx);
      } else {
        float w[4];
        for (int j = 0; j < 4; ++j) w[j] = idx + j < avail ? row[idx + j] : 0.0f;
        acc = acc + vec4_sum(w);
      }
    }
  }
  for (int64_t c = chunks * 4; c < cols; ++c) acc = acc + row[c];
  return acc;
}

/* Row reduce over a [rows, cols] matrix with row stride ldx.
 * op 0 = max, 1 = sum in the sequential order (unfused path, reduce.rs),
 * op 2 = sum in the fused load+reduce vec4 order (fused_reduce.rs).
 * x_len = elements of the buffer from x on (>= (rows-1)*ldx + cols): the
 * extent the vec4 loop's last window may read into. */
void cpuref_reduce_rows(int op, const float *x, float *out, int64_t rows, int64_t cols,
                        int64_t ldx, int64_t x_len) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float *row = x + r * ldx;
    if (op == 2 && cols >= 4)
      out[r] = fused_row_sum_vec4(row, cols, x_len - r * ldx);
    else
      out[r] = reduce_row_seq(row, cols, op == 0);
  }
}

/* ------------------------------------------------------------------------ */
/* a6 / a7: softmax.                                                         */
/* ------------------------------------------------------------------------ */

/* One program of the softmax DSL kernel (crates/sile/tests/backend_softmax.rs:3-15),
 * lowered as traced in crates/sile-tile-ir/src/passes/lowering/block.rs:458-513:
 *   tile_x = load_tile_like_2d(x, y): rows gid0*BM.., cols gid1*BN.., stride shape(x)[1]
 *            (crates/sile-tile-ir/src/lower.rs:551-573; tile_memory.rs:164-299)
 *   m_r    = fused load + max fold, x[r][0] first, `>` select (reduce.rs:10-30)
 *   num    = expf(x - m_r) materialised (tile_expr.rs:183-223; codegen.rs:696)
 *   s_r    = unfused sum: num[r][0] + num[r][1] + ... (reduce.rs:32-112)
 *   y      = num / s_r, IEEE division, stored at (gid0, gid1) with stride shape(y)[1]
 *            (tile_memory.rs:114-162) */
static void softmax_program(const float *x, float *y, int64_t ldx, int64_t ldy, int64_t bm,
                            int64_t bn, int64_t gid0, int64_t gid1, float *num) {
  for (int64_t r = 0; r < bm; ++r) {
    const float *xr = x + (gid0 * bm) * ldx + gid1 * bn + r * ldx;
    float *yr = y + (gid0 * bm) * ldy + gid1 * bn + r * ldy;
    float m = xr[0];
    for (int64_t c = 1; c < bn; ++c) m = combine_max(m, xr[c]);
    for (int64_t c = 0; c < bn; ++c) num[c] = expf(xr[c] - m);
    float s = num[0];
    for (int64_t c = 1; c < bn; ++c) s = s + num[c];
    for (int64_t c = 0; c < bn; ++c) yr[c] = num[c] / s;
  }
}

/* sile_kernel_softmax wrapper: buffers = {x, y}; shapes = shape(x) ++ shape(y);
 * tiles_n = shape(y)[1] / BN; total = (shape(y)[0] / BM) * tiles_n
 * (crates/sile-backend/src/cpu/codegen.rs:409-555). */
void cpuref_kernel_softmax(void **buffers, int64_t num_threadgroups, int64_t threads_per_group,
                           const int64_t *shapes, int64_t num_shapes, int64_t bm, int64_t bn) {
  (void)num_shapes;
  const float *x = (const float *)buffers[0];
  float *y = (float *)buffers[1];
  const int64_t tiles_n = shapes[3] / bn;
  const int64_t total = (shapes[2] / bm) * tiles_n;
#pragma omp parallel
  {
    float num_stack[4096];
    float *num = num_stack;
    float *heap = NULL;
    if (bn > 4096) {
      heap = (float *)__builtin_malloc((size_t)bn * sizeof(float));
      num = heap;
    }
#pragma omp for schedule(static)
    for (int64_t tg = 0; tg < num_threadgroups; ++tg) {
      int64_t base = tg * threads_per_group;
      for (int64_t t = 0; t < threads_per_group; ++t) {
        int64_t pid = base + t;
        if (pid < total)
          softmax_program(x, y, shapes[1], shapes[3], bm, bn, pid / tiles_n, pid % tiles_n, num);
      }
    }
    if (heap) __builtin_free(heap);
  }
}

/* Row softmax over a [rows, cols] matrix: the softmax program with BM = 1 and
 * BN = cols, one program per row (the only configuration in which the DSL
 * kernel is a row softmax: BN must equal the row width). */
void cpuref_softmax_rows(const float *x, float *y, int64_t rows, int64_t cols, int64_t ldx,
                         int64_t ldy) {
#pragma omp parallel
  {
    float *num = (float *)__builtin_malloc((size_t)cols * sizeof(float));
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; ++r) softmax_program(x, y, ldx, ldy, 1, cols, r, 0, num);
    __builtin_free(num);
  }
}

/* ------------------------------------------------------------------------ */
/* a8: parallel reduce with atomic add.                                      */
/* ------------------------------------------------------------------------ */

/* sile_kernel_parallel_reduce for crates/sile/examples/parallel_reduce.rs:3-9
 * (test crates/sile/tests/backend_parallel_reduce.rs:3-9):
 *   the output is only written by an atomic add, so infer_tile_plan finds no
 *   tile store (crates/sile-backend/src/emit.rs:241-296) and the wrapper falls
 *   back to total = shape(first buffer)[0], gid0 = pid
 *   (crates/sile-backend/src/cpu/codegen.rs:479-503, 517-531);
 *   tile = a[pid*TILE .. pid*TILE+TILE) (rank-1 addressing, tile_memory.rs:175-188);
 *   sum  = fused load+reduce in the vec4 order (fused_reduce.rs:80-113, 1182-1256),
 *          whose loop form reads up to 3 elements past the tile: the next
 *          program's first elements, or 0.0f past the end of a (see
 *          fused_row_sum_vec4);
 *   out[0] += sum under `#pragma omp atomic update` (codegen.rs:245-253).
 * The order of the atomic adds across programs is unspecified in the reference. */
void cpuref_kernel_parallel_reduce(void **buffers, int64_t num_threadgroups,
                                   int64_t threads_per_group, const int64_t *shapes,
                                   int64_t num_shapes, int64_t tile) {
  (void)num_shapes;
  const float *a = (const float *)buffers[0];
  float *out = (float *)buffers[1];
  const int64_t total = shapes[0];
#pragma omp parallel for schedule(static)
  for (int64_t tg = 0; tg < num_threadgroups; ++tg) {
    int64_t base = tg * threads_per_group;
    for (int64_t t = 0; t < threads_per_group; ++t) {
      int64_t pid = base + t;
      if (pid < total) {
        /* extent < 4 never takes the vec4 path (fused_reduce.rs:80) */
        float s = tile >= 4 ? fused_row_sum_vec4(a + pid * tile, tile, shapes[0] - pid * tile)
                            : reduce_row_seq(a + pid * tile, tile, 0);
#pragma omp atomic update
        out[0] += s;
      }
    }
  }
}

/* Per-program partial sums of parallel_reduce (the value each program adds
 * atomically) over a of `len` elements, so the in-tile order can be compared
 * bit for bit. */
void cpuref_parallel_reduce_partials(const float *a, float *partials, int64_t programs,
                                     int64_t tile, int64_t len) {
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < programs; ++p)
    partials[p] = tile >= 4 ? fused_row_sum_vec4(a + p * tile, tile, len - p * tile)
                            : reduce_row_seq(a + p * tile, tile, 0);
}

/* ------------------------------------------------------------------------ */
/* a9: causal attention forward (new; no reference kernel).                  */
/* ------------------------------------------------------------------------ */

/* The attention program written in sile's DSL (no causal mask: the DSL has
 * no iota or select on indices), K given transposed as kt [D, S_k]:
 *
 *   let pid = tile::id().0;
 *   let qt = q.load_tile([BM, D], [pid, 0]);
 *   let mut m = <m0 splat [BM, 1]>; let mut l = constant(0.0, [BM, 1]);
 *   let mut acc = constant(0.0, [BM, D]);
 *   for j in 0..kt.shape()[1] / BN {
 *       let s = mma(qt, kt.load_tile([D, BN], [0, j]), constant(0.0, [BM, BN]))
 *               * constant(scale, [BM, BN]);
 *       let m_new = max_tile(m, reduce_max(s, 1));
 *       let p = exp(s - m_new.broadcast([BM, BN]));
 *       let alpha = exp(m - m_new);
 *       l = l * alpha + reduce_sum(p, 1);
 *       acc = mma(p, v.load_tile([BN, D], [j, 0]), acc * alpha.broadcast([BM, D]));
 *       m = m_new;
 *   }
 *   o.store(acc / l.broadcast([BM, D]));
 *
 * with the reference's op semantics: mma = a per-cell chain from its seed,
 * s = s + a*b in increasing k with two roundings (tile_compute/mma.rs:25-739);
 * max_tile(a, b) = a >= b ? a : b (crates/sile-tile-ir/src/lower.rs:619-641);
 * the row max and row sum are the folds from element 0 (reduce.rs:10-112);
 * exp = expf; the maps round each operation.  Rows q_begin..q_end of
 * q [*, ldq], kt [D, ldkt], v [*, ldv], o [*, ldo]; keys
 * 0 .. (s_k / bn) * bn (the loop bound truncates). */
void cpuref_dsl_attention_f32(const float *q, int64_t ldq, const float *kt, int64_t ldkt,
                              const float *v, int64_t ldv, float *o, int64_t ldo, int64_t d,
                              int64_t s_k, int64_t bn, float scale, float m0, int64_t q_begin,
                              int64_t q_end) {
  const int64_t blocks = s_k / bn;
#pragma omp parallel
  {
    float *sc = (float *)__builtin_malloc((size_t)bn * sizeof(float));
    float *acc = (float *)__builtin_malloc((size_t)d * sizeof(float));
#pragma omp for schedule(dynamic, 4)
    for (int64_t i = q_begin; i < q_end; ++i) {
      const float *qi = q + i * ldq;
      float m = m0, l = 0.0f;
      for (int64_t t = 0; t < d; ++t) acc[t] = 0.0f;
      for (int64_t j = 0; j < blocks; ++j) {
        for (int64_t c = 0; c < bn; ++c) {
          float sum = 0.0f;
          for (int64_t t = 0; t < d; ++t) {
            float prod = qi[t] * kt[t * ldkt + j * bn + c];
            sum = sum + prod;
          }
          sc[c] = sum * scale;
        }
        const float rmax = reduce_row_seq(sc, bn, 1);
        const float m_new = m >= rmax ? m : rmax;
        for (int64_t c = 0; c < bn; ++c) sc[c] = expf(sc[c] - m_new);
        const float alpha = expf(m - m_new);
        const float rsum = reduce_row_seq(sc, bn, 0);
        const float la = l * alpha;
        l = la + rsum;
        for (int64_t t = 0; t < d; ++t) {
          float a = acc[t] * alpha;
          for (int64_t c = 0; c < bn; ++c) {
            float prod = sc[c] * v[(j * bn + c) * ldv + t];
            a = a + prod;
          }
          acc[t] = a;
        }
        m = m_new;
      }
      for (int64_t t = 0; t < d; ++t) o[i * ldo + t] = acc[t] / l;
    }
    __builtin_free(acc);
    __builtin_free(sc);
  }
}

/* The matvec program of crates/sile/examples/mlp.rs:26-44 (BM rows per
 * program; the row order does not matter, every row is independent):
 *   acc = constant(seed, [BM]); k_tiles = x.shape()[1] / BK;
 *   for k < k_tiles: acc = acc + reduce_sum(x[rows, k-tile] * broadcast(y[k-tile]), 1)
 * The product map feeds the reduce alone, so the reduce is the fused
 * map + reduce (crates/sile-tile-ir/src/passes/lowering/block.rs:491-510,
 * tile_compute/fused_reduce.rs:189-293): p = x0*y0, then p = p + xi*yi for
 * i = 1 .. BK-1 in order, every product and sum rounded (no contraction);
 * the carried add is the map addf of the [1, BM] accumulator and the
 * [BM, 1] reduce, element r of both (lower.rs:643-691; the [BM, 1] tile's
 * element (0, r) is its r-th element in row-major order).  Rows 0 .. m of
 * x [*, ldx], y [*], out [m]; tiles = k / bk whole tiles of K. */
void cpuref_dsl_matvec_f32(const float *x, int64_t ldx, const float *y, float *out, int64_t m,
                           int64_t k, int64_t bk, float seed) {
  const int64_t tiles = bk > 0 ? k / bk : 0;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < m; ++r) {
    const float *xr = x + r * ldx;
    float acc = seed;
    for (int64_t t = 0; t < tiles; ++t) {
      const float *xt = xr + t * bk, *yt = y + t * bk;
      float p = xt[0] * yt[0];
      for (int64_t i = 1; i < bk; ++i) {
        const float prod = xt[i] * yt[i];
        p = p + prod;
      }
      acc = acc + p;
    }
    out[r] = acc;
  }
}

/* Naive fp32 causal attention for one (batch, head) slice, queries
 * [q_begin, q_end).  Q, K, V, O are [S, D] row-major.  For query i:
 *   s_j = (sum_d q[i][d]*k[j][d], accumulated from 0.0f in increasing d with two
 *          roundings, as the canonical matmul, canonical_matmul.rs:226-370) * scale,
 *          for j <= i (causal: keys after the query are masked out)
 *   m   = max fold over s_0..s_i (reduce.rs:10-30)
 *   p_j = expf(s_j - m); l = p_0 + p_1 + ... (softmax composition of
 *         crates/sile/tests/backend_softmax.rs:3-15, as softmax_program above)
 *   o[d] = (sum_j p_j * v[j][d], from 0.0f in increasing j) / l
 * With causal = 0 every key is visible. */
void cpuref_attention_fwd(const float *q, const float *k, const float *v, float *o, int64_t s_len,
                          int64_t d, float scale, int causal, int64_t q_begin, int64_t q_end) {
#pragma omp parallel
  {
    float *sc = (float *)__builtin_malloc((size_t)s_len * sizeof(float));
#pragma omp for schedule(dynamic, 4)
    for (int64_t i = q_begin; i < q_end; ++i) {
      const int64_t nkeys = causal ? i + 1 : s_len;
      const float *qi = q + i * d;
      for (int64_t j = 0; j < nkeys; ++j) {
        const float *kj = k + j * d;
        float s = 0.0f;
        for (int64_t t = 0; t < d; ++t) {
          float p = qi[t] * kj[t];
          s = s + p;
        }
        sc[j] = s * scale;
      }
      float m = sc[0];
      for (int64_t j = 1; j < nkeys; ++j) m = combine_max(m, sc[j]);
      for (int64_t j = 0; j < nkeys; ++j) sc[j] = expf(sc[j] - m);
      float l = sc[0];
      for (int64_t j = 1; j < nkeys; ++j) l = l + sc[j];
      float *oi = o + i * d;
      for (int64_t t = 0; t < d; ++t) {
        float acc = 0.0f;
        for (int64_t j = 0; j < nkeys; ++j) {
          float p = sc[j] * v[j * d + t];
          acc = acc + p;
        }
        oi[t] = acc / l;
      }
    }
    __builtin_free(sc);
  }
}

/* ------------------------------------------------------------------------ */
/* Number formats of the new dtypes (bf16, fp8 e4m3fn).                      */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16, round to nearest even; NaN stays a (quiet) NaN. */
void cpuref_bf16_from_f32(const float *x, uint16_t *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u = f32_bits(x[i]);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      out[i] = (uint16_t)((u >> 16) | 0x40u);
    } else {
      uint32_t lsb = (u >> 16) & 1u;
      out[i] = (uint16_t)((u + 0x7fffu + lsb) >> 16);
    }
  }
}

void cpuref_f32_from_bf16(const uint16_t *x, float *out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = bits_f32((uint32_t)x[i] << 16);
}

/* OCP 8-bit e4m3fn ("fn": finite, no infinities): 1 sign, 4 exponent bits
 * (bias 7), 3 mantissa bits; exponent field 0 holds subnormals m * 2^-9;
 * S.1111.111 is NaN; the largest finite value is S.1111.110 = 448. */
static float e4m3_decode_one(uint8_t b) {
  const int sign = b >> 7, e = (b >> 3) & 0xf, m = b & 7;
  float mag;
  if (e == 15 && m == 7) return NAN;
  if (e == 0)
    mag = ldexpf((float)m, -9);
  else
    mag = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -mag : mag;
}

/* fp32 -> e4m3fn with round-to-nearest-even and saturation to +-448
 * ("rne_sat"); NaN encodes as 0x7F. */
static uint8_t e4m3_encode_one(float x) {
  if (isnan(x)) return 0x7f;
  const uint8_t sign = signbit(x) ? 0x80 : 0x00;
  float a = fabsf(x);
  if (a >= 464.0f) return sign | 0x7e; /* 464 = midpoint 448..480: everything above saturates */
  if (a < ldexpf(1.0f, -6)) {
    /* subnormal range: quantum 2^-9; nearbyintf rounds half to even.  A result
     * of 8 is the smallest normal (code 0x08), which the same code expresses. */
    float q = nearbyintf(ldexpf(a, 9));
    return sign | (uint8_t)q;
  }
  int e;
  float fr = frexpf(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  int ex = e - 1;           /* a = (2*fr) * 2^ex, 2*fr in [1, 2) */
  float mant = (2.0f * fr - 1.0f) * 8.0f;
  float q = nearbyintf(mant);
  if (q >= 8.0f) {
    q = 0.0f;
    ex += 1;
  }
  int field = ex + 7;
  if (field > 15 || (field == 15 && q > 6.0f)) return sign | 0x7e;
  return sign | (uint8_t)((field << 3) | (int)q);
}

/* q = rne_sat(x / scale), the per-tensor quantisation of the fp8 configuration
 * (scale = amax / 448). */
void cpuref_e4m3_encode(const float *x, uint8_t *out, int64_t n, float scale) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = e4m3_encode_one(x[i] / scale);
}

void cpuref_e4m3_decode(const uint8_t *x, float *out, int64_t n, float scale) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = e4m3_decode_one(x[i]) * scale;
}

/* Threads the OpenMP runtime will use (reported with every CPU timing). */
int cpuref_num_threads(void) { return omp_get_max_threads(); }
