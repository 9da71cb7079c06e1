// Row softmax and row reduce for gfx950 (HBM-bound).
//
// Semantics follow the softmax DSL kernel (crates/sile/tests/backend_softmax.rs:3-15)
// with BN equal to the row width, i.e. a row softmax, and the reduce ops
// ReduceMax / ReduceSum (crates/sile-tile-ir/src/ir.rs:128-262):
//   m = max_c x[c]; e[c] = exp(x[c] - m); s = sum_c e[c]; y[c] = e[c] / s
// with fp32 max, exp and sum for every input type.
//
// Every kernel reads x from HBM once and writes y once (4 bytes per fp16
// element in total), with non-temporal 128-bit loads and stores (streaming
// data, no reuse).  A lane's chunk is E consecutive elements (E = 8 for
// 16-bit inputs, 4 for fp32: one 128-bit access), and each load instruction
// of a wave reads one contiguous KiB of the row.
//  * rows of 256 / 512 / 1024 threads x 2 chunks (4096, 8192, 16384 16-bit
//    or 2048, 4096, 8192 fp32 elements): one row per workgroup, the shape of
//    the fastest copy measured on the device; the row max and sum are wave
//    all-reductions plus one exchange of per-wave partials through LDS;
//  * other widths: kL lanes per row for rows of up to 32 chunks (4..32 rows
//    per wave), one wave per row with the row in registers (whole chunks, or
//    a masked last chunk) up to 8192, one row per 1024-thread workgroup with
//    a masked last chunk up to 1024 * 8 chunks, two passes over the row by
//    one workgroup beyond that; a three-pass element-wise kernel when the
//    rows are not 16-byte aligned.
// Wave all-reductions use DPP row permutes (common.h); exp(x - m) is
// 2^((x - m) * log2 e) on v_exp_f32.
#include "common.h"

using namespace sile;

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

template <int kT>
struct Elem;
template <>
struct Elem<kF32> {
  using Storage = float;
  SILE_DEV static void load8(const float* p, float v[8]) {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 4));
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
    v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
  }
  SILE_DEV static void store8(float* p, const float v[8]) {
    f32x4 a = {v[0], v[1], v[2], v[3]}, b = {v[4], v[5], v[6], v[7]};
    __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p + 4));
  }
  SILE_DEV static void load4(const float* p, float v[4]) {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  }
  SILE_DEV static void store4(float* p, const float v[4]) {
    f32x4 a = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
  }
  SILE_DEV static float load1(const float* p) { return *p; }
  SILE_DEV static void store1(float* p, float v) { *p = v; }
};
template <>
struct Elem<kF16> {
  using Storage = uint16_t;
  SILE_DEV static void load8(const uint16_t* p, float v[8]) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // copy the element out first: hipcc's __builtin_bit_cast of an
      // ext_vector element reads element 0 whatever the index
      const uint32_t u = w[i];
      const f16x2 h = __builtin_bit_cast(f16x2, u);
      v[2 * i] = (float)h[0];
      v[2 * i + 1] = (float)h[1];
    }
  }
  SILE_DEV static void store8(uint16_t* p, const float v[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_f16x2(v[2 * i], v[2 * i + 1]);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  }
  SILE_DEV static float load1(const uint16_t* p) { return f16_to_f32(*p); }
  SILE_DEV static void store1(uint16_t* p, float v) { *p = f16_rne(v); }
};
template <>
struct Elem<kBF16> {
  using Storage = uint16_t;
  SILE_DEV static void load8(const uint16_t* p, float v[8]) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bits_f32(w[i] << 16);
      v[2 * i + 1] = bits_f32(w[i] & 0xffff0000u);
    }
  }
  SILE_DEV static void store8(uint16_t* p, const float v[8]) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
  }
  SILE_DEV static float load1(const uint16_t* p) { return bf16_to_f32(*p); }
  SILE_DEV static void store1(uint16_t* p, float v) { *p = bf16_rne(v); }
};

// Elements per lane chunk: one 16-byte access of the input, so that each
// load instruction of the wave reads 1 KiB of contiguous row.  fp32 -> fp32
// uses 4; the 16-bit inputs use 8.
template <int kIn, int kOut>
constexpr int chunk_elems() {
  return kIn == kF32 && kOut == kF32 ? 4 : 8;
}

template <int kT, int kE>
SILE_DEV void load_chunk(const typename Elem<kT>::Storage* p, float* v) {
  if constexpr (kE == 4)
    Elem<kT>::load4(p, v);
  else
    Elem<kT>::load8(p, v);
}
template <int kT, int kE>
SILE_DEV void store_chunk(typename Elem<kT>::Storage* p, const float* v) {
  if constexpr (kE == 4)
    Elem<kT>::store4(p, v);
  else
    Elem<kT>::store8(p, v);
}

// y = e / s.  fp32 outputs use IEEE division, as the reference's Div
// (crates/sile-tile-ir/src/passes/lowering/tile_expr.rs:646-813); a 16-bit
// output is rounded once more afterwards, so e * (1 / s), within an fp32 ulp
// of e / s, stands in for it there.  exp is the device's v_exp_f32, not the
// host libm expf of the reference (whose bits are not pinned by it).
template <int kOut>
SILE_DEV float normalise(float e, float s, float inv) {
  if constexpr (kOut == kF32)
    return e / s;
  else
    return e * inv;
}

// ---- register-resident row softmax: cols == kChunks * 64 * chunk_elems ----
template <int kIn, int kOut, int kChunks>
__device__ __forceinline__ void softmax_row_regs(const typename Elem<kIn>::Storage* __restrict__ xr,
                                                 typename Elem<kOut>::Storage* __restrict__ yr,
                                                 int lane) {
  constexpr int kE = chunk_elems<kIn, kOut>();
  float v[kChunks][kE];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) load_chunk<kIn, kE>(xr + (j * 64 + lane) * kE, v[j]);
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) m = fmax_ordered(m, v[j][i]);
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      v[j][i] = exp2_fast((v[j][i] - m) * kLog2e);
      s += v[j][i];
    }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
#pragma unroll
    for (int i = 0; i < kE; ++i) v[j][i] = normalise<kOut>(v[j][i], s, inv);
    store_chunk<kOut, kE>(yr + (j * 64 + lane) * kE, v[j]);
  }
}

// ---- register-resident row softmax of any width up to kChunks * 64 * E ----
// Chunks wholly inside the row are 128-bit accesses; the one chunk the row
// ends in is read and written element by element; positions past the row are
// -inf (exp 0) and never stored.
template <int kIn, int kOut, int kChunks>
__device__ __forceinline__ void softmax_row_masked(const typename Elem<kIn>::Storage* __restrict__ xr,
                                                   typename Elem<kOut>::Storage* __restrict__ yr,
                                                   int lane, int cols) {
  constexpr int kE = chunk_elems<kIn, kOut>();
  float v[kChunks][kE];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c0 = (j * 64 + lane) * kE;
    if (c0 + kE <= cols) {
      load_chunk<kIn, kE>(xr + c0, v[j]);
    } else {
#pragma unroll
      for (int i = 0; i < kE; ++i)
        v[j][i] = c0 + i < cols ? Elem<kIn>::load1(xr + c0 + i) : -__builtin_inff();
    }
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) m = fmax_ordered(m, v[j][i]);
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      v[j][i] = exp2_fast((v[j][i] - m) * kLog2e);  // -inf -> 0
      s += v[j][i];
    }
  s = wave_sum(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int c0 = (j * 64 + lane) * kE;
#pragma unroll
    for (int i = 0; i < kE; ++i) v[j][i] = normalise<kOut>(v[j][i], s, inv);
    if (c0 + kE <= cols) {
      store_chunk<kOut, kE>(yr + c0, v[j]);
    } else {
#pragma unroll
      for (int i = 0; i < kE; ++i)
        if (c0 + i < cols) Elem<kOut>::store1(yr + c0 + i, v[j][i]);
    }
  }
}

template <int kIn, int kOut, int kChunks>
__device__ __forceinline__ void softmax_rows_masked_kernel(const void* x, void* y, int64_t rows,
                                                           int64_t cols, int64_t ldx,
                                                           int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  softmax_row_masked<kIn, kOut, kChunks>(static_cast<const TI*>(x) + row * ldx,
                                         static_cast<TO*>(y) + row * ldy, lane, (int)cols);
}

template <int kIn, int kOut, int kChunks>
__device__ __forceinline__ void softmax_rows_regs_kernel(const void* x, void* y, int64_t rows,
                                                         int64_t ldx, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  softmax_row_regs<kIn, kOut, kChunks>(static_cast<const TI*>(x) + row * ldx,
                                       static_cast<TO*>(y) + row * ldy, lane);
}

// ---- any width: three passes over the row (L2-resident after the first) ----
template <int kIn, int kOut>
__device__ __forceinline__ void softmax_rows_generic_kernel(const void* x, void* y, int64_t rows,
                                                            int64_t cols, int64_t ldx,
                                                            int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  TO* yr = static_cast<TO*>(y) + row * ldy;
  float m = -__builtin_inff();
  for (int64_t c = lane; c < cols; c += 64) m = fmax_ordered(m, Elem<kIn>::load1(xr + c));
  m = wave_max(m);
  float s = 0.0f;
  for (int64_t c = lane; c < cols; c += 64) s += exp2_fast((Elem<kIn>::load1(xr + c) - m) * kLog2e);
  s = wave_sum(s);
  const float inv = 1.0f / s;
  for (int64_t c = lane; c < cols; c += 64)
    Elem<kOut>::store1(
        yr + c, normalise<kOut>(exp2_fast((Elem<kIn>::load1(xr + c) - m) * kLog2e), s, inv));
}

#define SILE_SOFTMAX_REGS(NAME, IN, OUT, CH)                                                 \
  extern "C" __global__ __launch_bounds__(256) void NAME(const void* x, void* y, int64_t rows, \
                                                         int64_t ldx, int64_t ldy) {         \
    softmax_rows_regs_kernel<IN, OUT, CH>(x, y, rows, ldx, ldy);                             \
  }
#define SILE_SOFTMAX_WIDTHS(TAG, IN, OUT)                      \
  SILE_SOFTMAX_REGS(sile_softmax_rows_##TAG##_c1, IN, OUT, 1)   \
  SILE_SOFTMAX_REGS(sile_softmax_rows_##TAG##_c2, IN, OUT, 2)   \
  SILE_SOFTMAX_REGS(sile_softmax_rows_##TAG##_c4, IN, OUT, 4)   \
  SILE_SOFTMAX_REGS(sile_softmax_rows_##TAG##_c8, IN, OUT, 8)   \
  SILE_SOFTMAX_REGS(sile_softmax_rows_##TAG##_c16, IN, OUT, 16) \
  extern "C" __global__ __launch_bounds__(256) void sile_softmax_rows_##TAG##_any(          \
      const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy) {      \
    softmax_rows_generic_kernel<IN, OUT>(x, y, rows, cols, ldx, ldy);                      \
  }

SILE_SOFTMAX_WIDTHS(f16_f16, kF16, kF16)
SILE_SOFTMAX_WIDTHS(bf16_bf16, kBF16, kBF16)
SILE_SOFTMAX_WIDTHS(f32_f32, kF32, kF32)
SILE_SOFTMAX_REGS(sile_softmax_rows_f32_f32_c32, kF32, kF32, 32)
SILE_SOFTMAX_WIDTHS(f16_f32, kF16, kF32)

#define SILE_SOFTMAX_MASKED(NAME, IN, OUT, CH)                                                 \
  extern "C" __global__ __launch_bounds__(256) void NAME(const void* x, void* y, int64_t rows,   \
                                                         int64_t cols, int64_t ldx, int64_t ldy) { \
    softmax_rows_masked_kernel<IN, OUT, CH>(x, y, rows, cols, ldx, ldy);                         \
  }
#define SILE_SOFTMAX_MASKED_WIDTHS(TAG, IN, OUT)                  \
  SILE_SOFTMAX_MASKED(sile_softmax_rows_##TAG##_m1, IN, OUT, 1)   \
  SILE_SOFTMAX_MASKED(sile_softmax_rows_##TAG##_m2, IN, OUT, 2)   \
  SILE_SOFTMAX_MASKED(sile_softmax_rows_##TAG##_m4, IN, OUT, 4)   \
  SILE_SOFTMAX_MASKED(sile_softmax_rows_##TAG##_m8, IN, OUT, 8)   \
  SILE_SOFTMAX_MASKED(sile_softmax_rows_##TAG##_m16, IN, OUT, 16)
SILE_SOFTMAX_MASKED_WIDTHS(f16_f16, kF16, kF16)
SILE_SOFTMAX_MASKED_WIDTHS(bf16_bf16, kBF16, kBF16)
SILE_SOFTMAX_MASKED_WIDTHS(f32_f32, kF32, kF32)
SILE_SOFTMAX_MASKED(sile_softmax_rows_f32_f32_m32, kF32, kF32, 32)
SILE_SOFTMAX_MASKED_WIDTHS(f16_f32, kF16, kF32)


// ---- one row per workgroup: cols == kThreads * kChunks * E ----
// The copy shape that moves the most bytes on MI355X (two 16-byte chunks per
// thread, 256-512 threads per 8-16 KiB) with the softmax's arithmetic in
// between: chunk j of thread t at column (j * kThreads + t) * E, loaded
// non-temporally, reduced to the row max and the row sum through a wave
// all-reduction and one exchange of the per-wave partials in LDS each, then
// exp, normalised and stored non-temporally.  The row is read once and
// written once, as in the wave-per-row kernels, but each wave keeps only
// kChunks chunks in flight and many more waves run.
template <int kIn, int kOut, int kThreads, int kChunks>
__device__ __forceinline__ void softmax_rows_block_kernel(const void* x, void* y, int64_t rows,
                                                          int64_t ldx, int64_t ldy) {
  constexpr int kE = chunk_elems<kIn, kOut>();
  constexpr int kWaves = kThreads / 64;
  __shared__ float part[2][kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  TO* yr = static_cast<TO*>(y) + row * ldy;
  float v[kChunks][kE];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) load_chunk<kIn, kE>(xr + (j * kThreads + t) * kE, v[j]);
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) m = fmax_ordered(m, v[j][i]);
  m = wave_max(m);
  if (lane == 0) part[0][wave] = m;
  __syncthreads();
  m = part[0][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmax_ordered(m, part[0][w]);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      v[j][i] = exp2_fast((v[j][i] - m) * kLog2e);
      s += v[j][i];
    }
  s = wave_sum(s);
  if (lane == 0) part[1][wave] = s;
  __syncthreads();
  s = part[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s += part[1][w];
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
#pragma unroll
    for (int i = 0; i < kE; ++i) v[j][i] = normalise<kOut>(v[j][i], s, inv);
    store_chunk<kOut, kE>(yr + (j * kThreads + t) * kE, v[j]);
  }
}

#define SILE_SOFTMAX_BLOCK(NAME, IN, OUT, T)                                                 \
  extern "C" __global__ __launch_bounds__(T) void NAME(const void* x, void* y, int64_t rows,   \
                                                       int64_t ldx, int64_t ldy) {           \
    softmax_rows_block_kernel<IN, OUT, T, 2>(x, y, rows, ldx, ldy);                          \
  }
#define SILE_SOFTMAX_BLOCK_WIDTHS(TAG, IN, OUT)                    \
  SILE_SOFTMAX_BLOCK(sile_softmax_rows_##TAG##_b256, IN, OUT, 256) \
  SILE_SOFTMAX_BLOCK(sile_softmax_rows_##TAG##_b512, IN, OUT, 512) \
  SILE_SOFTMAX_BLOCK(sile_softmax_rows_##TAG##_b1024, IN, OUT, 1024)
SILE_SOFTMAX_BLOCK_WIDTHS(f16_f16, kF16, kF16)
SILE_SOFTMAX_BLOCK_WIDTHS(bf16_bf16, kBF16, kBF16)
SILE_SOFTMAX_BLOCK_WIDTHS(f32_f32, kF32, kF32)
SILE_SOFTMAX_BLOCK_WIDTHS(f16_f32, kF16, kF32)

// ---- narrow rows: kL lanes per row, one chunk per lane ----
// cols <= kL * E; a wave holds 64 / kL rows and a workgroup of 4 waves
// 256 / kL, so short rows still fill whole load instructions.  The row max
// and sum are reductions inside kL-lane groups (DPP quad / half-row / row
// permutes, a 16-lane swizzle for 32); every lane takes part in them, rows
// past the last only neither load nor store.
template <int kL>
SILE_DEV float group_max(float v) {
  v = fmax_ordered(v, dpp<kDppXor1>(v));
  v = fmax_ordered(v, dpp<kDppXor2>(v));
  if constexpr (kL >= 8) v = fmax_ordered(v, dpp<kDppHalfMirror>(v));
  if constexpr (kL >= 16) v = fmax_ordered(v, dpp<kDppMirror>(v));
  if constexpr (kL >= 32) v = fmax_ordered(v, swizzle_xor16(v));
  return v;
}
template <int kL>
SILE_DEV float group_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  if constexpr (kL >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (kL >= 16) v += dpp<kDppMirror>(v);
  if constexpr (kL >= 32) v += swizzle_xor16(v);
  return v;
}

template <int kIn, int kOut, int kL>
__device__ __forceinline__ void softmax_rows_narrow_kernel(const void* x, void* y, int64_t rows,
                                                           int64_t cols, int64_t ldx,
                                                           int64_t ldy) {
  static_assert(kL == 4 || kL == 8 || kL == 16 || kL == 32, "lanes per row");
  constexpr int kE = chunk_elems<kIn, kOut>();
  const int lane = threadIdx.x & 63, li = lane % kL;
  const int64_t row = (int64_t)blockIdx.x * (256 / kL) + (threadIdx.x >> 6) * (64 / kL) + lane / kL;
  const bool live = row < rows;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  const int c0 = li * kE;
  float v[kE];
  if (live && c0 + kE <= cols) {
    load_chunk<kIn, kE>(static_cast<const TI*>(x) + row * ldx + c0, v);
  } else {
#pragma unroll
    for (int i = 0; i < kE; ++i)
      v[i] = live && c0 + i < cols ? Elem<kIn>::load1(static_cast<const TI*>(x) + row * ldx + c0 + i)
                                   : -__builtin_inff();
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kE; ++i) m = fmax_ordered(m, v[i]);
  m = group_max<kL>(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kE; ++i) {
    v[i] = exp2_fast((v[i] - m) * kLog2e);   // -inf -> 0
    s += v[i];
  }
  s = group_sum<kL>(s);
  if (!live) return;
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < kE; ++i) v[i] = normalise<kOut>(v[i], s, inv);
  TO* yr = static_cast<TO*>(y) + row * ldy;
  if (c0 + kE <= cols) {
    store_chunk<kOut, kE>(yr + c0, v);
  } else {
#pragma unroll
    for (int i = 0; i < kE; ++i)
      if (c0 + i < cols) Elem<kOut>::store1(yr + c0 + i, v[i]);
  }
}

#define SILE_SOFTMAX_NARROW(NAME, IN, OUT, L)                                                    \
  extern "C" __global__ __launch_bounds__(256) void NAME(const void* x, void* y, int64_t rows,   \
                                                         int64_t cols, int64_t ldx, int64_t ldy) { \
    softmax_rows_narrow_kernel<IN, OUT, L>(x, y, rows, cols, ldx, ldy);                          \
  }
#define SILE_SOFTMAX_NARROW_WIDTHS(TAG, IN, OUT)                 \
  SILE_SOFTMAX_NARROW(sile_softmax_rows_##TAG##_n4, IN, OUT, 4)   \
  SILE_SOFTMAX_NARROW(sile_softmax_rows_##TAG##_n8, IN, OUT, 8)   \
  SILE_SOFTMAX_NARROW(sile_softmax_rows_##TAG##_n16, IN, OUT, 16) \
  SILE_SOFTMAX_NARROW(sile_softmax_rows_##TAG##_n32, IN, OUT, 32)
SILE_SOFTMAX_NARROW_WIDTHS(f16_f16, kF16, kF16)
SILE_SOFTMAX_NARROW_WIDTHS(bf16_bf16, kBF16, kBF16)
SILE_SOFTMAX_NARROW_WIDTHS(f32_f32, kF32, kF32)
SILE_SOFTMAX_NARROW_WIDTHS(f16_f32, kF16, kF32)

// ---- wide rows: one row per workgroup of 1024 threads ----
// Masked form of the row-per-workgroup kernel for any width up to
// 1024 * kChunks * E: chunk j of thread t at column (j * 1024 + t) * E, whole
// chunks as 16-byte accesses, the chunk the row ends in element by element,
// positions past the row -inf (exp 0) and never stored.
template <int kIn, int kOut, int kChunks>
__device__ __forceinline__ void softmax_rows_wide_regs_kernel(const void* x, void* y,
                                                              int64_t rows, int64_t cols,
                                                              int64_t ldx, int64_t ldy) {
  constexpr int kT = 1024;
  constexpr int kE = chunk_elems<kIn, kOut>();
  constexpr int kWaves = kT / 64;
  __shared__ float part[2][kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  TO* yr = static_cast<TO*>(y) + row * ldy;
  float v[kChunks][kE];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int64_t c0 = ((int64_t)j * kT + t) * kE;
    if (c0 + kE <= cols) {
      load_chunk<kIn, kE>(xr + c0, v[j]);
    } else {
#pragma unroll
      for (int i = 0; i < kE; ++i)
        v[j][i] = c0 + i < cols ? Elem<kIn>::load1(xr + c0 + i) : -__builtin_inff();
    }
  }
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) m = fmax_ordered(m, v[j][i]);
  m = wave_max(m);
  if (lane == 0) part[0][wave] = m;
  __syncthreads();
  m = part[0][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmax_ordered(m, part[0][w]);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kChunks; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      v[j][i] = exp2_fast((v[j][i] - m) * kLog2e);
      s += v[j][i];
    }
  s = wave_sum(s);
  if (lane == 0) part[1][wave] = s;
  __syncthreads();
  s = part[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s += part[1][w];
  const float inv = 1.0f / s;
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int64_t c0 = ((int64_t)j * kT + t) * kE;
#pragma unroll
    for (int i = 0; i < kE; ++i) v[j][i] = normalise<kOut>(v[j][i], s, inv);
    if (c0 + kE <= cols) {
      store_chunk<kOut, kE>(yr + c0, v[j]);
    } else {
#pragma unroll
      for (int i = 0; i < kE; ++i)
        if (c0 + i < cols) Elem<kOut>::store1(yr + c0 + i, v[j][i]);
    }
  }
}

// Rows past 1024 * 8 * E: two passes over the row by one workgroup of 1024
// threads, 16-byte accesses.  Pass 1 keeps a running (max, sum) per thread
// (the sum rescaled when the max grows), then the workgroup combines them:
// M = max of the maxima, S = sum of sum_t * exp(m_t - M).  Pass 2 reads the
// row again (mostly from L2 / MALL) and writes exp(x - M) / S.  3 row
// accesses per element instead of 2.
template <int kIn, int kOut>
__device__ __forceinline__ void softmax_rows_wide_kernel(const void* x, void* y, int64_t rows,
                                                         int64_t cols, int64_t ldx,
                                                         int64_t ldy) {
  constexpr int kT = 1024;
  constexpr int kE = chunk_elems<kIn, kOut>();
  constexpr int kWaves = kT / 64;
  __shared__ float part[2][kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  using TO = typename Elem<kOut>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  TO* yr = static_cast<TO*>(y) + row * ldy;
  auto load = [&](int64_t c0, float (&v)[kE]) {
    if (c0 + kE <= cols) {
      load_chunk<kIn, kE>(xr + c0, v);
    } else {
#pragma unroll
      for (int i = 0; i < kE; ++i)
        v[i] = c0 + i < cols ? Elem<kIn>::load1(xr + c0 + i) : -__builtin_inff();
    }
  };
  float m = -__builtin_inff(), s = 0.0f;
  for (int64_t c0 = (int64_t)t * kE; c0 < cols; c0 += (int64_t)kT * kE) {
    float v[kE];
    load(c0, v);
    float cm = v[0];
#pragma unroll
    for (int i = 1; i < kE; ++i) cm = fmax_ordered(cm, v[i]);
    const float mn = fmax_ordered(m, cm);
    if (mn == -__builtin_inff()) continue;   // nothing but -inf so far: s stays 0
    s = (m == mn ? s : s * exp2_fast((m - mn) * kLog2e));   // m = -inf: s is 0
#pragma unroll
    for (int i = 0; i < kE; ++i) s += exp2_fast((v[i] - mn) * kLog2e);
    m = mn;
  }
  float M = wave_max(m);
  if (lane == 0) part[0][wave] = M;
  __syncthreads();
  M = part[0][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmax_ordered(M, part[0][w]);
  float S = wave_sum(m == -__builtin_inff() ? 0.0f : s * exp2_fast((m - M) * kLog2e));
  if (lane == 0) part[1][wave] = S;
  __syncthreads();
  S = part[1][0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) S += part[1][w];
  const float inv = 1.0f / S;
  for (int64_t c0 = (int64_t)t * kE; c0 < cols; c0 += (int64_t)kT * kE) {
    float v[kE];
    load(c0, v);
#pragma unroll
    for (int i = 0; i < kE; ++i) v[i] = normalise<kOut>(exp2_fast((v[i] - M) * kLog2e), S, inv);
    if (c0 + kE <= cols) {
      store_chunk<kOut, kE>(yr + c0, v);
    } else {
#pragma unroll
      for (int i = 0; i < kE; ++i)
        if (c0 + i < cols) Elem<kOut>::store1(yr + c0 + i, v[i]);
    }
  }
}

#define SILE_SOFTMAX_WIDE_REGS(NAME, IN, OUT, CH)                                              \
  extern "C" __global__ __launch_bounds__(1024) void NAME(const void* x, void* y, int64_t rows,  \
                                                          int64_t cols, int64_t ldx, int64_t ldy) { \
    softmax_rows_wide_regs_kernel<IN, OUT, CH>(x, y, rows, cols, ldx, ldy);                      \
  }
#define SILE_SOFTMAX_WIDE_WIDTHS(TAG, IN, OUT)                      \
  SILE_SOFTMAX_WIDE_REGS(sile_softmax_rows_##TAG##_w2, IN, OUT, 2)   \
  SILE_SOFTMAX_WIDE_REGS(sile_softmax_rows_##TAG##_w4, IN, OUT, 4)   \
  SILE_SOFTMAX_WIDE_REGS(sile_softmax_rows_##TAG##_w8, IN, OUT, 8)   \
  extern "C" __global__ __launch_bounds__(1024) void sile_softmax_rows_##TAG##_wide(          \
      const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy) {        \
    softmax_rows_wide_kernel<IN, OUT>(x, y, rows, cols, ldx, ldy);                           \
  }
SILE_SOFTMAX_WIDE_WIDTHS(f16_f16, kF16, kF16)
SILE_SOFTMAX_WIDE_WIDTHS(bf16_bf16, kBF16, kBF16)
SILE_SOFTMAX_WIDE_WIDTHS(f32_f32, kF32, kF32)
SILE_SOFTMAX_WIDE_WIDTHS(f16_f32, kF16, kF32)

// ---- row reduce (ReduceMax / ReduceSum along axis 1), fp32 result ----
// op 0 = max, the reference's fold from x0 bit for bit (first_max_* in
// common.h: NaN at column 0 gives NaN, other NaNs never enter, a +0 / -0 tie
// keeps the first in row order); op 1 = sum (a tree; the reference folds left
// to right).  The lane that stores a row's result always owns its column 0.
template <int kIn>
SILE_DEV float max_result(float v, const typename Elem<kIn>::Storage* xr) {
  const float x0 = Elem<kIn>::load1(xr);
  return x0 != x0 ? x0 : v;
}

template <int kIn>
__device__ __forceinline__ void reduce_rows_kernel(int op, int vec, const void* x, float* out,
                                                   int64_t rows, int64_t cols, int64_t ldx) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  constexpr int kE = chunk_elems<kIn, kF32>();  // one 16-byte load per lane
  const int64_t vec_cols = vec ? (cols & ~(int64_t)(kE - 1)) : 0;
  if (op == 0) {
    float m = -__builtin_inff();
    int mi = kNoCol;
    int64_t c = (int64_t)lane * kE;
    for (; c + kE <= vec_cols; c += 64 * kE) {
      float v[kE];
      load_chunk<kIn, kE>(xr + c, v);
#pragma unroll
      for (int i = 0; i < kE; ++i) first_max_fold(m, mi, v[i], (int)c + i);
    }
    for (int64_t cc = vec_cols + lane; cc < cols; cc += 64)
      first_max_fold(m, mi, Elem<kIn>::load1(xr + cc), (int)cc);
    wave_first_max(m, mi);
    if (lane == 0) out[row] = max_result<kIn>(m, xr);
    return;
  }
  float acc = 0.0f;
  int64_t c = (int64_t)lane * kE;
  for (; c + kE <= vec_cols; c += 64 * kE) {
    float v[kE];
    load_chunk<kIn, kE>(xr + c, v);
#pragma unroll
    for (int i = 0; i < kE; ++i) acc = acc + v[i];
  }
  for (int64_t cc = vec_cols + lane; cc < cols; cc += 64) acc = acc + Elem<kIn>::load1(xr + cc);
  acc = wave_sum(acc);
  if (lane == 0) out[row] = acc;
}

// Narrow rows (up to 32 chunks): kL lanes per row, one chunk per lane, 64 /
// kL rows per wave; rows of 16-byte aligned chunks only.
template <int kIn, int kL>
__device__ __forceinline__ void reduce_rows_narrow_kernel(int op, const void* x, float* out,
                                                          int64_t rows, int64_t cols,
                                                          int64_t ldx) {
  constexpr int kE = chunk_elems<kIn, kF32>();
  const int lane = threadIdx.x & 63, li = lane % kL;
  const int64_t row = (int64_t)blockIdx.x * (256 / kL) + (threadIdx.x >> 6) * (64 / kL) + lane / kL;
  const bool live = row < rows;
  using TI = typename Elem<kIn>::Storage;
  const TI* xr = static_cast<const TI*>(x) + (live ? row : 0) * ldx;
  const int c0 = li * kE;
  if (op == 0) {
    float m = -__builtin_inff();
    int mi = kNoCol;
    if (live && c0 + kE <= cols) {
      float v[kE];
      load_chunk<kIn, kE>(xr + c0, v);
#pragma unroll
      for (int i = 0; i < kE; ++i) first_max_fold(m, mi, v[i], c0 + i);
    } else if (live) {
      for (int i = 0; c0 + i < cols && i < kE; ++i)
        first_max_fold(m, mi, Elem<kIn>::load1(xr + c0 + i), c0 + i);
    }
    group_first_max<kL>(m, mi);
    if (live && li == 0) out[row] = max_result<kIn>(m, xr);
    return;
  }
  float acc = 0.0f;
  if (live && c0 + kE <= cols) {
    float v[kE];
    load_chunk<kIn, kE>(xr + c0, v);
#pragma unroll
    for (int i = 0; i < kE; ++i) acc = acc + v[i];
  } else if (live) {
    for (int i = 0; c0 + i < cols && i < kE; ++i) acc = acc + Elem<kIn>::load1(xr + c0 + i);
  }
  acc = group_sum<kL>(acc);
  if (live && li == 0) out[row] = acc;
}

// Wide rows, few of them: one row per workgroup of 1024 threads, 16-byte
// chunks strided by the workgroup, wave all-reductions plus one exchange of
// the per-wave partials through LDS.
template <int kIn>
__device__ __forceinline__ void reduce_rows_block_kernel(int op, const void* x, float* out,
                                                         int64_t rows, int64_t cols,
                                                         int64_t ldx) {
  constexpr int kT = 1024;
  constexpr int kE = chunk_elems<kIn, kF32>();
  __shared__ float part[kT / 64];
  __shared__ int part_col[kT / 64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  const int64_t vec_cols = cols & ~(int64_t)(kE - 1);
  if (op == 0) {
    float m = -__builtin_inff();
    int mi = kNoCol;
    for (int64_t c = (int64_t)t * kE; c < vec_cols; c += (int64_t)kT * kE) {
      float v[kE];
      load_chunk<kIn, kE>(xr + c, v);
#pragma unroll
      for (int i = 0; i < kE; ++i) first_max_fold(m, mi, v[i], (int)c + i);
    }
    for (int64_t c = vec_cols + t; c < cols; c += kT)
      first_max_fold(m, mi, Elem<kIn>::load1(xr + c), (int)c);
    wave_first_max(m, mi);
    if (lane == 0) {
      part[wave] = m;
      part_col[wave] = mi;
    }
    __syncthreads();
    if (t == 0) {
      for (int w = 1; w < kT / 64; ++w) first_max_merge(m, mi, part[w], part_col[w]);
      out[row] = max_result<kIn>(m, xr);
    }
    return;
  }
  float acc = 0.0f;
  for (int64_t c = (int64_t)t * kE; c < vec_cols; c += (int64_t)kT * kE) {
    float v[kE];
    load_chunk<kIn, kE>(xr + c, v);
#pragma unroll
    for (int i = 0; i < kE; ++i) acc = acc + v[i];
  }
  for (int64_t c = vec_cols + t; c < cols; c += kT) acc = acc + Elem<kIn>::load1(xr + c);
  acc = wave_sum(acc);
  if (lane == 0) part[wave] = acc;
  __syncthreads();
  if (t == 0) {
    float r = part[0];
    for (int w = 1; w < kT / 64; ++w) r = r + part[w];
    out[row] = r;
  }
}

// Rows of exactly 2 * kT chunks (the softmax's row-block widths): one row per
// workgroup of kT threads, both chunks of a thread loaded before either is
// folded (chunk j of thread t at column (j * kT + t) * E, folded in column
// order), wave all-reductions and one exchange of the per-wave partials.
template <int kIn, int kT>
__device__ __forceinline__ void reduce_rows_rowblock_kernel(int op, const void* x, float* out,
                                                            int64_t rows, int64_t ldx) {
  constexpr int kE = chunk_elems<kIn, kF32>();
  constexpr int kWaves = kT / 64;
  __shared__ float part[kWaves];
  __shared__ int part_col[kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  using TI = typename Elem<kIn>::Storage;
  const TI* xr = static_cast<const TI*>(x) + row * ldx;
  float v[2][kE];
#pragma unroll
  for (int j = 0; j < 2; ++j) load_chunk<kIn, kE>(xr + (j * kT + t) * kE, v[j]);
  if (op == 0) {
    float m = -__builtin_inff();
    int mi = kNoCol;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < kE; ++i) first_max_fold(m, mi, v[j][i], (j * kT + t) * kE + i);
    wave_first_max(m, mi);
    if (lane == 0) {
      part[wave] = m;
      part_col[wave] = mi;
    }
    __syncthreads();
    if (t == 0) {
#pragma unroll
      for (int w = 1; w < kWaves; ++w) first_max_merge(m, mi, part[w], part_col[w]);
      out[row] = max_result<kIn>(m, xr);
    }
    return;
  }
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < kE; ++i) acc = acc + v[j][i];
  acc = wave_sum(acc);
  if (lane == 0) part[wave] = acc;
  __syncthreads();
  if (t == 0) {
#pragma unroll
    for (int w = 1; w < kWaves; ++w) acc = acc + part[w];
    out[row] = acc;
  }
}

#define SILE_REDUCE_SHAPES(TAG, IN)                                                           \
  extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_##TAG##_n4(              \
      int op, const void* x, float* out, int64_t rows, int64_t cols, int64_t ldx) {          \
    reduce_rows_narrow_kernel<IN, 4>(op, x, out, rows, cols, ldx);                          \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_##TAG##_n8(              \
      int op, const void* x, float* out, int64_t rows, int64_t cols, int64_t ldx) {          \
    reduce_rows_narrow_kernel<IN, 8>(op, x, out, rows, cols, ldx);                          \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_##TAG##_n16(             \
      int op, const void* x, float* out, int64_t rows, int64_t cols, int64_t ldx) {          \
    reduce_rows_narrow_kernel<IN, 16>(op, x, out, rows, cols, ldx);                         \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_##TAG##_n32(             \
      int op, const void* x, float* out, int64_t rows, int64_t cols, int64_t ldx) {          \
    reduce_rows_narrow_kernel<IN, 32>(op, x, out, rows, cols, ldx);                         \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(1024) void sile_reduce_rows_##TAG##_block(          \
      int op, const void* x, float* out, int64_t rows, int64_t cols, int64_t ldx) {          \
    reduce_rows_block_kernel<IN>(op, x, out, rows, cols, ldx);                              \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_##TAG##_b256(            \
      int op, const void* x, float* out, int64_t rows, int64_t ldx) {                       \
    reduce_rows_rowblock_kernel<IN, 256>(op, x, out, rows, ldx);                            \
  }                                                                                         \
  extern "C" __global__ __launch_bounds__(512) void sile_reduce_rows_##TAG##_b512(            \
      int op, const void* x, float* out, int64_t rows, int64_t ldx) {                       \
    reduce_rows_rowblock_kernel<IN, 512>(op, x, out, rows, ldx);                            \
  }
SILE_REDUCE_SHAPES(f32, kF32)
SILE_REDUCE_SHAPES(f16, kF16)
SILE_REDUCE_SHAPES(bf16, kBF16)

extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_f32(int op, int vec, const void* x,
                                                                       float* out, int64_t rows,
                                                                       int64_t cols, int64_t ldx) {
  reduce_rows_kernel<kF32>(op, vec, x, out, rows, cols, ldx);
}
extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_f16(int op, int vec, const void* x,
                                                                       float* out, int64_t rows,
                                                                       int64_t cols, int64_t ldx) {
  reduce_rows_kernel<kF16>(op, vec, x, out, rows, cols, ldx);
}
extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_bf16(int op, int vec, const void* x,
                                                                        float* out, int64_t rows,
                                                                        int64_t cols,
                                                                        int64_t ldx) {
  reduce_rows_kernel<kBF16>(op, vec, x, out, rows, cols, ldx);
}

// ---- fp32 row sums in the order of the reference's fused load + reduce ----
// The CPU backend sums a row it loads straight from a buffer
// (crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:31-177)
// in 4-element windows, each ((v0 + v1) + v2) + v3, added in window order:
//  * cols <= 16: cols/4 windows, the accumulator starts at window 0 (:80-113);
//  * cols > 16: a step-4 loop from 0.0f while idx < cols (:1182-1256,
//    crates/sile-tile-ir/src/passes/lowering/core/emit/tile_loops/single_axis.rs:180-260),
//    so for cols % 4 != 0 the last window reads the next elements of the
//    buffer past the row;
// then a scalar tail from 4*(cols/4), which re-adds the row's elements of a
// partial last window.  cols < 4 is the plain fold from element 0.  Window
// elements at or past x_len (the buffer's end) are taken as 0.0f.
// Each row is one dependent chain, so one lane owns one row.
extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_fused_sum_f32(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows, int64_t cols, int64_t ldx,
    int64_t x_len) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const float* xr = x + row * ldx;
  const int64_t avail = x_len - row * ldx;
  float acc;
  if (cols < 4) {
    acc = xr[0];
    for (int64_t c = 1; c < cols; ++c) acc = acc + xr[c];
  } else {
    const int64_t chunks = cols / 4;
    if (cols <= 16) {
      acc = ((xr[0] + xr[1]) + xr[2]) + xr[3];
      for (int64_t i = 1; i < chunks; ++i) {
        const float* p = xr + 4 * i;
        acc = acc + (((p[0] + p[1]) + p[2]) + p[3]);
      }
    } else {
      acc = 0.0f;
      for (int64_t idx = 0; idx < cols; idx += 4) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = idx + j < avail ? xr[idx + j] : 0.0f;
        acc = acc + (((v[0] + v[1]) + v[2]) + v[3]);
      }
    }
    for (int64_t c = chunks * 4; c < cols; ++c) acc = acc + xr[c];
  }
  out[row] = acc;
}

// The same sums for cols > 16 at HBM rate (fused_sum_rows_tiled): the same
// arithmetic in the same order as sile_reduce_rows_fused_sum_f32, so
// bit-identical to it; _tiled for cols % 4 == 0 and 16-byte aligned rows
// (16-byte loads), _tiled_any for any cols, pitch and alignment.
extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_fused_sum_f32_tiled(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows, int64_t cols, int64_t ldx) {
  __shared__ __attribute__((aligned(16))) float w[kFsLds];
  const int64_t row0 = (int64_t)blockIdx.x * kFsRows;
  const int nrows = (int)min((int64_t)kFsRows, rows - row0);
  const float acc = fused_sum_rows_tiled<false>(x, cols, ldx, 0, row0, nrows, w);
  if ((int)threadIdx.x < nrows) out[row0 + threadIdx.x] = acc;
}
extern "C" __global__ __launch_bounds__(256) void sile_reduce_rows_fused_sum_f32_tiled_any(
    const float* __restrict__ x, float* __restrict__ out, int64_t rows, int64_t cols, int64_t ldx,
    int64_t x_len) {
  __shared__ __attribute__((aligned(16))) float w[kFsLds];
  const int64_t row0 = (int64_t)blockIdx.x * kFsRows;
  const int nrows = (int)min((int64_t)kFsRows, rows - row0);
  const float acc = fused_sum_rows_tiled<true>(x, cols, ldx, x_len, row0, nrows, w);
  if ((int)threadIdx.x < nrows) out[row0 + threadIdx.x] = acc;
}

// ---- 2-D copy: y[r][0, row_bytes) = x[r][0, row_bytes) ----
// Workgroup (r, s) of the grid copies segment s of row r: kCopySegB bytes, two 16-byte
// chunks per thread of 512 (chunk j of thread t at (j * 512 + t) * 16), both
// loaded (non-temporal) before either is stored, so each load or store
// instruction of a wave covers one contiguous KiB.  Of the copy shapes
// measured on MI355X (chunks per thread 1-16, 128-1024 threads, one wave per
// row, grid-stride; buffer loads / stores with every cache-policy
// combination), this one moved the most bytes: 6.25-6.35 TB/s for 128 MiB
// each way.  Rows and pitches are multiples of 16 bytes (checked by the host).
constexpr int kCopyThreads = 512;
constexpr int kCopySegB = kCopyThreads * 2 * 16;
extern "C" __global__ __launch_bounds__(kCopyThreads) void sile_copy_rows_b128(
    const uint8_t* __restrict__ x, uint8_t* __restrict__ y, int64_t rows, int64_t row_bytes,
    int64_t ldx, int64_t ldy) {
  const int64_t row = blockIdx.x, seg = blockIdx.y;
  if (row >= rows) return;
  const uint8_t* xr = x + row * ldx + seg * kCopySegB;
  uint8_t* yr = y + row * ldy + seg * kCopySegB;
  const int64_t n = (row_bytes - seg * kCopySegB) >> 4;  // chunks of this segment and beyond
  const int t = threadIdx.x;
  u32x4 w[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (j * kCopyThreads + t < n)
      w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xr + (j * kCopyThreads + t) * 16));
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (j * kCopyThreads + t < n)
      __builtin_nontemporal_store(w[j], reinterpret_cast<u32x4*>(yr + (j * kCopyThreads + t) * 16));
}

// Contiguous rows (pitch == row bytes): the matrix is one run of `chunks`
// 16-byte chunks, workgroup b copying chunks [b * 1024, b * 1024 + 1024).
extern "C" __global__ __launch_bounds__(kCopyThreads) void sile_copy_flat_b128(
    const uint8_t* __restrict__ x, uint8_t* __restrict__ y, int64_t chunks) {
  const int64_t c0 = (int64_t)blockIdx.x * (2 * kCopyThreads) + threadIdx.x;
  u32x4 w[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (c0 + j * kCopyThreads < chunks)
      w[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x) + c0 + j * kCopyThreads);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (c0 + j * kCopyThreads < chunks)
      __builtin_nontemporal_store(w[j], reinterpret_cast<u32x4*>(y) + c0 + j * kCopyThreads);
}

// ---- tile store of a splat (Splat + StorePtrTko): y[r][c] = v ----
// The write-only counterpart of the copy: contiguous 16-byte aligned rows are
// one run of `chunks` 16-byte chunks, each holding the element's bits
// repeated (`word`: one fp32, or two 16-bit elements), stored non-temporally
// in the copy's shape (512 threads x 2 chunks per workgroup).
extern "C" __global__ __launch_bounds__(kCopyThreads) void sile_fill_flat_b128(
    uint8_t* __restrict__ y, int64_t chunks, uint32_t word) {
  const int64_t c0 = (int64_t)blockIdx.x * (2 * kCopyThreads) + threadIdx.x;
  const u32x4 w = {word, word, word, word};
#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (c0 + j * kCopyThreads < chunks)
      __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(y) + c0 + j * kCopyThreads);
}
// Any rows, pitch and alignment: one wave per row, one element per lane;
// `bits` is the element (2 or 4 bytes wide, `eb`).
extern "C" __global__ __launch_bounds__(256) void sile_fill_rows_elem(uint8_t* y, int64_t rows,
                                                                     int64_t cols, int64_t ldy,
                                                                     uint32_t bits, int eb) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  if (eb == 4) {
    float* yr = reinterpret_cast<float*>(y) + row * ldy;
    for (int64_t c = lane; c < cols; c += 64) yr[c] = bits_f32(bits);
  } else {
    uint16_t* yr = reinterpret_cast<uint16_t*>(y) + row * ldy;
    for (int64_t c = lane; c < cols; c += 64) yr[c] = (uint16_t)bits;
  }
}

// Rows or pitches that are not multiples of 16 bytes: one byte per lane.
extern "C" __global__ __launch_bounds__(256) void sile_copy_rows_b8(const uint8_t* x, uint8_t* y,
                                                                   int64_t rows,
                                                                   int64_t row_bytes, int64_t ldx,
                                                                   int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= rows) return;
  for (int64_t c = lane; c < row_bytes; c += 64) y[row * ldy + c] = x[row * ldx + c];
}
