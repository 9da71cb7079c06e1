// Device-side helpers shared by the gfx950 kernels of libsile_hip.
//
// Everything here is written for CDNA4 (gfx950, wave64): vector types for the
// MFMA operands, round-to-nearest-even conversions to the 16-bit types, and
// wave-wide all-reductions built from DPP row permutes plus one cross-row
// exchange each for the 16- and 32-lane steps.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SILE_DEV __device__ __forceinline__

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

namespace sile {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

SILE_DEV uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
SILE_DEV float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// fp32 -> bf16 bits, round to nearest even (hardware v_cvt_pk_bf16_f32);
// NaN stays a quiet NaN.
SILE_DEV uint16_t bf16_rne(float f) {
  const __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
SILE_DEV float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// fp32 -> fp16 bits (hardware conversion, round to nearest even).
SILE_DEV uint16_t f16_rne(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}
SILE_DEV float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Packs two fp32 into one dword of two 16-bit values (lo in bits 0..15).
SILE_DEV uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
SILE_DEV uint32_t pack_f16x2(float lo, float hi) {
  f16x2 v = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- wave-wide all-reductions (DPP within 16-lane rows, then 2 exchanges) ----
template <int kCtrl>
SILE_DEV float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
// DPP controls: quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1] (xor 2),
// row_half_mirror (lane i <-> 7-i in each 8), row_mirror (i <-> 15-i in each 16).
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// ds_swizzle bit mode: and_mask 0x1f, xor_mask 0x10 -> lane ^ 16 within 32.
SILE_DEV float swizzle_xor16(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
// v_permlane32_swap on two copies of v: the upper half of one trades places
// with the lower half of the other, leaving v's lower half (lo) and upper half
// (hi) each broadcast to all 64 lanes.  Lane l then holds v[l % 32] and
// v[32 + l % 32], i.e. v of lanes l and l ^ 32.  (Each result is copied to a
// scalar before the bit cast: bit-casting a vector element directly reads
// element 0 with this compiler.)
SILE_DEV void half_swap(float v, float& lo, float& hi) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned a = r[0], b = r[1];
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}

SILE_DEV float fmax_ordered(float a, float b) { return (b > a) ? b : a; }

// max and sum of v over lanes l and l ^ 32 (the same value in both lanes)
SILE_DEV float pair32_max(float v) {
  float lo, hi;
  half_swap(v, lo, hi);
  return fmax_ordered(lo, hi);
}
SILE_DEV float pair32_sum(float v) {
  float lo, hi;
  half_swap(v, lo, hi);
  return lo + hi;
}

SILE_DEV float wave_max(float v) {
  v = fmax_ordered(v, dpp<kDppXor1>(v));
  v = fmax_ordered(v, dpp<kDppXor2>(v));
  v = fmax_ordered(v, dpp<kDppHalfMirror>(v));
  v = fmax_ordered(v, dpp<kDppMirror>(v));
  v = fmax_ordered(v, swizzle_xor16(v));
  return pair32_max(v);
}

SILE_DEV float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  v += swizzle_xor16(v);
  return pair32_sum(v);
}

// max and sum over each 16-lane row of the wave (all 16 lanes hold the result)
SILE_DEV float group_max16(float v) {
  v = fmax_ordered(v, dpp<kDppXor1>(v));
  v = fmax_ordered(v, dpp<kDppXor2>(v));
  v = fmax_ordered(v, dpp<kDppHalfMirror>(v));
  return fmax_ordered(v, dpp<kDppMirror>(v));
}
SILE_DEV float group_sum16(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  return v + dpp<kDppMirror>(v);
}

// ---- the reference's row max, computed in parallel ----
// ReduceMax folds from the row's first element, acc = x0; acc = x > acc ? x : acc
// (crates/sile-tile-ir/src/passes/lowering/tile_compute/reduce.rs:10-30), so
//  * x0 NaN gives NaN (no x compares greater than NaN);
//  * otherwise NaN elements never enter, and of the elements equal to the max
//    the first one in row order is kept (only +0 / -0 ties differ in bits).
// A lane folds its elements in increasing index order into (v, i), the value
// and column of its first maximum (start: -inf at column kNoCol); partials
// merge by the larger value, then the smaller column, an associative and
// commutative rule, so any reduction tree gives the fold's bits.  The caller
// returns x0 instead when x0 is NaN.
constexpr int kNoCol = 0x7fffffff;
SILE_DEV void first_max_fold(float& v, int& i, float x, int xi) {
  const bool gt = x > v;
  v = gt ? x : v;
  i = gt ? xi : i;
}
SILE_DEV void first_max_merge(float& v, int& i, float ov, int oi) {
  const bool take = ov > v || (ov == v && oi < i);
  v = take ? ov : v;
  i = take ? oi : i;
}
template <int kCtrl>
SILE_DEV int dpp_int(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xf, 0xf, false);
}
template <int kCtrl>
SILE_DEV void first_max_dpp(float& v, int& i) {
  first_max_merge(v, i, dpp<kCtrl>(v), dpp_int<kCtrl>(i));
}
SILE_DEV void first_max_swizzle16(float& v, int& i) {
  first_max_merge(v, i, swizzle_xor16(v), __builtin_amdgcn_ds_swizzle(i, 0x401F));
}
// (v, i) merged over groups of kL lanes (kL = 4 .. 32), all lanes of a group
// holding the result.
template <int kL>
SILE_DEV void group_first_max(float& v, int& i) {
  first_max_dpp<kDppXor1>(v, i);
  first_max_dpp<kDppXor2>(v, i);
  if constexpr (kL >= 8) first_max_dpp<kDppHalfMirror>(v, i);
  if constexpr (kL >= 16) first_max_dpp<kDppMirror>(v, i);
  if constexpr (kL >= 32) first_max_swizzle16(v, i);
}
SILE_DEV void wave_first_max(float& v, int& i) {
  group_first_max<32>(v, i);
  float lo, hi;
  half_swap(v, lo, hi);
  const unsigned iu = (unsigned)i;
  const auto r = __builtin_amdgcn_permlane32_swap(iu, iu, false, false);
  const unsigned ilo = r[0], ihi = r[1];
  v = lo;
  i = (int)ilo;
  first_max_merge(v, i, hi, (int)ihi);
}

// Instruction classes of __builtin_amdgcn_sched_group_barrier masks.
namespace sched {
constexpr int kValu = 0x002, kMfma = 0x008, kVmemRead = 0x020, kDsRead = 0x100;
}

// Fused load + vec4 sums of rows wider than 16 in the reference's loop form
// (windows ((v0 + v1) + v2) + v3 from 0.0f while idx < cols, added in window
// order, crates/sile-tile-ir/src/passes/lowering/tile_compute/fused_reduce.rs:1182-1256;
// then, for cols % 4 != 0, a scalar tail from 4 * (cols / 4) that re-adds
// the row's elements of the last window), at HBM rate.  The window sums are
// independent; only their accumulation is one chain per row.  A workgroup
// of 256 threads owns kFsRows rows and walks them kFsWin windows at a time:
// all threads form the next block's window sums into one half of LDS `w`
// (2 * kFsRows * kFsPitch floats) while lane r of wave 0 adds row r's window
// sums of the current block, from the other half, to its running sum in
// window order, four per LDS read (row pitch kFsWin + 4 floats: 16-byte
// aligned, rows 4 banks apart).  kAny = false: cols % 4 == 0 and 16-byte
// aligned rows, 16-byte loads; kAny = true: any cols, ldx and alignment,
// element loads, window elements at or past x_len (the buffer's end) taken
// as 0.0f, where the reference reads past its buffer (a last window past the
// row reads the next elements of the buffer, as the reference's does).
// Returns the sum of row row0 + tid for tid < nrows (0.0f elsewhere).
constexpr int kFsRows = 4;
constexpr int kFsWin = 256;                     // windows per row and block
constexpr int kFsPitch = kFsWin + 4;            // LDS floats per row
constexpr int kFsLds = 2 * kFsRows * kFsPitch;  // floats of `w`
template <bool kAny>
SILE_DEV float fused_sum_rows_tiled(const float* __restrict__ x, int64_t cols, int64_t ldx,
                                    int64_t x_len, int64_t row0, int nrows, float* w) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  const int64_t nwin = kAny ? (cols + 3) / 4 : cols / 4;
  // window sums of windows [wb, wb + kFsWin) of each row into buf
  auto fill = [&](int64_t wb, float* buf) {
    const int win = (int)(nwin - wb < kFsWin ? nwin - wb : kFsWin);
    for (int e = tid; e < nrows * win; e += 256) {
      const int r = e / win, i = e - r * win;
      const int64_t base = (row0 + r) * ldx + 4 * (wb + i);
      float v[4];
      if constexpr (kAny) {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = base + j < x_len ? x[base + j] : 0.0f;
      } else {
        const f32x4 q = *reinterpret_cast<const f32x4*>(x + base);
        v[0] = q[0]; v[1] = q[1]; v[2] = q[2]; v[3] = q[3];
      }
      buf[r * kFsPitch + i] = ((v[0] + v[1]) + v[2]) + v[3];
    }
  };
  float acc = 0.0f;
  fill(0, w);
  __syncthreads();
  int k = 0;
  for (int64_t wb = 0; wb < nwin; wb += kFsWin, ++k) {
    if (wb + kFsWin < nwin) fill(wb + kFsWin, w + ((k + 1) & 1) * kFsRows * kFsPitch);
    if (tid < nrows) {
      const float* wr = w + (k & 1) * kFsRows * kFsPitch + tid * kFsPitch;
      const int win = (int)(nwin - wb < kFsWin ? nwin - wb : kFsWin);
      const int win4 = win & ~3;
#pragma unroll 4
      for (int i = 0; i < win4; i += 4) {
        const f32x4 q = *reinterpret_cast<const f32x4*>(wr + i);
        acc = acc + q[0];
        acc = acc + q[1];
        acc = acc + q[2];
        acc = acc + q[3];
      }
      for (int i = win4; i < win; ++i) acc = acc + wr[i];
    }
    __syncthreads();
  }
  if constexpr (kAny) {
    if (tid < nrows)
      for (int64_t c = (cols / 4) * 4; c < cols; ++c) acc = acc + x[(row0 + tid) * ldx + c];
  }
  return acc;
}

// 2^x on the transcendental unit (v_exp_f32).
SILE_DEV float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace sile
