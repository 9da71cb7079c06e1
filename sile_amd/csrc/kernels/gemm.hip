// MFMA GEMM for gfx950:  C[M,N] = alpha * A[M,K] . B[K,N]
//   A row-major ([M,K], K contiguous), B column-major (stored [N,K], K
//   contiguous), fp32 accumulation in MFMA accumulators, output bf16 / fp16 /
//   fp32 with round-to-nearest-even.  alpha carries the per-tensor scales of
//   the fp8 path (scale_a * scale_b) and is 1 otherwise.
//
// This is the tile op `MmaF` of the canonical matmul
// (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:24-444) on the
// matrix cores; k runs over K' = (K / bk) * bk as there, which the host
// resolves before launch.  One body (gemm_ring_body) serves bf16, f16 (16 x 16
// MFMA blocks) and fp8 e4m3 (32 x 32 blocks) operands through a ring of 5
// LDS tiles; its design is described above it.  sile_gemm_f32_exact_{nn,nt}_t{128,64,32}
// are the fp32 path in the canonical order (bit-identical to the CPU backend).
#include <type_traits>

#include "common.h"

using namespace sile;

namespace {

enum Kind : int { kBF16 = 0, kF16 = 1, kFP8 = 2 };
enum Out : int { kOutBF16 = 0, kOutF16 = 1, kOutF32 = 2 };

// 16-bit C is written once and not read back by the kernel: non-temporal
// stores (streaming; 2-3 % faster for the staged 16-bit C than plain stores).
// fp32 C goes straight from the accumulators, 32 or 64 bytes of a row per
// instruction: plain stores, so that L2 merges a row's pieces into whole
// lines (non-temporal ones made the fp8 kernel's fp32 C 1.3x and its split-K
// planes up to 2.7x slower).
template <int kOut>
SILE_DEV void store_c4(void* C, int64_t idx, f32x4 v) {
  if constexpr (kOut == kOutF32) {
    *reinterpret_cast<f32x4*>(static_cast<float*>(C) + idx) = v;
  } else if constexpr (kOut == kOutBF16) {
    const u32x2 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(C) + idx));
  } else {
    const u32x2 w = {pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(C) + idx));
  }
}

struct GemmArgs {
  int64_t lda, ldb, ldc;  // in elements
  int32_t tiles_m, tiles_n, k_steps;
  float alpha;
  int32_t m, n;           // C extents (>= the tile edge kT, except m for kT = 128): the last tile
                          // row / column starts at m - kT / n - kT
  int32_t k_rem;          // elements of the last half k-step inside K' (1 .. a half k-step)
  int32_t split_steps;    // half k-steps per k-range (even, or k_steps when K is not split)
  int64_t c_split;        // elements between the C planes of consecutive k-ranges
  int64_t b_rows;         // B row-major [K, N]: rows of B's buffer (loads stay below them)
};

// The k-range of a workgroup: blockIdx.y selects half k-steps
// [y * split_steps, min((y + 1) * split_steps, k_steps)); only the range that
// ends at K' has a partial last half k-step.
struct KRange {
  int64_t byte0;          // first byte of the range in a row of A / B
  int32_t k_steps, k_rem;
};
template <int kEB>
SILE_DEV KRange k_range(const GemmArgs& g) {
  const int y = blockIdx.y;
  const int h0 = y * g.split_steps;
  KRange r;
  r.byte0 = (int64_t)h0 * 64;
  r.k_steps = min(g.split_steps, g.k_steps - h0);
  r.k_rem = h0 + r.k_steps == g.k_steps ? g.k_rem : 64 / kEB;
  return r;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One 32 x 32 output block over 64 k of fp8 e4m3: v_mfma_f32_32x32x64_f8f6f4
// on two 16-byte chunks per lane (e4m3 x e4m3, zero scale operands: the
// unscaled instruction).
SILE_DEV f32x16 mma32x32_fp8(const u32x4* a, const u32x4* b, f32x16 c) {
  const i32x8 av = {(int)a[0][0], (int)a[0][1], (int)a[0][2], (int)a[0][3],
                    (int)a[1][0], (int)a[1][1], (int)a[1][2], (int)a[1][3]};
  const i32x8 bv = {(int)b[0][0], (int)b[0][1], (int)b[0][2], (int)b[0][3],
                    (int)b[1][0], (int)b[1][1], (int)b[1][2], (int)b[1][3]};
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(av, bv, c, 0, 0, 0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Tile placement.
//
// kT x kT output tile per workgroup of 4 waves (2 x 2, kT/2 x kT/2 per wave),
// kT = 256 (one workgroup per CU) or 128 (two per CU).
// Tiles go from HBM straight into LDS (buffer_load_dwordx4 ... lds): one
// instruction of a wave fills 1 KiB of LDS, lane l writing bytes
// [16 l, 16 l + 16) of it, so each lane fetches the global chunk that belongs
// at its LDS slot under the swizzle.  A k-step is 128 bytes of each row (64
// 16-bit or 128 fp8 elements), so one instruction fetches 8 whole 128-byte
// lines, and one operand of one k-step is a kT x 128-byte tile (32 or 16 KiB).  Rows hold 8 chunks
// of 16 bytes; chunk c of row r sits at c ^ ((r >> 1) & 7), which puts the
// fragment reads of 16 or 32 consecutive rows (one chunk each) on distinct
// banks.  The buffer resources cover the tile's kT-row A and B panels (loads
// past a panel return zero).
// ---------------------------------------------------------------------------
constexpr int kRowB = 128;            // bytes of a tile row per k-step

struct TilePlan {
  int64_t row0, col0;                 // first row / column of the tile in C
  __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
  int a_rs, b_rs;                     // bytes per row of A / B
  int a_voff, b_voff;                 // this lane's byte offsets for the tile loads
  int b_voff1;                        // B row-major: the offset for odd load instructions
};

// ---------------------------------------------------------------------------
// B row-major ([K, N], N contiguous; the canonical matmul's own layout,
// canonical_matmul.rs:55-57).  A k-step's B tile is kept as it lies in
// memory, 64 rows of k by kT columns of n (kT * 2 bytes a row), and the MFMA
// fragments, which hold 8 consecutive k of one n, are read transposed with
// ds_read_b64_tr_b16: in each 16-lane group, result slot j of lane i is
// element (i & 3) of the 8 bytes addressed by lane 4 j + (i >> 2), so lane i
// addressing B[k0 + (i >> 2)][n0 + 4 (i & 3) .. + 4] receives
// B[k0 .. k0 + 3][n0 + i]; two such reads (k0 and k0 + 4) give a fragment.
// 16-byte chunk c of tile row k sits at c ^ swz_b(k), swz_b(k) =
// 2 ((k & 3) | ((k >> 1) & 4)): one transposing read touches 16 rows
// (k & 3 over the lane's quarter, k >> 3 over the 16-lane groups) with 32
// contiguous bytes each, and the swizzle puts those 16 pairs of chunks on
// each bank twice, the minimum for 512 bytes.
// ---------------------------------------------------------------------------
SILE_DEV int swz_b(int k) { return 2 * ((k & 3) | ((k >> 1) & 4)); }

template <int kEB, int kT, bool kBRow>
SILE_DEV TilePlan plan_tile(const uint8_t* A, const uint8_t* B, const GemmArgs& g, int64_t byte0,
                            int wave, int lane) {
  TilePlan p;
  // XCD-aware tile order: workgroups go round-robin to the 8 XCDs; each XCD
  // gets a contiguous range of tiles, grouped 8 tile-rows at a time
  const int num_tiles = g.tiles_m * g.tiles_n;
  const int bid = blockIdx.x;
  int lin = bid;
  if ((num_tiles & 7) == 0) lin = (bid & 7) * (num_tiles >> 3) + (bid >> 3);
  constexpr int kGroupM = 8;
  const int group_size = kGroupM * g.tiles_n;
  const int group = lin / group_size;
  const int first_m = group * kGroupM;
  const int rows_in_group = min(g.tiles_m - first_m, kGroupM);
  const int in_group = lin - group * group_size;
  const int tile_m = first_m + in_group % rows_in_group;
  const int tile_n = in_group / rows_in_group;
  // When M or N is not a multiple of kT the last tile is moved back to end
  // at M / N, so every load stays inside the operands; the rows or columns it
  // shares with its neighbour are computed in the same order by both
  // workgroups and written with the same values.
  // 128 x 128 tiles also take M below one tile: the tile starts at row 0 and
  // the rows past M load as zeros (outside A's buffer resource)
  p.row0 = kT == 256 || g.m >= kT ? min(tile_m * kT, g.m - kT) : 0;
  const int a_rows = kT == 256 ? kT : min(kT, g.m);
  p.col0 = min(tile_n * kT, g.n - kT);
  p.a_rs = (int)(g.lda * kEB);
  p.b_rs = (int)(g.ldb * kEB);
  // (a k-range that starts byte0 bytes into the rows moves the base, not the end)
  p.a_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)(A + p.row0 * p.a_rs + byte0), (short)0,
                                               (int)(a_rows * p.a_rs - byte0), 0x00020000);
  if constexpr (kBRow) {
    // the tile's columns of B from the k-range's first row to B's last row
    const int64_t base = byte0 / kEB * p.b_rs + p.col0 * kEB;
    p.b_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)(B + base), (short)0,
                                                 (int)(g.b_rows * p.b_rs - base), 0x00020000);
  } else {
    p.b_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)(B + p.col0 * p.b_rs + byte0), (short)0,
                                                 (int)(kT * p.b_rs - byte0), 0x00020000);
  }
  // wave w's load instruction i (0..7) of an operand fills rows
  // 8 (4 i + w) + (lane >> 3), position lane & 7, whose chunk is
  // (lane & 7) ^ ((row >> 1) & 7) with (row >> 1) & 7 = ((w & 1) << 2) | ((lane >> 4) & 3)
  const int dma_row = 8 * wave + (lane >> 3);
  const int dma_chunk = (lane & 7) ^ (((wave & 1) << 2) | ((lane >> 4) & 3));
  p.a_voff = dma_row * p.a_rs + dma_chunk * 16;
  p.b_voff = p.b_voff1 = dma_row * p.b_rs + dma_chunk * 16;
  if constexpr (kBRow) {
    // instruction i of wave w fills LDS KiB 4 i + w: rows kRI (4 i + w) ..,
    // kSlots chunks a row; lane l takes row kRI w + l / kSlots (plus 4 kRI i,
    // in the scalar offset) and slot l % kSlots, i.e. global chunk
    // slot ^ swz_b(row); swz_b of the row depends on i only through its
    // parity (bit 3 of the row, for 2 rows an instruction)
    constexpr int kSlots = kT * kEB / 16, kRI = 64 / kSlots;
    const int r0 = kRI * wave + lane / kSlots, slot = lane % kSlots;
    p.b_voff = r0 * p.b_rs + ((slot ^ swz_b(r0)) << 4);
    p.b_voff1 = r0 * p.b_rs + ((slot ^ swz_b(r0 + 4 * kRI)) << 4);
  }
  return p;
}

// One 16 x 16 output block over 32 k with the accumulator pinned in AGPRs
// ("+a"): for this shape the compiler's own allocation copies every
// accumulator through VGPRs around each MFMA.  As the instruction is opaque
// to the compiler, the caller pads before the accumulators are read.
template <int kKind>
SILE_DEV void mma16x16(const u32x4& a, const u32x4& b, f32x4& c) {
  static_assert(kKind != kFP8, "fp8 uses the 32 x 32 blocks");
  if constexpr (kKind == kBF16)
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  else
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// 16-bit C through LDS: a wave's kW x kW results (kW = 128 or 64) are put
// into LDS rows of 2 kW + 16 bytes (the pad puts the rows that one put
// instruction of the accumulator layouts writes on distinct banks), then
// written back so that each store instruction covers whole 2 kW-byte rows of
// C (16-byte stores, 512 / kW rows per instruction; 8-byte stores, half as
// many, when C's rows are not 16-byte aligned).  Writing straight from the accumulator layouts touches 16 or 32
// rows per instruction with 8 bytes each and ran 5 % slower at 8192^3, with
// twice C's size written to HBM.  fill(put) calls put(row, col, v) for 4
// consecutive columns of the wave's tile; the wave's LDS region is its own.
template <int kW> constexpr int kCRowB = 2 * kW + 16;
template <int kW> constexpr int kCStageB = kW * kCRowB<kW>;   // one wave's staged C (34 KiB at kW = 128)

// kGuardRows: only the first `rows` rows of the wave's tile are stored (C
// ends inside the tile).
template <int kOut, int kW, bool kGuardRows, typename Fill>
SILE_DEV void stage_and_store_c(void* C, int64_t ldc, int64_t m0, int64_t n0, uint8_t* cst,
                                int rows, Fill fill) {
  static_assert(kOut != kOutF32, "16-bit C");
  constexpr int kRowBytes = kCRowB<kW>;
  fill([&](int row, int col, f32x4 v) {
    const u32x2 w = kOut == kOutBF16 ? u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}
                                     : u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
    *reinterpret_cast<u32x2*>(cst + row * kRowBytes + col * 2) = w;
  });
  __builtin_amdgcn_s_waitcnt(0xf | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));  // lgkmcnt(0)
  __builtin_amdgcn_wave_barrier();
  const int lane = threadIdx.x & 63;
  uint16_t* cbase = static_cast<uint16_t*>(C) + m0 * ldc + n0;
  if ((ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(cbase) & 15) == 0) {
    constexpr int kLanesPerRow = kW / 8, kRowsPerStore = 64 / kLanesPerRow;
    const int lr = lane % kLanesPerRow, lg = lane / kLanesPerRow;
#pragma unroll 8
    for (int t = 0; t < kW / kRowsPerStore; ++t) {
      const int row = kRowsPerStore * t + lg;
      if (kGuardRows && row >= rows) continue;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(cst + row * kRowBytes + lr * 16),
                                  reinterpret_cast<u32x4*>(cbase + row * ldc + lr * 8));
    }
  } else {
    constexpr int kLanesPerRow = kW / 4, kRowsPerStore = 64 / kLanesPerRow;
    const int lr = lane % kLanesPerRow, lg = lane / kLanesPerRow;
#pragma unroll 8
    for (int t = 0; t < kW / kRowsPerStore; ++t) {
      const int row = kRowsPerStore * t + lg;
      if (kGuardRows && row >= rows) continue;
      __builtin_nontemporal_store(*reinterpret_cast<const u32x2*>(cst + row * kRowBytes + lr * 8),
                                  reinterpret_cast<u32x2*>(cbase + row * ldc + lr * 4));
    }
  }
}

// ---------------------------------------------------------------------------
// The GEMM body: a ring of 5 LDS tiles, tile loads spread over the k-step.
//
// A wave's kW x kW (kW = kT / 2) is kNB x kNB blocks of one MFMA (256 fp32
// accumulators per lane at kW = 128, 64 at kW = 64):
//   bf16 / f16: kW / 16 square blocks of v_mfma_f32_16x16x32_{bf16,f16};
//   fp8 e4m3:   kW / 32 square blocks of v_mfma_f32_32x32x64_f8f6f4
//               (unscaled: zero scale operands select the plain instruction).
// The MFMA is issued with the B fragment first, so accumulator register r of
// lane l is C[m = l % 16][n = 4 (l / 16) + r] of a 16 x 16 block and
// C[m = l % 32][n = 8 (r / 4) + 4 (l / 32) + r % 4] of a 32 x 32 block.  A
// k-step (128 bytes of a row: 64 16-bit or 128 fp8 elements) is two
// sub-steps of one MFMA depth; a fragment is row l % kBlk of a block, the kCh
// 16-byte chunks 4 sub + kCh (l / kBlk) + h of the row (kCh = 1 for 16-bit,
// 2 for fp8).  Sub-step 0's fragments go to register set X, sub-step 1's to Y.
//
// LDS holds a ring of 5 tiles (160 KiB; 80 at kT = 128): k-step ks's A tile is chunk 2 ks and
// its B tile chunk 2 ks + 1; chunk c sits in slot c % 5.  The barrier that
// starts k-step ks frees the slots of k-step ks - 1, which receive B of
// ks + 1 and A of ks + 2, so every tile load has one or two k-steps to land
// and a wave's kT / 16 load instructions of a k-step can be spread evenly
// over it (one per group of MFMAs).  (Two 64 KiB stages force the loads into the
// first half of the k-step, where they fill the load queue and stall the
// MFMAs issued behind them: 7-13 % slower.)
//
// Iteration ks, after the barrier that published A and B of ks:
//   phase 0, kNB/2 groups:   MFMA Y(ks - 1) rows kNB/2 .. kNB-1 | reads X(ks)
//   sub-step 1, kNB groups:  MFMA X(ks) rows 0 .. kNB-1         | reads Y(ks)
//   tail, kNB/2 groups:      MFMA Y(ks) rows 0 .. kNB/2-1
//   s_waitcnt (B of ks + 1 landed, A of ks + 2 may be in flight) + s_barrier
// A group is the kNB MFMAs of one accumulator row in quarters, with the
// fragment reads and tile loads at fixed places (Q MFMA, reads, Q MFMA,
// reads, Q MFMA, loads, Q MFMA), fenced so the compiler keeps that order;
// the first kT / 32 loads of a k-step are B of ks + 1, the rest A of ks + 2.  k_steps counts
// half k-steps (64 bytes of a row): an odd count ends with a half k-step
// whose sub-step 1 multiplies zero fragments.
// ---------------------------------------------------------------------------
// Keeps the elements e0 + j < k_rem of a 16-byte fragment chunk (8 16-bit or
// 16 fp8 elements, element j at byte j * size) and zeroes the rest: the
// last half k-step past K' holds whatever followed it in memory.
template <bool kFp8>
SILE_DEV u32x4 mask_k(u32x4 w, int e0, int k_rem) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t keep = 0;
    if constexpr (kFp8) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
        if (e0 + 4 * d + b < k_rem) keep |= 0xFFu << (8 * b);
    } else {
#pragma unroll
      for (int b = 0; b < 2; ++b)
        if (e0 + 2 * d + b < k_rem) keep |= 0xFFFFu << (16 * b);
    }
    w[d] &= keep;
  }
  return w;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

template <int kKind, int kOut, int kT, bool kBRow>
__device__ __forceinline__ void gemm_ring_body(const uint8_t* __restrict__ A,
                                               const uint8_t* __restrict__ B,
                                               void* __restrict__ C, const GemmArgs& g,
                                               uint8_t* smem) {
  static_assert(!kBRow || kKind != kFP8, "row-major B: 16-bit operands");
  constexpr bool kIsFP8 = kKind == kFP8;
  constexpr int kBlk = kIsFP8 ? 32 : 16;      // MFMA block edge
  constexpr int kW = kT / 2;                  // wave tile edge
  constexpr int kNB = kW / kBlk;              // blocks per wave edge
  constexpr int kTB = kT * kRowB;             // one operand tile of one k-step in LDS
  constexpr int kOpLoads = kT / 32;           // load instructions per operand, k-step and wave
  static_assert(kNB % 2 == 0, "two sub-step halves of fragments per row");
  constexpr int kCh = kIsFP8 ? 2 : 1;         // 16-byte chunks per lane per fragment
  // a group's MFMAs in quarters [kQ_s, kQ_{s+1}) (kNB = 2: quarters of 0 and 1)
  constexpr int kQ1 = kNB / 4, kQ2 = kNB / 2, kQ3 = 3 * kNB / 4;
  constexpr int kLoadsPerGroup = 2 * kOpLoads / (2 * kNB);
  using Acc = std::conditional_t<kIsFP8, f32x16, f32x4>;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const KRange kr = k_range<kIsFP8 ? 1 : 2>(g);
  const TilePlan p = plan_tile<kIsFP8 ? 1 : 2, kT, kBRow>(A, B, g, kr.byte0, wave, lane);
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);  // LDS-DMA bases in SGPRs

  Acc acc[kNB][kNB];
#pragma unroll
  for (int i = 0; i < kNB; ++i)
#pragma unroll
    for (int j = 0; j < kNB; ++j)
#pragma unroll
      for (int r = 0; r < (int)(sizeof(Acc) / 4); ++r) acc[i][j][r] = 0.0f;

  u32x4 xa[kNB][kCh], xb[kNB][kCh], ya[kNB][kCh], yb[kNB][kCh];
  const int last = (kr.k_steps - 1) >> 1;     // index of the last (possibly half) k-step
  const bool half_last = (kr.k_steps & 1) != 0;
  const int f_row = lane % kBlk, f_grp = lane / kBlk;
  const int f_swz = (f_row >> 1) & 7;         // block rows differ by multiples of 16
  const int a_fb = (wm * kW + f_row) * kRowB, b_fb = (wn * kW + f_row) * kRowB;
  // row-major B: a transposing read of lane l covers tile row
  // 32 sub + 8 (l >> 4) + 4 h + ((l >> 2) & 3) and chunk (n0 / 8 + ((l & 3) >> 1))
  // ^ swz_b(row), half l & 1, for the block at column n0 (swz_b(row) is fixed
  // per lane: row & 3 = (l >> 2) & 3, bit 3 of row = (l >> 4) & 1)
  constexpr int kBRowBytes = kT * 2;
  const int tr_row = 8 * (lane >> 4) + ((lane >> 2) & 3);
  const int tr_swz = swz_b(tr_row), tr_hi = (lane & 3) >> 1, tr_half = (lane & 1) << 3;

  // tile load instruction i (0..7) of operand B (or A) of k-step ks into slot
  auto load = [&](bool is_b, int ks, int slot, int i) {
    uint8_t* dst = smem + slot * kTB + wave_s * 1024 + i * 4096;
    if (is_b && kBRow)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(p.b_rsrc, (lds_ptr_t)dst, 16,
                                               (i & 1) ? p.b_voff1 : p.b_voff,
                                               (i * 4 * (1024 / kBRowBytes) + ks * 64) * p.b_rs,
                                               0, 0);
    else if (is_b)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(p.b_rsrc, (lds_ptr_t)dst, 16, p.b_voff,
                                               i * 32 * p.b_rs + ks * kRowB, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(p.a_rsrc, (lds_ptr_t)dst, 16, p.a_voff,
                                               i * 32 * p.a_rs + ks * kRowB, 0, 0);
  };
  // fragment q of sub-step sub: the A block q (q < kNB) or the B block q - kNB
  auto read = [&](int sa, int sb, int sub, int q, u32x4 (&fa)[kNB][kCh],
                  u32x4 (&fb)[kNB][kCh]) {
#pragma unroll
    for (int h = 0; h < kCh; ++h) {
      const int off = ((4 * sub + kCh * f_grp + h) ^ f_swz) << 4;
      if (q < kNB) {
        fa[q][h] = *reinterpret_cast<const u32x4*>(smem + sa * kTB + a_fb +
                                                   q * kBlk * kRowB + off);
      } else if constexpr (kBRow) {
        // 8 consecutive k of column n0 + (l & 15): two transposing reads
        const int n0 = wn * kW + (q - kNB) * kBlk;
        const int col = ((((n0 >> 3) | tr_hi) ^ tr_swz) << 4) | tr_half;
        uint32_t w[4];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int row = 32 * sub + 4 * t + tr_row;
          const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_ptr)(smem + sb * kTB + row * kBRowBytes + col));
          const short v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
          w[2 * t] = (uint16_t)v0 | ((uint32_t)(uint16_t)v1 << 16);
          w[2 * t + 1] = (uint16_t)v2 | ((uint32_t)(uint16_t)v3 << 16);
        }
        fb[q - kNB][h] = u32x4{w[0], w[1], w[2], w[3]};
      } else {
        fb[q - kNB][h] = *reinterpret_cast<const u32x4*>(smem + sb * kTB + b_fb +
                                                         (q - kNB) * kBlk * kRowB + off);
      }
    }
  };
  // MFMAs of accumulator row i, columns [j0, j1)
  auto mma = [&](const u32x4 (&fa)[kNB][kCh], const u32x4 (&fb)[kNB][kCh], int i, int j0,
                 int j1) {
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      if constexpr (kIsFP8)
        acc[i][j] = mma32x32_fp8(fb[i], fa[j], acc[i][j]);
      else
        mma16x16<kKind>(fb[i][0], fa[j][0], acc[i][j]);
    }
  };
  auto mod5 = [](int x) { return x >= 5 ? x - 5 : x; };
#define SILE_FENCE __builtin_amdgcn_sched_barrier(0)

  // k-step ks with its A tile in slot c0 and B tile in slot c0 + 1 (mod 5);
  // loads B of ks + 1 when kLoadB, A of ks + 2 when kLoadA
  auto iteration = [&](int ks, int c0, auto load_b_c, auto load_a_c, auto final_c) {
    constexpr bool kFinal = decltype(final_c)::value;
    constexpr bool kLoadB = decltype(load_b_c)::value, kLoadA = decltype(load_a_c)::value;
    const int sa = c0, sb = mod5(c0 + 1), lb = mod5(c0 + 3), la = mod5(c0 + 4);
    int n = 0;   // tile loads issued so far in this k-step
    auto loads = [&]() {
#pragma unroll
      for (int t = 0; t < kLoadsPerGroup; ++t, ++n) {
        if (n < kOpLoads) {
          if constexpr (kLoadB) load(true, ks + 1, lb, n);
        } else {
          if constexpr (kLoadA) load(false, ks + 2, la, n - kOpLoads);
        }
      }
    };
    // one group: row i of (fa, fb), reading fragments [q0, q0 + nq) of
    // sub-step sub into (ra, rb) in two halves
    auto group = [&](const u32x4 (&fa)[kNB][kCh], const u32x4 (&fb)[kNB][kCh], int i,
                     int sub, int q0, int nq, u32x4 (&ra)[kNB][kCh], u32x4 (&rb)[kNB][kCh]) {
      SILE_FENCE; mma(fa, fb, i, 0, kQ1); SILE_FENCE;
#pragma unroll
      for (int q = q0; q < q0 + nq / 2; ++q) read(sa, sb, sub, q, ra, rb);
      SILE_FENCE; mma(fa, fb, i, kQ1, kQ2); SILE_FENCE;
#pragma unroll
      for (int q = q0 + nq / 2; q < q0 + nq; ++q) read(sa, sb, sub, q, ra, rb);
      SILE_FENCE; mma(fa, fb, i, kQ2, kQ3); SILE_FENCE;
      loads();
      SILE_FENCE; mma(fa, fb, i, kQ3, kNB); SILE_FENCE;
    };
    // phase 0: MFMA Y(ks - 1) rows kNB/2 .. kNB-1 | reads X(ks), 4 fragments a group
#pragma unroll
    for (int r = 0; r < kNB / 2; ++r) group(ya, yb, kNB / 2 + r, 0, 4 * r, 4, xa, xb);
    if constexpr (kFinal) {
      // K' ends inside X (the first half of the final k-step): mask it
      if (half_last) {
#pragma unroll
        for (int q = 0; q < kNB; ++q)
#pragma unroll
          for (int h = 0; h < kCh; ++h) {
            xa[q][h] = mask_k<kIsFP8>(xa[q][h], (kCh * f_grp + h) * (kIsFP8 ? 16 : 8), kr.k_rem);
            xb[q][h] = mask_k<kIsFP8>(xb[q][h], (kCh * f_grp + h) * (kIsFP8 ? 16 : 8), kr.k_rem);
          }
      }
    }
    // sub-step 1: MFMA X(ks) | reads Y(ks), 2 fragments a group (A blocks
    // first: every MFMA of a row needs all of them)
#pragma unroll
    for (int r = 0; r < kNB; ++r) {
      group(xa, xb, r, 1, 2 * r, 2, ya, yb);
      if constexpr (kFinal) {
        // a half final k-step: sub-step 1 multiplies zeros (the LDS bytes past
        // the last half k-step hold whatever followed it in memory); else
        // K' ends inside Y: its elements past K' are zeroed
#pragma unroll
        for (int q = 2 * r; q < 2 * r + 2; ++q)
#pragma unroll
          for (int h = 0; h < kCh; ++h) {
            const int e0 = (kCh * f_grp + h) * (kIsFP8 ? 16 : 8);
            const int lim = half_last ? 0 : kr.k_rem;
            if (q < kNB) ya[q][h] = mask_k<kIsFP8>(ya[q][h], e0, lim);
            else yb[q - kNB][h] = mask_k<kIsFP8>(yb[q - kNB][h], e0, lim);
          }
      }
    }
    if constexpr (kFinal) {
#pragma unroll
      for (int r = 0; r < kNB; ++r) mma(ya, yb, r, 0, kNB);
      return;
    }
    // tail: MFMA Y(ks) rows 0 .. kNB/2-1
#pragma unroll
    for (int r = 0; r < kNB / 2; ++r) group(ya, yb, r, 1, 0, 0, ya, yb);
    // B of ks + 1 (and A of ks + 1, loaded a k-step earlier) landed: only the
    // kOpLoads loads of A of ks + 2 may still be in flight
    if constexpr (kLoadA)
      __builtin_amdgcn_s_waitcnt(kOpLoads | (0x7 << 4) | (0x0 << 8));
    else
      __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0x0 << 8));
    __builtin_amdgcn_s_barrier();
    SILE_FENCE;
  };
#undef SILE_FENCE

  // prologue: A of 0 -> slot 0, B of 0 -> slot 1, A of 1 -> slot 2; Y(-1) is zero
#pragma unroll
  for (int i = 0; i < kOpLoads; ++i) load(false, 0, 0, i);
#pragma unroll
  for (int i = 0; i < kOpLoads; ++i) load(true, 0, 1, i);
  if (last >= 1) {
#pragma unroll
    for (int i = 0; i < kOpLoads; ++i) load(false, 1, 2, i);
  }
#pragma unroll
  for (int i = 0; i < kNB; ++i)
#pragma unroll
    for (int h = 0; h < kCh; ++h) ya[i][h] = yb[i][h] = u32x4{0u, 0u, 0u, 0u};
  if (last >= 1)
    __builtin_amdgcn_s_waitcnt(kOpLoads | (0x7 << 4) | (0x0 << 8));   // A and B of 0 landed
  else
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0x0 << 8));
  __builtin_amdgcn_s_barrier();
  int ks = 0, c0 = 0;
  for (; ks + 2 <= last; ++ks) {
    iteration(ks, c0, std::true_type{}, std::true_type{}, std::false_type{});
    c0 = mod5(c0 + 2);
  }
  if (ks + 1 == last) {
    iteration(ks, c0, std::true_type{}, std::false_type{}, std::false_type{});
    c0 = mod5(c0 + 2);
    ++ks;
  }
  iteration(ks, c0, std::false_type{}, std::false_type{}, std::true_type{});

  // the 16 x 16 MFMAs are opaque to the compiler (inline assembly): pad the
  // wait states before their results are read (32 > what a 16x16x32 needs)
  if constexpr (!kIsFP8) asm volatile("s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");
  // ---- epilogue: calls f(row, col, v) for the 4 consecutive columns of each
  // accumulator register group (row, col within the wave's kW x kW) ----
  auto each_c4 = [&](auto f) {
#pragma unroll
    for (int i = 0; i < kNB; ++i)
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        if constexpr (kIsFP8) {
#pragma unroll
          for (int rg = 0; rg < 4; ++rg) {
            f32x4 v = {acc[i][j][4 * rg], acc[i][j][4 * rg + 1], acc[i][j][4 * rg + 2],
                       acc[i][j][4 * rg + 3]};
            if (g.alpha != 1.0f) v *= g.alpha;
            f(32 * j + (lane & 31), 32 * i + 8 * rg + 4 * (lane >> 5), v);
          }
        } else {
          f32x4 v = acc[i][j];
          if (g.alpha != 1.0f) v *= g.alpha;
          f(16 * j + (lane & 15), 16 * i + 4 * (lane >> 4), v);
        }
      }
  };
  const int64_t m0 = p.row0 + wm * kW, n0 = p.col0 + wn * kW;
  constexpr bool kGuardRows = kT == 128;   // M may end inside the tile
  const int rows = kGuardRows ? (int)min<int64_t>(kW, (int64_t)g.m - m0) : kW;
  if constexpr (kOut != kOutF32) {
    __syncthreads();   // every wave is done reading the ring
    stage_and_store_c<kOut, kW, kGuardRows>(C, g.ldc, m0, n0, smem + wave * kCStageB<kW>, rows,
                                            each_c4);
  } else {
    // fp32 C: the plane of this workgroup's k-range (plane 0 when K is not split)
    float* cz = static_cast<float*>(C) + (int64_t)blockIdx.y * g.c_split;
    each_c4([&](int row, int col, f32x4 v) {
      if (!kGuardRows || row < rows) store_c4<kOut>(cz, (m0 + row) * g.ldc + n0 + col, v);
    });
  }
}

}  // namespace

#define SILE_GEMM_KERNEL_B(NAME, KIND, OUT, KT, BROW)                                         \
  extern "C" __global__ __launch_bounds__(256, 256 / KT) void NAME(const void* A,              \
                                                                   const void* B, void* C,      \
                                                                   GemmArgs g) {               \
    static_assert(4 * kCStageB<KT / 2> <= 5 * KT * kRowB, "staged C fits the ring");           \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[5 * KT * kRowB];                   \
    gemm_ring_body<KIND, OUT, KT, BROW>(static_cast<const uint8_t*>(A),                       \
                                        static_cast<const uint8_t*>(B), C, g, smem);          \
  }
#define SILE_GEMM_KERNEL(NAME, KIND, OUT, KT) SILE_GEMM_KERNEL_B(NAME, KIND, OUT, KT, false)

// k_steps counts half k-steps: 32 elements (16-bit) or 64 (fp8)
SILE_GEMM_KERNEL(sile_gemm_nt_bf16_bf16, kBF16, kOutBF16, 256)
SILE_GEMM_KERNEL(sile_gemm_nt_bf16_f32, kBF16, kOutF32, 256)
SILE_GEMM_KERNEL(sile_gemm_nt_f16_f16, kF16, kOutF16, 256)
SILE_GEMM_KERNEL(sile_gemm_nt_f16_f32, kF16, kOutF32, 256)
SILE_GEMM_KERNEL(sile_gemm_nt_fp8_bf16, kFP8, kOutBF16, 256)
SILE_GEMM_KERNEL(sile_gemm_nt_fp8_f32, kFP8, kOutF32, 256)
// 128 x 128 tiles: shapes whose 256 x 256 tiles would leave CUs idle, and M
// or N below 256
SILE_GEMM_KERNEL(sile_gemm_nt128_bf16_bf16, kBF16, kOutBF16, 128)
SILE_GEMM_KERNEL(sile_gemm_nt128_bf16_f32, kBF16, kOutF32, 128)
SILE_GEMM_KERNEL(sile_gemm_nt128_f16_f16, kF16, kOutF16, 128)
SILE_GEMM_KERNEL(sile_gemm_nt128_f16_f32, kF16, kOutF32, 128)
SILE_GEMM_KERNEL(sile_gemm_nt128_fp8_bf16, kFP8, kOutBF16, 128)
SILE_GEMM_KERNEL(sile_gemm_nt128_fp8_f32, kFP8, kOutF32, 128)
// B row-major [K, N] (16-bit operands), the same two tile sizes
SILE_GEMM_KERNEL_B(sile_gemm_nn_bf16_bf16, kBF16, kOutBF16, 256, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn_bf16_f32, kBF16, kOutF32, 256, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn_f16_f16, kF16, kOutF16, 256, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn_f16_f32, kF16, kOutF32, 256, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn128_bf16_bf16, kBF16, kOutBF16, 128, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn128_bf16_f32, kBF16, kOutF32, 128, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn128_f16_f16, kF16, kOutF16, 128, true)
SILE_GEMM_KERNEL_B(sile_gemm_nn128_f16_f32, kF16, kOutF32, 128, true)

// out[c][r] = in[r][c] for r < rows, c < cols (elements of 1 or 2 bytes):
// a row-major B [K, N] written column-major ([N, K], K contiguous) for the
// GEMM shapes whose row-major kernels cannot take it.  A workgroup moves a
// tile of 128 x 128 bytes (128 rows of 128 or 64 elements) through LDS:
// 16-byte loads along the input rows, 16-byte stores along the output rows
// (each gathered from 16 / sizeof(T) input rows in LDS), when the tile lies
// inside both matrices and `vec` says rows start on 16-byte boundaries;
// element by element otherwise.  LDS rows are padded by 4 bytes, so the
// gathers of one column touch distinct banks.
template <typename T>
__device__ __forceinline__ void transpose_body(const T* __restrict__ in, int64_t ldi,
                                               T* __restrict__ out, int64_t ldo, int64_t rows,
                                               int64_t cols, int vec) {
  constexpr int kR = 128, kC = 128 / sizeof(T), kE = 16 / sizeof(T);  // tile rows, cols
  constexpr int kPitch = 128 + 4;                                       // LDS row bytes
  __shared__ __attribute__((aligned(16))) uint8_t tile[kR * kPitch];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * kR, c0 = (int64_t)blockIdx.x * kC;
  auto at = [&](int r, int c) -> T& { return *reinterpret_cast<T*>(tile + r * kPitch + c * sizeof(T)); };
  if (vec && r0 + kR <= rows && c0 + kC <= cols) {
    // 128 rows x 8 chunks in, 4 a thread
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = j * 256 + t, r = e >> 3, ch = e & 7;
      const u32x4 v = *reinterpret_cast<const u32x4*>(in + (r0 + r) * ldi + c0 + ch * kE);
      uint32_t* d = reinterpret_cast<uint32_t*>(tile + r * kPitch + ch * 16);
      d[0] = v[0]; d[1] = v[1]; d[2] = v[2]; d[3] = v[3];
    }
    __syncthreads();
    // kC output rows of kR elements, kCh chunks of kE each: 4 chunks a thread
    constexpr int kCh = kR / kE;
#pragma unroll
    for (int j = 0; j < kC * kCh / 256; ++j) {
      const int e = j * 256 + t, c = e / kCh, ch = e % kCh;
      T g[kE];
#pragma unroll
      for (int i = 0; i < kE; ++i) g[i] = at(ch * kE + i, c);
      u32x4 w;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t x = 0;
#pragma unroll
        for (int b = 0; b < 4 / (int)sizeof(T); ++b)
          x |= (uint32_t)g[q * (4 / sizeof(T)) + b] << (8 * sizeof(T) * b);
        w[q] = x;
      }
      *reinterpret_cast<u32x4*>(out + (c0 + c) * ldo + r0 + ch * kE) = w;
    }
    return;
  }
  for (int e = t; e < kR * kC; e += 256) {
    const int r = e / kC, c = e % kC;
    if (r0 + r < rows && c0 + c < cols) at(r, c) = in[(r0 + r) * ldi + c0 + c];
  }
  __syncthreads();
  for (int e = t; e < kR * kC; e += 256) {
    const int c = e / kR, r = e % kR;
    if (c0 + c < cols && r0 + r < rows) out[(c0 + c) * ldo + r0 + r] = at(r, c);
  }
}
extern "C" __global__ __launch_bounds__(256) void sile_transpose_e1(const uint8_t* in, int64_t ldi,
                                                                    uint8_t* out, int64_t ldo,
                                                                    int64_t rows, int64_t cols,
                                                                    int vec) {
  transpose_body<uint8_t>(in, ldi, out, ldo, rows, cols, vec);
}
extern "C" __global__ __launch_bounds__(256) void sile_transpose_e2(const uint16_t* in,
                                                                    int64_t ldi, uint16_t* out,
                                                                    int64_t ldo, int64_t rows,
                                                                    int64_t cols, int vec) {
  transpose_body<uint16_t>(in, ldi, out, ldo, rows, cols, vec);
}

// Split K: the ring kernel above writes one fp32 plane of C per k-range
// (planes `plane` elements apart, rows n elements long); this kernel adds the
// planes in k-range order, scales by alpha and writes C in its type.  N is a
// multiple of 4; workgroup (x, y) takes 4-element groups 256 x + t of rows
// y, y + gridDim.y, ...
template <int kOut>
__device__ __forceinline__ void splitk_reduce_body(const float* __restrict__ ws,
                                                   void* __restrict__ C, int64_t ldc, int64_t m,
                                                   int64_t n, int64_t plane, int splits,
                                                   float alpha) {
  const int64_t c4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (c4 >= n) return;
  for (int64_t row = blockIdx.y; row < m; row += gridDim.y) {
    const float* src = ws + row * n + c4;
    f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src));
    for (int z = 1; z < splits; ++z)
      v += __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + z * plane));
    if (alpha != 1.0f) v *= alpha;
    store_c4<kOut>(C, row * ldc + c4, v);
  }
}

#define SILE_GEMM_SPLITK_REDUCE(NAME, OUT)                                                    \
  extern "C" __global__ __launch_bounds__(256) void NAME(const float* ws, void* C, int64_t ldc, \
                                                         int64_t m, int64_t n, int64_t plane,   \
                                                         int splits, float alpha) {             \
    splitk_reduce_body<OUT>(ws, C, ldc, m, n, plane, splits, alpha);                          \
  }
SILE_GEMM_SPLITK_REDUCE(sile_gemm_splitk_reduce_bf16, kOutBF16)
SILE_GEMM_SPLITK_REDUCE(sile_gemm_splitk_reduce_f16, kOutF16)
SILE_GEMM_SPLITK_REDUCE(sile_gemm_splitk_reduce_f32, kOutF32)

// The same sum for the transposed form: the ring kernel ran C^T = B . A^T
// (A and B swapped), so plane z holds C^T as n rows of `pitch` fp32 (pitch a
// multiple of 4, at least m).  C[i][j] = alpha * sum_z plane_z[j][i], in plane
// order.  A workgroup moves one 32 (i) x 64 (j) block through LDS: 16-byte
// reads along i, element stores along j (C may have any pitch and alignment).
template <int kOut>
__device__ __forceinline__ void splitk_reduce_t_body(const float* __restrict__ ws,
                                                     void* __restrict__ C, int64_t ldc, int64_t m,
                                                     int64_t n, int64_t plane, int64_t pitch,
                                                     int splits, float alpha) {
  __shared__ float blk[64][33];
  const int tid = threadIdx.x;
  const int64_t i0 = (int64_t)blockIdx.x * 32, j0 = (int64_t)blockIdx.y * 64;
  const int iq = 4 * (tid & 7);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int jj = (tid >> 3) + 32 * p;
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (j0 + jj < n && i0 + iq < m) {
      const float* src = ws + (j0 + jj) * pitch + i0 + iq;
      v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src));
      for (int z = 1; z < splits; ++z)
        v += __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + z * plane));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) blk[jj][iq + e] = v[e];
  }
  __syncthreads();
  const int jj = tid & 63;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int ii = (tid >> 6) + 4 * q;
    const int64_t i = i0 + ii, j = j0 + jj;
    if (i >= m || j >= n) continue;
    const float x = alpha != 1.0f ? blk[jj][ii] * alpha : blk[jj][ii];
    if constexpr (kOut == kOutF32)
      static_cast<float*>(C)[i * ldc + j] = x;
    else if constexpr (kOut == kOutBF16)
      static_cast<uint16_t*>(C)[i * ldc + j] = bf16_rne(x);
    else
      static_cast<uint16_t*>(C)[i * ldc + j] = f16_rne(x);
  }
}

#define SILE_GEMM_SPLITK_REDUCE_T(NAME, OUT)                                                  \
  extern "C" __global__ __launch_bounds__(256) void NAME(                                     \
      const float* ws, void* C, int64_t ldc, int64_t m, int64_t n, int64_t plane,             \
      int64_t pitch, int splits, float alpha) {                                               \
    splitk_reduce_t_body<OUT>(ws, C, ldc, m, n, plane, pitch, splits, alpha);                 \
  }
SILE_GEMM_SPLITK_REDUCE_T(sile_gemm_splitk_reduce_t_bf16, kOutBF16)
SILE_GEMM_SPLITK_REDUCE_T(sile_gemm_splitk_reduce_t_f16, kOutF16)
SILE_GEMM_SPLITK_REDUCE_T(sile_gemm_splitk_reduce_t_f32, kOutF32)

// ---------------------------------------------------------------------------
// Any shape: M or N below one 256 x 256 tile, or N not a multiple of 4.
//
// 64 x 64 output tile per workgroup of 4 waves (2 x 2), a 32 x 32 block per
// wave on v_mfma_f32_32x32x16_{bf16,f16} (16 k per MFMA) or
// v_mfma_f32_32x32x64_f8f6f4 (64 k).  The operands are small, so each lane
// loads its fragments straight from global memory (L2): lane l supplies row
// (A) or column (B, stored [N, K]) l % 32 and the 8 (16-bit) or 32 (fp8)
// consecutive k of k-group l / 32, one or two 16-byte loads.  Rows past M,
// columns past N and k past K' are zero in both operands (the last k-step
// element by element), so NaN or Inf past K' never reaches a product.  The
// accumulator register i of lane l is C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]
// of the block; stores skip C outside [M, N].
// ---------------------------------------------------------------------------
struct SmallArgs {
  int64_t lda, ldb, ldc;  // in elements
  int64_t m, n, kp;
  float alpha;
};

template <int kKind, int kOut>
__device__ __forceinline__ void gemm_small_body(const uint8_t* __restrict__ A,
                                                const uint8_t* __restrict__ B, void* __restrict__ C,
                                                const SmallArgs& g) {
  constexpr bool kIsFP8 = kKind == kFP8;
  constexpr int kEB = kIsFP8 ? 1 : 2;        // bytes per element
  constexpr int kKStep = kIsFP8 ? 64 : 16;   // k per MFMA
  constexpr int kGrpK = kKStep / 2;          // k per lane group (16 or 32 bytes)
  constexpr int kCh = kGrpK * kEB / 16;      // 16-byte chunks per fragment
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31, grp = lane >> 5;
  const int64_t row0 = (int64_t)blockIdx.y * 64 + (wave >> 1) * 32;
  const int64_t col0 = (int64_t)blockIdx.x * 64 + (wave & 1) * 32;
  const int64_t arow = row0 + r, bcol = col0 + r;
  const bool a_ok = arow < g.m, b_ok = bcol < g.n;
  const uint8_t* ap = A + (a_ok ? arow : 0) * g.lda * kEB;
  const uint8_t* bp = B + (b_ok ? bcol : 0) * g.ldb * kEB;
  // one operand fragment at k = kg: whole 16-byte chunks inside K', else
  // element by element with zeros past K' (and everywhere for a row past M /
  // a column past N)
  auto frag = [&](const uint8_t* base, bool ok, int64_t kg, u32x4 (&f)[kCh]) {
    if (ok && kg + kGrpK <= g.kp) {
#pragma unroll
      for (int h = 0; h < kCh; ++h) f[h] = *reinterpret_cast<const u32x4*>(base + kg * kEB + 16 * h);
    } else {
#pragma unroll
      for (int h = 0; h < kCh; ++h) {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t v = 0;
#pragma unroll
          for (int e = 0; e < 4 / kEB; ++e) {
            const int64_t k = kg + (16 * h + 4 * q) / kEB + e;
            uint32_t x = 0;
            if (ok && k < g.kp)
              x = kEB == 1 ? base[k] : *reinterpret_cast<const uint16_t*>(base + 2 * k);
            v |= x << (8 * kEB * e);
          }
          w[q] = v;
        }
        f[h] = u32x4{w[0], w[1], w[2], w[3]};
      }
    }
  };
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
  auto mma = [&](const u32x4 (&fa)[kCh], const u32x4 (&fb)[kCh]) {
    if constexpr (kIsFP8) {
      acc = mma32x32_fp8(fa, fb, acc);
    } else if constexpr (kKind == kBF16) {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fa[0]),
                                                     __builtin_bit_cast(bf16x8, fb[0]), acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, fa[0]),
                                                    __builtin_bit_cast(f16x8, fb[0]), acc, 0, 0, 0);
    }
  };
  // Whole k-steps in blocks of kU, the loads of the next block in flight
  // while the current block's MFMAs run (two register sets), so the chain is
  // not held up by the global-load latency of each step; then the remaining
  // steps one at a time (the last may be partial).  The k order is the same.
  constexpr int kU = kIsFP8 ? 4 : 8;
  constexpr int64_t kBlk = (int64_t)kU * kKStep;
  const int64_t kfull = (g.kp / kBlk) * kBlk;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  auto load_blk = [&](int64_t k0, u32x4 (&fa)[kU][kCh], u32x4 (&fb)[kU][kCh]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t kg = k0 + u * kKStep + grp * kGrpK;
#pragma unroll
      for (int h = 0; h < kCh; ++h) {
        fa[u][h] = a_ok ? *reinterpret_cast<const u32x4*>(ap + kg * kEB + 16 * h) : zero4;
        fb[u][h] = b_ok ? *reinterpret_cast<const u32x4*>(bp + kg * kEB + 16 * h) : zero4;
      }
    }
  };
  auto mma_blk = [&](const u32x4 (&fa)[kU][kCh], const u32x4 (&fb)[kU][kCh]) {
#pragma unroll
    for (int u = 0; u < kU; ++u) mma(fa[u], fb[u]);
  };
  if (kfull > 0) {
    u32x4 fa0[kU][kCh], fb0[kU][kCh], fa1[kU][kCh], fb1[kU][kCh];
    load_blk(0, fa0, fb0);
    for (int64_t k0 = 0; k0 < kfull; k0 += 2 * kBlk) {
      const bool more = k0 + kBlk < kfull;
      if (more) load_blk(k0 + kBlk, fa1, fb1);
      mma_blk(fa0, fb0);
      if (!more) break;
      if (k0 + 2 * kBlk < kfull) load_blk(k0 + 2 * kBlk, fa0, fb0);
      mma_blk(fa1, fb1);
    }
  }
  for (int64_t k0 = kfull; k0 < g.kp; k0 += kKStep) {
    const int64_t kg = k0 + grp * kGrpK;
    u32x4 fa[kCh], fb[kCh];
    frag(ap, a_ok, kg, fa);
    frag(bp, b_ok, kg, fb);
    mma(fa, fb);
  }
  const int64_t col = col0 + r;
  if (col >= g.n) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t row = row0 + 8 * (i / 4) + 4 * grp + (i % 4);
    if (row >= g.m) continue;
    const float v = g.alpha != 1.0f ? acc[i] * g.alpha : acc[i];
    if constexpr (kOut == kOutF32)
      static_cast<float*>(C)[row * g.ldc + col] = v;
    else if constexpr (kOut == kOutBF16)
      static_cast<uint16_t*>(C)[row * g.ldc + col] = bf16_rne(v);
    else
      static_cast<uint16_t*>(C)[row * g.ldc + col] = f16_rne(v);
  }
}

#define SILE_GEMM_SMALL_KERNEL(NAME, KIND, OUT)                                                \
  extern "C" __global__ __launch_bounds__(256) void NAME(const void* A, const void* B, void* C, \
                                                         SmallArgs g) {                        \
    gemm_small_body<KIND, OUT>(static_cast<const uint8_t*>(A), static_cast<const uint8_t*>(B), \
                               C, g);                                                          \
  }
SILE_GEMM_SMALL_KERNEL(sile_gemm_small_bf16_bf16, kBF16, kOutBF16)
SILE_GEMM_SMALL_KERNEL(sile_gemm_small_bf16_f32, kBF16, kOutF32)
SILE_GEMM_SMALL_KERNEL(sile_gemm_small_f16_f16, kF16, kOutF16)
SILE_GEMM_SMALL_KERNEL(sile_gemm_small_f16_f32, kF16, kOutF32)
SILE_GEMM_SMALL_KERNEL(sile_gemm_small_fp8_bf16, kFP8, kOutBF16)
SILE_GEMM_SMALL_KERNEL(sile_gemm_small_fp8_f32, kFP8, kOutF32)

// C = 0 for K' = 0 (K below one BK): the canonical matmul's sums start at
// 0.0f and add no term (crates/sile-tile-ir/src/passes/lowering/canonical_matmul.rs:58-73,
// k_limit = 0).  C is addressed in 16-bit words: n16 words per row, ldc16
// words between rows (both exact for 16- and 32-bit C).
extern "C" __global__ __launch_bounds__(256) void sile_gemm_zero_c(uint16_t* C, int64_t ldc16,
                                                                   int64_t n16, int64_t m) {
  for (int64_t r = blockIdx.x; r < m; r += gridDim.x)
    for (int64_t c = threadIdx.x; c < n16; c += blockDim.x) C[r * ldc16 + c] = 0;
}

// fp32 GEMM on any shape in the canonical matmul's exact order: one thread per
// cell, s = s + a*b from 0.0f over k < kp with separate roundings (no FMA).
// A row-major [M,K]; B either row-major [K,N] (b_col_major = 0, the reference
// layout) or column-major (stored [N,K]).
// fp32 GEMM in the canonical order, register-tiled.  Each output keeps the
// reference's chain s = s + a[k] * b[k] from 0.0f in increasing k, the product
// and the sum rounded separately (no contraction), so the result is the same
// bit for bit as the CPU backend's.  The work is organised as T x T outputs
// per workgroup of 256 threads (T = 128, 64 or 32: the largest that still gives
// ~1024 workgroups), (T/16) x (T/16) independent chains per thread, operands staged in LDS
// in 16-deep k-tiles (64 for T = 32; double-buffered in LDS, with the global
// loads issued two k-tiles ahead into two register sets, 16-byte loads where a
// thread's run of a row is inside the operand), A and a column-major B
// transposed on the way in so a thread reads its 8 rows / 8 columns of one k as
// two 16-byte LDS reads.  Outside M, N and K' the staged A values are -0.0f and
// the staged B values +0.0f, so a padded term adds -0.0f, which leaves every
// sum unchanged (x + -0.0f == x for every x, +0.0f and -0.0f included).
// The chain starts from its seed: S[m][n] when S is given (the reference's
// tile MMA seeded from an accumulator tile, mma.rs:213-229; S may be C
// itself), otherwise the constant `seed` (0.0f for the canonical matmul, the
// splat value of a LoopCarriedSplat accumulator, mma.rs:483-558).
namespace f32t {
constexpr int kPad = 4;
}

// kT x kT outputs per workgroup of 256 threads, kR x kR per thread (kR = kT / 16);
// k-tiles 16 deep, 64 for the 32-wide tile (its 4 chains per thread overlap a
// load with the least work, so it waits for loads fewer times; measured
// 35 -> 32 us at 512^3, while 32-deep tiles made 64-wide ones slower)
template <bool kBCol, int kT>
__device__ __forceinline__ void gemm_f32_tiled_body(const float* __restrict__ A,
                                                    const float* __restrict__ B, float* C,
                                                    int64_t M, int64_t N, int64_t kp, int64_t lda,
                                                    int64_t ldb, int64_t ldc, const float* S,
                                                    int64_t lds, float seed) {
#pragma clang fp contract(off)
  using namespace f32t;
  constexpr int kK = kT == 32 ? 64 : 16;  // k-tile depth
  constexpr int kR = kT / 16;           // outputs per thread and dimension
  constexpr int kL = kT * kK / 256;     // staged elements per thread and operand
  static_assert(kR == 2 || kR == 4 || kR == 8, "tile sizes 32, 64, 128");
  __shared__ __attribute__((aligned(16))) float As[2][kK][kT + kPad];
  __shared__ __attribute__((aligned(16))) float Bs[2][kK][kT + kPad];
  const int t = threadIdx.x;
  const int tm = t >> 4, tn = t & 15;
  const int64_t m0 = (int64_t)blockIdx.y * kT, n0 = (int64_t)blockIdx.x * kT;
  // staging: A row m0 + la_r, k offsets la_k .. + kL; B likewise (column-major)
  // or B row k0 + lb_r, columns n0 + lb_c .. + kL (row-major)
  const int la_r = t / (kK / kL), la_k = (t % (kK / kL)) * kL;
  const int lb_r = kBCol ? la_r : t / (kT / kL);
  const int lb_c = kBCol ? la_k : (t % (kT / kL)) * kL;
  float ra_s[2][kL], rb_s[2][kL];
  // whole rows of 16-byte vectors: A (and a column-major B) rows start 16-byte aligned
  const bool vec_a = (lda & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0 && kL % 4 == 0;
  const bool vec_b = (ldb & 3) == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0 && kL % 4 == 0;
  auto gload = [&](int64_t k0, float (&ra)[kL], float (&rb)[kL]) {
    const int64_t am = m0 + la_r;
    if (vec_a && am < M && k0 + la_k + kL <= kp) {
#pragma unroll
      for (int i = 0; i < kL; i += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(A + am * lda + k0 + la_k + i);
        ra[i] = v[0]; ra[i + 1] = v[1]; ra[i + 2] = v[2]; ra[i + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kL; ++i) {
        const int64_t k = k0 + la_k + i;
        ra[i] = (am < M && k < kp) ? A[am * lda + k] : -0.0f;
      }
    }
    if constexpr (kBCol) {
      const int64_t bn = n0 + lb_r;
      if (vec_b && bn < N && k0 + lb_c + kL <= kp) {
#pragma unroll
        for (int i = 0; i < kL; i += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(B + bn * ldb + k0 + lb_c + i);
          rb[i] = v[0]; rb[i + 1] = v[1]; rb[i + 2] = v[2]; rb[i + 3] = v[3];
        }
      } else {
#pragma unroll
        for (int i = 0; i < kL; ++i) {
          const int64_t k = k0 + lb_c + i;
          rb[i] = (bn < N && k < kp) ? B[bn * ldb + k] : 0.0f;
        }
      }
    } else {
      const int64_t k = k0 + lb_r;
      if (vec_b && k < kp && n0 + lb_c + kL <= N) {
#pragma unroll
        for (int i = 0; i < kL; i += 4) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(B + k * ldb + n0 + lb_c + i);
          rb[i] = v[0]; rb[i + 1] = v[1]; rb[i + 2] = v[2]; rb[i + 3] = v[3];
        }
      } else {
#pragma unroll
        for (int i = 0; i < kL; ++i) {
          const int64_t bn = n0 + lb_c + i;
          rb[i] = (bn < N && k < kp) ? B[k * ldb + bn] : 0.0f;
        }
      }
    }
  };
  auto sstore = [&](int buf, const float (&ra)[kL], const float (&rb)[kL]) {
#pragma unroll
    for (int i = 0; i < kL; ++i) As[buf][la_k + i][la_r] = ra[i];
    if constexpr (kBCol) {
#pragma unroll
      for (int i = 0; i < kL; ++i) Bs[buf][lb_c + i][lb_r] = rb[i];
    } else {
#pragma unroll
      for (int i = 0; i < kL; ++i) Bs[buf][lb_r][lb_c + i] = rb[i];
    }
  };
  // kR consecutive floats of an LDS row
  auto lread = [&](const float* p, float (&v)[kR]) {
    if constexpr (kR == 2) {
      const f32x2 x = *reinterpret_cast<const f32x2*>(p);
      v[0] = x[0]; v[1] = x[1];
    } else {
#pragma unroll
      for (int h = 0; h < kR / 4; ++h) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(p + 4 * h);
        v[4 * h] = x[0]; v[4 * h + 1] = x[1]; v[4 * h + 2] = x[2]; v[4 * h + 3] = x[3];
      }
    }
  };

  float acc[kR][kR];
#pragma unroll
  for (int i = 0; i < kR; ++i)
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int64_t m = m0 + kR * tm + i, n = n0 + kR * tn + j;
      acc[i][j] = (S && m < M && n < N) ? S[m * lds + n] : seed;
    }

  const int64_t ktiles = (kp + kK - 1) / kK;
  if (ktiles > 0) {
    gload(0, ra_s[0], rb_s[0]);
    sstore(0, ra_s[0], rb_s[0]);
  }
  if (ktiles > 1) gload(kK, ra_s[1], rb_s[1]);
  __syncthreads();
  // k-tile kt is computed from LDS buffer kt & 1 while the global loads of
  // k-tile kt + 2 are in flight into register set kt & 1; k-tile kt + 1 (in
  // set (kt + 1) & 1 since the previous iteration) is stored after the compute
  auto ktile = [&](int64_t kt, auto set_c) {
    constexpr int kSet = decltype(set_c)::value;
    const int buf = kSet;
    if (kt + 2 < ktiles) gload((kt + 2) * kK, ra_s[kSet], rb_s[kSet]);
    // the 32-wide tile (one wave per SIMD, 4 chains a thread) waits on its
    // LDS reads unless they run several k ahead: unrolled 8 (512^3: 32 -> 21 us);
    // the larger tiles keep 2 (their chains hide the reads, and deeper unrolling
    // hoists their reads into too many registers)
#pragma unroll (kT == 32 ? 8 : 2)
    for (int kk = 0; kk < kK; ++kk) {
      float av[kR], bv[kR];
      lread(&As[buf][kk][kR * tm], av);
      lread(&Bs[buf][kk][kR * tn], bv);
#pragma unroll
      for (int i = 0; i < kR; ++i)
#pragma unroll
        for (int j = 0; j < kR; ++j) {
          const float p = av[i] * bv[j];
          acc[i][j] = acc[i][j] + p;
        }
    }
    if (kt + 1 < ktiles) sstore(buf ^ 1, ra_s[kSet ^ 1], rb_s[kSet ^ 1]);
    __syncthreads();
  };
  int64_t kt = 0;
  for (; kt + 2 <= ktiles; kt += 2) {
    ktile(kt, std::integral_constant<int, 0>{});
    ktile(kt + 1, std::integral_constant<int, 1>{});
  }
  if (kt < ktiles) ktile(kt, std::integral_constant<int, 0>{});
#pragma unroll
  for (int i = 0; i < kR; ++i) {
    const int64_t m = m0 + kR * tm + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < kR; ++j) {
      const int64_t n = n0 + kR * tn + j;
      if (n < N) C[m * ldc + n] = acc[i][j];
    }
  }
}

#define SILE_GEMM_F32_TILED(NAME, BCOL, T)                                                     \
  extern "C" __global__ __launch_bounds__(256, 2) void NAME(                                   \
      const float* __restrict__ A, const float* __restrict__ B, float* C, int64_t M,          \
      int64_t N, int64_t kp, int64_t lda, int64_t ldb, int64_t ldc, const float* S,           \
      int64_t lds, float seed) {                                                               \
    gemm_f32_tiled_body<BCOL, T>(A, B, C, M, N, kp, lda, ldb, ldc, S, lds, seed);             \
  }
SILE_GEMM_F32_TILED(sile_gemm_f32_exact_nn_t128, false, 128)
SILE_GEMM_F32_TILED(sile_gemm_f32_exact_nn_t64, false, 64)
SILE_GEMM_F32_TILED(sile_gemm_f32_exact_nn_t32, false, 32)
SILE_GEMM_F32_TILED(sile_gemm_f32_exact_nt_t128, true, 128)
SILE_GEMM_F32_TILED(sile_gemm_f32_exact_nt_t64, true, 64)
SILE_GEMM_F32_TILED(sile_gemm_f32_exact_nt_t32, true, 32)

