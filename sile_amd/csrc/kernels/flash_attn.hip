// Flash-attention forward on the gfx950 matrix cores, head_dim 128.
//
//   O = softmax(Q K^T * scale [+ causal mask]) V     Q, K, V, O: [B*H, S, 128] 16-bit
//
// sile's DSL has no attention kernel (no mask, iota or transpose); this is
// the composition of its tile ops MmaF, ReduceMax, Exp, ReduceSum and the
// softmax Map (crates/sile-tile-ir/src/ir.rs:128-262) fused into one pass
// with an fp32 online softmax (running max m, running sum l, rescaled
// accumulator), so S and P never leave registers.
//
// Work split: a workgroup of 4 waves owns a block of 4 * kQT * 32 queries of
// one (batch, head); each wave owns kQT * 32 of them.  The workgroup walks the
// keys in blocks of kNK, staged through LDS (double-buffered: the next block's
// global loads are in flight while the matrix cores work on the current one).
//
// Orientation of the two products (v_mfma_f32_32x32x16_{f16,bf16}):
//   * S^T = K . Q^T : the A operand is K (rows = keys, k = d, read from LDS),
//     the B operand Q^T (k = d, cols = queries, kept in registers for the
//     whole kernel).  The accumulator of lane l holds 16 keys of ONE query
//     (l % 32), so the online-softmax max and sum are in-register folds plus
//     one exchange with lane l ^ 32 for the max.
//   * O^T = V^T . P^T : the A operand is V^T (rows = d, k = keys), the B
//     operand P^T straight from the S^T accumulators converted to 16 bits.
//     The output accumulator of lane l again holds one query (l % 32), so the
//     rescale by exp(m_old - m_new) is a per-lane scalar.
//   32x32 accumulator layout: register i of lane l is row 8*(i/4) + 4*(l/32) + i%4,
//   column l % 32.  A/B operand: lane l supplies row/column l % 32 and 8
//   consecutive k slots of k-group l / 32.
//   P's 8 values for k-group g of a 16-key chunk are the keys
//   {4g..4g+3, 8+4g..8+4g+3} of that chunk (accumulator rows).  V^T is
//   therefore stored in LDS with bits 2 and 3 of the key index swapped inside
//   every 16-key chunk, so that k-group g reads its 8 keys as one 16-byte
//   vector.  V is transposed while it is written to LDS (4 keys x 1 d packed
//   per 8-byte store).
//
// LDS layout per stage: K [kNK][256 B] with 16-byte chunk c of row r at
// c ^ (r & 15); V^T [128][kNK * 2 B] with chunk c of row d at c ^ swz8(d).
// Both make the fragment reads (one row per lane) conflict-free.
//
// Launch order: workgroups are dispatched round-robin over the 8 XCDs, so
// workgroup i runs on XCD i % 8.  Head h is pinned to XCD h % 8 and its query
// blocks are issued together (largest causal block first), so the K/V stream
// of a head is shared in one XCD's L2 by all of its query blocks.
#include <type_traits>

#include "common.h"

using namespace sile;

namespace {

constexpr int kD = 128;
constexpr int kRowB = kD * 2;  // bytes of one K row
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold: p <= 2^8
// fast-path limit on one lane's block sum of p (pipelined kernel): below it
// every p of the block is <= 2^kRescaleLog2
constexpr float kBlockSumLimit = 256.0f;

template <bool kBF16>
SILE_DEV f32x16 mma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (kBF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool kBF16>
SILE_DEV uint32_t pack2(float lo, float hi) {
  return kBF16 ? pack_bf16x2(lo, hi) : pack_f16x2(lo, hi);
}

SILE_DEV int swz8(int d) { return (d ^ (d >> 3)) & 7; }
// bits 2 and 3 of a key index swapped
SILE_DEV int kperm(int k) { return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1); }

struct AttnArgs {
  int64_t seq;          // S
  int32_t bh;           // B * H
  int32_t q_blocks;     // S / kBQ
  float scale_log2;     // softmax scale * log2(e)
  int32_t causal;
  int32_t xcd_map;      // 1: head-per-XCD launch order (bh % 8 == 0)
  int32_t pair;         // 1: causal query blocks in balanced pairs (v2 kernels)
};

// Block kernel for any S (and head_dim 64 or 128): 4 waves x kQT * 32 queries,
// kNK-key blocks staged through LDS by plain loads (double-buffered through
// registers).  Keys and queries past S are zero in the staged operands, keys
// past S are masked to -inf, and queries past S are not stored, so S need
// not be a multiple of any block.
template <bool kBF16, int kQT, int kNK, int kDh>
__device__ __forceinline__ void attn_fwd_body(const uint16_t* __restrict__ Q,
                                              const uint16_t* __restrict__ K,
                                              const uint16_t* __restrict__ V,
                                              uint16_t* __restrict__ O, const AttnArgs& a,
                                              uint8_t* smem) {
  constexpr int kBQ = kWaves * kQT * 32;
  constexpr int kKT = kNK / 32;                     // 32-key tiles per block
  constexpr int kRB = kDh * 2;                      // bytes of one K / V row
  constexpr int kRC = kDh / 8;                      // 16-byte chunks per row
  constexpr int kKBytes = kNK * kRB;                // K stage bytes
  constexpr int kVRowB = kNK * 2;                   // V^T row bytes
  constexpr int kStageB = 2 * kKBytes;              // K + V^T (same size)
  constexpr int kRowsPerPass = kThreads / kRC;      // K rows one pass of the workgroup loads
  constexpr int kKLoads = kNK / kRowsPerPass;       // 16-byte K chunks per thread
  constexpr int kVItems = kNK * kRC / 4 / kThreads; // (4 keys x 8 d) items per thread
  constexpr int kDT = kDh / 32;                     // 32-row tiles of O^T
  constexpr int kDK = kDh / 16;                     // MFMA k-steps over d
  static_assert(kKLoads >= 1 && kVItems >= 1, "block too small for the workgroup");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;

  // ---- which (head, query block) ----
  int bh, qb;
  const int bid = blockIdx.x;
  if (a.xcd_map) {
    const int xcd = bid & 7, idx = bid >> 3;
    bh = ((idx / a.q_blocks) << 3) + xcd;
    qb = idx % a.q_blocks;
  } else {
    bh = bid % a.bh;
    qb = bid / a.bh;
  }
  if (a.causal) qb = a.q_blocks - 1 - qb;  // largest causal blocks first
  const int64_t S = a.seq;
  const int S32 = (int)S;
  const int64_t head_off = (int64_t)bh * S * kDh;
  const uint16_t* Qh = Q + head_off;
  const uint8_t* Kh = reinterpret_cast<const uint8_t*>(K + head_off);
  const uint8_t* Vh = reinterpret_cast<const uint8_t*>(V + head_off);
  const int q0 = qb * kBQ;
  const int wq0 = q0 + wave * kQT * 32;  // first query of this wave

  // ---- Q^T fragments: lane holds query wq0 + 32 qt + l32, d = 16 kk + 8 g + [0, 8) ----
  u32x4 qf[kQT][kDK];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const int q = wq0 + qt * 32 + l32;
    const uint16_t* qrow = Qh + (int64_t)(q < S32 ? q : 0) * kDh + 8 * g;
#pragma unroll
    for (int kk = 0; kk < kDK; ++kk)
      qf[qt][kk] = q < S32 ? *reinterpret_cast<const u32x4*>(qrow + 16 * kk) : u32x4{0u, 0u, 0u, 0u};
  }

  // ---- K / V global -> register staging (rows past S: zero) ----
  // K: thread moves chunk (tid % kRC) of rows tid / kRC + kRowsPerPass i.
  // V: item (key group kg = 4 keys, d chunk dc = 8 d): dc = tid % kRC,
  //    kg = tid / kRC + kRowsPerPass i.
  const int k_chunk = tid % kRC, k_row = tid / kRC;
  u32x4 kreg[kKLoads];
  u32x4 vreg[kVItems][4];
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  auto global_load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < kKLoads; ++i) {
      const int key = kb + k_row + kRowsPerPass * i;
      kreg[i] = key < S32 ? *reinterpret_cast<const u32x4*>(Kh + (int64_t)key * kRB + k_chunk * 16)
                          : zero4;
    }
#pragma unroll
    for (int i = 0; i < kVItems; ++i) {
      const int kg = k_row + kRowsPerPass * i;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = kb + 4 * kg + r;
        vreg[i][r] = key < S32 ? *reinterpret_cast<const u32x4*>(Vh + (int64_t)key * kRB + k_chunk * 16)
                               : zero4;
      }
    }
  };
  auto lds_store = [&](int stage) {
    uint8_t* ks = smem + stage * kStageB;
    uint8_t* vs = ks + kKBytes;
#pragma unroll
    for (int i = 0; i < kKLoads; ++i) {
      const int row = k_row + kRowsPerPass * i;
      *reinterpret_cast<u32x4*>(ks + row * kRB + ((k_chunk ^ (row & (kRC - 1))) << 4)) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < kVItems; ++i) {
      const int kg = k_row + kRowsPerPass * i;
      const int kp = kperm(4 * kg);          // 4 keys stay contiguous
      const int chunk = kp >> 3, half = (kp >> 2) & 1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * k_chunk + e;
        const int w = e >> 1, sh = (e & 1) * 16;
        const uint32_t v0 = (vreg[i][0][w] >> sh) & 0xffffu, v1 = (vreg[i][1][w] >> sh) & 0xffffu;
        const uint32_t v2 = (vreg[i][2][w] >> sh) & 0xffffu, v3 = (vreg[i][3][w] >> sh) & 0xffffu;
        const u32x2 pk = {v0 | (v1 << 16), v2 | (v3 << 16)};
        *reinterpret_cast<u32x2*>(vs + d * kVRowB + ((chunk ^ swz8(d)) << 4) + 8 * half) = pk;
      }
    }
  };

  f32x16 oacc[kQT][kDT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[qt][dt][i] = 0.0f;
  float m_run[kQT], l_run[kQT];
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    m_run[qt] = -__builtin_inff();
    l_run[qt] = 0.0f;
  }

  const int key_end = a.causal ? min(q0 + kBQ, S32) : S32;  // keys any query here sees
  const int nblocks = (key_end + kNK - 1) / kNK;
  const float c = a.scale_log2;

  global_load(0);
  lds_store(0);
  __syncthreads();

  for (int jb = 0; jb < nblocks; ++jb) {
    const int stage = jb & 1;
    const int kb = jb * kNK;
    if (jb + 1 < nblocks) global_load(kb + kNK);
    const bool active = (!a.causal || kb <= wq0 + kQT * 32 - 1) && wq0 < S32;
    if (active) {
      const uint8_t* ks = smem + stage * kStageB;
      const uint8_t* vs = ks + kKBytes;
      // ---- S^T = K . Q^T ----
      f32x16 sacc[kKT][kQT];
#pragma unroll
      for (int t = 0; t < kKT; ++t)
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
#pragma unroll
          for (int i = 0; i < 16; ++i) sacc[t][qt][i] = 0.0f;
#pragma unroll
      for (int t = 0; t < kKT; ++t) {
        const int row = 32 * t + l32;
        const uint8_t* krow = ks + row * kRB;
#pragma unroll
        for (int kk = 0; kk < kDK; ++kk) {
          const u32x4 kf =
              *reinterpret_cast<const u32x4*>(krow + (((2 * kk + g) ^ (row & (kRC - 1))) << 4));
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt) sacc[t][qt] = mma32<kBF16>(kf, qf[qt][kk], sacc[t][qt]);
        }
      }
      // ---- causal mask on the diagonal blocks, keys past S ----
      if ((a.causal && kb + kNK - 1 > wq0) || kb + kNK > S32) {
#pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          const int q = wq0 + 32 * qt + l32;
          const int lim = a.causal ? min(q, S32 - 1) : S32 - 1;  // last visible key
#pragma unroll
          for (int t = 0; t < kKT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int key = kb + 32 * t + 8 * (i >> 2) + 4 * g + (i & 3);
              if (key > lim) sacc[t][qt][i] = -__builtin_inff();
            }
        }
      }
      // ---- online softmax ----
      // The running max m only moves when some lane's block max exceeds it
      // by more than kRescaleLog2 (in log2 units); otherwise exponents are
      // taken against the stale m, so p <= 2^kRescaleLog2 and the rescale of
      // O and l (a pass over all accumulators) is skipped for the block.
      u32x4 pf[kQT][kKT * 2];
#pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        float mx = -__builtin_inff();
#pragma unroll
        for (int t = 0; t < kKT; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = __builtin_fmaxf(mx, sacc[t][qt][i]);
        mx = pair32_max(mx);
        const bool grow = (mx - m_run[qt]) * c > kRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float m_new = __builtin_fmaxf(m_run[qt], mx);
          const float alpha = exp2_fast((m_run[qt] - m_new) * c);
          m_run[qt] = m_new;
          l_run[qt] *= alpha;
#pragma unroll
          for (int dt = 0; dt < kDT; ++dt) oacc[qt][dt] *= alpha;
        }
        const float mc = m_run[qt] * c;
        float rs = 0.0f;
#pragma unroll
        for (int t = 0; t < kKT; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float p = exp2_fast(__builtin_fmaf(sacc[t][qt][i], c, -mc));
            sacc[t][qt][i] = p;
            rs += p;
          }
        l_run[qt] += rs;
#pragma unroll
        for (int t = 0; t < kKT; ++t)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              w[j] = pack2<kBF16>(sacc[t][qt][8 * h + 2 * j], sacc[t][qt][8 * h + 2 * j + 1]);
            pf[qt][2 * t + h] = w;
          }
      }
      // ---- O^T += V^T . P^T ----
#pragma unroll
      for (int dt = 0; dt < kDT; ++dt) {
        const int d = 32 * dt + l32;
        const uint8_t* vrow = vs + d * kVRowB;
#pragma unroll
        for (int cc = 0; cc < kKT * 2; ++cc) {
          const u32x4 vf =
              *reinterpret_cast<const u32x4*>(vrow + (((2 * cc + g) ^ swz8(d)) << 4));
#pragma unroll
          for (int qt = 0; qt < kQT; ++qt) oacc[qt][dt] = mma32<kBF16>(vf, pf[qt][cc], oacc[qt][dt]);
        }
      }
    }
    if (jb + 1 < nblocks) lds_store(stage ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O[q][d] = O^T[d][q] / l (queries past S not stored) ----
#pragma unroll
  for (int qt = 0; qt < kQT; ++qt) {
    const float l = pair32_sum(l_run[qt]);
    const float inv = 1.0f / l;
    const int q = wq0 + 32 * qt + l32;
    if (q >= S32) continue;
    uint16_t* orow = O + head_off + (int64_t)q * kDh;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 32 * dt + 8 * r + 4 * g;
        const f32x16& acc = oacc[qt][dt];
        const u32x2 w = {pack2<kBF16>(acc[4 * r] * inv, acc[4 * r + 1] * inv),
                         pack2<kBF16>(acc[4 * r + 2] * inv, acc[4 * r + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = w;
      }
  }
}

}  // namespace

// ===========================================================================
// Pipelined kernel (any S): 8 waves x 32 queries, 32-key blocks.
//
// Iteration j of the key loop issues, as one scheduling region,
//   * on the matrix cores: S_{j+1} = K_{j+1} . Q^T  and  O^T += V_{j-1}^T . P_{j-1}
//   * on the VALU: the online softmax of S_j (mask, exp against the running
//     max, row sum) -> P_j
// so the softmax of one block runs while the matrix cores work on its
// neighbours.  The block max is taken only when a lane's block sum of p
// exceeds 2^8 (a row's first block, or a max that has moved): that rare path
// recomputes P_j against the new max and rescales O lazily.  K and V tiles go
// from HBM straight into LDS (buffer_load_dwordx4 ... lds), double-buffered:
// iteration j loads K_{j+2} and V_j.
//
// V is kept in LDS in its natural [key][d] layout and read with
// ds_read_b64_tr_b16: in each 16-lane group, result slot j of lane i is
// 16-bit element (i & 3) of the 8 bytes addressed by lane 4 j + (i >> 2).
// Lane i of a group addresses V[k0 + (i >> 2)][d0 + 4 (i & 3) .. + 4], so it
// receives V[k0 .. k0 + 3][d0 + i]: four consecutive keys of one d, i.e. four
// k slots of the V^T A operand.  Two such reads (k0 = 16 cc + 4 g and
// 16 cc + 8 + 4 g for k-group g = lane / 32) give the 8 slots whose keys are
// exactly those P's accumulator rows hold for that k-group.
//
// LDS per stage: K [32][256 B], chunk c of row r at c ^ (r & 15);
//                V [32][256 B], chunk c of row r at c ^ 4 (r & 3).
// ===========================================================================
namespace v2 {

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_ptr;

template <bool kBF16>
SILE_DEV float pair_sum(uint32_t pk, float acc) {
  if constexpr (kBF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(__bf16 __attribute__((ext_vector_type(2))), pk),
                                           __builtin_bit_cast(__bf16 __attribute__((ext_vector_type(2))), 0x3f803f80u),
                                           acc, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk), f16x2{(_Float16)1.0f, (_Float16)1.0f}, acc,
                                  false);
}

// LDS bytes of the two stages (K and V tiles of kNK keys each)
template <int kNK>
constexpr int lds_bytes() { return 2 * 2 * kNK * kRowB; }

// kQT 32-query tiles per wave, kW waves per workgroup: kW * kQT * 32 queries
// per workgroup (256 for every instantiation); kNK keys per block (32 or 64),
// i.e. kST = kNK / 32 S tiles of 32 keys x 32 queries per query tile.
template <bool kBF16, int kQT, int kW, int kNK>
__device__ __forceinline__ void attn_fwd_v2(const uint16_t* __restrict__ Q,
                                            const uint16_t* __restrict__ K,
                                            const uint16_t* __restrict__ V,
                                            uint16_t* __restrict__ O, const AttnArgs& a,
                                            uint8_t* smem) {
  constexpr int kBQ = kW * kQT * 32;
  constexpr int kST = kNK / 32;
  constexpr int kTileB = kNK * kRowB;    // one K or V tile
  constexpr int kStageB = 2 * kTileB;    // K + V
  constexpr int kDmaPerWave = kTileB / 1024 / kW;  // 1 KiB DMA instructions per wave per tile
  static_assert(kNK % 32 == 0 && kDmaPerWave >= 1 && (kTileB / 1024) % kW == 0,
                "tiles in 1 KiB slices, evenly over the waves");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;

  // Work unit u of a head: query block u, or with a.pair (causal) the pair of
  // query blocks (q_blocks - 1 - u, u), whose key ranges add up to the same
  // length for every u, so all workgroups carry equal work.  Causal blocks
  // run largest first.
  const int units = a.pair ? (a.q_blocks + 1) / 2 : a.q_blocks;
  int bh, u;
  const int bid = blockIdx.x;
  if (a.xcd_map) {
    const int xcd = bid & 7, idx = bid >> 3;
    bh = ((idx / units) << 3) + xcd;
    u = idx % units;
  } else {
    bh = bid % a.bh;
    u = bid / a.bh;
  }
  const int qb_first = a.causal ? a.q_blocks - 1 - u : u;
  const int qb_second = a.pair ? u : qb_first;
  const int64_t S = a.seq;
  const int64_t head_off = (int64_t)bh * S * kD;

  for (int pass = 0; pass < (qb_second == qb_first ? 1 : 2); ++pass) {
    const int qb = pass ? qb_second : qb_first;
    // the previous block's last reads of both LDS stages are done before the
    // prologue below refills them
    if (pass) __syncthreads();
    const int q0 = qb * kBQ;
    const int wq0 = q0 + wave * kQT * 32;

    // ---- Q^T fragments (B operand of S^T = K . Q^T) ----
    u32x4 qf[kQT][8];
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      // queries past S (the last block of an S that is not a multiple of
      // 256) read row S - 1 and are not stored
      const int64_t qr = min((int64_t)(wq0 + qt * 32 + l32), S - 1);
      const uint16_t* qrow = Q + head_off + qr * kD + 8 * g;
  #pragma unroll
      for (int kk = 0; kk < 8; ++kk) qf[qt][kk] = *reinterpret_cast<const u32x4*>(qrow + 16 * kk);
    }

    // ---- LDS-DMA addressing: wave w's instruction i fills rows 4 (w + kW i) + (lane >> 4) ----
    // (the swizzles depend on row & 15 and row & 3, the same for every i)
    const int dma_row = 4 * wave + (lane >> 4), dma_pos = lane & 15;
    const int k_voff = dma_row * kRowB + ((dma_pos ^ (dma_row & 15)) << 4);
    const int v_voff = dma_row * kRowB + ((dma_pos ^ (4 * (dma_row & 3))) << 4);
    const int kv_bytes = (int)(S * kRowB);
    const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(K + head_off), (short)0, kv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(V + head_off), (short)0, kv_bytes, 0x00020000);
    auto dma_k = [&](int blk, int stage) {
      uint8_t* base = smem + stage * kStageB + wave * 1024;
  #pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(k_rsrc, (lds_ptr_t)(base + i * kW * 1024), 16,
                                                 k_voff, (blk * kNK + 4 * kW * i) * kRowB, 0, 0);
    };
    auto dma_v = [&](int blk, int stage) {
      uint8_t* base = smem + stage * kStageB + kTileB + wave * 1024;
  #pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(v_rsrc, (lds_ptr_t)(base + i * kW * 1024), 16,
                                                 v_voff, (blk * kNK + 4 * kW * i) * kRowB, 0, 0);
    };

    // ---- fragment reads ----
    // K fragment of S tile st, d-step kk: row 32 st + l32 (row & 15 == l32 & 15)
    const int kf_off = l32 * kRowB;
    const int kf_swz = l32 & 15;
    auto k_frag = [&](const uint8_t* ks, int st, int kk) {
      return *reinterpret_cast<const u32x4*>(ks + 32 * st * kRowB + (((2 * kk + g) ^ kf_swz) << 4));
    };
    auto s_block = [&](int stage, f32x16 (&sacc)[kQT][kST]) {
      const uint8_t* ks = smem + stage * kStageB + kf_off;
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
        for (int st = 0; st < kST; ++st)
  #pragma unroll
          for (int i = 0; i < 16; ++i) sacc[qt][st][i] = 0.0f;
  #pragma unroll
      for (int st = 0; st < kST; ++st)
  #pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const u32x4 kf = k_frag(ks, st, kk);
  #pragma unroll
          for (int qt = 0; qt < kQT; ++qt) sacc[qt][st] = mma32<kBF16>(kf, qf[qt][kk], sacc[qt][st]);
        }
    };
    // V^T fragment for d-tile dt, 16-key chunk cc: two transposing reads
    const int tr_i = lane & 15, tr_s = (lane >> 4) & 1;
    auto v_frag = [&](const uint8_t* vs, int dt, int cc) {
      u32x4 out;
  #pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int key = 16 * cc + 8 * hh + 4 * g + (tr_i >> 2);
        const int d = 32 * dt + 16 * tr_s + 4 * (tr_i & 3);
        const int chunk = d >> 3;
        const int off = key * kRowB + ((chunk ^ (4 * (key & 3))) << 4) + 8 * (tr_i & 1);
        const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(vs + off));
        const u32x2 w = __builtin_bit_cast(u32x2, v);
        out[2 * hh] = w[0];
        out[2 * hh + 1] = w[1];
      }
      return out;
    };
    auto pv_block = [&](int stage, const u32x4 (&pf)[kQT][2 * kST], f32x16 (&oacc)[kQT][4]) {
      const uint8_t* vs = smem + stage * kStageB + kTileB;
  #pragma unroll
      for (int dt = 0; dt < 4; ++dt)
  #pragma unroll
        for (int cc = 0; cc < 2 * kST; ++cc) {
          const u32x4 vf = v_frag(vs, dt, cc);
  #pragma unroll
          for (int qt = 0; qt < kQT; ++qt) oacc[qt][dt] = mma32<kBF16>(vf, pf[qt][cc], oacc[qt][dt]);
        }
    };

    // S_{j+1} over (S tile, d-step) and PV_{j-1} over (d-tile, key chunk), one
    // step of each at a time: S step (st, kk) runs at step 8 st + kk, PV
    // (dt, cc) at step dt + 4 cc
    auto mma_block = [&](int kstage, int vstage, f32x16 (&sacc)[kQT][kST],
                         const u32x4 (&pf)[kQT][2 * kST], f32x16 (&oa)[kQT][4]) {
      const uint8_t* ks = smem + kstage * kStageB + kf_off;
      const uint8_t* vs = smem + vstage * kStageB + kTileB;
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
        for (int st = 0; st < kST; ++st)
  #pragma unroll
          for (int i = 0; i < 16; ++i) sacc[qt][st][i] = 0.0f;
  #pragma unroll
      for (int step = 0; step < 8 * kST; ++step) {
        const int st = step >> 3, kk = step & 7;
        const u32x4 kf = k_frag(ks, st, kk);
        const int dt = step & 3, cc = step >> 2;
        const u32x4 vf = v_frag(vs, dt, cc);
  #pragma unroll
        for (int qt = 0; qt < kQT; ++qt) sacc[qt][st] = mma32<kBF16>(kf, qf[qt][kk], sacc[qt][st]);
  #pragma unroll
        for (int qt = 0; qt < kQT; ++qt) oa[qt][dt] = mma32<kBF16>(vf, pf[qt][cc], oa[qt][dt]);
      }
    };

    f32x16 oacc[kQT][4];
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
      for (int dt = 0; dt < 4; ++dt)
  #pragma unroll
        for (int i = 0; i < 16; ++i) oacc[qt][dt][i] = 0.0f;
    float m_run[kQT], l_run[kQT];
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      m_run[qt] = -__builtin_inff();
      l_run[qt] = 0.0f;
    }
    u32x4 pprev[kQT][2 * kST];
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
      for (int cc = 0; cc < 2 * kST; ++cc) pprev[qt][cc] = u32x4{0u, 0u, 0u, 0u};

    // key blocks: through the block's last query (causal) or S, rounded up
    // to even (the loop runs in pairs); keys past S load as zeros (outside
    // the K / V buffer resources) and are masked
    const int64_t kend = a.causal ? min((int64_t)(q0 + kBQ), S) : S;
    int nb = (int)((kend + kNK - 1) / kNK);
    nb += nb & 1;
    const int last = nb - 1;
    const float c = a.scale_log2;

    // Stages: iteration j reads K_{j+1} and V_{j-1} (stage (j + 1) & 1) and loads
    // K_{j+2} and V_j into stage j & 1, whose previous contents were read in
    // iteration j - 1; the barrier closing iteration j waits for those loads.
    // The key loop is unrolled by two so that stage indices and the roles of
    // the two S and P register sets are compile-time constants (nb is even,
    // rounded up above).
    // Prologue: K_0, K_1 and a finite V tile in stage 1 for the empty PV_{-1}
    // (its P is zero).
    dma_k(0, 0);
    dma_k(min(1, last), 1);
    dma_v(0, 1);
    __syncthreads();
    f32x16 sa[kQT][kST], sb[kQT][kST];
    u32x4 pb[kQT][2 * kST];
    s_block(0, sa);
    __syncthreads();

    // One iteration: everything up to the optional O rescale is one basic block,
    // so the scheduler interleaves the softmax VALU work of block j with the
    // MFMAs of blocks j + 1 (S) and j - 1 (PV).  kMasked selects the causal-mask
    // code, needed only on the workgroup's diagonal.
    auto iteration = [&](int j, auto stage_c, auto masked, f32x16 (&scur)[kQT][kST],
                         f32x16 (&snext)[kQT][kST], const u32x4 (&pprev)[kQT][2 * kST],
                         u32x4 (&pnew)[kQT][2 * kST]) {
      constexpr int kS = decltype(stage_c)::value;
      constexpr bool kMasked = decltype(masked)::value;
      dma_k(min(j + 2, last), kS);
      dma_v(j, kS);
      // matrix cores: S_{j+1} and PV_{j-1}, interleaved step by step so that
      // consecutive MFMAs never accumulate into the same registers
      mma_block(kS ^ 1, kS ^ 1, snext, pprev, oacc);
      // VALU: online softmax of S_j -> P_j
      if constexpr (kMasked) {
        const int kb = j * kNK;
  #pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          // last key this lane's query sees: the query itself (causal) or S - 1
          const int lim = a.causal ? min(wq0 + 32 * qt + l32, (int)S - 1) : (int)S - 1;
          const int q = lim - kb - 4 * g;  // key offset limit for this lane
  #pragma unroll
          for (int st = 0; st < kST; ++st)
  #pragma unroll
            for (int i = 0; i < 16; ++i)
              scur[qt][st][i] =
                  (32 * st + 8 * (i >> 2) + (i & 3) > q) ? -__builtin_inff() : scur[qt][st][i];
        }
      }
      // Fast path: P_j against the running max, with no block max.  Every p
      // of a lane stays <= 2^kRescaleLog2 as long as the lane's block sum of p
      // does.  A lane whose block sum is larger, or NaN (a row's first block,
      // where the running max is -inf), sends the wave to the block-max update
      // below, which recomputes P_j exactly as a max-first softmax would.
      bool slow = false;
      float rs_blk[kQT];
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
        const float mc = m_run[qt] * c;
        float rs = 0.0f;
  #pragma unroll
        for (int st = 0; st < kST; ++st)
  #pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4 w;
  #pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              const float p0 = exp2_fast(__builtin_fmaf(scur[qt][st][8 * h + 2 * jj], c, -mc));
              const float p1 = exp2_fast(__builtin_fmaf(scur[qt][st][8 * h + 2 * jj + 1], c, -mc));
              const uint32_t pk = pack2<kBF16>(p0, p1);
              w[jj] = pk;
              rs = pair_sum<kBF16>(pk, rs);
            }
            pnew[qt][2 * st + h] = w;
          }
        slow |= __builtin_amdgcn_ballot_w64(!(rs <= kBlockSumLimit)) != 0;
        rs_blk[qt] = rs;
      }
      if (slow) {
        // Rare: the running max moves only when a block max exceeds it by more
        // than kRescaleLog2 for some lane of the wave (lazy rescale of O).  The
        // scores pass through an empty asm so that the block max is not
        // computed ahead of the branch.
  #pragma unroll
        for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
          for (int st = 0; st < kST; ++st) asm volatile("" : "+v"(scur[qt][st]));
        bool grow_any = false;
        float mx[kQT];
  #pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          float m = scur[qt][0][0];
  #pragma unroll
          for (int st = 0; st < kST; ++st)
  #pragma unroll
            for (int i = 0; i < 16; ++i) m = __builtin_fmaxf(m, scur[qt][st][i]);
          mx[qt] = pair32_max(m);
          grow_any |= __builtin_amdgcn_ballot_w64((mx[qt] - m_run[qt]) * c > kRescaleLog2) != 0;
        }
  #pragma unroll
        for (int qt = 0; qt < kQT; ++qt) {
          const float m_new = grow_any ? __builtin_fmaxf(m_run[qt], mx[qt]) : m_run[qt];
          const float alpha = exp2_fast((m_run[qt] - m_new) * c);
          m_run[qt] = m_new;
          const float mc = m_new * c;
          float rs = 0.0f;
  #pragma unroll
          for (int st = 0; st < kST; ++st)
  #pragma unroll
            for (int h = 0; h < 2; ++h) {
              u32x4 w;
  #pragma unroll
              for (int jj = 0; jj < 4; ++jj) {
                const float p0 = exp2_fast(__builtin_fmaf(scur[qt][st][8 * h + 2 * jj], c, -mc));
                const float p1 = exp2_fast(__builtin_fmaf(scur[qt][st][8 * h + 2 * jj + 1], c, -mc));
                const uint32_t pk = pack2<kBF16>(p0, p1);
                w[jj] = pk;
                rs = pair_sum<kBF16>(pk, rs);
              }
              pnew[qt][2 * st + h] = w;
            }
          rs_blk[qt] = rs;
          l_run[qt] *= alpha;
          // O rescale after PV_{j-1} (issued above), before PV_j
          if (grow_any) {
  #pragma unroll
            for (int dt = 0; dt < 4; ++dt) oacc[qt][dt] *= alpha;
          }
        }
      }
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt) l_run[qt] += rs_blk[qt];
      // keep P_j and l in this region, beside the MFMAs
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt) {
  #pragma unroll
        for (int cc = 0; cc < 2 * kST; ++cc) asm volatile("" : "+v"(pnew[qt][cc]));
        asm volatile("" : "+v"(l_run[qt]));
      }
      __syncthreads();
    };
    // blocks left of the workgroup's diagonal (causal) or of the block that
    // holds key S (S not a multiple of the block) need no mask
    const int j_diag = a.causal ? q0 / kNK : (int)(S / kNK) & ~1;
    using Z = std::integral_constant<int, 0>;
    using One = std::integral_constant<int, 1>;
    int j = 0;
    for (; j < j_diag; j += 2) {
      iteration(j, Z{}, std::false_type{}, sa, sb, pprev, pb);
      iteration(j + 1, One{}, std::false_type{}, sb, sa, pb, pprev);
    }
    for (; j < nb; j += 2) {
      iteration(j, Z{}, std::true_type{}, sa, sb, pprev, pb);
      iteration(j + 1, One{}, std::true_type{}, sb, sa, pb, pprev);
    }
    // PV of the last block (nb is even: P_{nb-1} is in pprev, V_{nb-1} in stage 1)
    pv_block(1, pprev, oacc);

    // ---- epilogue: O[q][d] = O^T[d][q] / l ----
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const float l = pair32_sum(l_run[qt]);
      const float inv = 1.0f / l;
      const int q = wq0 + 32 * qt + l32;
      if (q >= S) continue;
      uint16_t* orow = O + head_off + (int64_t)q * kD;
  #pragma unroll
      for (int dt = 0; dt < 4; ++dt)
  #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 32 * dt + 8 * r + 4 * g;
          const f32x16& acc = oacc[qt][dt];
          const u32x2 w = {pack2<kBF16>(acc[4 * r] * inv, acc[4 * r + 1] * inv),
                           pack2<kBF16>(acc[4 * r + 2] * inv, acc[4 * r + 3] * inv)};
          *reinterpret_cast<u32x2*>(orow + d) = w;
        }
    }
  }  // pass
}

}  // namespace v2

#define SILE_FA_V2_KERNEL(NAME, BF, QT, W, NK)                                                \
  extern "C" __global__ __launch_bounds__(W * 64, 1) void NAME(                               \
      const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O, AttnArgs a) {     \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[v2::lds_bytes<NK>()];              \
    v2::attn_fwd_v2<BF, QT, W, NK>(Q, K, V, O, a, smem);                                      \
  }
// 8 waves x 32 queries (two waves per SIMD) over 32-key blocks
SILE_FA_V2_KERNEL(sile_flash_attn_fwd_f16_v2w8, false, 1, 8, 32)
SILE_FA_V2_KERNEL(sile_flash_attn_fwd_bf16_v2w8, true, 1, 8, 32)

#define SILE_FA_KERNEL(NAME, BF, QT, NK, DH)                                                  \
  extern "C" __global__ __launch_bounds__(kThreads, 1) void NAME(                             \
      const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O, AttnArgs a) {     \
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * NK * DH * 2];                \
    attn_fwd_body<BF, QT, NK, DH>(Q, K, V, O, a, smem);                                       \
  }

// 128 queries per workgroup, any S, head_dim 64 over 128-key blocks
SILE_FA_KERNEL(sile_flash_attn_fwd_f16_q1_k128_d64, false, 1, 128, 64)
SILE_FA_KERNEL(sile_flash_attn_fwd_bf16_q1_k128_d64, true, 1, 128, 64)
