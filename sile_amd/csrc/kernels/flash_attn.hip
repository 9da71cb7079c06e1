// Flash-attention forward on the gfx950 matrix cores, any sequence length,
// head_dim a multiple of 16 up to 256.
//
//   O = softmax(Q K^T * scale [+ causal mask]) V     Q, K, V, O: [B*H, S, D] 16-bit
//
// sile's DSL has no attention kernel (no mask, iota or transpose); this is
// the composition of its tile ops MmaF, ReduceMax, Exp, ReduceSum and the
// softmax Map (crates/sile-tile-ir/src/ir.rs:128-262) fused into one pass
// with an fp32 online softmax (running max m, running sum l, rescaled
// accumulator), so S and P never leave registers.
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
//
// Launch order: workgroups are dispatched round-robin over the 8 XCDs, so
// workgroup i runs on XCD i % 8.  Head h is pinned to XCD h % 8 and its query
// blocks are issued together (largest causal block first), so the K/V stream
// of a head is shared in one XCD's L2 by all of its query blocks.
#include <type_traits>

#include "common.h"

using namespace sile;

namespace {

constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold: p <= 2^8
// fast-path limit on one lane's block sum of p: below it every p of the
// block is <= 2^kRescaleLog2
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

struct AttnArgs {
  int64_t seq;          // S
  int32_t bh;           // B * H
  int32_t q_blocks;     // S / kBQ
  float scale_log2;     // softmax scale * log2(e)
  int32_t causal;
  int32_t xcd_map;      // 1: head-per-XCD launch order (bh % 8 == 0)
  int32_t pair;         // 1: causal query blocks in balanced pairs
};

}  // namespace

// ===========================================================================
// Pipelined kernel (any S): 8 waves x 32 queries = 256 queries per
// workgroup, two waves per SIMD, for head_dim up to 128 (32-key blocks over
// 256-byte LDS rows, 64-key blocks over 128-byte rows: the same LDS bytes and
// MFMAs per block); 4 waves x 32 queries over 512-byte rows up to 256.
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
// LDS per stage: K and V [kNK][2 kDh B]; with 256-byte rows chunk c of row
// r at c ^ (r & 15) (K) and c ^ 4 (r & 3) (V), with 128-byte rows at
// c ^ ((r >> 1) & 7) and c ^ 2 (r & 3).
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

// LDS bytes of the two stages (K and V tiles of kNK keys, rows of kDp
// 16-bit elements each)
template <int kNK, int kDp>
constexpr int lds_bytes() { return 2 * 2 * kNK * 2 * kDp; }

// kQT 32-query tiles per wave, kW waves per workgroup: kW * kQT * 32 queries
// per workgroup (256 for every instantiation); kNK keys per block (32 or 64),
// i.e. kST = kNK / 32 S tiles of 32 keys x 32 queries per query tile.
// kDh: the head dimension (a multiple of 16); kDp: the LDS row length (64,
// 128 or 256 elements, at least kDh): the chunks of a row past kDh are
// loaded as zeros (outside the buffer resources), so the products over them
// add nothing and the O^T rows past kDh are zero and not stored.
template <bool kBF16, int kQT, int kW, int kNK, int kDh, int kDp>
__device__ __forceinline__ void attn_fwd_v2(const uint16_t* __restrict__ Q,
                                            const uint16_t* __restrict__ K,
                                            const uint16_t* __restrict__ V,
                                            uint16_t* __restrict__ O, const AttnArgs& a,
                                            uint8_t* smem) {
  constexpr int kBQ = kW * kQT * 32;
  constexpr int kST = kNK / 32;
  constexpr int kRow = 2 * kDp;          // bytes of a K or V row in LDS
  constexpr int kRowG = 2 * kDh;         // bytes of a K or V row in HBM
  constexpr int kChunks = kRow / 16;     // 16-byte chunks per LDS row
  constexpr int kChunksG = kRowG / 16;   // of them holding data
  constexpr int kKK = kDh / 16;          // d-steps of S^T = K . Q^T
  constexpr int kDT = (kDh + 31) / 32;   // 32-d tiles of O^T
  constexpr int kDmaRows = 1024 / kRow;  // rows one 1 KiB DMA instruction fills
  static_assert(kDh % 16 == 0 && kDh <= kDp && (kDp == 64 || kDp == 128 || kDp == 256),
                "head_dim a multiple of 16 up to the LDS row");
  constexpr int kTileB = kNK * kRow;     // one K or V tile
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
  const int64_t head_off = (int64_t)bh * S * kDh;
  // K: chunk c of row r at c ^ kswz(r); V: at c ^ vswz(r).  With rows of
  // 256 bytes or more a row spans every bank and r & 15 separates 16 rows;
  // with 128-byte rows two rows share the banks, so (r >> 1) & 7 separates
  // the 8 pairs.  V's swizzle puts the four keys of a transposing read on
  // distinct banks.
  auto kswz = [](int r) { return kChunks == 8 ? ((r >> 1) & 7) : (r & 15); };
  auto vswz = [](int r) { return (kChunks == 8 ? 2 : 4) * (r & 3); };

  for (int pass = 0; pass < (qb_second == qb_first ? 1 : 2); ++pass) {
    const int qb = pass ? qb_second : qb_first;
    // the previous block's last reads of both LDS stages are done before the
    // prologue below refills them
    if (pass) __syncthreads();
    const int q0 = qb * kBQ;
    const int wq0 = q0 + wave * kQT * 32;

    // ---- Q^T fragments (B operand of S^T = K . Q^T) ----
    u32x4 qf[kQT][kKK];
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      // queries past S (the last block of an S that is not a multiple of
      // 256) read row S - 1 and are not stored
      const int64_t qr = min((int64_t)(wq0 + qt * 32 + l32), S - 1);
      const uint16_t* qrow = Q + head_off + qr * kDh + 8 * g;
  #pragma unroll
      for (int kk = 0; kk < kKK; ++kk) qf[qt][kk] = *reinterpret_cast<const u32x4*>(qrow + 16 * kk);
    }

    // ---- LDS-DMA addressing: wave w's instruction i fills LDS rows
    // kDmaRows (w + kW i) + lane / kChunks; lane l writes slot l % kChunks of
    // its row, so it fetches the HBM chunk that belongs there under the
    // swizzle, or, for a chunk past the row's data, an offset past the
    // buffer (zeros) ----
    const int kv_bytes = (int)(S * kRowG);
    int k_voff[kDmaPerWave], v_voff[kDmaPerWave];
  #pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
      const int row = kDmaRows * (wave + kW * i) + lane / kChunks, pos = lane % kChunks;
      const int kc = pos ^ kswz(row), vc = pos ^ vswz(row);
      k_voff[i] = kc < kChunksG ? row * kRowG + kc * 16 : kv_bytes;
      v_voff[i] = vc < kChunksG ? row * kRowG + vc * 16 : kv_bytes;
    }
    const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(K + head_off), (short)0, kv_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(V + head_off), (short)0, kv_bytes, 0x00020000);
    auto dma_k = [&](int blk, int stage) {
      uint8_t* base = smem + stage * kStageB + wave * 1024;
  #pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(k_rsrc, (lds_ptr_t)(base + i * kW * 1024), 16,
                                                 k_voff[i], blk * kNK * kRowG, 0, 0);
    };
    auto dma_v = [&](int blk, int stage) {
      uint8_t* base = smem + stage * kStageB + kTileB + wave * 1024;
  #pragma unroll
      for (int i = 0; i < kDmaPerWave; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(v_rsrc, (lds_ptr_t)(base + i * kW * 1024), 16,
                                                 v_voff[i], blk * kNK * kRowG, 0, 0);
    };

    // ---- fragment reads ----
    // K fragment of S tile st, d-step kk: row 32 st + l32 (kswz(row) == kswz(l32))
    const int kf_off = l32 * kRow;
    const int kf_swz = kswz(l32);
    auto k_frag = [&](const uint8_t* ks, int st, int kk) {
      return *reinterpret_cast<const u32x4*>(ks + 32 * st * kRow + (((2 * kk + g) ^ kf_swz) << 4));
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
        for (int kk = 0; kk < kKK; ++kk) {
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
        const int off = key * kRow + ((chunk ^ vswz(key)) << 4) + 8 * (tr_i & 1);
        const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(vs + off));
        const u32x2 w = __builtin_bit_cast(u32x2, v);
        out[2 * hh] = w[0];
        out[2 * hh + 1] = w[1];
      }
      return out;
    };
    auto pv_block = [&](int stage, const u32x4 (&pf)[kQT][2 * kST], f32x16 (&oacc)[kQT][kDT]) {
      const uint8_t* vs = smem + stage * kStageB + kTileB;
  #pragma unroll
      for (int dt = 0; dt < kDT; ++dt)
  #pragma unroll
        for (int cc = 0; cc < 2 * kST; ++cc) {
          const u32x4 vf = v_frag(vs, dt, cc);
  #pragma unroll
          for (int qt = 0; qt < kQT; ++qt) oacc[qt][dt] = mma32<kBF16>(vf, pf[qt][cc], oacc[qt][dt]);
        }
    };

    // S_{j+1} over (S tile, d-step) and PV_{j-1} over (d-tile, key chunk), one
    // step of each at a time: S step (st, kk) runs at step kKK st + kk, PV
    // (dt, cc) at step dt + kDT cc (kST kKK and 2 kST kDT steps: equal
    // unless kDh % 32 == 16)
    auto mma_block = [&](int kstage, int vstage, f32x16 (&sacc)[kQT][kST],
                         const u32x4 (&pf)[kQT][2 * kST], f32x16 (&oa)[kQT][kDT]) {
      const uint8_t* ks = smem + kstage * kStageB + kf_off;
      const uint8_t* vs = smem + vstage * kStageB + kTileB;
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
        for (int st = 0; st < kST; ++st)
  #pragma unroll
          for (int i = 0; i < 16; ++i) sacc[qt][st][i] = 0.0f;
      constexpr int kSSteps = kKK * kST, kPSteps = 2 * kDT * kST;
  #pragma unroll
      for (int step = 0; step < (kSSteps > kPSteps ? kSSteps : kPSteps); ++step) {
        if (step < kSSteps) {
          const int st = step / kKK, kk = step % kKK;
          const u32x4 kf = k_frag(ks, st, kk);
  #pragma unroll
          for (int qt = 0; qt < kQT; ++qt) sacc[qt][st] = mma32<kBF16>(kf, qf[qt][kk], sacc[qt][st]);
        }
        if (step < kPSteps) {
          const int dt = step % kDT, cc = step / kDT;
          const u32x4 vf = v_frag(vs, dt, cc);
  #pragma unroll
          for (int qt = 0; qt < kQT; ++qt) oa[qt][dt] = mma32<kBF16>(vf, pf[qt][cc], oa[qt][dt]);
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

    // The online softmax of S_j -> P_j on the VALU (causal / past-S mask
    // first when kMasked).
    auto softmax_block = [&](int j, auto masked, f32x16 (&scur)[kQT][kST],
                             u32x4 (&pnew)[kQT][2 * kST]) {
      constexpr bool kMasked = decltype(masked)::value;
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
            for (int dt = 0; dt < kDT; ++dt) oacc[qt][dt] *= alpha;
          }
        }
      }
  #pragma unroll
      for (int qt = 0; qt < kQT; ++qt) l_run[qt] += rs_blk[qt];
    };
    // Last key block this wave needs: the one holding its last query (causal)
    // or key S - 1.  On the diagonal the wave skips iteration j once block
    // j - 1 is past it: S_{j+1}, P_j and PV_{j-1} are then all of masked keys
    // (their P is zero), and the block's DMA and barrier stay.  (Skipping the
    // unneeded half of iterations jw and jw + 1 as well keeps registers of the
    // skipped branches live and spills.)
    const int jw = __builtin_amdgcn_readfirstlane(
        (int)((a.causal ? min((int64_t)(wq0 + 32 * kQT - 1), S - 1) : S - 1) / kNK));

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
      if constexpr (kMasked) {
        // From S_{jw+1} on this wave's scores are all masked: its Q^T
        // operand is zeroed, so the S products it still issues run on zeros
        // (the matrix cores draw far less power on zero data).
        if (j == jw) {
  #pragma unroll
          for (int qt = 0; qt < kQT; ++qt)
  #pragma unroll
            for (int kk = 0; kk < kKK; ++kk) qf[qt][kk] = u32x4{0u, 0u, 0u, 0u};
        }
      }
      if (!kMasked || j - 1 <= jw) {
        // matrix cores: S_{j+1} and PV_{j-1}, interleaved step by step so that
        // consecutive MFMAs never accumulate into the same registers
        mma_block(kS ^ 1, kS ^ 1, snext, pprev, oacc);
        softmax_block(j, masked, scur, pnew);
      }
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
    if (last <= jw) pv_block(1, pprev, oacc);

    // ---- epilogue: O[q][d] = O^T[d][q] / l ----
  #pragma unroll
    for (int qt = 0; qt < kQT; ++qt) {
      const float l = pair32_sum(l_run[qt]);
      const float inv = 1.0f / l;
      const int q = wq0 + 32 * qt + l32;
      if (q >= S) continue;
      uint16_t* orow = O + head_off + (int64_t)q * kDh;
  #pragma unroll
      for (int dt = 0; dt < kDT; ++dt)
  #pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 32 * dt + 8 * r + 4 * g;
          if (d >= kDh) continue;   // O^T rows past the head dimension (zero)
          const f32x16& acc = oacc[qt][dt];
          const u32x2 w = {pack2<kBF16>(acc[4 * r] * inv, acc[4 * r + 1] * inv),
                           pack2<kBF16>(acc[4 * r + 2] * inv, acc[4 * r + 3] * inv)};
          *reinterpret_cast<u32x2*>(orow + d) = w;
        }
    }
  }  // pass
}

}  // namespace v2

#define SILE_FA_V2_KERNEL(NAME, BF, QT, W, NK, DH, DP)                                        \
  extern "C" __global__ __launch_bounds__(W * 64, 1) void NAME(                               \
      const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O, AttnArgs a) {     \
    __shared__ __attribute__((aligned(1024))) uint8_t smem[v2::lds_bytes<NK, DP>()];          \
    v2::attn_fwd_v2<BF, QT, W, NK, DH, DP>(Q, K, V, O, a, smem);                              \
  }
// 8 waves x 32 queries (two waves per SIMD) for head_dim up to 128: 32-key
// blocks over 256-byte LDS rows, 64-key blocks over 128-byte rows (the same
// LDS bytes and MFMAs per block); 4 waves (one per SIMD, room for the O
// accumulators) over 512-byte rows for head_dim up to 256.
#define SILE_FA_V2_DTYPES(SUFFIX, W, NK, DH, DP)                                              \
  SILE_FA_V2_KERNEL(sile_flash_attn_fwd_f16_##SUFFIX, false, 1, W, NK, DH, DP)                  \
  SILE_FA_V2_KERNEL(sile_flash_attn_fwd_bf16_##SUFFIX, true, 1, W, NK, DH, DP)
// every head dimension that is a multiple of 16 from 16 to 256
SILE_FA_V2_DTYPES(v2w8_d16, 8, 64, 16, 64)
SILE_FA_V2_DTYPES(v2w8_d32, 8, 64, 32, 64)
SILE_FA_V2_DTYPES(v2w8_d48, 8, 64, 48, 64)
SILE_FA_V2_DTYPES(v2w8_d64, 8, 64, 64, 64)
SILE_FA_V2_DTYPES(v2w8_d80, 8, 32, 80, 128)
SILE_FA_V2_DTYPES(v2w8_d96, 8, 32, 96, 128)
SILE_FA_V2_DTYPES(v2w8_d112, 8, 32, 112, 128)
SILE_FA_V2_DTYPES(v2w8, 8, 32, 128, 128)
SILE_FA_V2_DTYPES(v2w4_d144, 4, 32, 144, 256)
SILE_FA_V2_DTYPES(v2w4_d160, 4, 32, 160, 256)
SILE_FA_V2_DTYPES(v2w4_d176, 4, 32, 176, 256)
SILE_FA_V2_DTYPES(v2w4_d192, 4, 32, 192, 256)
SILE_FA_V2_DTYPES(v2w4_d208, 4, 32, 208, 256)
SILE_FA_V2_DTYPES(v2w4_d224, 4, 32, 224, 256)
SILE_FA_V2_DTYPES(v2w4_d240, 4, 32, 240, 256)
SILE_FA_V2_DTYPES(v2w4_d256, 4, 32, 256, 256)
