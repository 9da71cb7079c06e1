// Attention forward for gfx950.
//
// sile_attn_fwd_rowwise_*: one wave per query row with an fp32 online softmax
// (running max m, running sum l, rescaled accumulator), any head_dim <= 256.
// Used for shapes the MFMA flash kernel does not take.
#include "common.h"

using namespace sile;

template <bool kBF16>
SILE_DEV float ld16(const uint16_t* p) {
  return kBF16 ? bf16_to_f32(*p) : f16_to_f32(*p);
}
template <bool kBF16>
SILE_DEV uint16_t st16(float v) {
  return kBF16 ? bf16_rne(v) : f16_rne(v);
}

template <bool kBF16>
__device__ __forceinline__ void attn_rowwise(const uint16_t* __restrict__ q,
                                             const uint16_t* __restrict__ k,
                                             const uint16_t* __restrict__ v,
                                             uint16_t* __restrict__ o, int64_t bh_count,
                                             int64_t seq, int64_t d, float scale, int causal) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= bh_count * seq) return;
  const int64_t bh = row / seq, i = row % seq;
  const uint16_t* qi = q + (bh * seq + i) * d;
  const uint16_t* kb = k + bh * seq * d;
  const uint16_t* vb = v + bh * seq * d;
  float qv[4], acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t dd = lane + 64 * t;
    qv[t] = dd < d ? ld16<kBF16>(qi + dd) * (scale * kLog2e) : 0.0f;
    acc[t] = 0.0f;
  }
  float m = -__builtin_inff(), l = 0.0f;
  const int64_t nkeys = causal ? i + 1 : seq;
  for (int64_t j = 0; j < nkeys; ++j) {
    const uint16_t* kj = kb + j * d;
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t dd = lane + 64 * t;
      if (dd < d) s += qv[t] * ld16<kBF16>(kj + dd);
    }
    s = wave_sum(s);  // score in log2 units
    const float m_new = fmax_ordered(m, s);
    const float alpha = exp2_fast(m - m_new);
    const float p = exp2_fast(s - m_new);
    l = l * alpha + p;
    const uint16_t* vj = vb + j * d;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t dd = lane + 64 * t;
      if (dd < d) acc[t] = acc[t] * alpha + p * ld16<kBF16>(vj + dd);
    }
    m = m_new;
  }
  uint16_t* oi = o + (bh * seq + i) * d;
  const float inv = 1.0f / l;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int64_t dd = lane + 64 * t;
    if (dd < d) oi[dd] = st16<kBF16>(acc[t] * inv);
  }
}

extern "C" __global__ __launch_bounds__(256) void sile_attn_fwd_rowwise_f16(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int64_t bh_count,
    int64_t seq, int64_t d, float scale, int causal) {
  attn_rowwise<false>(q, k, v, o, bh_count, seq, d, scale, causal);
}
extern "C" __global__ __launch_bounds__(256) void sile_attn_fwd_rowwise_bf16(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o, int64_t bh_count,
    int64_t seq, int64_t d, float scale, int causal) {
  attn_rowwise<true>(q, k, v, o, bh_count, seq, d, scale, causal);
}

// ---- fp32 attention with K given transposed: the DSL attention program ----
// O = softmax(Q Kt * scale) V over keys [0, n_k), online, with the running
// max starting at m0 (the program's initial max tile) and updated as
// m_new = m >= rowmax ? m : rowmax (max_tile, crates/sile-tile-ir/src/lower.rs:619-641);
// q [n_q, ldq], kt [d, ldkt] (key j of dim t at kt[t * ldkt + j]), v [n_k, ldv],
// o [n_q, ldo], fp32 throughout.  A workgroup of 256 threads owns 64 queries
// and walks the keys in blocks of 64: Q^T, the block's K^T and V, and P^T sit
// in LDS; thread t computes the 4 x 4 scores of queries 4 (t / 16) .. + 3 and
// keys 4 (t % 16) .. + 3, the row max and sum over the 16 lanes that share its
// queries (DPP), and then O for its 4 queries and dims (t % 16) * kDp / 16 ..
// + kDp / 16.  kDp is the head dim padded to a multiple of 16 (dims past d
// load as 0 and are not stored); keys past n_k in the last block have p = 0.
template <int kDp>
__device__ __forceinline__ void attn_f32_kt(const float* __restrict__ q, int64_t ldq,
                                            const float* __restrict__ kt, int64_t ldkt,
                                            const float* __restrict__ v, int64_t ldv,
                                            float* __restrict__ o, int64_t ldo, int64_t n_q,
                                            int64_t n_k, int d, float scale, float m0) {
  constexpr int kQ = 64, kK = 64, kDg = kDp / 16, kPp = kQ + 4;
  __shared__ __attribute__((aligned(16))) float qT[kDp][kQ];
  __shared__ __attribute__((aligned(16))) float kT[kDp][kK];
  __shared__ __attribute__((aligned(16))) float vS[kK][kDp];
  __shared__ __attribute__((aligned(16))) float pT[kK][kPp];
  const int t = threadIdx.x, qg = t >> 4, kg = t & 15;
  const int64_t q0 = (int64_t)blockIdx.x * kQ;
  for (int e = t; e < kQ * kDp; e += 256) {
    const int qi = e / kDp, dd = e % kDp;
    qT[dd][qi] = q0 + qi < n_q && dd < d ? q[(q0 + qi) * ldq + dd] : 0.0f;
  }
  float m[4], l[4], acc[4][kDg];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = m0;
    l[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < kDg; ++c) acc[i][c] = 0.0f;
  }
  for (int64_t kb = 0; kb < n_k; kb += kK) {
    __syncthreads();  // the previous block's LDS reads are done
    for (int e = t; e < kDp * kK; e += 256) {
      const int dd = e / kK, kk = e % kK;
      kT[dd][kk] = dd < d && kb + kk < n_k ? kt[dd * ldkt + kb + kk] : 0.0f;
    }
    for (int e = t; e < kK * kDp; e += 256) {
      const int kk = e / kDp, dd = e % kDp;
      vS[kk][dd] = dd < d && kb + kk < n_k ? v[(kb + kk) * ldv + dd] : 0.0f;
    }
    __syncthreads();
    float s[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) s[i][j] = 0.0f;
#pragma unroll 8
    for (int dd = 0; dd < kDp; ++dd) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(&qT[dd][4 * qg]);
      const f32x4 b = *reinterpret_cast<const f32x4*>(&kT[dd][4 * kg]);
      const float av[4] = {a[0], a[1], a[2], a[3]}, bv[4] = {b[0], b[1], b[2], b[3]};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) s[i][j] += av[i] * bv[j];
    }
    bool live[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) live[j] = kb + 4 * kg + j < n_k;
    float p[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float rmax = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[i][j] *= scale;
        if (live[j]) rmax = fmax_ordered(rmax, s[i][j]);
      }
      rmax = group_max16(rmax);
      const float m_new = m[i] >= rmax ? m[i] : rmax;
      float rsum = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        p[i][j] = live[j] ? exp2_fast((s[i][j] - m_new) * kLog2e) : 0.0f;
        rsum += p[i][j];
      }
      rsum = group_sum16(rsum);
      const float alpha = exp2_fast((m[i] - m_new) * kLog2e);
      l[i] = l[i] * alpha + rsum;
#pragma unroll
      for (int c = 0; c < kDg; ++c) acc[i][c] *= alpha;
      m[i] = m_new;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 col = {p[0][j], p[1][j], p[2][j], p[3][j]};
      *reinterpret_cast<f32x4*>(&pT[4 * kg + j][4 * qg]) = col;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < kK; ++kk) {
      const f32x4 pv = *reinterpret_cast<const f32x4*>(&pT[kk][4 * qg]);
      const float pw[4] = {pv[0], pv[1], pv[2], pv[3]};
      float vv[kDg];
#pragma unroll
      for (int c = 0; c < kDg; ++c) vv[c] = vS[kk][kg * kDg + c];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < kDg; ++c) acc[i][c] += pw[i] * vv[c];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t qi = q0 + 4 * qg + i;
    if (qi >= n_q) continue;
#pragma unroll
    for (int c = 0; c < kDg; ++c) {
      const int dd = kg * kDg + c;
      if (dd < d) o[qi * ldo + dd] = acc[i][c] / l[i];
    }
  }
}

#define SILE_ATTN_F32_KT(DP)                                                                   \
  extern "C" __global__ __launch_bounds__(256) void sile_attn_f32_kt_d##DP(                    \
      const float* q, int64_t ldq, const float* kt, int64_t ldkt, const float* v, int64_t ldv, \
      float* o, int64_t ldo, int64_t n_q, int64_t n_k, int d, float scale, float m0) {         \
    attn_f32_kt<DP>(q, ldq, kt, ldkt, v, ldv, o, ldo, n_q, n_k, d, scale, m0);                 \
  }
SILE_ATTN_F32_KT(16)
SILE_ATTN_F32_KT(32)
SILE_ATTN_F32_KT(48)
SILE_ATTN_F32_KT(64)
SILE_ATTN_F32_KT(80)
SILE_ATTN_F32_KT(96)
SILE_ATTN_F32_KT(112)
SILE_ATTN_F32_KT(128)
