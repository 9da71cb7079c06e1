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
