// Merge of split-KV decode attention segments, shared by the attention merge
// kernel and the projection that takes the merged rows as its input, so both
// produce the same bits.
//
// Segment s of virtual head vh left f32 partial numerators
// partials[vh, s, g, 0..128) and statistics stats[vh, s, 0, g] = running
// maximum m_s (log2 domain), stats[vh, s, 1, g] = denominator l_s.  The merged
// row is
//   M = max_s m_s,  w_s = l_s > 0 ? 2^(m_s - M) : 0,
//   out = bf16( (sum_s w_s * partial_s) / (sum_s w_s * l_s) )
// with both sums taken in segment order (a zero denominator gives zeros).
#pragma once

#include "qf_device.h"

namespace qf {

constexpr int kMaxSegments = 32;  // most key segments a virtual head may have
constexpr int kMergeBatch = 16;   // partial rows loaded before any is combined

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// One wave merges query row g of virtual head vh; lane l gets dims 2l and
// 2l + 1 as one dword of two bf16.  Lane s holds segment s's statistics and
// computes its weight (lanes s >= S hold weight 0); the combine loops
// broadcast them with readlane, so the wave spends a few vector registers on
// statistics and 2 * kMergeBatch on partials.  Segments go in batches of
// kMergeBatch whose loads are all in flight before any is combined (one
// memory latency for S <= kMergeBatch); a batch's loads past S re-read
// segment S - 1 and are not combined, so the code has no per-segment
// branch.  Split in two so a caller can issue other loads between the
// first batch's loads (merge_issue) and their use (merge_finish): vector
// loads complete in order, so loads issued after the first batch do not
// delay its combine.  Must be called by all 64 lanes of a wave.
template <int NB = kMergeBatch>
struct SegmentLoads {
  float2 p[NB];
  float m, l;  // lane s: segment s's running maximum and denominator
};

template <int NB>
__device__ __forceinline__ void merge_load_batch(SegmentLoads<NB>& L, const float* partials,
                                                 int64_t vh, int S, int G, int g, int lane, int s0) {
  const float* base = partials + (vh * S * G + g) * 128 + 2 * lane;
  const int seg_stride = G * 128;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int s = s0 + i < S ? s0 + i : S - 1;
    L.p[i] = *reinterpret_cast<const float2*>(base + s * seg_stride);
  }
}

template <int NB>
__device__ __forceinline__ void merge_issue(SegmentLoads<NB>& L, const float* partials,
                                            const float* stats, int64_t vh, int S, int G, int g,
                                            int lane) {
  merge_load_batch(L, partials, vh, S, G, g, lane, 0);
  const float* st = stats + vh * S * 2 * G + g;
  L.m = lane < S ? st[lane * 2 * G] : -__builtin_inff();
  L.l = lane < S ? st[lane * 2 * G + G] : 0.0f;
}

// NB segments per batch (up to kMergeBatch): a caller that knows S <= NB
// issues no loads for slots it does not need; the sums are the same for
// every NB (each term added in segment order).
template <int NB>
__device__ __forceinline__ uint32_t merge_finish(SegmentLoads<NB>& L, const float* partials,
                                                 int64_t vh, int S, int G, int g, int lane) {
  static_assert(NB >= 1 && NB <= kMergeBatch && kMaxSegments == 32, "batch within a wave");
  // M = max over lanes 0..31 (lane s >= S holds -inf): a max within each
  // 16-lane row by DPP, then rows 0 and 1 (a max is exact in any order).
  float rm = L.m;
  rm = fmaxf(rm, __uint_as_float(dpp_u32<kQuadXor1>(__float_as_uint(rm))));
  rm = fmaxf(rm, __uint_as_float(dpp_u32<kQuadXor2>(__float_as_uint(rm))));
  rm = fmaxf(rm, __uint_as_float(dpp_u32<kRowHalfMirror>(__float_as_uint(rm))));
  rm = fmaxf(rm, __uint_as_float(dpp_u32<kRowMirror>(__float_as_uint(rm))));
  float M = fmaxf(lane_value(rm, 0), lane_value(rm, 16));
  if (M == -__builtin_inff()) M = 0.0f;
  const float w_own = L.l > 0.0f ? __builtin_amdgcn_exp2f(L.m - M) : 0.0f;
  const float lw_own = L.l * w_own;
  float total = 0.0f, acc0 = 0.0f, acc1 = 0.0f;
  auto combine = [&](int s0) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const bool on = s0 + i < S;
      const float w = lane_value(w_own, s0 + i);
      const float lw = lane_value(lw_own, s0 + i);
      total = on ? total + lw : total;
      acc0 = on ? acc0 + L.p[i].x * w : acc0;
      acc1 = on ? acc1 + L.p[i].y * w : acc1;
    }
  };
  combine(0);
  for (int s0 = NB; s0 < S; s0 += NB) {
    merge_load_batch(L, partials, vh, S, G, g, lane, s0);
    combine(s0);
  }
  const float den = total > 0.0f ? total : 1.0f;
  return pack2(acc0 / den, acc1 / den);
}

template <int NB = kMergeBatch>
__device__ __forceinline__ uint32_t merge_segments_row(const float* partials, const float* stats,
                                                       int64_t vh, int S, int G, int g, int lane) {
  SegmentLoads<NB> L;
  merge_issue(L, partials, stats, vh, S, G, g, lane);
  return merge_finish(L, partials, vh, S, G, g, lane);
}

}  // namespace qf
