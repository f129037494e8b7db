// Per-head RMSNorm + NeoX rotate-half RoPE on one 128-wide head row held by
// a 16-lane DPP row (lane l holds elements 8l..8l+7), shared by the Q/K
// kernels and the decode attention prologue so both produce the same bits.
//
//   inv = 1 / sqrt(f32(sum(x^2)) / 128 + eps)   (sum exact in f64, rounded once)
//   n   = bf16(bf16(x * inv) * w)
//   rot = [-n[64:], n[:64]]
//   out = bf16(bf16(n * cos) + bf16(rot * sin))
#pragma once

#include "qf_device.h"

namespace qf {

__device__ __forceinline__ uint4 zero4() { return make_uint4(0, 0, 0, 0); }

// Component-wise select (a whole-struct ?: is lowered through a stack slot).
__device__ __forceinline__ uint4 select4(bool c, const uint4& a, const uint4& b) {
  return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

// Norm + gain + RoPE of one head row held as 8 f32 per lane (values already
// representable in bf16).  w, c are this lane's gains and cos values; sr is
// its sin values with the rotate-half sign folded in (-sin on lanes 0..7 of
// the DPP row, whose partner values come from the second half):
// (-p) * s == p * (-s) exactly, so bf16(rot * sin) is unchanged.
// Returns the 8 bf16 outputs of this lane.
__device__ __forceinline__ uint4 norm_rope_f(const float* x, const float* w, const float* c,
                                             const float* sr, float eps) {
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += (double)(x[j] * x[j]);  // exact squares, exact sum
  const float inv = inv_rms(group_sum_f64<16>(ss), 128.0f, eps);

  float n[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] = x[j] * inv;
  round8(n);
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] *= w[j];
  const uint4 nb = pack8(n);
  unpack8(nb, n);

  // Partner half: lane l <-> lane l^8 inside the 16-lane DPP row.
  uint4 pb;
  pb.x = dpp_u32<kRowRor8>(nb.x);
  pb.y = dpp_u32<kRowRor8>(nb.y);
  pb.z = dpp_u32<kRowRor8>(nb.z);
  pb.w = dpp_u32<kRowRor8>(nb.w);
  float p[8], left[8];
  unpack8(pb, p);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    left[j] = n[j] * c[j];
    p[j] *= sr[j];
  }
  round8(left);
  round8(p);
#pragma unroll
  for (int j = 0; j < 8; ++j) left[j] += p[j];
  return pack8(left);
}

// Negate both bf16 of every dword (sign bit flip) when `neg`.
__device__ __forceinline__ uint4 negate_if(uint4 v, bool neg) {
  const uint32_t m = neg ? 0x80008000u : 0u;
  return make_uint4(v.x ^ m, v.y ^ m, v.z ^ m, v.w ^ m);
}

// Same with gains / cos / sin still packed.
__device__ __forceinline__ uint4 norm_rope(const float* x, uint4 wv, uint4 cv, uint4 sv,
                                           float eps, int l16) {
  float w[8], c[8], sr[8];
  unpack8(wv, w);
  unpack8(cv, c);
  unpack8(negate_if(sv, l16 < 8), sr);
  return norm_rope_f(x, w, c, sr, eps);
}

}  // namespace qf
