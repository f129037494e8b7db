// bf16-exact SiLU for gfx950, shared by the packed SiLU * up kernel and the
// SiLU epilogue of the decode gate/up projection.
//
// silu_f32(g) returns g / (1 + exp(-g)) as the f32 formula evaluates it with
// every step correctly rounded, up to a few f32 ulps; it is only ever rounded
// to bf16 afterwards, and it returns the exact f32 formula's value whenever
// that rounding could depend on those ulps.  exp(-g) = 2^t on the hardware
// exp2 (v_exp_f32) with t = fl(-g * log2 e), and g / d as g * (1 / d) on the
// hardware reciprocal (v_rcp_f32).  For |g| < 22 (|t| < 32) t's rounding
// error is below 2^-20, a relative error below ln 2 * 2^-20 (~5.5 f32 ulps)
// in 2^t and so in the quotient; with the two hardware ops and two rounded
// steps that stays under ~9 ulps, inside kBand.  At g >= 22 the denominator
// rounds to exactly 1 and the quotient is g.  An element within kBand f32
// ulps of a bf16 rounding midpoint, below -22 (where t's error grows past the
// band), or NaN is recomputed with expf and an IEEE divide, so
// bf16(silu_f32(g)) == bf16(g / (1 + expf(-g))) for every bf16 g (checked on
// all 65,536 bf16 gate values).
#pragma once

#include "qf_device.h"

namespace qf {
namespace {

constexpr float kLog2e = 0x1.715476p+0f;     // log2(e) rounded to f32
constexpr int kBand = 16;                    // f32 ulps around a bf16 midpoint
constexpr float kFastBelow = -22.0f;         // gates below take the exact path

// g / (1 + exp(-g)) with every step correctly rounded in f32.
__device__ __attribute__((noinline)) float silu_exact(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float silu_f32(float g) {
  const float e = __builtin_amdgcn_exp2f(-g * kLog2e);                // v_exp_f32
  const float a = g * __builtin_amdgcn_rcpf(1.0f + e);                // v_rcp_f32
  const int low = (int)(__float_as_uint(a) & 0xffffu);                // bits below bf16
  if (__builtin_expect(abs(low - 0x8000) < kBand || !(g >= kFastBelow), 0)) return silu_exact(g);
  return a;
}

}  // namespace
}  // namespace qf
