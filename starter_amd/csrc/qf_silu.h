// bf16-exact SiLU for gfx950, shared by the packed SiLU * up kernel and the
// SiLU epilogue of the decode gate/up projection.
//
// silu_f32(g) returns g / (1 + exp(-g)) as the f32 formula evaluates it with
// every step correctly rounded, up to a few f32 ulps; it is only ever rounded
// to bf16 afterwards, and it returns the exact f32 formula's value whenever
// that rounding could depend on those ulps.  exp(-g) = 2^t on the hardware
// exp2 (v_exp_f32) with t = -g * log2 e, the rounding error of t restored by
// one FMA (2^(t + dt) ~= 2^t * (1 + dt ln 2)), and g / d as g * (1 / d) on the
// hardware reciprocal (v_rcp_f32).  An element within kBand f32 ulps of a bf16
// rounding midpoint - or whose reciprocal would be denormal (g < -86.6) - is
// recomputed with expf and an IEEE divide (~0.05% of elements), so
// bf16(silu_f32(g)) == bf16(g / (1 + expf(-g))) for every bf16 g.
#pragma once

#include "qf_device.h"

namespace qf {
namespace {

constexpr float kLog2e = 0x1.715476p+0f;     // log2(e) rounded to f32
constexpr float kLog2eLo = 0x1.4ae0c0p-26f;  // log2(e) - kLog2e
constexpr float kLn2 = 0x1.62e430p-1f;
constexpr int kBand = 16;                    // f32 ulps around a bf16 midpoint

// g / (1 + exp(-g)) with every step correctly rounded in f32.
__device__ __attribute__((noinline)) float silu_exact(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ float silu_f32(float g) {
  const float t = -g * kLog2e;
  const float dt = __builtin_fmaf(-g, kLog2e, -t) + (-g) * kLog2eLo;  // t's rounding error
  const float e0 = __builtin_amdgcn_exp2f(t);                         // v_exp_f32
  const float e = __builtin_fmaf(e0, dt * kLn2, e0);
  const float d = 1.0f + e;
  const float a = g * __builtin_amdgcn_rcpf(d);                       // v_rcp_f32
  const int low = (int)(__float_as_uint(a) & 0xffffu);                // bits below bf16
  if (__builtin_expect(abs(low - 0x8000) < kBand || !(d < 0x1p125f), 0)) return silu_exact(g);
  return a;
}

}  // namespace
}  // namespace qf
