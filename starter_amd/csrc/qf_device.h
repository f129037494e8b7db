// Device helpers shared by the gfx950 kernels: bf16 <-> f32 conversion on
// packed dwords, wavefront-64 DPP reductions, and the host-side launch
// plumbing (status codes, stream casts).
//
// Numerics: every kernel is compiled with -ffp-contract=off so that no
// multiply/add pair is fused into an FMA behind the source's back, and with
// HIP's default correctly rounded f32 divide and sqrt.  f32 -> bf16 uses the
// gfx950 v_cvt_pk_bf16_f32 instruction (round to nearest even).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qwen_fused.h"

namespace qf {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kBlock = 256;  // 4 waves per workgroup everywhere
constexpr int kCUs = 256;    // MI355X compute units (sizes launch plans)
constexpr int kXCDs = 8;     // MI355X dies; workgroup i of a grid runs on XCD i % 8

// ---- bf16 <-> f32 -----------------------------------------------------------

// Low / high bf16 of a packed dword, widened exactly to f32.
__device__ __forceinline__ float lo_f32(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float hi_f32(uint32_t d) { return __uint_as_float(d & 0xffff0000u); }

// Two f32 -> one dword of two bf16 (lo first), round to nearest even.
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint16_t to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ float from_bf16(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}

// 8 bf16 (one 16-byte vector) <-> 8 f32.
__device__ __forceinline__ void unpack8(const uint4& u, float* f) {
  f[0] = lo_f32(u.x); f[1] = hi_f32(u.x);
  f[2] = lo_f32(u.y); f[3] = hi_f32(u.y);
  f[4] = lo_f32(u.z); f[5] = hi_f32(u.z);
  f[6] = lo_f32(u.w); f[7] = hi_f32(u.w);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 u;
  u.x = pack2(f[0], f[1]);
  u.y = pack2(f[2], f[3]);
  u.z = pack2(f[4], f[5]);
  u.w = pack2(f[6], f[7]);
  return u;
}
// Round 8 f32 to bf16 and widen back: the value a bf16 tensor would hold.
__device__ __forceinline__ void round8(float* f) {
  uint4 u = pack8(f);
  unpack8(u, f);
}

// 2^x on the transcendental unit (v_exp_f32); the softmax kernels feed it
// arguments <= 0.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Orders one wave's LDS writes before its reads of other lanes' data (and the
// reads before the next writes); LDS executes a wave's operations in order,
// so this costs no instruction.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- 16-byte global loads / stores ------------------------------------------

// NT = true marks the access nontemporal (streamed once: the "nt" bit of
// global_load/store_dwordx4), which measurably raises streaming bandwidth on
// gfx950; NT = false is an ordinary cached access (for data re-read soon,
// such as gains and rotary rows).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 load16(const void* p) {
  if constexpr (NT) {
    const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *static_cast<const uint4*>(p);
  }
}
template <bool NT>
__device__ __forceinline__ void store16(void* p, const uint4& v) {
  if constexpr (NT) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, static_cast<u32x4*>(p));
  } else {
    *static_cast<uint4*>(p) = v;
  }
}

// Calls that touch at least this many bytes stream their row data with
// nontemporal accesses; smaller (decode-size) calls keep ordinary cached
// accesses so the next kernel finds their outputs in L2 / Infinity Cache.
constexpr int64_t kStreamBytes = 32ll << 20;

// ---- DPP / cross-lane -------------------------------------------------------

// DPP control words (GFX9 encoding).
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowRor8 = 0x128;     // row_ror:8, lane i <- lane (i+8) mod 16

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __double_as_longlong(v);
  const uint32_t lo = dpp_u32<CTRL>((uint32_t)u);
  const uint32_t hi = dpp_u32<CTRL>((uint32_t)(u >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// All-reduce sum over aligned lane groups of 8/16/32/64 lanes, in f64.  Every
// lane of a group ends with the same bits (each step adds a commutative pair);
// all lanes of the wave must be active.  The RMSNorm kernels feed it exact f32 squares of
// bf16 values (at most 16 significant bits each), so for any realistic row the
// f64 partial sums are exact and the result does not depend on the reduction
// order: rounding it once to f32 gives the correctly rounded f32 sum of
// squares, bit-identical to any other exact evaluation.
template <int LANES>
__device__ __forceinline__ double group_sum_f64(double v) {
  static_assert(LANES == 8 || LANES == 16 || LANES == 32 || LANES == 64, "group");
  v += dpp_f64<kQuadXor1>(v);
  v += dpp_f64<kQuadXor2>(v);
  v += dpp_f64<kRowHalfMirror>(v);
  if constexpr (LANES >= 16) v += dpp_f64<kRowMirror>(v);
  if constexpr (LANES >= 32) v += __shfl_xor(v, 16);
  if constexpr (LANES >= 64) v += __shfl_xor(v, 32);
  return v;
}

// 1 / sqrt(mean + eps) from an exact f64 sum of squares over n elements, with
// every f32 step correctly rounded (IEEE divide and sqrt):
//   var = f32(sum) / n;  inv = 1 / sqrt(var + eps).
__device__ __forceinline__ float inv_rms(double sum_sq, float n, float eps) {
  const float var = (float)sum_sq / n;
  return 1.0f / sqrtf(var + eps);
}

// ---- f32 split-K partials ---------------------------------------------------

// y[0..8) = f32 sum of `splits` partials of 8 consecutive columns, in split
// order starting from 0: (((0 + p[0]) + p[1]) + ...), partial s at
// p + s * stride.  Up to P partials are loaded before any of them is added,
// so a call waits ceil(splits / P) memory latencies rather than `splits`.
// Lanes with live == false load nothing and return zeros.
template <int P>
__device__ __forceinline__ void sum_partials8(const float* p, int64_t stride, int splits, bool live,
                                              float* y) {
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = 0.0f;
  for (int s0 = 0; s0 < splits; s0 += P) {
    float4 lo[P], hi[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      lo[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      hi[i] = lo[i];
      if (live && s0 + i < splits) {
        const float4* q = reinterpret_cast<const float4*>(p + (int64_t)(s0 + i) * stride);
        lo[i] = q[0];
        hi[i] = q[1];
      }
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if (s0 + i < splits) {
        y[0] += lo[i].x; y[1] += lo[i].y; y[2] += lo[i].z; y[3] += lo[i].w;
        y[4] += hi[i].x; y[5] += hi[i].y; y[6] += hi[i].z; y[7] += hi[i].w;
      }
    }
  }
}

// ---- integer helpers --------------------------------------------------------

// Unsigned 32-bit division by a run-time constant d >= 1 via a multiply-high
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994): q = (umulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)((((1ull << s) - d) << 32) / d + 1);
  return f;
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  uint64_t t = (uint64_t)__umulhi(n, f.m) + n;
  return (uint32_t)(t >> f.s);
}

// ---- host-side plumbing -----------------------------------------------------

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Status of the launch just enqueued on this thread.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? QF_OK : (int)e;
}

}  // namespace qf
