// Per-head Q/K RMSNorm fused with NeoX rotate-half RoPE for gfx950, in the
// three layouts the engine calls it with:
//   qf_qk_norm_rope         module path, separate (possibly strided) q and k
//                           and per-sequence cos/sin rows
//                           (engine/kernels/qk_norm_rope.py:8-73)
//   qf_qkv_norm_rope_cache  packed [q|k|v] decode row, device position, K/V
//                           written to cache slot `position`, optional f32
//                           split-K partials (engine/kernels/decode_fused.py:59-118)
//   qf_prefill_qkv          packed prefill rows, slot = token index, K/V
//                           written to cache slots [0, T) (engine/kernels/prefill.py:19-63)
//
// Arithmetic per head row x[0..127] (same cast chain in every layout):
//   inv = 1 / sqrt(f32(sum(x^2)) / 128 + eps)   (sum exact in f64, rounded once)
//   n   = bf16(bf16(x * inv) * w)
//   rot = [-n[64:], n[:64]]
//   out = bf16(bf16(n * cos) + bf16(rot * sin))
// which is Qwen3RMSNorm followed by apply_rotary_pos_emb (transformers
// models/qwen3/modeling_qwen3.py) on bf16 tensors.
//
// Layout: a head row is 256 bytes = 16 lanes x 16 bytes, i.e. one DPP row.
// Lane l holds elements 8l..8l+7; its rotate-half partner (element +-64) sits
// in lane l^8 of the same DPP row, so one row_ror:8 per dword exchanges the
// already-rounded n values; nothing is loaded twice.  A wave covers 4 head
// rows, a 256-thread workgroup 16.  All 64 lanes always run the arithmetic
// (DPP needs every lane of a row active); only loads and stores of rows past
// the end are predicated off.
#include "qf_device.h"
#include "qf_rope.h"

namespace qf {
namespace {

constexpr int kD = 128;
constexpr int kLanes = 16;                      // lanes per head row
constexpr int kRowsPerBlock = kBlock / kLanes;  // 16 head rows
// The decode-size kernels (qk_norm_rope, qkv_norm_rope_cache) run one-wave
// workgroups of 4 head rows, spreading a call over 4x as many CUs (config 3,
// B = 32: 2.28 -> 2.21 us; the batch-64 packed call 2.39 -> 2.33).
constexpr int kDecodeThreads = kWave;
constexpr int kDecodeRows = kDecodeThreads / kLanes;

// ---------------------------------------------------------------- module path
struct QkArgs {
  const uint16_t* q;
  const uint16_t* k;
  int64_t q_bs, q_hs, k_bs, k_hs;
  const uint16_t* qw;
  const uint16_t* kw;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t cs_bs;
  float q_eps, k_eps;
  uint16_t* oq;
  uint16_t* ok;
  uint32_t rows;   // batch * (nq + nk)
  uint32_t nq, nk;
  FastDiv heads;   // nq + nk
};

__global__ __launch_bounds__(kDecodeThreads) void qk_norm_rope_kernel(QkArgs a) {
  const uint32_t g = blockIdx.x * kDecodeRows + threadIdx.x / kLanes;
  const int l = threadIdx.x % kLanes;
  const bool live = g < a.rows;
  const uint32_t gg = live ? g : 0;
  const uint32_t b = fdiv(gg, a.heads);
  const uint32_t h = gg - b * a.heads.d;
  const bool is_q = h < a.nq;
  const uint16_t* src = is_q ? a.q + b * a.q_bs + (int64_t)h * a.q_hs
                             : a.k + b * a.k_bs + (int64_t)(h - a.nq) * a.k_hs;
  uint16_t* dst = is_q ? a.oq + ((uint64_t)b * a.nq + h) * kD
                       : a.ok + ((uint64_t)b * a.nk + (h - a.nq)) * kD;
  const uint4 xv = live ? reinterpret_cast<const uint4*>(src)[l] : zero4();
  const uint4 wv = reinterpret_cast<const uint4*>(is_q ? a.qw : a.kw)[l];
  const uint4 cv = reinterpret_cast<const uint4*>(a.cos + b * a.cs_bs)[l];
  const uint4 sv = reinterpret_cast<const uint4*>(a.sin + b * a.cs_bs)[l];
  float x[8];
  unpack8(xv, x);
  const uint4 o = norm_rope(x, wv, cv, sv, is_q ? a.q_eps : a.k_eps, l);
  if (live) reinterpret_cast<uint4*>(dst)[l] = o;
}

// ------------------------------------------------------- packed decode + cache
struct QkvArgs {
  const void* qkv;         // bf16 [batch, W] or f32 [splits, batch, W]
  int32_t splits;
  int64_t split_stride;    // batch * W
  uint32_t rows;           // batch * heads
  uint32_t nq, nk;
  FastDiv heads;           // nq + 2 nk
  const uint16_t* qw;
  const uint16_t* kw;
  float q_eps, k_eps;
  const uint16_t* cos;
  const uint16_t* sin;
  const int64_t* position;
  int64_t capacity;
  uint16_t* q_out;
  uint16_t* kc;
  uint16_t* vc;
};

__global__ __launch_bounds__(kDecodeThreads) void qkv_norm_rope_cache_kernel(QkvArgs a) {
  const uint32_t g = blockIdx.x * kDecodeRows + threadIdx.x / kLanes;
  const int l = threadIdx.x % kLanes;
  const bool live = g < a.rows;
  const uint32_t gg = live ? g : 0;
  const uint32_t b = fdiv(gg, a.heads);
  const uint32_t h = gg - b * a.heads.d;
  const int64_t width = (int64_t)a.heads.d * kD;

  const int64_t pos = *a.position;
  const bool pos_ok = pos >= 0 && pos < a.capacity;
  const int64_t slot = pos_ok ? pos : 0;

  const int64_t off = (int64_t)b * width + (int64_t)h * kD + l * 8;
  uint4 xv;
  float x[8];
  if (a.splits == 0) {
    xv = live ? *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.qkv) + off)
              : zero4();
    unpack8(xv, x);
  } else {
    sum_partials8<16>(static_cast<const float*>(a.qkv) + off, a.split_stride, a.splits, live, x);
    xv = pack8(x);  // one rounding of the f32 sum
    unpack8(xv, x);
  }

  const bool is_q = h < a.nq;
  const bool is_k = !is_q && h < a.nq + a.nk;
  const uint4 wv = reinterpret_cast<const uint4*>(is_q ? a.qw : a.kw)[l];
  const uint4 cv = reinterpret_cast<const uint4*>(a.cos + slot * kD)[l];
  const uint4 sv = reinterpret_cast<const uint4*>(a.sin + slot * kD)[l];
  const uint4 o = norm_rope(x, wv, cv, sv, is_q ? a.q_eps : a.k_eps, l);

  if (!live) return;  // no cross-lane work below
  if (is_q) {
    const uint4 nan4 = make_uint4(0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u);
    reinterpret_cast<uint4*>(a.q_out + ((uint64_t)b * a.nq + h) * kD)[l] = select4(pos_ok, o, nan4);
  } else if (pos_ok) {
    const uint32_t kvh = is_k ? h - a.nq : h - a.nq - a.nk;
    const int64_t row = ((int64_t)b * a.nk + kvh) * a.capacity + slot;
    uint16_t* dst = (is_k ? a.kc : a.vc) + row * kD;
    reinterpret_cast<uint4*>(dst)[l] = select4(is_k, o, xv);
  }
}

// ------------------------------------------------------------ packed prefill
struct PrefillArgs {
  const uint16_t* qkv;     // [batch * length, W]
  uint32_t rows;           // batch * length * heads          (generic kernel)
  uint32_t waves;          // tokens * waves per token        (unit kernel)
  uint32_t nq, nk;
  uint32_t q_units, k_units, units;  // nq / 8, nk / 8, (nq + 2 nk) / 8
  FastDiv heads;           // nq + 2 nk
  FastDiv waves_per_token; // ceil(units / kUnitsPerWave)
  FastDiv length;
  const uint16_t* qw;
  const uint16_t* kw;
  float q_eps, k_eps;
  const uint16_t* cos;
  const uint16_t* sin;
  int64_t capacity;
  uint16_t* q_out;         // [batch, length, nq, 128]
  uint16_t* kc;
  uint16_t* vc;
};

// Unit kernel (nq and nk multiples of 8).  A lane holds 16 elements of one
// head row: [8l, 8l+8) and their rotate-half partners [64+8l, 64+8l+8), so
// the partner exchange needs no cross-lane traffic and a row is reduced over
// 8 lanes (3 DPP steps).  A "unit" is 8 consecutive head rows of one token
// with one role (q, k or v), one per 8-lane group of a wave.  A wave owns up
// to kUnitsPerWave consecutive units of one token: its loads all issue first,
// the token's cos/sin row and both gains are unpacked once per wave, roles
// are wave-uniform (scalar branches) and v units are pure copies.
// Qwen3-4B: 6 units per token -> 3 waves of 2 units.
constexpr int kUnitsPerWave = 2;
constexpr int kRowLanes = 8;  // lanes per head row in the unit kernel

// Norm + gain + RoPE of one head row spread as 16 elements per lane over 8
// lanes: x[0..7] are elements 8l+j, x[8..15] their partners 64+8l+j.  sr is
// sin with the rotate-half sign folded in (negated for the first half).
__device__ __forceinline__ void norm_rope16(const float* x, const float* w, const float* c,
                                            const float* sr, float eps, uint4& lo, uint4& hi) {
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < 16; ++j) ss += (double)(x[j] * x[j]);  // exact squares, exact sum
  const float inv = inv_rms(group_sum_f64<kRowLanes>(ss), (float)kD, eps);
  float n[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) n[j] = x[j] * inv;
  round8(n);
  round8(n + 8);
#pragma unroll
  for (int j = 0; j < 16; ++j) n[j] *= w[j];
  round8(n);
  round8(n + 8);
  float left[16], right[16];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    left[j] = n[j] * c[j];
    right[j] = n[j + 8] * sr[j];          // rot = -n[e + 64] for the first half
    left[j + 8] = n[j + 8] * c[j + 8];
    right[j + 8] = n[j] * sr[j + 8];      // rot = n[e - 64] for the second half
  }
  round8(left);
  round8(left + 8);
  round8(right);
  round8(right + 8);
#pragma unroll
  for (int j = 0; j < 16; ++j) left[j] += right[j];
  lo = pack8(left);
  hi = pack8(left + 8);
}

// FULL: every wave's UPW units exist (units % UPW == 0), so the loads and the
// unit loop carry no bounds branch; measured on the Qwen3-4B 4 x 2048 call
// 34.0 us against 35.2 us with the checks (a copy with this kernel's loads and
// stores and no arithmetic takes 33.0 us).
template <bool NT, bool FULL, int UPW = kUnitsPerWave, int MIN_WAVES = 1>
__global__ __launch_bounds__(kBlock, MIN_WAVES) void prefill_qkv_unit_kernel(PrefillArgs a) {
  const uint32_t wave =
      __builtin_amdgcn_readfirstlane(blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave);
  if (wave >= a.waves) return;  // wave-uniform
  const uint32_t token = __builtin_amdgcn_readfirstlane(fdiv(wave, a.waves_per_token));
  const uint32_t first =
      __builtin_amdgcn_readfirstlane((wave - token * a.waves_per_token.d) * UPW);
  const uint32_t b = __builtin_amdgcn_readfirstlane(fdiv(token, a.length));
  const uint32_t t = token - b * a.length.d;
  const int lane = threadIdx.x % kWave;
  const int grp = lane / kRowLanes;  // head within the unit
  const int l = lane % kRowLanes;

  const int64_t width = (int64_t)a.heads.d * kD;
  const uint16_t* src = a.qkv + (int64_t)token * width + grp * kD + l * 8;
  uint4 xlo[UPW], xhi[UPW];
#pragma unroll
  for (int u = 0; u < UPW; ++u) {
    if (FULL || first + u < a.units) {
      const uint16_t* p = src + (int64_t)(first + u) * kRowLanes * kD;
      xlo[u] = load16<NT>(p);
      xhi[u] = load16<NT>(p + kD / 2);
    }
  }

  float c[16], sr[16], wq[16], wk[16];
  const int64_t trow = (int64_t)t * kD + l * 8;
  unpack8(load16<false>(a.cos + trow), c);
  unpack8(load16<false>(a.cos + trow + kD / 2), c + 8);
  unpack8(negate_if(load16<false>(a.sin + trow), true), sr);
  unpack8(load16<false>(a.sin + trow + kD / 2), sr + 8);
  unpack8(load16<false>(a.qw + l * 8), wq);
  unpack8(load16<false>(a.qw + l * 8 + kD / 2), wq + 8);
  unpack8(load16<false>(a.kw + l * 8), wk);
  unpack8(load16<false>(a.kw + l * 8 + kD / 2), wk + 8);

#pragma unroll
  for (int u = 0; u < UPW; ++u) {
    const uint32_t unit = first + u;
    if (!FULL && unit >= a.units) break;  // wave-uniform
    uint16_t* dst;
    uint4 lo = xlo[u], hi = xhi[u];
    if (unit < a.q_units + a.k_units) {
      float x[16];
      unpack8(xlo[u], x);
      unpack8(xhi[u], x + 8);
      if (unit < a.q_units) {
        norm_rope16(x, wq, c, sr, a.q_eps, lo, hi);
        dst = a.q_out + ((uint64_t)token * a.nq + unit * kRowLanes + grp) * kD;
      } else {
        norm_rope16(x, wk, c, sr, a.k_eps, lo, hi);
        const uint32_t kvh = (unit - a.q_units) * kRowLanes + grp;
        dst = a.kc + (((int64_t)b * a.nk + kvh) * a.capacity + t) * kD;
      }
    } else {
      const uint32_t kvh = (unit - a.q_units - a.k_units) * kRowLanes + grp;
      dst = a.vc + (((int64_t)b * a.nk + kvh) * a.capacity + t) * kD;  // raw copy
    }
    store16<NT>(dst + l * 8, lo);
    store16<NT>(dst + l * 8 + kD / 2, hi);
  }
}

// Generic kernel (any nq, nk): one head row per 16-lane group.
__global__ __launch_bounds__(kBlock) void prefill_qkv_kernel(PrefillArgs a) {
  const uint32_t g = blockIdx.x * kRowsPerBlock + threadIdx.x / kLanes;
  const int l = threadIdx.x % kLanes;
  const bool live = g < a.rows;
  const uint32_t gg = live ? g : 0;
  const uint32_t token = fdiv(gg, a.heads);
  const uint32_t h = gg - token * a.heads.d;
  const uint32_t b = fdiv(token, a.length);
  const uint32_t t = token - b * a.length.d;

  const int64_t width = (int64_t)a.heads.d * kD;
  const uint4 xv =
      live ? reinterpret_cast<const uint4*>(a.qkv + (int64_t)token * width + (int64_t)h * kD)[l]
           : zero4();
  float x[8];
  unpack8(xv, x);

  const bool is_q = h < a.nq;
  const bool is_k = !is_q && h < a.nq + a.nk;
  const uint4 wv = reinterpret_cast<const uint4*>(is_q ? a.qw : a.kw)[l];
  const uint4 cv = reinterpret_cast<const uint4*>(a.cos + (int64_t)t * kD)[l];
  const uint4 sv = reinterpret_cast<const uint4*>(a.sin + (int64_t)t * kD)[l];
  const uint4 o = norm_rope(x, wv, cv, sv, is_q ? a.q_eps : a.k_eps, l);

  if (!live) return;
  if (is_q) {
    reinterpret_cast<uint4*>(a.q_out + ((uint64_t)token * a.nq + h) * kD)[l] = o;
  } else {
    const uint32_t kvh = is_k ? h - a.nq : h - a.nq - a.nk;
    const int64_t row = ((int64_t)b * a.nk + kvh) * a.capacity + t;
    uint16_t* dst = (is_k ? a.kc : a.vc) + row * kD;
    reinterpret_cast<uint4*>(dst)[l] = select4(is_k, o, xv);
  }
}

inline unsigned blocks_for(uint64_t rows, int per_block = kRowsPerBlock) {
  return (unsigned)((rows + per_block - 1) / per_block);
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int qf_qk_norm_rope(const void* q, const void* k, int64_t batch, int32_t nq,
                               int32_t nk, int64_t q_bstride, int64_t q_hstride,
                               int64_t k_bstride, int64_t k_hstride, const void* q_weight,
                               const void* k_weight, const void* cos, const void* sin,
                               int64_t cs_bstride, float q_eps, float k_eps, void* out_q,
                               void* out_k, void* stream) {
  if (batch < 0 || nq < 1 || nk < 1 || cs_bstride < 0) return QF_E_ARG;
  if (batch == 0) return QF_OK;
  if (!q || !k || !q_weight || !k_weight || !cos || !sin || !out_q || !out_k) return QF_E_ARG;
  const uint64_t rows = (uint64_t)batch * (uint64_t)(nq + nk);
  if (rows >= (uint64_t)UINT32_MAX - kRowsPerBlock) return QF_E_SHAPE;
  const bool aligned = aligned16(q) && aligned16(k) && aligned16(q_weight) &&
                       aligned16(k_weight) && aligned16(cos) && aligned16(sin) &&
                       aligned16(out_q) && aligned16(out_k) && q_bstride % 8 == 0 &&
                       q_hstride % 8 == 0 && k_bstride % 8 == 0 && k_hstride % 8 == 0 &&
                       cs_bstride % 8 == 0;
  if (!aligned) return QF_E_ALIGN;
  QkArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.q_bs = q_bstride; a.q_hs = q_hstride; a.k_bs = k_bstride; a.k_hs = k_hstride;
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.cs_bs = cs_bstride;
  a.q_eps = q_eps; a.k_eps = k_eps;
  a.oq = static_cast<uint16_t*>(out_q);
  a.ok = static_cast<uint16_t*>(out_k);
  a.rows = (uint32_t)rows;
  a.nq = (uint32_t)nq; a.nk = (uint32_t)nk;
  a.heads = make_fastdiv((uint32_t)(nq + nk));
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(blocks_for(rows, kDecodeRows)),
                     dim3(kDecodeThreads), 0, as_stream(stream), a);
  return launch_status();
}

extern "C" int qf_qkv_norm_rope_cache(const void* qkv, int32_t splits, int64_t batch, int32_t nq,
                                      int32_t nk, const void* q_weight, const void* k_weight,
                                      float q_eps, float k_eps, const void* cos, const void* sin,
                                      const int64_t* position, int64_t capacity, void* q_out,
                                      void* key_cache, void* value_cache, void* stream) {
  if (batch < 0 || nq < 1 || nk < 1 || splits < 0 || capacity < 1) return QF_E_ARG;
  if (batch == 0) return QF_OK;
  if (!qkv || !q_weight || !k_weight || !cos || !sin || !position || !q_out || !key_cache ||
      !value_cache)
    return QF_E_ARG;
  const uint64_t heads = (uint64_t)nq + 2 * (uint64_t)nk;
  const uint64_t rows = (uint64_t)batch * heads;
  if (rows >= (uint64_t)UINT32_MAX - kRowsPerBlock) return QF_E_SHAPE;
  if (!(aligned16(qkv) && aligned16(q_weight) && aligned16(k_weight) && aligned16(cos) &&
        aligned16(sin) && aligned16(q_out) && aligned16(key_cache) && aligned16(value_cache)) ||
      (reinterpret_cast<uintptr_t>(position) & 7u))
    return QF_E_ALIGN;
  QkvArgs a{};
  a.qkv = qkv;
  a.splits = splits;
  a.split_stride = batch * (int64_t)heads * kD;
  a.rows = (uint32_t)rows;
  a.nq = (uint32_t)nq; a.nk = (uint32_t)nk;
  a.heads = make_fastdiv((uint32_t)heads);
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.q_eps = q_eps; a.k_eps = k_eps;
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.position = position;
  a.capacity = capacity;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.kc = static_cast<uint16_t*>(key_cache);
  a.vc = static_cast<uint16_t*>(value_cache);
  hipLaunchKernelGGL(qkv_norm_rope_cache_kernel, dim3(blocks_for(rows, kDecodeRows)),
                     dim3(kDecodeThreads), 0,
                     as_stream(stream), a);
  return launch_status();
}

extern "C" int qf_prefill_qkv(const void* qkv, int64_t batch, int64_t length, int32_t nq,
                              int32_t nk, const void* q_weight, const void* k_weight, float q_eps,
                              float k_eps, const void* cos, const void* sin, int64_t capacity,
                              void* q_out, void* key_cache, void* value_cache, void* stream) {
  if (batch < 0 || length < 0 || nq < 1 || nk < 1 || capacity < 1) return QF_E_ARG;
  if (length > capacity) return QF_E_SHAPE;
  if (batch == 0 || length == 0) return QF_OK;
  if (!qkv || !q_weight || !k_weight || !cos || !sin || !q_out || !key_cache || !value_cache)
    return QF_E_ARG;
  const uint64_t heads = (uint64_t)nq + 2 * (uint64_t)nk;
  const uint64_t tokens = (uint64_t)batch * (uint64_t)length;
  const uint64_t rows = tokens * heads;
  if (rows >= (uint64_t)UINT32_MAX - kRowsPerBlock || length >= (int64_t)UINT32_MAX)
    return QF_E_SHAPE;
  if (!(aligned16(qkv) && aligned16(q_weight) && aligned16(k_weight) && aligned16(cos) &&
        aligned16(sin) && aligned16(q_out) && aligned16(key_cache) && aligned16(value_cache)))
    return QF_E_ALIGN;
  PrefillArgs a{};
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.rows = (uint32_t)rows;
  a.nq = (uint32_t)nq; a.nk = (uint32_t)nk;
  a.heads = make_fastdiv((uint32_t)heads);
  a.length = make_fastdiv((uint32_t)length);
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.q_eps = q_eps; a.k_eps = k_eps;
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.capacity = capacity;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.kc = static_cast<uint16_t*>(key_cache);
  a.vc = static_cast<uint16_t*>(value_cache);
  hipStream_t s = as_stream(stream);
  if (nq % kRowLanes == 0 && nk % kRowLanes == 0) {
    a.q_units = (uint32_t)nq / kRowLanes;
    a.k_units = (uint32_t)nk / kRowLanes;
    a.units = (uint32_t)heads / kRowLanes;
    const uint32_t per_token = (a.units + kUnitsPerWave - 1) / kUnitsPerWave;
    a.waves_per_token = make_fastdiv(per_token);
    const uint64_t waves = tokens * per_token;
    a.waves = (uint32_t)waves;
    const uint64_t blocks = (waves + kBlock / kWave - 1) / (kBlock / kWave);
    const bool stream = (int64_t)rows * kD * 4 >= kStreamBytes;
    const bool full = a.units % kUnitsPerWave == 0;
    if (stream && full)
      hipLaunchKernelGGL((prefill_qkv_unit_kernel<true, true>), dim3((unsigned)blocks),
                         dim3(kBlock), 0, s, a);
    else if (stream)
      hipLaunchKernelGGL((prefill_qkv_unit_kernel<true, false>), dim3((unsigned)blocks),
                         dim3(kBlock), 0, s, a);
    else if (full)
      hipLaunchKernelGGL((prefill_qkv_unit_kernel<false, true>), dim3((unsigned)blocks),
                         dim3(kBlock), 0, s, a);
    else
      hipLaunchKernelGGL((prefill_qkv_unit_kernel<false, false>), dim3((unsigned)blocks),
                         dim3(kBlock), 0, s, a);
    return launch_status();
  }
  hipLaunchKernelGGL(prefill_qkv_kernel, dim3(blocks_for(rows)), dim3(kBlock), 0, s, a);
  return launch_status();
}
