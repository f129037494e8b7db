// Decode projections at one to four rows, one workgroup per compute unit.
//
// The engine's decode step (engine/decode_step.py:40-59) runs every
// projection as split-K partials (engine/kernels/skinny_gemm.py:100-109) and
// then a separate residual-add + RMSNorm launch over the partials
// (engine/kernels/decode_fused.py:140-160).  At one to four rows that
// launch is pure latency (a few microseconds for 10 KB per row).  Here a
// projection instead runs as 256 workgroups (one per MI355X compute unit),
// each over the WHOLE K range of n / 256 consecutive columns, so every
// output is complete inside one workgroup and the add + norm split in two:
//
// * qf_linear_residual (the residual add, as the producer's epilogue):
//     y = bf16(x W^T);  total = bf16(residual + y)
//   and per workgroup g the f64 sum of total^2 over its columns,
//   sq[r][g] (exact: squares of bf16 values, at most 16 significant bits).
// * qf_linear_normed (the RMSNorm, as the consumer's prologue):
//     inv = 1 / sqrt(f32(sum_g sq[r][g]) / k + eps)
//     x   = bf16(bf16(total * inv) * gain);  out = bf16(x W^T)
//   with the same rounding steps as qf_add_rms_norm, so x is bit-identical
//   to the normalised row that launch would have written (the f64 sum is
//   exact, so its order does not matter).
//
// Work per workgroup: C = n / 256 weight rows of k bf16 (contiguous), read
// once with nontemporal 16-byte loads; thread t takes 8-element chunks
// t, t + 256, ... of K for every column and every input row, with the next
// chunk's loads issued before this chunk's dot products (v_dot2c_f32_bf16,
// f32 accumulation), eight waves per workgroup.  The per-thread sums of each
// output go through LDS (column-major, one float per thread) and are added
// in a fixed order.  Measured on the Qwen3-4B down projection (49.8 MB):
// 8 waves 9.7 us against 10.2 with 4; nontemporal weight loads 5-15% faster
// than cached ones; input rows staged in LDS instead of loaded per chunk
// 0.5 us slower (the staging's round trip sits before the stream).
// Per-CU streaming rate rather than workgroup count bounds this shape: one
// workgroup of full-K rows per CU keeps every CU's request queue full.
#include "qf_device.h"

namespace qf {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kGroups = QF_ROW_GROUPS;  // workgroups per launch = sq entries per row
constexpr int kRowThreads = 512;        // 8 waves: two per SIMD
constexpr int kMaxRows = 4;
static_assert(kGroups <= kRowThreads, "the prologue loads one sum of squares per thread");

struct RowArgs {
  const uint16_t* x;         // bf16 [rows, k]: input rows, or (NORMED) the residual stream
  const double* sq;          // NORMED: f64 [rows, kGroups]
  const uint16_t* gain;      // NORMED: bf16 [k]
  float eps;
  const uint16_t* w;         // bf16 [n, k]
  int64_t k;
  int32_t rows, n;
  int32_t chunks;            // k / 8
  uint16_t* out;             // bf16 [rows, n]: y, or (RESIDUAL) residual + y
  const uint16_t* residual;  // RESIDUAL: bf16 [rows, n]
  double* sq_out;            // RESIDUAL: f64 [rows, kGroups]
};

__device__ __forceinline__ float dot8(const uint4& x, const uint4& w, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.x), __builtin_bit_cast(bf16x2, w.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.y), __builtin_bit_cast(bf16x2, w.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.z), __builtin_bit_cast(bf16x2, w.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.w), __builtin_bit_cast(bf16x2, w.w), acc, false);
  return acc;
}

// R: rows (padded: rows >= a.rows are skipped at the stores); C: columns per
// workgroup; PF: weight chunks in flight per thread (1 or 2).
//
// Order of the memory operations matters: a wave waits for its global loads
// in issue order (one vmcnt counter), so each chunk's input-row (and gain)
// loads are issued before its weight loads, and the next chunk's before this
// chunk's arithmetic; the sums of squares and the first chunk's loads are all
// in flight before the prologue waits for the sums.
template <int R, int C, bool NORMED, bool RESIDUAL>
__global__ __launch_bounds__(kRowThreads) void row_gemv_kernel(RowArgs a) {
  constexpr int V = R * C;  // outputs per workgroup
  constexpr int PF = C * 8 + V <= 224 ? 2 : 1;
  constexpr int kWaves = kRowThreads / kWave;
  constexpr int kStride = kRowThreads + 4;  // floats per LDS column (16-byte aligned rows)
  constexpr int kPer = kRowThreads / 8;     // per-thread values each reducing thread adds
  static_assert(V <= 32, "at most 32 outputs per workgroup (8 reducing threads each)");
  __shared__ __attribute__((aligned(16))) float red[V * kStride];
  __shared__ double wsum[kWaves][R];
  __shared__ double sq_cols[V];
  const int t = threadIdx.x;
  const int g = blockIdx.x;
  const int64_t n0 = (int64_t)g * C;
  const uint16_t* wbase = a.w + n0 * a.k;
  const int chunks = a.chunks;

  uint4 wv[PF][C];
  uint4 xr[PF][R], gr[PF];
  auto load_w = [&](int slot, int ch) {
#pragma unroll
    for (int j = 0; j < C; ++j) wv[slot][j] = load16<true>(wbase + j * a.k + 8 * ch);
  };
  auto load_x = [&](int slot, int ch) {
    if constexpr (NORMED) gr[slot] = load16<false>(a.gain + 8 * ch);
#pragma unroll
    for (int r = 0; r < R; ++r) xr[slot][r] = load16<false>(a.x + (int64_t)(r < a.rows ? r : 0) * a.k + 8 * ch);
  };

  double sqv[R];
  if constexpr (NORMED) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      sqv[r] = r < a.rows && t < kGroups ? a.sq[(int64_t)r * kGroups + t] : 0.0;
  }
  if (t < chunks) {
    load_x(0, t);
    load_w(0, t);
  }
  float inv[R];
  if constexpr (NORMED) {
    // inv_rms of each row from the producer's per-workgroup sums of squares.
#pragma unroll
    for (int r = 0; r < R; ++r) sqv[r] = group_sum_f64<kWave>(sqv[r]);
    if (t % kWave == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) wsum[t / kWave][r] = sqv[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      double s = 0.0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) s += wsum[w][r];
      inv[r] = inv_rms(s, (float)a.k, a.eps);
    }
  }

  float acc[R][C];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < C; ++j) acc[r][j] = 0.0f;
  auto consume = [&](int slot) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint4 xv = xr[slot][r];
      if constexpr (NORMED) {
        float f[8], gf[8];
        unpack8(xv, f);
        unpack8(gr[slot], gf);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= inv[r];
        round8(f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= gf[e];
        xv = pack8(f);
      }
#pragma unroll
      for (int j = 0; j < C; ++j) acc[r][j] = dot8(xv, wv[slot][j], acc[r][j]);
    }
  };
  if constexpr (PF == 2) {
    for (int ch = t; ch < chunks; ch += 2 * kRowThreads) {
      if (ch + kRowThreads < chunks) {
        load_x(1, ch + kRowThreads);
        load_w(1, ch + kRowThreads);
      }
      consume(0);
      if (ch + kRowThreads >= chunks) break;
      if (ch + 2 * kRowThreads < chunks) {
        load_x(0, ch + 2 * kRowThreads);
        load_w(0, ch + 2 * kRowThreads);
      }
      consume(1);
    }
  } else {
    for (int ch = t; ch < chunks; ch += kRowThreads) {
      if (ch != t) {
        load_x(0, ch);
        load_w(0, ch);
      }
      consume(0);
    }
  }

  // Sum of the per-thread values of each output, in a fixed order: threads
  // 8v .. 8v + 7 add kPer consecutive entries each, then pairwise.
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < C; ++j) red[(r * C + j) * kStride + t] = acc[r][j];
  __syncthreads();
  const int v = t / 8, part = t % 8;
  float s = 0.0f;
  if (v < V) {
    const float4* p = reinterpret_cast<const float4*>(red + v * kStride + kPer * part);
#pragma unroll
    for (int i = 0; i < kPer / 4; ++i) {
      const float4 q = p[i];
      s += q.x;
      s += q.y;
      s += q.z;
      s += q.w;
    }
  }
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  const int r = v / C, j = v % C;
  const bool live = v < V && part == 0 && r < a.rows;
  const int64_t col = n0 + j;
  if constexpr (RESIDUAL) {
    float tot = 0.0f;
    if (live) {
      const float y = from_bf16(to_bf16(s));
      tot = from_bf16(to_bf16(from_bf16(a.residual[(int64_t)r * a.n + col]) + y));
      a.out[(int64_t)r * a.n + col] = to_bf16(tot);
    }
    if (v < V && part == 0) sq_cols[v] = (double)(tot * tot);
    __syncthreads();
    if (t < R && t < a.rows) {
      double q = 0.0;
#pragma unroll
      for (int c = 0; c < C; ++c) q += sq_cols[t * C + c];
      a.sq_out[(int64_t)t * kGroups + g] = q;
    }
  } else {
    if (live) a.out[(int64_t)r * a.n + col] = to_bf16(s);
  }
}

template <int R, bool NORMED, bool RESIDUAL>
int launch_rows_c(RowArgs a, int c, hipStream_t s) {
  switch (c) {
#define QF_ROW_CASE(CC)                                                                          \
  case CC:                                                                                       \
    if constexpr (R * CC <= 32) {                                                                \
      hipLaunchKernelGGL((row_gemv_kernel<R, CC, NORMED, RESIDUAL>), dim3(kGroups),              \
                         dim3(kRowThreads), 0, s, a);                                            \
      return launch_status();                                                                    \
    }                                                                                            \
    return QF_E_SHAPE;
    QF_ROW_CASE(2)
    QF_ROW_CASE(4)
    QF_ROW_CASE(8)
    QF_ROW_CASE(10)
    QF_ROW_CASE(16)
    QF_ROW_CASE(24)
    QF_ROW_CASE(32)
#undef QF_ROW_CASE
    default:
      return QF_E_SHAPE;
  }
}

template <bool NORMED, bool RESIDUAL>
int launch_rows(RowArgs a, hipStream_t s) {
  const int c = a.n / kGroups;
  switch (a.rows) {
    case 1: return launch_rows_c<1, NORMED, RESIDUAL>(a, c, s);
    case 2: return launch_rows_c<2, NORMED, RESIDUAL>(a, c, s);
    default: return launch_rows_c<4, NORMED, RESIDUAL>(a, c, s);
  }
}

bool row_columns_ok(int64_t n, int32_t rows) {
  if (n < kGroups || n % kGroups != 0) return false;
  const int64_t c = n / kGroups;
  const int padded = rows <= 2 ? rows : 4;
  return (c == 2 || c == 4 || c == 8 || c == 10 || c == 16 || c == 24 || c == 32) && padded * c <= 32;
}

int row_shape_status(int32_t rows, int64_t k, int64_t n) {
  if (rows < 1 || rows > kMaxRows || k < 8 || k % 8 != 0 || k / 8 > INT32_MAX || n > INT32_MAX)
    return QF_E_SHAPE;
  return row_columns_ok(n, rows) ? QF_OK : QF_E_SHAPE;
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int qf_row_supported(int32_t rows, int64_t k, int64_t n) {
  return row_shape_status(rows, k, n) == QF_OK ? 1 : 0;
}

extern "C" int qf_linear_rows(const void* x, int32_t rows, int64_t k, const void* weight, int64_t n,
                              void* out, void* stream) {
  const int st = row_shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!x || !weight || !out) return QF_E_ARG;
  if (!aligned16(x) || !aligned16(weight)) return QF_E_ALIGN;
  RowArgs a = {};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(weight);
  a.k = k;
  a.rows = rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)(k / 8);
  a.out = static_cast<uint16_t*>(out);
  return launch_rows<false, false>(a, as_stream(stream));
}

extern "C" int qf_linear_residual(const void* x, int32_t rows, int64_t k, const void* weight,
                                  int64_t n, const void* residual, void* total, double* sq,
                                  void* stream) {
  const int st = row_shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!x || !weight || !residual || !total || !sq) return QF_E_ARG;
  if (!aligned16(x) || !aligned16(weight) || (reinterpret_cast<uintptr_t>(sq) & 7u) != 0)
    return QF_E_ALIGN;
  RowArgs a = {};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(weight);
  a.k = k;
  a.rows = rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)(k / 8);
  a.out = static_cast<uint16_t*>(total);
  a.residual = static_cast<const uint16_t*>(residual);
  a.sq_out = sq;
  return launch_rows<false, true>(a, as_stream(stream));
}

extern "C" int qf_linear_normed(const void* total, const double* sq, const void* gain, float eps,
                                int32_t rows, int64_t k, const void* weight, int64_t n, void* out,
                                void* stream) {
  const int st = row_shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!total || !sq || !gain || !weight || !out) return QF_E_ARG;
  if (!(eps == eps) || eps < 0.0f || eps == __builtin_inff()) return QF_E_ARG;
  if (!aligned16(total) || !aligned16(gain) || !aligned16(weight) ||
      (reinterpret_cast<uintptr_t>(sq) & 7u) != 0)
    return QF_E_ALIGN;
  RowArgs a = {};
  a.x = static_cast<const uint16_t*>(total);
  a.sq = sq;
  a.gain = static_cast<const uint16_t*>(gain);
  a.eps = eps;
  a.w = static_cast<const uint16_t*>(weight);
  a.k = k;
  a.rows = rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)(k / 8);
  a.out = static_cast<uint16_t*>(out);
  return launch_rows<true, false>(a, as_stream(stream));
}
