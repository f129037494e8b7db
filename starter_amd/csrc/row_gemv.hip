// Decode projections at one to four rows, one workgroup per compute unit.
//
// The engine's decode step (engine/decode_step.py:40-59) runs every
// projection as split-K partials (engine/kernels/skinny_gemm.py:100-109) and
// then a separate residual-add + RMSNorm launch over the partials
// (engine/kernels/decode_fused.py:140-160).  At one to four rows that
// launch is pure latency (a few microseconds for 10 KB per row).  Here a
// projection instead runs as 256 workgroups (one per MI355X compute unit),
// each over the WHOLE K range of a block of columns, so every output is
// complete inside one workgroup and the add + norm split in two:
//
// * residual epilogue (qf_linear_residual, qf_linear_residual_merged):
//     y = bf16(x W^T);  total = bf16(residual + y)
//   and per workgroup g the f64 sum of total^2 over its columns, sq[r][g]
//   (squares of bf16 values have at most 16 significant bits, so the sums
//   are exact while a row's squares span less than about 53 - 16 - log2(k)
//   bits of exponent).
// * normalising prologue (qf_linear_normed, qf_linear_silu_mul_normed):
//     inv = 1 / sqrt(f32(sum_g sq[r][g]) / k + eps)
//     x   = bf16(bf16(total * inv) * gain);  out = bf16(x W^T)
//   with the same rounding steps as qf_add_rms_norm, so x is bit-identical
//   to the normalised row that launch would have written whenever the f64
//   sums are exact.  Rows with a wider spread (Qwen3's massive activations
//   next to near-zero values) add their squares in a different order from
//   qf_add_rms_norm; the two totals then differ by far less than an f32 ulp
//   and round to the same f32 except in rare near-tie cases.
//
// Two more ends complete a decoder layer: the SiLU * up epilogue of the
// packed gate/up projection (bf16(bf16(silu(bf16(g))) * bf16(u)), as
// qf_linear_silu_mul; workgroup g owns gate rows [gH, gH + H) and the
// matching up rows), and a prologue that merges the decode attention's key
// segments into the input row (qf_merge.h, the bits of the attention's own
// merge), for o_proj.
//
// Work per workgroup: C weight rows of k bf16 (contiguous), read once with
// nontemporal 16-byte loads.  The 8 waves form NG column groups of C / NG
// columns; thread t of a group takes 8-element chunks t, t + 512 / NG, ...
// of K for its columns and every input row (NG > 1 keeps every wave busy
// when K is short), with each chunk's input loads issued before its weight
// loads and the next chunk's before this chunk's dot products
// (v_dot2c_f32_bf16, f32 accumulation).  The per-thread sums of each output
// go through LDS (one float per thread) and are added in a fixed order.
// Measured on the Qwen3-4B down projection (49.8 MB): 8 waves 9.7 us against
// 10.2 with 4; nontemporal weight loads 5-15% faster than cached ones; input
// rows staged in LDS instead of loaded per chunk 0.5 us slower (the
// staging's round trip sits before the stream).  Per-CU streaming rate
// rather than workgroup count bounds this shape: one workgroup of full-K
// rows per CU keeps every CU's request queue full.
#include "qf_device.h"
#include "qf_merge.h"
#include "qf_silu.h"

namespace qf {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kGroups = QF_ROW_GROUPS;  // workgroups per launch = sq entries per row
constexpr int kRowThreads = 512;        // 8 waves: two per SIMD
constexpr int kRowWaves = kRowThreads / kWave;
constexpr int kMaxRows = 4;
constexpr int kMaxOutputs = 128;        // rows x columns per workgroup
static_assert(kGroups <= kRowThreads, "the prologue loads one sum of squares per thread");

// Input row source and output epilogue.
constexpr int kInPlain = 0;   // x rows from memory
constexpr int kInNormed = 1;  // RMSNorm of the residual stream (sq from a residual epilogue)
constexpr int kInMerged = 2;  // merge of the attention's key segments (staged in LDS)
constexpr int kOutPlain = 0;
constexpr int kOutResidual = 1;
constexpr int kOutSiluMul = 2;

struct RowArgs {
  const uint16_t* x;         // bf16 [rows, k]: input rows, or (normed) the residual stream
  const double* sq;          // normed: f64 [rows, kGroups]
  const uint16_t* gain;      // normed: bf16 [k]
  float eps;
  const float* seg_partials; // merged: [rows * kv_heads, segments, G, 128]
  const float* seg_stats;    // merged: [rows * kv_heads, segments, 2, G]
  int32_t segments, q_heads, kv_heads;
  const uint16_t* w;         // bf16 [n, k] ([2 n_out, k] for SiLU * up)
  int64_t k;
  int32_t rows, n;           // n: weight rows
  int32_t chunks;            // k / 8
  uint16_t* out;             // bf16 [rows, n]: y; residual: residual + y; SiLU: [rows, n / 2]
  const uint16_t* residual;  // residual: bf16 [rows, n]
  double* sq_out;            // residual: f64 [rows, kGroups]
};

__device__ __forceinline__ float dot8(const uint4& x, const uint4& w, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.x), __builtin_bit_cast(bf16x2, w.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.y), __builtin_bit_cast(bf16x2, w.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.z), __builtin_bit_cast(bf16x2, w.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.w), __builtin_bit_cast(bf16x2, w.w), acc, false);
  return acc;
}

// Merged attention rows (vh, g) for several query rows at once: lane l gets
// dims 2l, 2l + 1 of each as two packed bf16.  The arithmetic and its order
// are those of merge_segments_row (qf_merge.h), so the bits are the
// attention merge's:
//   M = max_s m_s (0 if every m_s is -inf),  w_s = l_s > 0 ? 2^(m_s - M) : 0,
//   out = bf16((sum_s w_s * p_s) / (sum_s w_s * l_s))  (sums in segment
//   order, unfused multiply then add; a zero denominator gives zeros).
// Lane s loads segment s's statistics and computes its weights, which the
// wave shares through its own LDS table (wl: NR x 64 floats); the partials
// of NR rows and kSegBatch segments are all in flight before any is combined.
template <int NR>
__device__ __forceinline__ void merge_rows(const float* partials, const float* stats, const int64_t* vh,
                                           const int* g, int S, int G, int lane, float* wl,
                                           uint32_t* out) {
  constexpr int kSegBatch = 8;
  float2 pv[NR][kSegBatch];
  auto load_batch = [&](int s0) {
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const float* base = partials + (vh[i] * S * G + g[i]) * 128 + 2 * lane;
#pragma unroll
      for (int j = 0; j < kSegBatch; ++j) {
        const int sj = s0 + j < S ? s0 + j : S - 1;
        pv[i][j] = *reinterpret_cast<const float2*>(base + (int64_t)sj * G * 128);
      }
    }
  };
  load_batch(0);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float* st = stats + vh[i] * S * 2 * G + g[i];
    const float m = lane < S ? st[lane * 2 * G] : -__builtin_inff();
    const float l = lane < S ? st[lane * 2 * G + G] : 0.0f;
    float M = m;
#pragma unroll
    for (int off = 1; off < kWave; off *= 2) M = fmaxf(M, __shfl_xor(M, off));
    if (M == -__builtin_inff()) M = 0.0f;
    const float w = l > 0.0f ? __builtin_amdgcn_exp2f(m - M) : 0.0f;
    if (lane < 32) {
      wl[i * 64 + lane] = w;
      wl[i * 64 + 32 + lane] = l * w;
    }
  }
  wave_lds_fence();
  float total[NR], acc0[NR], acc1[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) total[i] = acc0[i] = acc1[i] = 0.0f;
  for (int s0 = 0; s0 < S; s0 += kSegBatch) {
    if (s0 > 0) load_batch(s0);
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
      for (int j = 0; j < kSegBatch; ++j) {
        if (s0 + j >= S) break;  // wave-uniform
        const float w = wl[i * 64 + s0 + j], lw = wl[i * 64 + 32 + s0 + j];
        total[i] = total[i] + lw;
        acc0[i] = acc0[i] + pv[i][j].x * w;
        acc1[i] = acc1[i] + pv[i][j].y * w;
      }
  }
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float den = total[i] > 0.0f ? total[i] : 1.0f;
    out[i] = pack2(acc0[i] / den, acc1[i] / den);
  }
  wave_lds_fence();  // the table is read before the next call's writes
}

// Column groups per workgroup for C columns: short K ranges need several
// groups to keep all eight waves streaming (qkv and gate/up: K = 2560).
constexpr int column_groups(int c) { return c % 4 == 0 && c >= 16 ? 4 : c % 2 == 0 && c >= 8 ? 2 : 1; }

// R: rows (padded: rows >= a.rows are skipped at the stores); C: columns per
// workgroup; IN / OUT: input source and epilogue.  PF: weight chunks in
// flight per thread (1 or 2).
//
// Order of the memory operations matters: a wave waits for its global loads
// in issue order (one vmcnt counter), so each chunk's input-row (and gain)
// loads are issued before its weight loads, and the next chunk's before this
// chunk's arithmetic; the sums of squares and the first chunk's loads are all
// in flight before the prologue waits for the sums.
template <int R, int C, int IN, int OUT>
__global__ __launch_bounds__(kRowThreads) void row_gemv_kernel(RowArgs a) {
  // (SiLU * up: at least two groups, so no group straddles gate and up rows)
  constexpr int NG = OUT == kOutSiluMul && column_groups(C) < 2 ? 2 : column_groups(C);
  constexpr int CG = C / NG;                   // columns per group
  constexpr int TG = kRowThreads / NG;         // threads per group
  constexpr int V = R * C;                     // outputs per workgroup
  constexpr int RT = V <= 64 ? 8 : 4;          // threads that add up one output
  constexpr int kPer = TG / RT;                // per-thread values each of them adds
  constexpr int kStride = TG + 4;              // floats per output's LDS column
  constexpr int PF = CG * 8 + R * CG <= 224 ? 2 : 1;
  constexpr bool kLdsX = IN == kInMerged;
  static_assert(V <= kMaxOutputs && V * RT <= kRowThreads, "outputs per workgroup");
  static_assert(OUT != kOutSiluMul || (C % 2 == 0 && (C / 2) % CG == 0), "gate / up column groups");
  extern __shared__ uint4 xs[];                // merged: [R][chunks] input rows
  __shared__ __attribute__((aligned(16))) float red[V * kStride];
  __shared__ double wsum[kRowWaves][R];
  __shared__ double sq_cols[V];
  __shared__ float fin[OUT == kOutSiluMul ? V : 1];
  __shared__ float merge_w[IN == kInMerged ? kRowWaves : 1][4 * 64];  // merge_rows' tables
  const int t = threadIdx.x;
  const int lane = t % kWave, wave = t / kWave;
  const int gi = t / TG, tl = t % TG;
  const int g = blockIdx.x;
  const int chunks = a.chunks;

  // Weight row of this thread's column j (local column gi * CG + j).
  auto wrow = [&](int j) -> int64_t {
    const int c = gi * CG + j;
    if constexpr (OUT == kOutSiluMul) {
      constexpr int H = C / 2;
      return c < H ? (int64_t)g * H + c : (int64_t)a.n / 2 + (int64_t)g * H + (c - H);
    } else {
      return (int64_t)g * C + c;
    }
  };
  const uint16_t* wrows[CG];
#pragma unroll
  for (int j = 0; j < CG; ++j) wrows[j] = a.w + wrow(j) * a.k;

  uint4 wv[PF][CG];
  uint4 xr[PF][R], gr[PF];
  auto load_w = [&](int slot, int ch) {
#pragma unroll
    for (int j = 0; j < CG; ++j) wv[slot][j] = load16<true>(wrows[j] + 8 * ch);
  };
  auto load_x = [&](int slot, int ch) {
    if constexpr (!kLdsX) {
      if constexpr (IN == kInNormed) gr[slot] = load16<false>(a.gain + 8 * ch);
#pragma unroll
      for (int r = 0; r < R; ++r)
        xr[slot][r] = load16<false>(a.x + (int64_t)(r < a.rows ? r : 0) * a.k + 8 * ch);
    }
  };

  double sqv[R];
  if constexpr (IN == kInNormed) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      sqv[r] = r < a.rows && t < kGroups ? a.sq[(int64_t)r * kGroups + t] : 0.0;
  }
  if constexpr (IN == kInNormed) {
    // Issued unconditionally (a thread past the last chunk reloads it and
    // never consumes it): behind a branch the compiler cannot count these
    // loads, and the prologue's wait for the sums would wait for them too
    // (s_waitcnt vmcnt(0)), leaving the weight stream idle during the
    // prologue.  Qwen3-4B qkv at one row: 7.7 -> 6.8 us.
    const int c0 = tl < chunks ? tl : chunks - 1;
    load_x(0, c0);
    load_w(0, c0);
  } else if (tl < chunks) {
    load_x(0, tl);
    load_w(0, tl);
  }
  float inv[R];
  if constexpr (IN == kInNormed) {
    // inv_rms of each row from the producer's per-workgroup sums of squares.
#pragma unroll
    for (int r = 0; r < R; ++r) sqv[r] = group_sum_f64<kWave>(sqv[r]);
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) wsum[wave][r] = sqv[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
      double s = 0.0;
#pragma unroll
      for (int w = 0; w < kRowWaves; ++w) s += wsum[w][r];
      inv[r] = inv_rms(s, (float)a.k, a.eps);
    }
  }
  if constexpr (IN == kInMerged) {
    // Merged attention rows (row r, query head h) into LDS while the first
    // weight chunks are in flight: wave w takes rows w, w + 8, ...,
    // kMergeRows at a time (all their loads in flight together).
    constexpr int kMergeRows = 4;
    const int G = a.q_heads / a.kv_heads;
    const int total_rows = a.rows * a.q_heads;
    uint32_t* xw = reinterpret_cast<uint32_t*>(xs);
    for (int base = wave; base < total_rows; base += kMergeRows * kRowWaves) {
      int64_t vh[kMergeRows];
      int gq[kMergeRows], dst[kMergeRows];
#pragma unroll
      for (int i = 0; i < kMergeRows; ++i) {
        const int idx = base + i * kRowWaves < total_rows ? base + i * kRowWaves : base;
        const int r = idx / a.q_heads, h = idx % a.q_heads;
        vh[i] = __builtin_amdgcn_readfirstlane((int)((int64_t)r * a.kv_heads + h / G));
        gq[i] = __builtin_amdgcn_readfirstlane(h % G);
        dst[i] = (r * (int)a.k + h * 128) / 2;
      }
      uint32_t merged[kMergeRows];
      merge_rows<kMergeRows>(a.seg_partials, a.seg_stats, vh, gq, a.segments, G, lane,
                             merge_w[wave], merged);
#pragma unroll
      for (int i = 0; i < kMergeRows; ++i)
        if (base + i * kRowWaves < total_rows) xw[dst[i] + lane] = merged[i];
    }
    __syncthreads();
  }

  float acc[R][CG];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < CG; ++j) acc[r][j] = 0.0f;
  auto consume = [&](int slot, int ch) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint4 xv;
      if constexpr (kLdsX) {
        xv = xs[(r < a.rows ? r : 0) * chunks + ch];
      } else {
        xv = xr[slot][r];
      }
      if constexpr (IN == kInNormed) {
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
      for (int j = 0; j < CG; ++j) acc[r][j] = dot8(xv, wv[slot][j], acc[r][j]);
    }
  };
  if constexpr (PF == 2) {
    for (int ch = tl; ch < chunks; ch += 2 * TG) {
      if (ch + TG < chunks) {
        load_x(1, ch + TG);
        load_w(1, ch + TG);
      }
      consume(0, ch);
      if (ch + TG >= chunks) break;
      if (ch + 2 * TG < chunks) {
        load_x(0, ch + 2 * TG);
        load_w(0, ch + 2 * TG);
      }
      consume(1, ch + TG);
    }
  } else {
    for (int ch = tl; ch < chunks; ch += TG) {
      if (ch != tl) {
        load_x(0, ch);
        load_w(0, ch);
      }
      consume(0, ch);
    }
  }

  // Sum of the per-thread values of each output (v = r * C + column), in a
  // fixed order: threads RT v .. RT v + RT - 1 add kPer consecutive entries
  // each, then pairwise.
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < CG; ++j) red[(r * C + gi * CG + j) * kStride + tl] = acc[r][j];
  __syncthreads();
  const int v = t / RT, part = t % RT;
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
  if constexpr (RT == 8) s += __shfl_xor(s, 4);
  const int r = v / C, c = v % C;
  const bool lead = v < V && part == 0;
  const bool live = lead && r < a.rows;
  if constexpr (OUT == kOutResidual) {
    const int64_t col = (int64_t)g * C + c;
    float tot = 0.0f;
    if (live) {
      const float y = from_bf16(to_bf16(s));
      tot = from_bf16(to_bf16(from_bf16(a.residual[(int64_t)r * a.n + col]) + y));
      a.out[(int64_t)r * a.n + col] = to_bf16(tot);
    }
    if (lead) sq_cols[v] = (double)(tot * tot);
    __syncthreads();
    if (t < R && t < a.rows) {
      double q = 0.0;
#pragma unroll
      for (int cc = 0; cc < C; ++cc) q += sq_cols[t * C + cc];
      a.sq_out[(int64_t)t * kGroups + g] = q;
    }
  } else if constexpr (OUT == kOutSiluMul) {
    constexpr int H = C / 2;
    if (lead) fin[v] = s;
    __syncthreads();
    if (t < R * H && t / H < a.rows) {
      const int rr = t / H, i = t % H;
      const float gate = from_bf16(to_bf16(fin[rr * C + i]));
      const float up = from_bf16(to_bf16(fin[rr * C + H + i]));
      const float y = from_bf16(to_bf16(silu_f32(gate))) * up;
      a.out[(int64_t)rr * (a.n / 2) + (int64_t)g * H + i] = to_bf16(y);
    }
  } else {
    if (live) a.out[(int64_t)r * a.n + (int64_t)g * C + c] = to_bf16(s);
  }
}

// Columns per workgroup served by each epilogue.
constexpr bool served_columns(int c, bool silu) {
  return silu ? (c == 4 || c == 8 || c == 16 || c == 32 || c == 76)
              : (c == 2 || c == 4 || c == 8 || c == 10 || c == 16 || c == 24 || c == 32);
}

constexpr int padded_rows(int rows) { return rows <= 2 ? rows : 4; }

constexpr bool outputs_fit(int v) { return v <= kMaxOutputs && v * (v <= 64 ? 8 : 4) <= kRowThreads; }

template <int R, int IN, int OUT>
int launch_rows_c(RowArgs a, int c, size_t lds, hipStream_t s) {
  switch (c) {
#define QF_ROW_CASE(CC)                                                                           \
  case CC:                                                                                        \
    if constexpr (served_columns(CC, OUT == kOutSiluMul) && outputs_fit(R * CC)) {                \
      hipLaunchKernelGGL((row_gemv_kernel<R, CC, IN, OUT>), dim3(kGroups), dim3(kRowThreads),     \
                         lds, s, a);                                                              \
      return launch_status();                                                                     \
    }                                                                                             \
    return QF_E_SHAPE;
    QF_ROW_CASE(2)
    QF_ROW_CASE(4)
    QF_ROW_CASE(8)
    QF_ROW_CASE(10)
    QF_ROW_CASE(16)
    QF_ROW_CASE(24)
    QF_ROW_CASE(32)
    QF_ROW_CASE(76)
#undef QF_ROW_CASE
    default:
      return QF_E_SHAPE;
  }
}

template <int IN, int OUT>
int launch_rows(RowArgs a, size_t lds, hipStream_t s) {
  const int c = a.n / kGroups;
  switch (padded_rows(a.rows)) {
    case 1: return launch_rows_c<1, IN, OUT>(a, c, lds, s);
    case 2: return launch_rows_c<2, IN, OUT>(a, c, lds, s);
    default: return launch_rows_c<4, IN, OUT>(a, c, lds, s);
  }
}

// n: weight rows (2 n_out for SiLU * up).
int row_shape_status(int32_t rows, int64_t k, int64_t n, bool silu = false) {
  if (rows < 1 || rows > kMaxRows || k < 8 || k % 8 != 0 || k / 8 > INT32_MAX || n > INT32_MAX ||
      n < kGroups || n % kGroups != 0)
    return QF_E_SHAPE;
  const int64_t c = n / kGroups;
  return served_columns((int)c, silu) && outputs_fit(padded_rows(rows) * (int)c) ? QF_OK : QF_E_SHAPE;
}

RowArgs row_args(const void* x, int32_t rows, int64_t k, const void* weight, int64_t n, void* out) {
  RowArgs a = {};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(weight);
  a.k = k;
  a.rows = rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)(k / 8);
  a.out = static_cast<uint16_t*>(out);
  return a;
}

bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
bool eps_ok(float eps) { return eps == eps && eps >= 0.0f && eps != __builtin_inff(); }

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
  return launch_rows<kInPlain, kOutPlain>(row_args(x, rows, k, weight, n, out), 0, as_stream(stream));
}

extern "C" int qf_linear_residual(const void* x, int32_t rows, int64_t k, const void* weight,
                                  int64_t n, const void* residual, void* total, double* sq,
                                  void* stream) {
  const int st = row_shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!x || !weight || !residual || !total || !sq) return QF_E_ARG;
  if (!aligned16(x) || !aligned16(weight) || !aligned8(sq)) return QF_E_ALIGN;
  RowArgs a = row_args(x, rows, k, weight, n, total);
  a.residual = static_cast<const uint16_t*>(residual);
  a.sq_out = sq;
  return launch_rows<kInPlain, kOutResidual>(a, 0, as_stream(stream));
}

extern "C" int qf_linear_normed(const void* total, const double* sq, const void* gain, float eps,
                                int32_t rows, int64_t k, const void* weight, int64_t n, void* out,
                                void* stream) {
  const int st = row_shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!total || !sq || !gain || !weight || !out || !eps_ok(eps)) return QF_E_ARG;
  if (!aligned16(total) || !aligned16(gain) || !aligned16(weight) || !aligned8(sq)) return QF_E_ALIGN;
  RowArgs a = row_args(total, rows, k, weight, n, out);
  a.sq = sq;
  a.gain = static_cast<const uint16_t*>(gain);
  a.eps = eps;
  return launch_rows<kInNormed, kOutPlain>(a, 0, as_stream(stream));
}

extern "C" int qf_row_silu_supported(int32_t rows, int64_t k, int64_t n) {
  return n >= 1 && n <= INT32_MAX / 2 && row_shape_status(rows, k, 2 * n, true) == QF_OK ? 1 : 0;
}

extern "C" int qf_linear_silu_mul_normed(const void* total, const double* sq, const void* gain,
                                         float eps, int32_t rows, int64_t k, const void* gate_up,
                                         int64_t n, void* out, void* stream) {
  if (!qf_row_silu_supported(rows, k, n)) return QF_E_SHAPE;
  if (!total || !sq || !gain || !gate_up || !out || !eps_ok(eps)) return QF_E_ARG;
  if (!aligned16(total) || !aligned16(gain) || !aligned16(gate_up) || !aligned8(sq))
    return QF_E_ALIGN;
  RowArgs a = row_args(total, rows, k, gate_up, 2 * n, out);
  a.sq = sq;
  a.gain = static_cast<const uint16_t*>(gain);
  a.eps = eps;
  return launch_rows<kInNormed, kOutSiluMul>(a, 0, as_stream(stream));
}

extern "C" int qf_row_merged_supported(int32_t rows, int32_t segments, int32_t q_heads,
                                       int32_t kv_heads, int64_t n) {
  if (segments < 2 || segments > kMaxSegments || q_heads < 1 || kv_heads < 1 ||
      q_heads % kv_heads != 0 || q_heads > INT32_MAX / 128)
    return 0;
  const int64_t k = (int64_t)q_heads * 128;
  if (padded_rows(rows) * k * 2 > (64 << 10)) return 0;  // staged rows in LDS
  return row_shape_status(rows, k, n) == QF_OK ? 1 : 0;
}

extern "C" int qf_linear_residual_merged(const float* seg_partials, const float* seg_stats,
                                         int32_t segments, int32_t rows, int32_t q_heads,
                                         int32_t kv_heads, const void* weight, int64_t n,
                                         const void* residual, void* total, double* sq,
                                         void* stream) {
  if (!qf_row_merged_supported(rows, segments, q_heads, kv_heads, n)) return QF_E_SHAPE;
  if (!seg_partials || !seg_stats || !weight || !residual || !total || !sq) return QF_E_ARG;
  if (!aligned8(seg_partials) || !aligned16(weight) || !aligned8(sq)) return QF_E_ALIGN;
  const int64_t k = (int64_t)q_heads * 128;
  RowArgs a = row_args(nullptr, rows, k, weight, n, total);
  a.seg_partials = seg_partials;
  a.seg_stats = seg_stats;
  a.segments = segments;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.residual = static_cast<const uint16_t*>(residual);
  a.sq_out = sq;
  return launch_rows<kInMerged, kOutResidual>(a, (size_t)padded_rows(rows) * k * 2,
                                              as_stream(stream));
}
