// Decode projections y = x @ W^T for at most 64 rows of x, on the gfx950
// matrix cores (engine/kernels/skinny_gemm.py:28-121 is the reference:
// _partials_kernel :28-46, _silu_mul_kernel :49-72).
//
// A decode step multiplies a few rows by every layer weight, so each call is
// a weight stream: W ([N, K] bf16, K contiguous) is read once from HBM and x
// (at most 64 x K bf16) comes from L2.  The arithmetic is small next to the
// bytes (2*M flops per weight byte), but at M = 64 it is beyond what the VALU
// does at HBM speed, so every product runs on v_mfma_f32_16x16x32_bf16:
//
//   A operand = 16 rows of W (one n-tile), B operand = 16 rows of x (one
//   m-tile), 32 k per instruction.  Lane l holds A row (l % 16) and B column
//   (l % 16), k = 8*(l / 16) .. +8 of the step.  The f32 result lane l holds
//   is D[4*(l/16) + i][l % 16] = y[m0 + l%16][n0 + 4*(l/16) + i]: four
//   consecutive output columns of one x row, one 16-byte store.
//
// Loading W straight into that layout would make every 16 lanes of a load
// touch 16 different rows; HBM streams far better when each row is read a
// whole 128-byte line at a time.  So W moves in 64-wide k chunks: one
// 16-byte load per lane reads 8 rows x 128 contiguous bytes (two loads per
// 16-row tile), the wave writes the chunk to its own LDS staging tile
// (XOR-swizzled, conflict-free both ways) and reads it back in MFMA layout.  Only the wave itself touches its staging tile, so no
// workgroup barrier is needed in the loop.  Each wave keeps D chunks of loads
// in flight (software pipelined).
//
// A workgroup owns NT n-tiles and one K range (its split); its four waves
// take interleaved chunks of that range, so together they read consecutive
// bytes of every row, and reduce their f32 tiles through LDS in wave order.
// Rows of x beyond M are never stored.
//
// Two epilogues, as in the reference:
//   * qf_linear_partials: the workgroup's f32 tile is split `split`'s partial
//     [S, M, N]; the consumers (qf_add_rms_norm, qf_qkv_norm_rope_cache) add
//     the S partials in order and round once to bf16.  No atomics, no extra
//     reduction launch.
//   * qf_linear_silu_mul: the workgroup owns gate rows [c, c+16h) and the
//     matching up rows [N + c, ...) of the packed [2N, K] weight over all of
//     K, and writes bf16(bf16(silu(bf16(gate))) * bf16(up)).
//
// Numerics: bf16 x bf16 products are exact in f32; the MFMA adds them in f32
// in an order fixed by the hardware, and the wave hand-off adds the four
// waves' sums in wave order.  Results are deterministic run to run; they
// equal the exactly rounded dot product whenever every partial sum is an
// exactly representable f32 (e.g. integer inputs below 2^24), and otherwise
// differ from it by f32 accumulation error only.
#include <mutex>

#include "qf_device.h"
#include "qf_merge.h"
#include "qf_silu.h"

namespace qf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 16;    // rows of W (output columns) per n-tile; rows of x per m-tile
constexpr int kStep = 32;    // k per MFMA
constexpr int kChunk = 64;   // k per wave chunk; the shape rule's k granularity
constexpr int kWaves = kBlock / kWave;
constexpr int kMaxRows = 64;
constexpr int kColAlign = 32;  // N granularity of the shape rule

// Epilogues.
constexpr int kEpiPartials = 0;  // f32 split-K partials [S, M, N]
constexpr int kEpiSiluMul = 1;   // packed gate/up -> bf16 silu(gate) * up [M, N]
constexpr int kEpiArgmax = 2;    // bf16 logits (optional) + argmax candidates per 16-column tile

// Sources of x in skinny_kernel.
constexpr int kXDirect = 0;  // global loads straight into MFMA layout (up to 4 rows)
constexpr int kXStaged = 1;  // loaded like W, transposed through the wave's LDS tile
constexpr int kXMerged = 2;  // merged from attention segments into LDS by a prologue
constexpr int kXNormed = 3;  // RMSNorm of the residual stream, into LDS by a prologue
constexpr int kNormRows = 4; // most rows kXNormed takes (f64 sums of squares per thread)

// Is (v, i) ahead of (bv, bi) in argmax order: larger value, NaN above
// everything, the lower index on equal values (torch.argmax's first maximum)?
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

struct SkinnyArgs {
  const uint16_t* x;   // [m, k]
  const uint16_t* w;   // [n, k], or [2n, k] gate rows then up rows
  float* partials;     // [splits, m, n]; argmax: (value, index) pairs [m, workgroups]
  uint16_t* out;       // [m, n] (argmax: optional bf16 logits, may be null)
  int64_t k;
  int32_t m;
  int32_t n;           // output columns
  int32_t chunks;      // 64-wide k chunks per split
  int32_t splits_major; // 1: blockIdx.x is the split and blockIdx.y the column block
  // kXMerged only: x row m, columns [128 h, 128 h + 128), is the merge of the
  // attention segments of virtual head m * seg_kv_heads + h / seg_groups,
  // query group h % seg_groups (partials [V, S, G, 128], stats [V, S, 2, G]).
  const float* seg_partials;
  const float* seg_stats;
  int32_t seg_splits;
  int32_t seg_groups;
  int32_t seg_kv_heads;
  // kXNormed only: x (the residual stream `total`, bf16 [m, k]) enters as
  //   inv = 1 / sqrt(f32(sum_g sq[m][g]) / k + eps),  bf16(bf16(x * inv) * gain)
  // with sq f64 [m, QF_ROW_GROUPS] (per-workgroup sums of squares from
  // qf_linear_residual) and gain bf16 [k].
  const double* sq;
  const uint16_t* gain;
  float eps;
};

__device__ __forceinline__ f32x4 mfma(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Staging tiles: 128-byte rows, 16-byte piece c of row r stored at piece
// c ^ ((r >> 1) & 7).  Both access patterns then touch 16 distinct 16-byte
// bank groups per 16 lanes: the chunk loads' writes (rows r, r + 1, all
// eight pieces) and the MFMA-layout reads (rows 0..15, one piece).  Same
// bits as padded 144-byte rows, 2-3% faster at 64 rows.
constexpr int kLdsRow = kChunk * 2;            // staging row bytes
constexpr int kTileLds = kTile * kLdsRow;      // one 16-row staging tile
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kLdsRow + 16 * (chunk ^ ((row >> 1) & 7));
}
constexpr int kRowsPerLoad = kWave * 16 / (kChunk * 2);  // 8 rows x 128 B per load

// Wave hand-off and epilogue shared by the kernel variants: waves wk > 0 of
// each n-tile group pass their f32 tiles through LDS to wave wk = 0, which
// adds them in wave order and writes the partials, the SiLU * up product or
// the argmax candidates.  Called by every wave of the workgroup.
template <int MT, int NT, int WK, int EPI>
__device__ __forceinline__ void finish(const SkinnyArgs& a, f32x4 (&acc)[NT][MT], uint8_t* lds,
                                       int lane, int wk, int wn, int col0, bool live, int split) {
  constexpr bool PAIRS = EPI == kEpiSiluMul;
  constexpr bool HALF = PAIRS && NT == 1;  // one tile: 8 gate rows over 8 up rows
  constexpr int kCols = PAIRS ? NT / 2 : NT;
  const int r = lane % kTile;
  const int g = lane / kTile;
  // Waves wk = 1..WK-1 of each group hand their tiles to the group's wave
  // wk = 0, which adds them in wave order.
  if constexpr (WK > 1) {
    __syncthreads();
    f32x4* handoff = reinterpret_cast<f32x4*>(lds);
    constexpr int kPer = NT * MT * kWave;
    if (wk > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          handoff[(wn * (WK - 1) + wk - 1) * kPer + (t * MT + mt) * kWave + lane] = acc[t][mt];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll
    for (int w = 0; w < WK - 1; ++w)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[t][mt] += handoff[(wn * (WK - 1) + w) * kPer + (t * MT + mt) * kWave + lane];
  }

  if constexpr (EPI == kEpiArgmax) {
    // bf16 logits of this wave's 16*NT columns; per row and 16-column tile
    // the largest, lowest column on ties (NaN counts as largest), reduced
    // over the four lanes that hold a row of the tile (all lanes take part in
    // the shuffles); one candidate per row and tile.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = kTile * mt + r;
      const bool row_ok = live && m < a.m;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        float best = -__builtin_inff();
        int besti = INT32_MAX;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = from_bf16(to_bf16(acc[t][mt][i]));
          const int col = col0 + kTile * t + 4 * g + i;
          if (better(v[i], col, best, besti)) {
            best = v[i];
            besti = col;
          }
        }
        if (row_ok && a.out)
          *reinterpret_cast<uint2*>(a.out + (int64_t)m * a.n + col0 + kTile * t + 4 * g) =
              make_uint2(pack2(v[0], v[1]), pack2(v[2], v[3]));
#pragma unroll
        for (int mask = 16; mask <= 32; mask *= 2) {
          const float ov = __shfl_xor(best, mask);
          const int oi = __shfl_xor(besti, mask);
          if (better(ov, oi, best, besti)) {
            best = ov;
            besti = oi;
          }
        }
        if (row_ok && g == 0) {
          uint2* cand = reinterpret_cast<uint2*>(a.partials) + (int64_t)m * (a.n / kTile) +
                        col0 / kTile + t;
          *cand = make_uint2(__float_as_uint(best), (uint32_t)besti);
        }
      }
    }
    return;
  }
  if (!live) return;
  if constexpr (!PAIRS) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = kTile * mt + r;
      if (m >= a.m) continue;
      float* dst = a.partials + ((int64_t)split * a.m + m) * a.n + col0 + 4 * g;
#pragma unroll
      for (int t = 0; t < NT; ++t) *reinterpret_cast<f32x4*>(dst + kTile * t) = acc[t][mt];
    }
  } else if constexpr (HALF) {
    // Lanes of groups g = 0, 1 hold gate columns col0 + 4g .. +4; groups
    // 2, 3 the matching up columns, fetched across the wave's halves.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float up[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) up[i] = __shfl_xor(acc[0][mt][i], 32);
      const int m = kTile * mt + r;
      if (g >= 2 || m >= a.m) continue;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float gate = from_bf16(to_bf16(acc[0][mt][i]));
        y[i] = from_bf16(to_bf16(silu_f32(gate))) * from_bf16(to_bf16(up[i]));
      }
      *reinterpret_cast<uint2*>(a.out + (int64_t)m * a.n + col0 + 4 * g) =
          make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = kTile * mt + r;
      if (m >= a.m) continue;
      uint16_t* dst = a.out + (int64_t)m * a.n + col0 + 4 * g;
#pragma unroll
      for (int h = 0; h < kCols; ++h) {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // Each projection is a bf16 tensor in the reference; SiLU is
          // rounded to bf16 before the bf16 product.
          const float gate = from_bf16(to_bf16(acc[h][mt][i]));
          const float up = from_bf16(to_bf16(acc[kCols + h][mt][i]));
          y[i] = from_bf16(to_bf16(silu_f32(gate))) * up;
        }
        *reinterpret_cast<uint2*>(dst + kTile * h) = make_uint2(pack2(y[0], y[1]), pack2(y[2], y[3]));
      }
    }
  }
}

// MT m-tiles of x (M <= 16*MT); NT n-tiles of W per wave (for PAIRS the
// first NT/2 are gate tiles, the rest the matching up tiles; a single PAIRS
// tile holds 8 gate rows over the matching 8 up rows, its two 8-row loads
// taken from the two halves of the weight); the four waves
// form WN = 4/WK groups of distinct n-tiles, each group WK waves that split
// the chunks; D chunks in flight per wave; NTL = nontemporal weight loads;
// XS = source of x (kXDirect, kXStaged, kXMerged, kXNormed).  Waves of
// different groups read the same x chunk at about the same time, so x is
// fetched from L2 once per workgroup rather than once per wave.
//
// kXMerged (MT = 1): the workgroup's x slice, M rows x (chunks * 64)
// columns = whole heads of the attention output, is merged from the
// attention segments by the workgroup itself into dynamic LDS (row stride
// chunks * 128 + 16 bytes), one wave per (row, head), after the first D
// weight chunks are issued, so the merge's loads overlap the weight loads.
// kXNormed (M <= kNormRows): the same slice, normalised from the residual
// stream with qf_add_rms_norm's rounding steps (inverse RMS from the
// producer's per-workgroup sums of squares) into the same LDS layout, PPT
// 16-byte pieces per thread.  MFMA operands and their order are those of
// kXDirect: a normalised x equal to qf_add_rms_norm's output gives the bits
// of qf_linear_partials / qf_linear_silu_mul on it.
template <int MT, int NT, int WK, int D, int EPI, bool NTL, int XS, int PPT = 0>
__global__ __launch_bounds__(kBlock) void skinny_kernel(SkinnyArgs a) {
  constexpr bool PAIRS = EPI == kEpiSiluMul;
  constexpr bool HALF = PAIRS && NT == 1;
  constexpr bool XT = XS == kXStaged;
  constexpr bool XM = XS == kXMerged;
  constexpr bool XN = XS == kXNormed;
  constexpr bool XL = XM || XN;  // x read from the prologue's LDS slice
  static_assert(kWaves % WK == 0, "wave split");
  static_assert(!XL || MT == 1, "an LDS x slice holds at most 16 rows");
  static_assert(!XN || (kBlock == QF_ROW_GROUPS && PPT >= 1), "normed x: one sum per thread and row");
  constexpr int WN = kWaves / WK;
  constexpr int kCols = PAIRS ? NT / 2 : NT;  // output n-tiles per wave
  constexpr int kColW = HALF ? kTile / 2 : kTile * kCols;  // output columns per wave
  constexpr int kStageTiles = NT + (XT ? MT : 0);
  constexpr int kStageBytes = kWaves * kStageTiles * kTileLds;
  constexpr int kHandoffBytes = WN * (WK - 1) * NT * MT * kWave * 16;
  __shared__ __attribute__((aligned(16)))
      uint8_t lds[kStageBytes > kHandoffBytes ? kStageBytes : kHandoffBytes];
  extern __shared__ __attribute__((aligned(16))) uint8_t xm_lds[];
  __shared__ double xn_wsum[XN ? kWaves : 1][kNormRows];

  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int r = lane % kTile;
  const int g = lane / kTile;
  const int wk = wave % WK;  // position among the waves sharing n-tiles
  const int wn = wave / WK;  // n-tile group
  const int col0 = ((a.splits_major ? blockIdx.y : blockIdx.x) * WN + wn) * kColW;
  const bool live = col0 < a.n;  // the last workgroup's groups may lie past N
  const int split = a.splits_major ? blockIdx.x : blockIdx.y;
  const int64_t kbase = (int64_t)split * a.chunks * kChunk;

  // Chunk loads: lane reads row (lane / 8) + 8*i of the tile, 16 bytes at
  // column 8 * (lane % 8) of the chunk (a half-pair tile: gate row
  // col0 + lane / 8, then the up row n further on).
  const uint16_t* wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int row = col0 + kTile * t;
    if (PAIRS && !HALF && t >= kCols) row = a.n + col0 + kTile * (t - kCols);
    wp[t] = a.w + (int64_t)(row + lane / 8) * a.k + kbase + 8 * (lane % 8);
  }
  const int64_t wstep = HALF ? (int64_t)a.n * a.k : (int64_t)kRowsPerLoad * a.k;
  // Lanes of x rows beyond M read row 0 instead: the MFMA keeps every
  // output column separate, and those columns are never stored.
  const uint16_t* xp[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if constexpr (XT) {  // coalesced like W, transposed through LDS
        const int row = kTile * mt + kRowsPerLoad * i + lane / 8;
        xp[mt][i] = a.x + (int64_t)(row < a.m ? row : 0) * a.k + kbase + 8 * (lane % 8);
      } else if constexpr (!XL) {  // straight into MFMA layout
        const int row = kTile * mt + r;
        xp[mt][i] = a.x + (int64_t)(row < a.m ? row : 0) * a.k + kbase + 8 * g + kStep * i;
      }
    }
  uint8_t* stage = lds + wave * kStageTiles * kTileLds;
  const int wr_off[2] = {lds_off(lane / 8, lane % 8), lds_off(lane / 8 + kRowsPerLoad, lane % 8)};
  const int rd_off[2] = {lds_off(r, g), lds_off(r, g + 4)};
  const int xm_row = a.chunks * kChunk * 2 + 16;
  const int xm_off = (r < a.m ? r : 0) * xm_row + 16 * g;

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 wv[D][NT][2], xv[D][MT][2];
  // This wave's chunks are wk, wk + WK, ...: n_own of them.
  const int n_own = live && a.chunks > wk ? (a.chunks - wk + WK - 1) / WK : 0;

  auto issue = [&](int d, int j) {
    const int64_t off = (int64_t)(wk + WK * j) * kChunk;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 2; ++i) wv[d][t][i] = load16<NTL>(wp[t] + off + i * wstep);
    if constexpr (!XL) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 2; ++i) xv[d][mt][i] = load16<false>(xp[mt][i] + off);
    }
  };
  // The normed-x prologue: 16-byte piece p of the slice is row p / per_row,
  // columns kbase + 8 * (p % per_row) .. +8.  Thread t loads sq[q][t] of
  // every row q and its PPT pieces t, t + 256, ... (x and gain) before the
  // first weight loads - a fixed count with no branch, so the waits below
  // cover only these loads and the weight chunks stay in flight; pieces past
  // the slice re-read piece 0 and are not stored.  After the weight loads the
  // f64 sums are reduced (in wave, then wave order through LDS: exact) and
  // the pieces normalised into the LDS slice.
  const int xn_per_row = a.chunks * (kChunk / 8);
  const int xn_pieces = XN ? a.m * xn_per_row : 0;
  double sqv[XN ? kNormRows : 1];
  uint4 xnv[XN ? PPT : 1], gnv[XN ? PPT : 1];
  auto norm_first = [&]() {
    if constexpr (XN) {
#pragma unroll
      for (int q = 0; q < kNormRows; ++q)
        sqv[q] = a.sq[(int64_t)(q < a.m ? q : 0) * QF_ROW_GROUPS + threadIdx.x];
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int p = (int)threadIdx.x + kBlock * i;
        const int pc = p < xn_pieces ? p : 0;
        const int row = pc / xn_per_row, col = pc - row * xn_per_row;
        xnv[i] = load16<false>(a.x + (int64_t)row * a.k + kbase + 8 * col);
        gnv[i] = load16<false>(a.gain + kbase + 8 * col);
      }
    }
  };
  auto norm_x = [&]() {
    if constexpr (XN) {
#pragma unroll
      for (int q = 0; q < kNormRows; ++q) sqv[q] = group_sum_f64<kWave>(sqv[q]);
      if (lane == 0) {
#pragma unroll
        for (int q = 0; q < kNormRows; ++q) xn_wsum[wave][q] = sqv[q];
      }
      __syncthreads();
      float inv[kNormRows];
#pragma unroll
      for (int q = 0; q < kNormRows; ++q) {
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) sum += xn_wsum[w][q];
        inv[q] = inv_rms(sum, (float)a.k, a.eps);
      }
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int p = (int)threadIdx.x + kBlock * i;
        const int row = p / xn_per_row, col = p - row * xn_per_row;
        float iv = inv[0];
#pragma unroll
        for (int q = 1; q < kNormRows; ++q) iv = row == q ? inv[q] : iv;
        // The rounding steps of qf_add_rms_norm: bf16(bf16(t * inv) * gain).
        float f[8], gf[8];
        unpack8(xnv[i], f);
        unpack8(gnv[i], gf);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= iv;
        round8(f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] *= gf[e];
        if (p < xn_pieces) *reinterpret_cast<uint4*>(xm_lds + row * xm_row + 16 * col) = pack8(f);
      }
      __syncthreads();
    }
  };
  // The merged-x prologue: wave w merges (row, head) pairs w, w + 4, ... of
  // the split's K range.  The first pair's loads are issued before the
  // weight loads (merge_first, from the pipeline) and combined after them
  // (merge_x), so the merge overlaps the weight fetch.  Every thread of the
  // workgroup takes part.
  const int heads = XM ? a.chunks * kChunk / 128 : 0;  // heads in this split's K range
  const int q0 = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform by construction
  SegmentLoads<> seg;
  auto pair = [&](int q, int64_t& vh, int& g, int& off) {
    const int m = q / heads, hl = q - m * heads, h = (int)(kbase / 128) + hl;
    vh = (int64_t)m * a.seg_kv_heads + h / a.seg_groups;
    g = h % a.seg_groups;
    off = m * xm_row + hl * 256;
  };
  auto merge_first = [&]() {
    if constexpr (XM) {
      if (q0 < a.m * heads) {
        int64_t vh; int g, off;
        pair(q0, vh, g, off);
        merge_issue(seg, a.seg_partials, a.seg_stats, vh, a.seg_splits, a.seg_groups, g, lane);
      }
    }
  };
  auto merge_x = [&]() {
    if constexpr (XM) {
      for (int q = q0; q < a.m * heads; q += kWaves) {
        int64_t vh; int g, off;
        pair(q, vh, g, off);
        if (q != q0) merge_issue(seg, a.seg_partials, a.seg_stats, vh, a.seg_splits, a.seg_groups, g, lane);
        reinterpret_cast<uint32_t*>(xm_lds + off)[lane] =
            merge_finish(seg, a.seg_partials, vh, a.seg_splits, a.seg_groups, g, lane);
      }
      __syncthreads();
    }
  };
  auto consume = [&](int d, int j) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        *reinterpret_cast<uint4*>(stage + t * kTileLds + wr_off[i]) =
            wv[d][t][i];
    if constexpr (XT) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          *reinterpret_cast<uint4*>(stage + (NT + mt) * kTileLds + wr_off[i]) =
              xv[d][mt][i];
    }
    wave_lds_fence();
    uint4 fw[NT][2], fx[MT][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        fw[t][s] = *reinterpret_cast<const uint4*>(stage + t * kTileLds + rd_off[s]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (XT)
          fx[mt][s] = *reinterpret_cast<const uint4*>(stage + (NT + mt) * kTileLds + rd_off[s]);
        else if constexpr (XL)
          fx[mt][s] = *reinterpret_cast<const uint4*>(xm_lds + xm_off + (wk + WK * j) * kChunk * 2 + s * kStep * 2);
        else
          fx[mt][s] = xv[d][mt][s];
      }
    }
    wave_lds_fence();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma(fw[t][s], fx[mt][s], acc[t][mt]);
  };

  // Software pipeline with D chunks in flight.  The steady-state loop issues
  // unconditionally, so the compiler's wait counts stay exact (each consume
  // waits only for its own chunk); only the last 2*D chunks take branches.
  merge_first();
  norm_first();
  if (n_own >= D) {
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    merge_x();
    norm_x();
    int j = 0;
    for (; j + 2 * D <= n_own; j += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        consume(d, j + d);
        issue(d, j + d + D);
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(d, j + d);
      if (j + d + D < n_own) issue(d, j + d + D);
    }
    j += D;
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (j + d < n_own) consume(d, j + d);
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < n_own) issue(d, d);
    merge_x();
    norm_x();
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < n_own) consume(d, d);
  }

  finish<MT, NT, WK, EPI>(a, acc, lds, lane, wk, wn, col0, live, split);
}

// Variant for 17..64 rows of x, where re-reading x dominates: with the
// waves of a workgroup splitting K, every workgroup reads its whole x slice
// from L2 for only 16*NT output columns.  Here the WN = 4 / WK wave groups
// take distinct n-tiles of the same chunks, and the workgroup stages each x
// chunk once, cooperatively and coalesced, in a shared LDS ring of two
// buffers (one barrier per step: a buffer is rewritten only after every wave
// has passed the barrier that follows its last read).  A step covers WK
// chunks, one per wave of a group; W still goes through each wave's private
// staging tile.  All waves run the same number of steps (chunks % WK == 0);
// waves whose n-tiles lie past N stream row 0 and store nothing.
template <int MT, int NT, int WK, int D, int EPI, bool NTL>
__global__ __launch_bounds__(kBlock) void skinny_xs_kernel(SkinnyArgs a) {
  constexpr bool PAIRS = EPI == kEpiSiluMul;
  static_assert(!PAIRS || NT % 2 == 0, "gate/up tiles come in pairs here");
  static_assert(kWaves % WK == 0, "wave split");
  constexpr int WN = kWaves / WK;
  constexpr int kCols = PAIRS ? NT / 2 : NT;
  constexpr int kRows = kTile * MT;                       // staged x rows (M padded)
  constexpr int kPieces = WK * kRows * (kChunk * 2 / 16);  // 16-byte pieces per step
  constexpr int XL = (kPieces + kBlock - 1) / kBlock;      // x loads per thread per step
  constexpr int kXStep = WK * kRows * kLdsRow;             // one ring buffer
  constexpr int kWStage = kWaves * NT * kTileLds;
  constexpr int kStageBytes = 2 * kXStep + kWStage;
  constexpr int kHandoffBytes = WN * (WK - 1) * NT * MT * kWave * 16;
  __shared__ __attribute__((aligned(16)))
      uint8_t lds[kStageBytes > kHandoffBytes ? kStageBytes : kHandoffBytes];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int r = lane % kTile;
  const int g = lane / kTile;
  const int wk = wave % WK;
  const int wn = wave / WK;
  const int col0 = ((a.splits_major ? blockIdx.y : blockIdx.x) * WN + wn) * (kTile * kCols);
  const bool live = col0 < a.n;
  const int split = a.splits_major ? blockIdx.x : blockIdx.y;
  const int64_t kbase = (int64_t)split * a.chunks * kChunk;

  const uint16_t* wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int row = col0 + kTile * t;
    if (PAIRS && t >= kCols) row = a.n + col0 + kTile * (t - kCols);
    if (!live) row = 0;
    wp[t] = a.w + (int64_t)(row + lane / 8) * a.k + kbase + 8 * (lane % 8);
  }
  const int64_t wstep = (int64_t)kRowsPerLoad * a.k;

  // Piece p = tid + 256 i of a step: chunk wk' = p / (8 kRows) of the step,
  // x row (p / 8) % kRows (row 0 stands in for rows past M), 16 bytes at
  // column 8 * (p % 8) of the chunk.
  const uint16_t* xp[XL];
  int xoff[XL];
  bool xon[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int p = tid + kBlock * i;
    xon[i] = p < kPieces;
    const int pc = xon[i] ? p : 0;
    const int wkp = pc / (8 * kRows);
    const int row = (pc / 8) % kRows;
    xp[i] = a.x + (int64_t)(row < a.m ? row : 0) * a.k + kbase + (int64_t)wkp * kChunk + 8 * (pc % 8);
    xoff[i] = lds_off(wkp * kRows + row, pc % 8);
  }
  uint8_t* xring = lds;
  uint8_t* stage = lds + 2 * kXStep + wave * NT * kTileLds;
  const int wr_off[2] = {lds_off(lane / 8, lane % 8), lds_off(lane / 8 + kRowsPerLoad, lane % 8)};
  const int rd_off[2] = {lds_off(r, g), lds_off(r, g + 4)};
  const int xrd_base = wk * kRows * kLdsRow;  // rows of a multiple of 16 keep the swizzle

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  uint4 wv[D][NT][2], xv[D][XL];
  const int steps = a.chunks / WK;  // the same for every wave

  auto issue = [&](int d, int j) {
    const int64_t off = (int64_t)(wk + WK * j) * kChunk;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 2; ++i) wv[d][t][i] = load16<NTL>(wp[t] + off + i * wstep);
    const int64_t xstep = (int64_t)WK * j * kChunk;
#pragma unroll
    for (int i = 0; i < XL; ++i) xv[d][i] = xon[i] ? load16<false>(xp[i] + xstep) : make_uint4(0, 0, 0, 0);
  };
  auto consume = [&](int d, int j) {
    uint8_t* xb = xring + (j & 1) * kXStep;
#pragma unroll
    for (int i = 0; i < XL; ++i)
      if (xon[i]) *reinterpret_cast<uint4*>(xb + xoff[i]) = xv[d][i];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 2; ++i)
        *reinterpret_cast<uint4*>(stage + t * kTileLds + wr_off[i]) =
            wv[d][t][i];
    __syncthreads();
    uint4 fw[NT][2], fx[MT][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        fw[t][s] = *reinterpret_cast<const uint4*>(stage + t * kTileLds + rd_off[s]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        fx[mt][s] = *reinterpret_cast<const uint4*>(xb + xrd_base + mt * kTileLds + rd_off[s]);
    }
    wave_lds_fence();
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma(fw[t][s], fx[mt][s], acc[t][mt]);
  };

  // The same software pipeline as skinny_kernel, D steps in flight.
  if (steps >= D) {
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, d);
    int j = 0;
    for (; j + 2 * D <= steps; j += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        consume(d, j + d);
        issue(d, j + d + D);
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
      consume(d, j + d);
      if (j + d + D < steps) issue(d, j + d + D);
    }
    j += D;
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (j + d < steps) consume(d, j + d);
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < steps) issue(d, d);
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (d < steps) consume(d, d);
  }

  finish<MT, NT, WK, EPI>(a, acc, lds, lane, wk, wn, col0, live, split);
}

// ---- launch plans -----------------------------------------------------------

int shape_status(int64_t rows, int64_t k, int64_t n) {
  if (rows < 1 || rows > kMaxRows || k <= 0 || n <= 0) return QF_E_SHAPE;
  if (k % kChunk != 0 || n % kColAlign != 0) return QF_E_SHAPE;
  if (k > (int64_t)INT32_MAX || n > (int64_t)INT32_MAX / 2) return QF_E_SHAPE;
  return QF_OK;
}

// Shared-x wave layout for 17..64 rows (measured on the Qwen3-4B shapes at
// M = 32 and 64 over tile widths 1-4, wave splits and split counts): each
// wave all of its workgroup's K range (WK = 1), four steps in flight, and two
// n-tiles per wave (128 columns per workgroup, half the x re-reads of one)
// while the grid stays within one workgroup per CU, else one tile.  A CU
// keeps a bounded number of L1 misses in flight, so the stream needs the
// workgroups spread over all CUs more than it needs the fewest x re-reads.
constexpr int64_t kPlanCUs = 256;  // MI355X compute units
struct XsPlan {
  int nt, wk, d;
};
XsPlan xs_plan(int64_t n, int64_t splits) {
  const int64_t wide = (n + 8 * kTile - 1) / (8 * kTile) * splits;
  return wide <= kPlanCUs ? XsPlan{2, 1, 4} : XsPlan{1, 1, 4};
}

// Power-of-two K splits (measured on the Qwen3-4B projection shapes).  Up to
// 16 rows: as many as keep every wave at least one chunk, the grid at most
// 3072 workgroups of 16 columns (~12 per CU), and the partials (written here,
// read by the consumer) small: splits * min(M, 16) <= K / 32, at most 8 (o_proj
// takes the same time at 8 and 16 splits, and its consumer, one workgroup per
// row, reads half the bytes).  Beyond 16 rows (shared-x kernel): K ranges
// of at most 512 (eight chunks) per workgroup, the fewest splits that give
// them (Qwen3-4B: qkv 5, o_proj 8, down 19 splits; 10-17% faster at 32 and
// 64 rows than ~150 workgroups of longer ranges, consumers included).
int plan_splits(int64_t rows, int64_t k, int64_t n) {
  const int64_t chunks = k / kChunk;
  const int64_t mrows = rows < kTile ? rows : kTile;
  int64_t s = 1;
  if (rows > kTile) {
    while (chunks / s > 8 || chunks % s != 0) ++s;
    return (int)s;
  }
  const int64_t tiles = n / kTile;
  while (s < 8 && chunks % (2 * s) == 0 && chunks / (2 * s) >= kWaves && tiles * 2 * s <= 3072 &&
         2 * s * mrows <= k / 32)
    s *= 2;
  return (int)s;
}

// Grid order: workgroups are dispatched x-fastest.  Where K is at least N
// (o_proj, down) the splits of one column block go in consecutive
// workgroups, so the grid streams each weight row's K ranges together
// (measured with the Qwen3-4B weights: o_proj 6.40 -> 6.05 us at 16 rows,
// down 10.01 -> 9.44 at one row and 14.97 -> 14.71 at 64; same bits); qkv
// (K < N) keeps column blocks fastest (6.83 against 6.88 us at one row).
dim3 skinny_grid(SkinnyArgs& a, int64_t grid_x, int splits) {
  a.splits_major = splits > 1 && a.k >= a.n && grid_x <= 65535 ? 1 : 0;
  return a.splits_major ? dim3((unsigned)splits, (unsigned)grid_x)
                        : dim3((unsigned)grid_x, (unsigned)splits);
}

template <int MT, int NT, int WK, int D, int EPI, bool NTL, int XS, int PPT = 0>
int launch(const SkinnyArgs& args, int splits, hipStream_t s, size_t dyn_lds = 0) {
  constexpr bool PAIRS = EPI == kEpiSiluMul;
  constexpr int kColsPerBlock =
      (PAIRS && NT == 1 ? kTile / 2 : kTile * (PAIRS ? NT / 2 : NT)) * (kWaves / WK);
  SkinnyArgs a = args;
  const int64_t grid_x = (a.n + kColsPerBlock - 1) / kColsPerBlock;
  const dim3 grid = skinny_grid(a, grid_x, splits);
  hipLaunchKernelGGL((skinny_kernel<MT, NT, WK, D, EPI, NTL, XS, PPT>), grid, dim3(kBlock),
                     dyn_lds, s, a);
  return launch_status();
}

// The normed-x kernels, instantiated for 1..kMaxPiecesPerThread slice pieces
// per thread (the prologue's loads are a fixed count).
constexpr int kMaxPiecesPerThread = 5;  // 4 rows x 2560 columns of slice
template <int D, int EPI>
int launch_normed(const SkinnyArgs& a, int splits, hipStream_t s) {
  const int64_t pieces = (int64_t)a.m * a.chunks * (kChunk / 8);
  const size_t lds = (size_t)a.m * (size_t)(a.chunks * kChunk * 2 + 16);
  switch ((pieces + kBlock - 1) / kBlock) {
    case 1: return launch<1, 1, 4, D, EPI, true, kXNormed, 1>(a, splits, s, lds);
    case 2: return launch<1, 1, 4, D, EPI, true, kXNormed, 2>(a, splits, s, lds);
    case 3: return launch<1, 1, 4, D, EPI, true, kXNormed, 3>(a, splits, s, lds);
    case 4: return launch<1, 1, 4, D, EPI, true, kXNormed, 4>(a, splits, s, lds);
    case 5: return launch<1, 1, 4, D, EPI, true, kXNormed, 5>(a, splits, s, lds);
    default: return QF_E_SHAPE;
  }
}

template <int MT, int NT, int WK, int D, int EPI>
int launch_xs(const SkinnyArgs& args, int splits, hipStream_t s) {
  constexpr int kColsPerBlock = kTile * (EPI == kEpiSiluMul ? NT / 2 : NT) * (kWaves / WK);
  SkinnyArgs a = args;
  const int64_t grid_x = (a.n + kColsPerBlock - 1) / kColsPerBlock;
  const dim3 grid = skinny_grid(a, grid_x, splits);
  hipLaunchKernelGGL((skinny_xs_kernel<MT, NT, WK, D, EPI, true>), grid, dim3(kBlock), 0, s, a);
  return launch_status();
}

template <int MT>
int dispatch_xs_partials(const SkinnyArgs& a, const XsPlan& p, int splits, hipStream_t s) {
  if (p.nt == 2) return launch_xs<MT, 2, 1, 4, kEpiPartials>(a, splits, s);
  return launch_xs<MT, 1, 1, 4, kEpiPartials>(a, splits, s);
}

// Tile plans (measured): up to 4 rows of x arrive as one broadcast line per
// load, so x goes straight into MFMA layout; up to 16 x is loaded like W and
// transposed through LDS by each wave; beyond 16 rows the shared-x kernel
// stages each x chunk once per workgroup (the plain kernel remains for
// splits whose chunk count does not divide into the plan's steps).
int dispatch_partials(const SkinnyArgs& a, int splits, hipStream_t s) {
  const int mt = (a.m + kTile - 1) / kTile;
  if (mt > 1) {
    const XsPlan p = xs_plan(a.n, splits);
    if (a.chunks % p.wk == 0) {
      if (mt == 2) return dispatch_xs_partials<2>(a, p, splits, s);
      if (mt == 3) return dispatch_xs_partials<3>(a, p, splits, s);
      return dispatch_xs_partials<4>(a, p, splits, s);
    }
  }
  switch (mt) {
    case 1:
      if (a.m <= 4) return launch<1, 1, 4, 2, kEpiPartials, true, kXDirect>(a, splits, s);
      if (a.n / kTile >= 256) return launch<1, 2, 4, 2, kEpiPartials, true, kXStaged>(a, splits, s);
      return launch<1, 1, 4, 2, kEpiPartials, true, kXStaged>(a, splits, s);
    case 2: return launch<2, 2, 4, 2, kEpiPartials, true, kXStaged>(a, splits, s);
    case 3: return launch<3, 2, 4, 2, kEpiPartials, true, kXStaged>(a, splits, s);
    default: return launch<4, 2, 4, 2, kEpiPartials, true, kXStaged>(a, splits, s);
  }
}

// Gate/up + SiLU: all of K per workgroup.  Up to 12 rows one tile of 8 gate
// over 8 up rows per workgroup (1,216 workgroups for Qwen3-4B: 10% faster at
// 1-4 rows than a gate and an up tile per wave, whose 608 larger workgroups
// leave the stream's end unbalanced, 4% at 9-10 rows, even at 12-14, 1%
// slower at 16; same bits); 13..16 rows the tile pair; beyond 16 rows one
// gate and one up tile per wave, four waves sharing each staged x chunk.
int dispatch_silu(const SkinnyArgs& a, hipStream_t s) {
  switch ((a.m + kTile - 1) / kTile) {
    case 1:
      if (a.m <= 4) return launch<1, 1, 4, 4, kEpiSiluMul, true, kXDirect>(a, 1, s);
      if (a.m <= 12) return launch<1, 1, 4, 4, kEpiSiluMul, true, kXStaged>(a, 1, s);
      return launch<1, 2, 4, 4, kEpiSiluMul, true, kXStaged>(a, 1, s);
    case 2: return launch_xs<2, 2, 1, 4, kEpiSiluMul>(a, 1, s);
    case 3: return launch_xs<3, 2, 1, 4, kEpiSiluMul>(a, 1, s);
    default: return launch_xs<4, 2, 1, 4, kEpiSiluMul>(a, 1, s);
  }
}

// Final argmax over a row's candidates: one 1024-thread workgroup per row,
// each thread four candidates in flight per round (9,496 candidates for
// Qwen3-4B: three rounds instead of 37 loads in turn per thread).  The
// order (larger value, NaN largest, then the lower index) is total, so the
// reduction order does not change the result.
constexpr int kFinThreads = 1024;
constexpr int kFinUnroll = 4;
// With `position` set, workgroup 0 also advances the decode position and
// the per-head lengths by one (the step's last writes, in the same launch).
__global__ __launch_bounds__(kFinThreads) void argmax_finalize_kernel(const uint2* cand,
                                                                     int64_t blocks,
                                                                     int64_t* tokens,
                                                                     int64_t* position,
                                                                     int32_t* lengths,
                                                                     int64_t length_count) {
  if (position != nullptr && blockIdx.x == 0) {
    if (threadIdx.x == 0) position[0] += 1;
    for (int64_t i = threadIdx.x; i < length_count; i += kFinThreads) lengths[i] += 1;
  }
  __shared__ float wv[kFinThreads / kWave];
  __shared__ int wi[kFinThreads / kWave];
  const int64_t row = blockIdx.x;
  const uint2* c = cand + row * blocks;
  float best = -__builtin_inff();
  int besti = INT32_MAX;
  for (int64_t j0 = threadIdx.x; j0 < blocks; j0 += (int64_t)kFinThreads * kFinUnroll) {
    uint2 v[kFinUnroll];
#pragma unroll
    for (int u = 0; u < kFinUnroll; ++u) {
      const int64_t j = j0 + (int64_t)u * kFinThreads;
      v[u] = j < blocks ? c[j] : make_uint2(__float_as_uint(-__builtin_inff()), (uint32_t)INT32_MAX);
    }
#pragma unroll
    for (int u = 0; u < kFinUnroll; ++u) {
      const float val = __uint_as_float(v[u].x);
      const int idx = (int)v[u].y;
      if (better(val, idx, best, besti)) {
        best = val;
        besti = idx;
      }
    }
  }
#pragma unroll
  for (int mask = 1; mask < kWave; mask *= 2) {
    const float ov = __shfl_xor(best, mask);
    const int oi = __shfl_xor(besti, mask);
    if (better(ov, oi, best, besti)) {
      best = ov;
      besti = oi;
    }
  }
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) {
    wv[wave] = best;
    wi[wave] = besti;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kFinThreads / kWave; ++w)
      if (better(wv[w], wi[w], best, besti)) {
        best = wv[w];
        besti = wi[w];
      }
    tokens[row] = besti;
  }
}

// LM head plans (measured on the Qwen3-4B head, 151936 x 2560, at 1, 4, 8,
// 16, 32 and 64 rows): up to 4 rows x straight into MFMA layout with four
// chunks in flight (two n-tiles per wave from 2 rows); 5..16 rows the
// shared-x kernel with two n-tiles per wave and wave pairs splitting K (20%
// faster at 16 rows than per-wave x staging); beyond 16 rows two n-tiles
// per wave, each wave all of K (10% faster at 32 rows and 18% at 64 than one
// tile: every workgroup re-reads x, so wider workgroups halve that traffic).
// Two-tile plans need vocab % 32 == 0.
int dispatch_argmax(const SkinnyArgs& a, hipStream_t s) {
  const bool two = a.n % (2 * kTile) == 0;
  switch ((a.m + kTile - 1) / kTile) {
    case 1:
      // Up to 4 rows (x as broadcast lines): one 16-column tile per
      // workgroup, the most workgroups (Qwen3-4B head at 2 and 3 rows: 117.8
      // -> 114.8 and 118.3 -> 115.7 us against two tiles; even at 4).
      if (a.m <= 4) return launch<1, 1, 4, 4, kEpiArgmax, true, kXDirect>(a, 1, s);
      if (!two) return launch_xs<1, 1, 1, 4, kEpiArgmax>(a, 1, s);
      // 5-16 rows share each staged x chunk among the waves: 32 columns per
      // workgroup (two wave groups of one tile) up to 8 rows, 128 (four
      // groups of two) beyond, where x's re-reads weigh more (measured on
      // the Qwen3-4B head against 64 columns: 122.6 -> 119.1 us at 5 rows,
      // 124.5 -> 122.3 at 8, 129.0 -> 126.0 at 16).
      if (a.m <= 8) return launch_xs<1, 1, 2, 4, kEpiArgmax>(a, 1, s);
      return launch_xs<1, 2, 1, 4, kEpiArgmax>(a, 1, s);
    case 2: return two ? launch_xs<2, 2, 1, 4, kEpiArgmax>(a, 1, s) : launch_xs<2, 1, 1, 4, kEpiArgmax>(a, 1, s);
    case 3: return two ? launch_xs<3, 2, 1, 4, kEpiArgmax>(a, 1, s) : launch_xs<3, 1, 1, 4, kEpiArgmax>(a, 1, s);
    default: return two ? launch_xs<4, 2, 1, 4, kEpiArgmax>(a, 1, s) : launch_xs<4, 1, 1, 4, kEpiArgmax>(a, 1, s);
  }
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int64_t qf_lm_head_blocks(int64_t vocab) {
  return vocab > 0 && vocab % kTile == 0 ? vocab / kTile : QF_E_SHAPE;
}

namespace qf {
namespace {
// Host checks of the LM head arguments other than the candidate buffer.
int lm_head_status(const void* x, int64_t rows, int64_t k, const void* weight, int64_t vocab,
                   const int64_t* tokens, const void* logits) {
  if (rows < 1 || rows > kMaxRows || k <= 0 || k % kChunk != 0 || k > (int64_t)INT32_MAX ||
      vocab <= 0 || vocab % kTile != 0 || vocab > (int64_t)INT32_MAX / 2)
    return QF_E_SHAPE;
  if (!x || !weight || !tokens) return QF_E_ARG;
  if (!aligned16(x) || !aligned16(weight) || (reinterpret_cast<uintptr_t>(logits) & 7u) != 0)
    return QF_E_ALIGN;
  return QF_OK;
}
}  // namespace
}  // namespace qf

namespace {

int lm_head_argmax(const void* x, int64_t rows, int64_t k, const void* weight, int64_t vocab,
                   void* candidates, int64_t* tokens, void* logits, int64_t* position,
                   int32_t* lengths, int64_t length_count, void* stream) {
  const int checked = lm_head_status(x, rows, k, weight, vocab, tokens, logits);
  if (checked != QF_OK) return checked;
  if (!candidates) return QF_E_ARG;
  if ((reinterpret_cast<uintptr_t>(candidates) & 7u) != 0) return QF_E_ALIGN;
  SkinnyArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(weight);
  a.partials = static_cast<float*>(candidates);
  a.out = static_cast<uint16_t*>(logits);
  a.k = k;
  a.m = (int32_t)rows;
  a.n = (int32_t)vocab;
  a.chunks = (int32_t)(k / kChunk);
  hipStream_t s = as_stream(stream);
  const int st = dispatch_argmax(a, s);
  if (st != QF_OK) return st;
  hipLaunchKernelGGL(argmax_finalize_kernel, dim3((unsigned)rows), dim3(kFinThreads), 0, s,
                     static_cast<const uint2*>(candidates), vocab / kTile, tokens, position,
                     lengths, length_count);
  return launch_status();
}

}  // namespace

extern "C" int qf_lm_head_argmax(const void* x, int64_t rows, int64_t k, const void* weight,
                                 int64_t vocab, void* candidates, int64_t* tokens, void* logits,
                                 void* stream) {
  return lm_head_argmax(x, rows, k, weight, vocab, candidates, tokens, logits, nullptr, nullptr, 0,
                        stream);
}

extern "C" int qf_lm_head_argmax_advance(const void* x, int64_t rows, int64_t k,
                                         const void* weight, int64_t vocab, void* candidates,
                                         int64_t* tokens, void* logits, int64_t* position,
                                         int32_t* lengths, int64_t length_count, void* stream) {
  if (!position || length_count < 0 || (length_count > 0 && !lengths)) return QF_E_ARG;
  if ((reinterpret_cast<uintptr_t>(position) & 7u) != 0 ||
      (reinterpret_cast<uintptr_t>(lengths) & 3u) != 0)
    return QF_E_ALIGN;
  return lm_head_argmax(x, rows, k, weight, vocab, candidates, tokens, logits, position, lengths,
                        length_count, stream);
}

// Candidate scratch of qf_lm_head_argmax_static: a file-scope device array,
// one copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): each device's address comes from hipGetSymbolAddress, taken once
// per device with that device current, and only that address is used.
static __device__ __align__(256) uint2 scratch[QF_LM_HEAD_STATIC_SLOTS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

// The address of `scratch` on the device `stream` belongs to (the current
// device for the null stream); nullptr and a status on failure.  The lookup
// runs with that device current - hipGetSymbolAddress answers for the current
// device - and the caller's current device is restored afterwards.
void* scratch_address(hipStream_t stream, int* status) {
  int current = 0;
  hipError_t e = hipGetDevice(&current);
  int dev = current;
  if (e == hipSuccess && stream != nullptr) e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) {
    *status = static_cast<int>(e);
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *status = QF_E_ARG;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    if (dev != current && (e = hipSetDevice(dev)) != hipSuccess) {
      *status = static_cast<int>(e);
      return nullptr;
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t restored = dev != current ? hipSetDevice(current) : hipSuccess;
    if (e == hipSuccess) e = restored;
    if (e != hipSuccess || ptr == nullptr) {
      *status = e != hipSuccess ? static_cast<int>(e) : QF_E_ARG;
      return nullptr;
    }
    g_scratch[dev] = ptr;
  }
  *status = QF_OK;
  return g_scratch[dev];
}
}  // namespace

extern "C" int qf_lm_head_argmax_static(const void* x, int64_t rows, int64_t k,
                                        const void* weight, int64_t vocab, int64_t* tokens,
                                        void* logits, void* stream) {
  const int checked = lm_head_status(x, rows, k, weight, vocab, tokens, logits);
  if (checked != QF_OK) return checked;
  if (rows * (vocab / kTile) > QF_LM_HEAD_STATIC_SLOTS) return QF_E_CAPACITY;
  int status = QF_OK;
  void* candidates = scratch_address(static_cast<hipStream_t>(stream), &status);
  if (candidates == nullptr) return status;
  // Every candidate slot the finalize kernel reads is written first by the
  // projection's epilogue, so nothing left by an earlier call is read.
  return qf_lm_head_argmax(x, rows, k, weight, vocab, candidates, tokens, logits, stream);
}

extern "C" int qf_linear_splits(int64_t rows, int64_t k, int64_t n) {
  const int st = shape_status(rows, k, n);
  return st != QF_OK ? st : plan_splits(rows, k, n);
}

extern "C" int qf_linear_partials(const void* x, int64_t rows, int64_t k, const void* weight,
                                  int64_t n, int32_t splits, void* partials, void* stream) {
  const int st = shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!x || !weight || !partials) return QF_E_ARG;
  if (splits < 1 || (k / kChunk) % splits != 0) return QF_E_ARG;
  if (!aligned16(x) || !aligned16(weight) || !aligned16(partials)) return QF_E_ALIGN;
  SkinnyArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(weight);
  a.partials = static_cast<float*>(partials);
  a.out = nullptr;
  a.k = k;
  a.m = (int32_t)rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)(k / kChunk / splits);
  return dispatch_partials(a, splits, as_stream(stream));
}

extern "C" int qf_linear_partials_merged(const float* seg_partials, const float* seg_stats,
                                         int32_t seg_splits, int64_t batch, int32_t q_heads,
                                         int32_t kv_heads, const void* weight, int64_t n,
                                         int32_t splits, void* partials, void* stream) {
  if (batch < 1 || batch > kTile || q_heads < 1 || kv_heads < 1 || q_heads % kv_heads != 0 ||
      q_heads / kv_heads > 16)
    return QF_E_SHAPE;
  const int64_t k = (int64_t)q_heads * 128;
  const int st = shape_status(batch, k, n);
  if (st != QF_OK) return st;
  if (!seg_partials || !seg_stats || !weight || !partials) return QF_E_ARG;
  if (seg_splits < 2 || seg_splits > kMaxSegments) return QF_E_ARG;
  if (splits < 1 || (k / kChunk) % splits != 0 || (k / kChunk / splits) % 2 != 0) return QF_E_ARG;
  const int64_t chunks = k / kChunk / splits;
  const size_t lds = (size_t)batch * (size_t)(chunks * kChunk * 2 + 16);
  if (lds > (64u << 10)) return QF_E_SHAPE;
  if ((reinterpret_cast<uintptr_t>(seg_partials) & 7u) != 0 ||
      (reinterpret_cast<uintptr_t>(seg_stats) & 3u) != 0 || !aligned16(weight) ||
      !aligned16(partials))
    return QF_E_ALIGN;
  SkinnyArgs a;
  a.x = nullptr;
  a.w = static_cast<const uint16_t*>(weight);
  a.partials = static_cast<float*>(partials);
  a.out = nullptr;
  a.k = k;
  a.m = (int32_t)batch;
  a.n = (int32_t)n;
  a.chunks = (int32_t)chunks;
  a.seg_partials = seg_partials;
  a.seg_stats = seg_stats;
  a.seg_splits = seg_splits;
  a.seg_groups = q_heads / kv_heads;
  a.seg_kv_heads = kv_heads;
  // The same tile plan (and so the same f32 addition order) as
  // qf_linear_partials for up to 16 rows: one 16-row x tile, four waves
  // splitting each workgroup's chunks, two chunks in flight.
  return launch<1, 1, 4, 2, kEpiPartials, true, kXMerged>(a, splits, as_stream(stream), lds);
}

namespace qf {
namespace {
// Checks and arguments shared by the normed-input entry points.
int normed_args(SkinnyArgs& a, const void* total, const double* sq, const void* gain, float eps,
                int64_t rows, int64_t k, const void* weight, int64_t n, int64_t chunks) {
  const int st = shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (rows > kNormRows || rows * chunks * (kChunk / 8) > (int64_t)kMaxPiecesPerThread * kBlock)
    return QF_E_SHAPE;
  if (!total || !sq || !gain || !weight) return QF_E_ARG;
  if (!(eps == eps) || eps < 0.0f || eps == __builtin_inff()) return QF_E_ARG;
  if (!aligned16(total) || !aligned16(gain) || !aligned16(weight) ||
      (reinterpret_cast<uintptr_t>(sq) & 7u) != 0)
    return QF_E_ALIGN;
  a = SkinnyArgs{};
  a.x = static_cast<const uint16_t*>(total);
  a.w = static_cast<const uint16_t*>(weight);
  a.k = k;
  a.m = (int32_t)rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)chunks;
  a.sq = sq;
  a.gain = static_cast<const uint16_t*>(gain);
  a.eps = eps;
  return QF_OK;
}
}  // namespace
}  // namespace qf

extern "C" int qf_linear_partials_normed(const void* total, const double* sq, const void* gain,
                                         float eps, int64_t rows, int64_t k, const void* weight,
                                         int64_t n, int32_t splits, void* partials, void* stream) {
  if (splits < 1 || k <= 0 || k % kChunk != 0 || (k / kChunk) % splits != 0) return QF_E_ARG;
  SkinnyArgs a;
  const int st = normed_args(a, total, sq, gain, eps, rows, k, weight, n, k / kChunk / splits);
  if (st != QF_OK) return st;
  if (!partials) return QF_E_ARG;
  if (!aligned16(partials)) return QF_E_ALIGN;
  a.partials = static_cast<float*>(partials);
  // qf_linear_partials' plan for up to 4 rows (the same tiles, waves and
  // chunks in flight, so the same f32 addition order).
  return launch_normed<2, kEpiPartials>(a, splits, as_stream(stream));
}

extern "C" int qf_linear_silu_mul_normed_tiled(const void* total, const double* sq,
                                               const void* gain, float eps, int64_t rows,
                                               int64_t k, const void* gate_up, int64_t n,
                                               void* out, void* stream) {
  if (k <= 0 || k % kChunk != 0) return QF_E_SHAPE;
  SkinnyArgs a;
  const int st = normed_args(a, total, sq, gain, eps, rows, k, gate_up, n, k / kChunk);
  if (st != QF_OK) return st;
  if (!out) return QF_E_ARG;
  if ((reinterpret_cast<uintptr_t>(out) & 7u) != 0) return QF_E_ALIGN;
  a.out = static_cast<uint16_t*>(out);
  // qf_linear_silu_mul's plan for up to 4 rows: 8 gate over 8 up rows per
  // workgroup, four waves splitting K, four chunks in flight.
  return launch_normed<4, kEpiSiluMul>(a, 1, as_stream(stream));
}

extern "C" int qf_linear_silu_mul(const void* x, int64_t rows, int64_t k, const void* gate_up,
                                  int64_t n, void* out, void* stream) {
  const int st = shape_status(rows, k, n);
  if (st != QF_OK) return st;
  if (!x || !gate_up || !out) return QF_E_ARG;
  if (!aligned16(x) || !aligned16(gate_up) || (reinterpret_cast<uintptr_t>(out) & 7u) != 0)
    return QF_E_ALIGN;
  SkinnyArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(gate_up);
  a.partials = nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.k = k;
  a.m = (int32_t)rows;
  a.n = (int32_t)n;
  a.chunks = (int32_t)(k / kChunk);
  return dispatch_silu(a, as_stream(stream));
}
