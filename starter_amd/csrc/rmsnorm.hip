// RMSNorm and residual-add + RMSNorm for gfx950.
//
// Arithmetic (engine/kernels/rmsnorm.py:19-36, engine/kernels/decode_fused.py:26-44;
// Qwen3RMSNorm.forward in transformers models/qwen3/modeling_qwen3.py):
//   total  = bf16(float(residual) + float(branch))          (add variant only)
//   var    = f32(sum(float(t)^2)) / cols   (squares exact in f32, summed exactly in f64)
//   n      = bf16(float(t) * (1 / sqrt(var + eps)))          (IEEE sqrt and divide)
//   out    = bf16(float(n) * float(w))
// Split-K branch: branch = bf16(((0 + p0) + p1) + ... ) in f32, in split order.
//
// Layout: a group of LPR lanes owns one row; lane i holds the 16-byte vectors
// i, i+LPR, ..., so each wave-wide load instruction covers LPR*16 contiguous
// bytes.  The row stays in registers between the reduction and the output, so
// every input byte is read once and every output byte written once.  The sum
// of squares is reduced in f64 with DPP inside 16-lane rows and ds_bpermute
// across them; no LDS allocation and no barrier.  Split-K partials (decode)
// take rms_partials_kernel, one workgroup per row.  Rows that are whole
// multiples of 64 vectors (plain or bf16-branch add) take rms_stream_kernel:
// every load (gain included) issued before the first store, several rows per
// wave with nontemporal accesses for large calls, one row per wave with
// cached accesses for decode sizes.
#include "qf_device.h"

namespace qf {
namespace {

struct RmsArgs {
  const uint16_t* x;       // residual (add) or input rows (plain)
  const void* branch;      // bf16 [rows, cols] or f32 [splits, rows, cols]
  const uint16_t* w;
  uint16_t* total;         // add variant only
  uint16_t* out;
  int64_t rows, cols;
  int64_t inner, outer_stride, inner_stride;  // plain variant row walk
  int64_t split_stride;    // rows * cols
  int32_t splits;
  int32_t nvec;            // cols / 8
  float eps;
};

template <bool ADD>
__device__ __forceinline__ const uint16_t* row_base(const RmsArgs& a, int64_t r) {
  if constexpr (ADD) {
    return a.x + r * a.cols;
  } else {
    return a.x + (r / a.inner) * a.outer_stride + (r % a.inner) * a.inner_stride;
  }
}

// Vector path: cols % 8 == 0 and every pointer / row stride 16-byte aligned.
// MODE: 0 = plain RMSNorm, 1 = add a bf16 branch, 2 = add f32 split-K partials.
// A wave owns RPW rows (LPR == 64) and issues all of their loads before any
// arithmetic; NT selects nontemporal row loads / stores for large calls.
template <int LPR, int VPL, int MODE, int RPW, bool NT>
__global__ __launch_bounds__(kBlock) void rms_vec_kernel(RmsArgs a) {
  constexpr bool ADD = MODE != 0;
  constexpr int kRowsPerBlock = kBlock / LPR * RPW;
  const int lane = threadIdx.x % LPR;
  const int64_t row0 = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x / LPR) * RPW;

  uint4 xv[RPW][VPL], bv[RPW][VPL];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool live = row < a.rows;
    const uint4* xin = reinterpret_cast<const uint4*>(row_base<ADD>(a, live ? row : 0));
    const uint4* bin = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.branch) +
                                                      (live ? row : 0) * a.cols);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + k * LPR;
      const bool on = live && v < a.nvec;
      xv[r][k] = on ? load16<NT>(xin + v) : make_uint4(0, 0, 0, 0);
      if constexpr (MODE == 1) bv[r][k] = on ? load16<NT>(bin + v) : make_uint4(0, 0, 0, 0);
    }
  }

#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool live = row < a.rows;
    const int64_t rr = live ? row : 0;
    float t[VPL][8];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + k * LPR;
      const bool on = live && v < a.nvec;
      unpack8(xv[r][k], t[k]);
      if constexpr (ADD) {
        float y[8];
        if constexpr (MODE == 1) {
          unpack8(bv[r][k], y);
        } else {
          // f32 partials: two 16-byte halves per 8 columns, summed in split order.
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = 0.0f;
          const float* p = static_cast<const float*>(a.branch) + rr * a.cols + (int64_t)v * 8;
          for (int s = 0; s < a.splits; ++s) {
            const uint4 p0 = on ? load16<NT>(p) : make_uint4(0, 0, 0, 0);
            const uint4 p1 = on ? load16<NT>(p + 4) : make_uint4(0, 0, 0, 0);
            y[0] += __uint_as_float(p0.x); y[1] += __uint_as_float(p0.y);
            y[2] += __uint_as_float(p0.z); y[3] += __uint_as_float(p0.w);
            y[4] += __uint_as_float(p1.x); y[5] += __uint_as_float(p1.y);
            y[6] += __uint_as_float(p1.z); y[7] += __uint_as_float(p1.w);
            p += a.split_stride;
          }
          round8(y);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) t[k][j] += y[j];
        const uint4 tv = pack8(t[k]);
        unpack8(tv, t[k]);
        if (on) store16<NT>(reinterpret_cast<uint4*>(a.total + rr * a.cols) + v, tv);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += (double)(t[k][j] * t[k][j]);
    }

    const float inv = inv_rms(group_sum_f64<LPR>(ss), (float)a.cols, a.eps);
    const uint4* wv = reinterpret_cast<const uint4*>(a.w);
    uint4* o = reinterpret_cast<uint4*>(a.out + rr * a.cols);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + k * LPR;
      const bool on = live && v < a.nvec;
      float n[8], w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) n[j] = t[k][j] * inv;
      round8(n);
      unpack8(on ? wv[v] : make_uint4(0, 0, 0, 0), w);
#pragma unroll
      for (int j = 0; j < 8; ++j) n[j] *= w[j];
      if (on) store16<NT>(o + v, pack8(n));
    }
  }
}

// MODE 0 or 1, rows of at most 16 vectors per lane: R rows of one wave (R > 1
// for large calls, NT = nontemporal accesses; R = 1 with cached accesses for
// decode sizes), with every load issued before the first store - the gain
// first, then each row's inputs.  gfx950 counts loads and stores on one in-order
// counter, so a load issued after a store can only be waited for together
// with that store; here every wait covers older loads only, and row r's
// arithmetic starts while rows r+1.. are still arriving.  Loads are
// unconditional (a lane past the row end re-reads the row's last vector and
// contributes zero), so the compiler has no branch to sink them under.
template <int VPL, int R, int MODE, bool FULL, bool NT>
__device__ __forceinline__ void stream_rows(const RmsArgs& a, int64_t row0, int64_t rstride,
                                            int lane) {
  constexpr bool ADD = MODE == 1;
  const int last = a.nvec - 1;
  const uint4* wv4 = reinterpret_cast<const uint4*>(a.w);
  uint4 wv[VPL], xv[R][VPL], bv[R][VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    wv[k] = wv4[FULL || v < a.nvec ? v : last];
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint4* xin = reinterpret_cast<const uint4*>(row_base<ADD>(a, row0 + r * rstride));
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + k * kWave;
      const int vv = FULL || v < a.nvec ? v : last;
      xv[r][k] = load16<NT>(xin + vv);
      if constexpr (ADD) {
        const uint4* bin = reinterpret_cast<const uint4*>(
            static_cast<const uint16_t*>(a.branch) + (row0 + r * rstride) * a.cols);
        bv[r][k] = load16<NT>(bin + vv);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t row = row0 + r * rstride;
    float t[VPL][8];
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + k * kWave;
      const bool on = FULL || v < a.nvec;
      unpack8(xv[r][k], t[k]);
      if constexpr (ADD) {
        float y[8];
        unpack8(bv[r][k], y);
#pragma unroll
        for (int j = 0; j < 8; ++j) t[k][j] += y[j];
        const uint4 tv = pack8(t[k]);
        unpack8(tv, t[k]);
        if (on) store16<NT>(reinterpret_cast<uint4*>(a.total + row * a.cols) + v, tv);
      }
      if (!on) {
#pragma unroll
        for (int j = 0; j < 8; ++j) t[k][j] = 0.0f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += (double)(t[k][j] * t[k][j]);
    }
    const float inv = inv_rms(group_sum_f64<kWave>(ss), (float)a.cols, a.eps);
    uint4* o = reinterpret_cast<uint4*>(a.out + row * a.cols);
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = lane + k * kWave;
      float n[8], w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) n[j] = t[k][j] * inv;
      round8(n);
      unpack8(wv[k], w);
#pragma unroll
      for (int j = 0; j < 8; ++j) n[j] *= w[j];
      if (FULL || v < a.nvec) store16<NT>(o + v, pack8(n));
    }
  }
}

// A wave takes RPW rows, run by run (ILV false: rows RPW w .. RPW w + RPW - 1)
// or interleaved: the grid's waves go in rounds of kCUs * 4 waves (one 4-wave
// workgroup per CU), and wave i of a round of n waves takes rows base + i,
// base + i + n, .., base + i + (RPW - 1) n, so each round streams one
// contiguous front of rows.  A wave whose last row would run past a.rows
// takes its rows one at a time.
// WPB: waves per workgroup (4, or 1 for decode sizes).
template <int VPL, int RPW, int MODE, bool FULL, bool NT = true, bool ILV = false,
          int WPB = kBlock / kWave>
__global__ __launch_bounds__(kBlock) void rms_stream_kernel(RmsArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t w = __builtin_amdgcn_readfirstlane(
      (int64_t)blockIdx.x * WPB + threadIdx.x / kWave);
  int64_t row0 = w * RPW, step = 1;
  if constexpr (ILV) {
    constexpr int64_t kRound = (int64_t)kCUs * WPB;
    const int64_t waves = (int64_t)gridDim.x * WPB;
    const int64_t q = w / kRound;
    step = waves - q * kRound < kRound ? waves - q * kRound : kRound;
    row0 = q * kRound * RPW + w % kRound;
  }
  if (row0 + (RPW - 1) * step < a.rows) {
    stream_rows<VPL, RPW, MODE, FULL, NT>(a, row0, step, lane);
  } else {
    for (int64_t row = row0; row < a.rows; row += step)  // wave-uniform
      stream_rows<VPL, 1, MODE, FULL, NT>(a, row, step, lane);
  }
}

// Element value entering the norm: x, or bf16(x + branch) for the add variant.
template <bool ADD>
__device__ __forceinline__ float scalar_value(const RmsArgs& a, const uint16_t* x, int64_t row,
                                              int64_t c) {
  float t = from_bf16(x[c]);
  if constexpr (ADD) {
    float y;
    if (a.splits == 0) {
      y = from_bf16(static_cast<const uint16_t*>(a.branch)[row * a.cols + c]);
    } else {
      const float* p = static_cast<const float*>(a.branch) + row * a.cols + c;
      y = 0.0f;
      for (int s = 0; s < a.splits; ++s) y += p[(int64_t)s * a.split_stride];
      y = from_bf16(to_bf16(y));
    }
    t = from_bf16(to_bf16(t + y));
  }
  return t;
}

// Scalar path for any width / alignment: one wave per row, two passes over
// the inputs (the second recomputes the element instead of reading back the
// stored sum).  Only odd shapes take it.
template <bool ADD>
__global__ __launch_bounds__(kBlock) void rms_scalar_kernel(RmsArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
  if (row >= a.rows) return;  // wave-uniform
  const uint16_t* x = row_base<ADD>(a, row);
  double ss = 0.0;
  for (int64_t c = lane; c < a.cols; c += kWave) {
    const float t = scalar_value<ADD>(a, x, row, c);
    if constexpr (ADD) a.total[row * a.cols + c] = to_bf16(t);
    ss += (double)(t * t);
  }
  const float inv = inv_rms(group_sum_f64<kWave>(ss), (float)a.cols, a.eps);
  for (int64_t c = lane; c < a.cols; c += kWave) {
    const float n = from_bf16(to_bf16(scalar_value<ADD>(a, x, row, c) * inv));
    a.out[row * a.cols + c] = to_bf16(n * from_bf16(a.w[c]));
  }
}

template <int LPR, int VPL, int MODE, int RPW, bool NT>
int launch_rows(const RmsArgs& a, hipStream_t s) {
  constexpr int64_t per_block = kBlock / LPR * RPW;
  const int64_t blocks = (a.rows + per_block - 1) / per_block;
  hipLaunchKernelGGL((rms_vec_kernel<LPR, VPL, MODE, RPW, NT>), dim3((unsigned)blocks), dim3(kBlock),
                     0, s, a);
  return launch_status();
}

// Large calls stream with nontemporal accesses and, for rows of at most five
// vectors per lane (<= 2560 columns) with a bf16 or no branch, two rows per
// wave; decode-size calls keep one row per wave and cached accesses.
// Interleaved rows (ILV) for rows of at most five vectors per lane once the
// grid fills every CU, measured on the residual add + norm: [8192, 2560]
// 28.2 -> 27.0 us, [16384, 2560] 62.8 -> 59.3, [32768, 2560] 126.4 -> 120.3,
// [4096, 2560] 14.2 -> 13.9; wider rows ([8192, 4096]: 45.5 -> 48.1) and
// grids under one workgroup per CU ([3000, 2560]: 11.2 -> 12.2) keep runs.
template <int VPL, int RPW, int MODE>
int launch_stream(const RmsArgs& a, hipStream_t s) {
  constexpr int64_t per_block = kBlock / kWave * RPW;
  const int64_t blocks = (a.rows + per_block - 1) / per_block;
  if (VPL <= 5 && RPW > 1 && blocks >= kCUs)
    hipLaunchKernelGGL((rms_stream_kernel<VPL, RPW, MODE, true, true, true>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, s, a);
  else
    hipLaunchKernelGGL((rms_stream_kernel<VPL, RPW, MODE, true>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, s, a);
  return launch_status();
}

// Large calls whose rows are whole multiples of 64 vectors take
// rms_stream_kernel with the fewest rows per wave (1, 2, 4 or 8, at most 40
// vectors of each input per lane) that keep the grid within one 4-wave
// workgroup per CU.  Measured on the [8192, 2560] residual add + norm: 8 rows
// per wave (256 workgroups) 28.5 us against 29.0 us for rms_vec_kernel's two
// rows per wave; rows that end mid-vector-group keep rms_vec_kernel, which
// was faster for them.
template <int VPL, int MODE>
int launch_full_stream(const RmsArgs& a, hipStream_t s) {
  constexpr int kMaxRows = 40 / VPL >= 8 ? 8 : 40 / VPL >= 4 ? 4 : 40 / VPL >= 2 ? 2 : 1;
  const int64_t waves_per_grid = (int64_t)kCUs * (kBlock / kWave);
  int rows = 1;
  while (rows < kMaxRows && (int64_t)rows * waves_per_grid < a.rows) rows *= 2;
  switch (rows) {
    case 1: return launch_stream<VPL, 1, MODE>(a, s);
    case 2: return launch_stream<VPL, (kMaxRows >= 2 ? 2 : 1), MODE>(a, s);
    case 4: return launch_stream<VPL, (kMaxRows >= 4 ? 4 : 1), MODE>(a, s);
    default: return launch_stream<VPL, kMaxRows, MODE>(a, s);
  }
}

template <int LPR, int VPL, int MODE>
int launch_vec(const RmsArgs& a, hipStream_t s) {
  const int64_t bytes = a.rows * a.cols * 2 * (MODE == 0 ? 2 : 4);
  if (bytes < kStreamBytes) {
    // Decode sizes: one row per wave, cached accesses; whole-group rows take
    // the loads-before-stores kernel with one wave per workgroup, so the rows
    // spread over as many CUs as there are rows (the 36-call [64, 2560]
    // add + norm chain: 2.89 -> 2.66 us per call against four waves per
    // workgroup; [16, 2560] 2.84 -> 2.62).
    if constexpr (LPR == 64 && MODE != 2) {
      if (a.nvec == VPL * kWave) {
        hipLaunchKernelGGL((rms_stream_kernel<VPL, 1, MODE, true, false, false, 1>),
                           dim3((unsigned)a.rows), dim3(kWave), 0, s, a);
        return launch_status();
      }
    }
    return launch_rows<LPR, VPL, MODE, 1, false>(a, s);
  }
  if constexpr (LPR == 64 && MODE != 2)
    if (a.nvec == VPL * kWave) return launch_full_stream<VPL, MODE>(a, s);
  if constexpr (LPR == 64 && VPL <= 5 && MODE != 2) return launch_rows<LPR, VPL, MODE, 2, true>(a, s);
  return launch_rows<LPR, VPL, MODE, 1, true>(a, s);
}

// Residual add of f32 split-K partials + RMSNorm for decode-size calls: one
// workgroup per row, one thread per 16-byte vector of the row (cols / 8 <= 1024
// threads), up to P partials of a vector loaded before any is added (split
// order kept), the f64 sum of squares reduced across waves through LDS in
// wave order (exact, so order-free).  A wave-per-row kernel would walk the
// splits one memory latency at a time for each of its vectors.
template <int P, int MAXT, int FIXED = 0>
__global__ __launch_bounds__(MAXT) void rms_partials_kernel(RmsArgs a) {
  __shared__ double wave_sums[MAXT / kWave];
  __shared__ double row_sum;
  const int64_t row = blockIdx.x;
  const int v = threadIdx.x;
  // Every argument the loads need is fetched in one round of scalar loads
  // (the empty asm takes them all as operands): left to itself the compiler
  // fetches the struct's fields in three dependent rounds, between the first
  // global loads.
  const uint16_t* x = a.x;
  const uint16_t* gain = a.w;
  const float* branch = static_cast<const float*>(a.branch);
  const int64_t cols = a.cols, split_stride = a.split_stride;
  const int splits = FIXED ? FIXED : a.splits;
  const int nvec = a.nvec;
  asm volatile("" ::"s"(x), "s"(gain), "s"(branch), "s"(cols), "s"(split_stride), "s"(splits),
               "s"(nvec));
  const bool on = v < nvec;
  const int vi = on ? v : 0;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  // The gain is loaded first: a load issued after the total store below
  // could only be waited for together with that store (one in-order counter).
  // Loads are unconditional (vi keeps idle lanes in range; their values are
  // zeroed below), so no exec-mask branch separates them.
  const uint4 wv = reinterpret_cast<const uint4*>(gain)[vi];
  const uint4 xv = load16<false>(reinterpret_cast<const uint4*>(x + row * cols) + vi);
  float y[8], t[8];
  sum_partials8<P>(branch + row * cols + (int64_t)vi * 8, split_stride, splits, true, y);
  round8(y);
  unpack8(xv, t);
  if (!on) {
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = t[j] = 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) t[j] += y[j];
  const uint4 tv = pack8(t);
  unpack8(tv, t);
  if (on) store16<false>(reinterpret_cast<uint4*>(a.total + row * a.cols) + v, tv);
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += (double)(t[j] * t[j]);
  ss = group_sum_f64<kWave>(ss);
  if (lane == 0) wave_sums[wave] = ss;
  __syncthreads();
  if (threadIdx.x == 0) {
    double tot = 0.0;
    for (int w = 0; w < (int)(blockDim.x / kWave); ++w) tot += wave_sums[w];
    row_sum = tot;
  }
  __syncthreads();
  if (!on) return;
  const float inv = inv_rms(row_sum, (float)a.cols, a.eps);
  float n[8], w[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] = t[j] * inv;
  round8(n);
  unpack8(wv, w);
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] *= w[j];
  store16<false>(reinterpret_cast<uint4*>(a.out + row * a.cols) + v, pack8(n));
}

template <int MODE>
int dispatch(RmsArgs a, bool vec_ok, hipStream_t s) {
  constexpr bool ADD = MODE != 0;
  if (a.rows == 0) return QF_OK;
  if (vec_ok) {
    a.nvec = (int32_t)(a.cols / 8);
    const int nv = a.nvec;
    if (MODE == 2 && nv <= 1024 && a.rows <= (int64_t)UINT32_MAX) {
      // 16 partials in flight per thread up to 4096 columns (512 threads);
      // 8 beyond, where 1024 threads leave 128 registers each.
      // 8 splits (every split-K projection of the engine up to 16 rows, and
      // o_proj beyond) and 19 (the down projection beyond 16 rows) take
      // instantiations with the count fixed: their loads issue with no branch
      // between them (10.5 -> 10.2 us per Qwen3-4B add+norm + qkv pair at batch 1).
      const int threads = (nv + kWave - 1) / kWave * kWave;
      if (nv <= 512 && a.splits == 8)
        hipLaunchKernelGGL((rms_partials_kernel<8, 512, 8>), dim3((unsigned)a.rows), dim3(threads), 0, s, a);
      else if (nv <= 512 && a.splits == 19)
        hipLaunchKernelGGL((rms_partials_kernel<19, 512, 19>), dim3((unsigned)a.rows), dim3(threads), 0, s, a);
      else if (nv <= 512)
        hipLaunchKernelGGL((rms_partials_kernel<16, 512>), dim3((unsigned)a.rows), dim3(threads), 0, s, a);
      else
        hipLaunchKernelGGL((rms_partials_kernel<8, 1024>), dim3((unsigned)a.rows), dim3(threads), 0, s, a);
      return launch_status();
    }
    if (nv <= 8) return launch_vec<8, 1, MODE>(a, s);
    if (nv <= 16) return launch_vec<16, 1, MODE>(a, s);
    if (nv <= 32) return launch_vec<32, 1, MODE>(a, s);
    switch ((nv + 63) / 64) {
      case 1: return launch_vec<64, 1, MODE>(a, s);
      case 2: return launch_vec<64, 2, MODE>(a, s);
      case 3: return launch_vec<64, 3, MODE>(a, s);
      case 4: return launch_vec<64, 4, MODE>(a, s);
      case 5: return launch_vec<64, 5, MODE>(a, s);
      case 6: return launch_vec<64, 6, MODE>(a, s);
      case 7: return launch_vec<64, 7, MODE>(a, s);
      case 8: return launch_vec<64, 8, MODE>(a, s);
      case 9: case 10: return launch_vec<64, 10, MODE>(a, s);
      case 11: case 12: return launch_vec<64, 12, MODE>(a, s);
      case 13: case 14: return launch_vec<64, 14, MODE>(a, s);
      case 15: case 16: return launch_vec<64, 16, MODE>(a, s);
      default: break;  // wider than 8192 columns: the scalar path handles any width
    }
  }
  const int64_t blocks = (a.rows + 3) / 4;
  hipLaunchKernelGGL((rms_scalar_kernel<ADD>), dim3((unsigned)blocks), dim3(kBlock), 0, s, a);
  return launch_status();
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int qf_rms_norm(const void* x, int64_t rows, int64_t cols, int64_t inner,
                           int64_t outer_stride, int64_t inner_stride,
                           const void* weight, float eps, void* out, void* stream) {
  if (rows < 0 || cols <= 0 || inner <= 0) return QF_E_ARG;
  if (rows == 0) return QF_OK;
  if (!x || !weight || !out) return QF_E_ARG;
  if (rows > (int64_t)UINT32_MAX * 4) return QF_E_SHAPE;
  RmsArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(weight);
  a.out = static_cast<uint16_t*>(out);
  a.rows = rows;
  a.cols = cols;
  a.inner = inner;
  a.outer_stride = outer_stride;
  a.inner_stride = inner_stride;
  a.eps = eps;
  const bool vec_ok = cols % 8 == 0 && outer_stride % 8 == 0 && inner_stride % 8 == 0 &&
                      aligned16(x) && aligned16(weight) && aligned16(out);
  return dispatch<0>(a, vec_ok, as_stream(stream));
}

extern "C" int qf_add_rms_norm(const void* residual, const void* branch, int32_t splits,
                               const void* weight, int64_t rows, int64_t cols, float eps,
                               void* total, void* normed, void* stream) {
  if (rows < 0 || cols <= 0 || splits < 0) return QF_E_ARG;
  if (rows == 0) return QF_OK;
  if (!residual || !branch || !weight || !total || !normed) return QF_E_ARG;
  if (rows > (int64_t)UINT32_MAX * 4) return QF_E_SHAPE;
  RmsArgs a{};
  a.x = static_cast<const uint16_t*>(residual);
  a.branch = branch;
  a.splits = splits;
  a.split_stride = rows * cols;
  a.w = static_cast<const uint16_t*>(weight);
  a.total = static_cast<uint16_t*>(total);
  a.out = static_cast<uint16_t*>(normed);
  a.rows = rows;
  a.cols = cols;
  a.inner = 1;
  a.eps = eps;
  const bool vec_ok = cols % 8 == 0 && aligned16(residual) && aligned16(branch) &&
                      aligned16(weight) && aligned16(total) && aligned16(normed);
  return splits == 0 ? dispatch<1>(a, vec_ok, as_stream(stream))
                     : dispatch<2>(a, vec_ok, as_stream(stream));
}
