// Token embedding gather (bit-exact row copy) and the rotary cos/sin table
// builder for gfx950.
//
// Embedding: out[i, :] = table[ids[i], :] - the nn.Embedding lookup of
// engine/decode_step.py:38, engine/prefill.py:34, engine/decode.py:19.  A wave
// copies one row (decode sizes) or up to 8 consecutive rows (large calls)
// with 16-byte loads and stores (lane i moves vectors i, i+64, ...); the ids
// are read with scalar loads.  Rows are copied as raw bits, so the result is
// bit-exact by construction.  Out-of-range ids give zero rows.
//
// Rotary table: the Qwen3 default RoPE table that engine/decode.py:52-59
// builds from Qwen3RotaryEmbedding.forward:
//   ang = inv_freq[j] * float(pos)   (one f32 product)
//   cos[p, j] = cos[p, j + half] = bf16(cos(ang)); sin likewise.
#include "qf_device.h"

namespace qf {
namespace {

// Copies rows row0 .. row0+R-1 (all < n_ids): their ids come in scalar
// loads, then every row's table loads are issued before the first store, so
// the wave waits for the id load once and keeps R * VPL 16-byte loads in
// flight.  Every load is unconditional - an invalid id reads row 0 and a lane
// past the row end re-reads the last vector, and the stores write zeros /
// nothing there - and so are the stores of complete rows, so the compiler has
// no branch to sink a later row's loads below an earlier row's stores.
template <int VPL, int R, bool NT, bool FULL>
__device__ __forceinline__ void copy_rows(const int64_t* __restrict__ ids,
                                          const uint4* __restrict__ table,
                                          uint4* __restrict__ out, int64_t row0, int64_t vocab,
                                          int32_t nvec, int lane) {
  int64_t id[R];
#pragma unroll
  for (int r = 0; r < R; ++r) id[r] = ids[row0 + r];
  uint4 v[R][VPL];
  bool valid[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    valid[r] = id[r] >= 0 && id[r] < vocab;
    const uint4* src = table + (valid[r] ? id[r] : 0) * nvec;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int c = lane + k * kWave;
      v[r][k] = load16<false>(src + (FULL || c < nvec ? c : nvec - 1));
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint4* dst = out + (row0 + r) * nvec;
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int c = lane + k * kWave;
      if (FULL || c < nvec) store16<NT>(dst + c, valid[r] ? v[r][k] : make_uint4(0, 0, 0, 0));
    }
  }
}

// A wave owns RPW consecutive rows; the last wave of the grid, whose rows may
// run past n_ids, copies its rows one at a time.
// NT: nontemporal stores for large calls (the gathered table rows are read
// with ordinary cached loads - measured faster for this random-row pattern).
// FULL: the row is exactly VPL vectors per lane (nvec == VPL * 64), so no lane
// needs a column bound.
// WPB: waves per workgroup (4; 1 for decode sizes, which spreads their rows
// over as many CUs: 64 ids 2.11 -> 2.02 us).
template <int VPL, int RPW, bool NT, bool FULL = false, int WPB = kBlock / kWave>
__global__ __launch_bounds__(kBlock) void embedding_vec_kernel(const int64_t* __restrict__ ids,
                                                              const uint4* __restrict__ table,
                                                              uint4* __restrict__ out,
                                                              int64_t n_ids, int64_t vocab,
                                                              int32_t nvec) {
  const int lane = threadIdx.x % kWave;
  const int64_t row0 = __builtin_amdgcn_readfirstlane(
      ((int64_t)blockIdx.x * WPB + threadIdx.x / kWave) * RPW);
  if (row0 + RPW <= n_ids) {
    copy_rows<VPL, RPW, NT, FULL>(ids, table, out, row0, vocab, nvec, lane);
  } else {
    for (int64_t row = row0; row < n_ids; ++row)  // wave-uniform
      copy_rows<VPL, 1, NT, FULL>(ids, table, out, row, vocab, nvec, lane);
  }
}

// Any width / alignment: one wave per row, 2-byte elements.
__global__ __launch_bounds__(kBlock) void embedding_scalar_kernel(const int64_t* __restrict__ ids,
                                                                 const uint16_t* __restrict__ table,
                                                                 uint16_t* __restrict__ out,
                                                                 int64_t n_ids, int64_t vocab,
                                                                 int64_t cols) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
  if (row >= n_ids) return;
  const int64_t id = ids[row];
  const bool valid = id >= 0 && id < vocab;
  for (int64_t c = lane; c < cols; c += kWave)
    out[row * cols + c] = valid ? table[id * cols + c] : (uint16_t)0;
}

template <int VPL, int RPW, bool NT, bool FULL>
int launch_rows(const int64_t* ids, const void* table, void* out, int64_t n_ids, int64_t vocab,
                int32_t nvec, hipStream_t s) {
  constexpr int WPB = RPW == 1 && !NT ? 1 : kBlock / kWave;
  constexpr int64_t per_block = WPB * RPW;
  const int64_t blocks = (n_ids + per_block - 1) / per_block;
  hipLaunchKernelGGL((embedding_vec_kernel<VPL, RPW, NT, FULL, WPB>), dim3((unsigned)blocks),
                     dim3(WPB * kWave), 0, s, ids, static_cast<const uint4*>(table),
                     static_cast<uint4*>(out), n_ids, vocab, nvec);
  return launch_status();
}

template <int VPL, int RPW>
int launch_streaming(const int64_t* ids, const void* table, void* out, int64_t n_ids,
                     int64_t vocab, int32_t nvec, hipStream_t s) {
  if (nvec == VPL * kWave)
    return launch_rows<VPL, RPW, true, true>(ids, table, out, n_ids, vocab, nvec, s);
  return launch_rows<VPL, RPW, true, false>(ids, table, out, n_ids, vocab, nvec, s);
}

// Decode-size calls: one row per wave, cached stores (the next kernel reads
// the rows).  Large calls: nontemporal stores, and the fewest rows per wave
// (1, 2, 4 or 8, at most 40 vectors per lane in flight) that keep the grid
// within one 4-wave workgroup per CU.  Measured on the 8192-id Qwen3-4B
// gather (2560 columns): 8 rows per wave (256 workgroups) 14.2-14.5 us,
// against 15.1 us with one row per wave (2048 workgroups); row counts that
// leave the CUs unevenly loaded (3 or 5 per wave: 683 or 410 workgroups)
// take 16.3-16.7 us.
template <int VPL>
int launch_embedding(const int64_t* ids, const void* table, void* out, int64_t n_ids,
                     int64_t vocab, int32_t nvec, hipStream_t s) {
  if (n_ids * nvec * 32 < kStreamBytes)
    return launch_rows<VPL, 1, false, false>(ids, table, out, n_ids, vocab, nvec, s);
  constexpr int kMaxRows = 40 / VPL >= 8 ? 8 : 40 / VPL >= 4 ? 4 : 40 / VPL >= 2 ? 2 : 1;
  const int64_t waves_per_grid = (int64_t)kCUs * (kBlock / kWave);
  int rows = 1;
  while (rows < kMaxRows && (int64_t)rows * waves_per_grid < n_ids) rows *= 2;
  switch (rows) {
    case 1: return launch_streaming<VPL, 1>(ids, table, out, n_ids, vocab, nvec, s);
    case 2: return launch_streaming<VPL, (kMaxRows >= 2 ? 2 : 1)>(ids, table, out, n_ids, vocab, nvec, s);
    case 4: return launch_streaming<VPL, (kMaxRows >= 4 ? 4 : 1)>(ids, table, out, n_ids, vocab, nvec, s);
    default: return launch_streaming<VPL, kMaxRows>(ids, table, out, n_ids, vocab, nvec, s);
  }
}

__global__ __launch_bounds__(kBlock) void rope_table_kernel(const float* __restrict__ inv_freq,
                                                           int32_t half,
                                                           const int64_t* __restrict__ positions,
                                                           int64_t start, int64_t n_pos,
                                                           uint16_t* __restrict__ cos_out,
                                                           uint16_t* __restrict__ sin_out) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n_pos * half) return;
  const int64_t p = i / half;
  const int j = (int)(i - p * half);
  const int64_t pos = positions ? positions[p] : start + p;
  const float ang = inv_freq[j] * (float)pos;
  const uint16_t c = to_bf16(cosf(ang));
  const uint16_t s = to_bf16(sinf(ang));
  const int64_t base = p * 2 * half;
  cos_out[base + j] = c;
  cos_out[base + j + half] = c;
  sin_out[base + j] = s;
  sin_out[base + j + half] = s;
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int qf_embedding(const int64_t* ids, int64_t n_ids, const void* table, int64_t vocab,
                            int64_t cols, void* out, void* stream) {
  if (n_ids < 0 || vocab < 0 || cols <= 0) return QF_E_ARG;
  if (n_ids == 0) return QF_OK;
  if (!ids || !out || (!table && vocab > 0)) return QF_E_ARG;
  if ((reinterpret_cast<uintptr_t>(ids) & 7u)) return QF_E_ALIGN;
  hipStream_t s = as_stream(stream);
  // The vector kernel always loads row 0 for invalid ids, so it needs a
  // non-empty table; an empty one (every id invalid) takes the scalar kernel.
  if (vocab > 0 && cols % 8 == 0 && aligned16(table) && aligned16(out) && cols / 8 <= 16 * kWave) {
    const int32_t nvec = (int32_t)(cols / 8);
    switch ((nvec + kWave - 1) / kWave) {
      case 1: return launch_embedding<1>(ids, table, out, n_ids, vocab, nvec, s);
      case 2: return launch_embedding<2>(ids, table, out, n_ids, vocab, nvec, s);
      case 3: return launch_embedding<3>(ids, table, out, n_ids, vocab, nvec, s);
      case 4: return launch_embedding<4>(ids, table, out, n_ids, vocab, nvec, s);
      case 5: return launch_embedding<5>(ids, table, out, n_ids, vocab, nvec, s);
      case 6: return launch_embedding<6>(ids, table, out, n_ids, vocab, nvec, s);
      case 7: case 8: return launch_embedding<8>(ids, table, out, n_ids, vocab, nvec, s);
      default: return launch_embedding<16>(ids, table, out, n_ids, vocab, nvec, s);
    }
  }
  const int64_t blocks = (n_ids + 3) / 4;
  hipLaunchKernelGGL(embedding_scalar_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s, ids,
                     static_cast<const uint16_t*>(table), static_cast<uint16_t*>(out), n_ids,
                     vocab, cols);
  return launch_status();
}

extern "C" int qf_rope_table(const float* inv_freq, int32_t half, const int64_t* positions,
                             int64_t start, int64_t n_pos, void* cos, void* sin, void* stream) {
  if (half < 1 || n_pos < 0) return QF_E_ARG;
  if (n_pos == 0) return QF_OK;
  if (!inv_freq || !cos || !sin) return QF_E_ARG;
  const int64_t n = n_pos * half;
  const int64_t blocks = (n + kBlock - 1) / kBlock;
  if (blocks > (int64_t)INT32_MAX) return QF_E_SHAPE;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, as_stream(stream),
                     inv_freq, half, positions, start, n_pos, static_cast<uint16_t*>(cos),
                     static_cast<uint16_t*>(sin));
  return launch_status();
}

extern "C" int qf_version(void) { return 100; }

extern "C" const char* qf_error_string(int status) {
  switch (status) {
    case QF_OK: return "success";
    case QF_E_ARG: return "invalid argument (null pointer, negative size or stride)";
    case QF_E_SHAPE: return "unsupported shape";
    case QF_E_ALIGN: return "pointer or stride not aligned for the kernel";
    case QF_E_CAPACITY: return "input exceeds the static scratch capacity";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
