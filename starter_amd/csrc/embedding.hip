// Token embedding gather (bit-exact row copy) and the rotary cos/sin table
// builder for gfx950.
//
// Embedding: out[i, :] = table[ids[i], :] - the nn.Embedding lookup of
// engine/decode_step.py:38, engine/prefill.py:34, engine/decode.py:19.  One
// wave copies one row with 16-byte loads and stores (lane i moves vectors i,
// i+64, ...); the id is read once per wave with a scalar load.  Rows are copied as raw bits, so
// the result is bit-exact by construction.  Out-of-range ids give zero rows.
//
// Rotary table: the Qwen3 default RoPE table that engine/decode.py:52-59
// builds from Qwen3RotaryEmbedding.forward:
//   ang = inv_freq[j] * float(pos)   (one f32 product)
//   cos[p, j] = cos[p, j + half] = bf16(cos(ang)); sin likewise.
#include "qf_device.h"

namespace qf {
namespace {

// NT: nontemporal stores for large calls (the gathered table rows are read
// with ordinary cached loads - measured faster for this random-row pattern).
template <int VPL, bool NT>
__global__ __launch_bounds__(kBlock) void embedding_vec_kernel(const int64_t* __restrict__ ids,
                                                              const uint4* __restrict__ table,
                                                              uint4* __restrict__ out,
                                                              int64_t n_ids, int64_t vocab,
                                                              int32_t nvec) {
  const int lane = threadIdx.x % kWave;
  // Wave-uniform row: the id is fetched with one scalar load.
  const int64_t row = __builtin_amdgcn_readfirstlane(blockIdx.x * (kBlock / kWave) +
                                                     threadIdx.x / kWave);
  if (row >= n_ids) return;
  const int64_t id = ids[row];
  const bool valid = id >= 0 && id < vocab;
  const uint4* src = table + (valid ? id : 0) * nvec;
  uint4* dst = out + row * nvec;
  uint4 v[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = lane + k * kWave;
    v[k] = (valid && c < nvec) ? load16<false>(src + c) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = lane + k * kWave;
    if (c < nvec) store16<NT>(dst + c, v[k]);
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

template <int VPL>
int launch_embedding(const int64_t* ids, const void* table, void* out, int64_t n_ids,
                     int64_t vocab, int32_t nvec, hipStream_t s) {
  const int64_t blocks = (n_ids + 3) / 4;
  if (n_ids * nvec * 32 >= kStreamBytes)
    hipLaunchKernelGGL((embedding_vec_kernel<VPL, true>), dim3((unsigned)blocks), dim3(kBlock), 0, s,
                       ids, static_cast<const uint4*>(table), static_cast<uint4*>(out), n_ids,
                       vocab, nvec);
  else
    hipLaunchKernelGGL((embedding_vec_kernel<VPL, false>), dim3((unsigned)blocks), dim3(kBlock), 0,
                       s, ids, static_cast<const uint4*>(table), static_cast<uint4*>(out), n_ids,
                       vocab, nvec);
  return launch_status();
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
  if (cols % 8 == 0 && aligned16(table) && aligned16(out) && cols / 8 <= 16 * kWave) {
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
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}
