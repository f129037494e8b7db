// SiLU(gate) * up on a packed [rows, 2*cols] projection for gfx950.
//
// Arithmetic (engine/kernels/decode_fused.py:52-56; F.silu(gate) * up on bf16
// tensors in engine/mlp.py:19-21):
//   a   = bf16(g / (1 + exp(-g)))
//   out = bf16(float(a) * float(u))
// The f32 SiLU is silu_f32 (qf_silu.h): hardware exp2 and reciprocal with an
// exact fallback near bf16 rounding midpoints, so bf16(silu) matches the f32
// formula for every bf16 gate; the tests check all 65,536 gate values against
// the oracle bit for bit.  The cheap path costs ~9 VALU instructions per
// element instead of ~25 for expf and an IEEE divide, which would make the
// kernel VALU-bound.
//
// Layout: the output is a flat sequence of 16-byte vectors (8 columns).  A
// thread owns U vectors spaced one workgroup apart, so each wave-wide access
// covers 1 KiB of consecutive gate, up or output bytes.  Row / column of a
// vector come from a multiply-high division by the per-row vector count.
#include "qf_device.h"
#include "qf_silu.h"

namespace qf {
namespace {

__device__ __forceinline__ uint4 silu_mul8(const uint4& gv, const uint4& uv) {
  float g[8], u[8];
  unpack8(gv, g);
  unpack8(uv, u);
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = silu_f32(g[j]);
  round8(g);  // SiLU rounded to bf16 before the product, as the reference does
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] *= u[j];
  return pack8(g);
}

template <int U, bool NT>
__global__ __launch_bounds__(kBlock) void silu_mul_vec_kernel(const uint4* __restrict__ gu,
                                                             uint4* __restrict__ out,
                                                             uint32_t total_vec, FastDiv per_row) {
  const uint32_t base = blockIdx.x * (uint32_t)(kBlock * U) + threadIdx.x;
  uint4 gv[U], uv[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const uint32_t i = base + k * kBlock;
    if (i < total_vec) {
      const uint32_t row = fdiv(i, per_row);
      const uint32_t col = i - row * per_row.d;
      const uint4* g = gu + (uint64_t)row * (2 * per_row.d) + col;
      gv[k] = load16<NT>(g);
      uv[k] = load16<NT>(g + per_row.d);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const uint32_t i = base + k * kBlock;
    if (i < total_vec) store16<NT>(out + i, silu_mul8(gv[k], uv[k]));
  }
}

// Any width / alignment: one element per thread, grid-stride.
__global__ __launch_bounds__(kBlock) void silu_mul_scalar_kernel(const uint16_t* __restrict__ gu,
                                                                uint16_t* __restrict__ out,
                                                                int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kBlock) {
    const int64_t r = i / cols, c = i - r * cols;
    const float g = from_bf16(gu[r * 2 * cols + c]);
    const float u = from_bf16(gu[r * 2 * cols + cols + c]);
    out[i] = to_bf16(from_bf16(to_bf16(silu_f32(g))) * u);
  }
}

template <int U, bool NT>
int launch_silu_vec(const void* gate_up, void* out, int64_t nvec_total, int64_t cols,
                    hipStream_t s) {
  const FastDiv per_row = make_fastdiv((uint32_t)(cols / 8));
  const int64_t blocks = (nvec_total + kBlock * U - 1) / (kBlock * U);
  hipLaunchKernelGGL((silu_mul_vec_kernel<U, NT>), dim3((unsigned)blocks), dim3(kBlock), 0, s,
                     static_cast<const uint4*>(gate_up), static_cast<uint4*>(out),
                     (uint32_t)nvec_total, per_row);
  return launch_status();
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int qf_silu_mul(const void* gate_up, int64_t rows, int64_t cols, void* out,
                           void* stream) {
  if (rows < 0 || cols <= 0) return QF_E_ARG;
  if (rows == 0) return QF_OK;
  if (!gate_up || !out) return QF_E_ARG;
  hipStream_t s = as_stream(stream);
  const int64_t nvec_total = rows * (cols / 8);
  if (cols % 8 == 0 && aligned16(gate_up) && aligned16(out) &&
      nvec_total < (int64_t)UINT32_MAX - 4 * kBlock) {
    if (nvec_total * 48 >= kStreamBytes)
      return launch_silu_vec<1, true>(gate_up, out, nvec_total, cols, s);
    return launch_silu_vec<1, false>(gate_up, out, nvec_total, cols, s);
  }
  const int64_t n = rows * cols;
  int64_t blocks = (n + kBlock - 1) / kBlock;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(silu_mul_scalar_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, s,
                     static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), rows,
                     cols);
  return launch_status();
}
