/*
 * qf_oracle.c - CPU ORACLE (test infrastructure only).
 *
 * A plain-C restatement of the reference arithmetic of the fused layer ops of
 * the Qwen3-4B engine (jadenpxrk/starter), used as the checker for the HIP
 * kernels in starter_amd/.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load this library; the product path never
 * does.  Compile with -ffp-contract=off (no FMA contraction) and without
 * -ffast-math; see oracle/build.py.
 *
 * bf16 values are uint16_t bit patterns.  Rounding f32 -> bf16 is round to
 * nearest even with NaN -> 0x7FC0, which is what torch's c10::BFloat16
 * conversion does; every "bf16(...)" below is that rounding.
 *
 * Where the reference reduces in f32 (the sum of squares of RMSNorm), the
 * oracle accumulates the exact f32 squares in double and rounds the sum once
 * to f32.  Any f32 summation order (torch's CPU cascade, a Triton tree, a
 * wavefront DPP tree) differs from that sum by a few f32 ulps, which moves a
 * bf16 output by at most one ulp.
 *
 * Pinning of each function (tests/test_oracle.py):
 *   or_rms_norm            transformers Qwen3RMSNorm on CPU; golden fixture;
 *                          known answers (constant rows with eps 0 -> weight
 *                          exactly; zero rows -> 0); planted cast-placement
 *                          mistake must be detected.
 *   or_add_rms_norm        bf16 add is exact (atol 0); split-K fold equals
 *                          sequential f32 sum + one rounding; norm as above.
 *   or_silu_mul            F.silu(gate) * up on CPU; special values
 *                          -40,-12,-1,0,1,12,40,88; f64 bounds.
 *   or_qk_norm_rope etc.   Qwen3RMSNorm + apply_rotary_pos_emb on CPU;
 *                          position 0 identity; constant rows eps 0 exact;
 *                          zeros -> zeros; dropping the product rounding must
 *                          change bits.
 *   or_embedding           F.embedding on CPU, bit-exact.
 *   or_rope_table          Qwen3RotaryEmbedding.forward on CPU, <= 1 bf16 ulp.
 *   or_linear_partials     integer inputs against an int64 matmul, bit-exact
 *                          per split; torch float64 F.linear per chunk;
 *                          dropped-chunk and transposed-operand mistakes
 *                          must be detected.
 *   or_decode_attention    torch float64 softmax attention per (sequence, kv
 *                          head); known answers (zero queries -> mean of V,
 *                          one dominant key block -> its V); wrong head
 *                          mapping and reading past `used` are detected.
 *   or_prefill_attention   torch float64 scaled_dot_product_attention with
 *                          is_causal and grouped K/V heads; known answers
 *                          (zero queries -> running mean of V, a dominant key
 *                          -> its V from that position on); attending one
 *                          key past the diagonal is detected.
 *   or_lm_head_argmax      logits bit-equal to torch float64 F.linear rounded
 *                          to bf16; token = torch.argmax of them (first
 *                          maximum) on integer inputs full of exact ties.
 *   or_linear_silu_mul     composition of exactly rounded projections with
 *                          or_silu_mul (bit-exact), torch float64 projections
 *                          + F.silu; skipping the projection rounding must
 *                          change bits (the reference's negative control).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ bf16 */

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* f32 -> bf16, round to nearest even; NaN -> 0x7FC0 (c10::BFloat16). */
EXPORT uint16_t or_bf16(float f) {
  if (isnan(f)) return 0x7FC0;
  uint32_t u = f32_bits(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
EXPORT float or_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }
static inline float rbf(float f) { return or_f32(or_bf16(f)); }

/* --------------------------------------------------------------- RMSNorm */

/* 1 / sqrt(mean(t^2) + eps) of one row of f32 values (bf16-representable).
 * engine/kernels/rmsnorm.py:21-23; Qwen3RMSNorm.forward lines
 * "variance = hidden_states.pow(2).mean(-1)" and "* torch.rsqrt(variance + eps)". */
static float inv_rms(const float* t, int64_t cols, float eps) {
  double acc = 0.0;
  for (int64_t c = 0; c < cols; ++c) acc += (double)(t[c] * t[c]); /* exact squares */
  const float var = (float)acc / (float)cols;
  return 1.0f / sqrtf(var + eps);
}

/* n = bf16(t * inv); out = bf16(n * w): the cast sits BEFORE the gain
 * (engine/kernels/rmsnorm.py:25-36; "self.weight * hidden_states.to(input_dtype)"). */
static void norm_gain(const float* t, int64_t cols, float inv, const uint16_t* w, uint16_t* out) {
  for (int64_t c = 0; c < cols; ++c) out[c] = or_bf16(rbf(t[c] * inv) * or_f32(w[c]));
}

/* engine/kernels/rmsnorm.py:12-62 (rms_norm): x is contiguous [rows, cols]. */
EXPORT void or_rms_norm(const uint16_t* x, int64_t rows, int64_t cols, const uint16_t* w,
                        float eps, float* scratch, uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) scratch[c] = or_f32(x[r * cols + c]);
    norm_gain(scratch, cols, inv_rms(scratch, cols, eps), w, out + r * cols);
  }
}

/* engine/kernels/decode_fused.py:19-44 (_add_rms_norm_kernel) and :140-158.
 * branch: bf16 [rows, cols] (splits == 0) or f32 partials [splits, rows, cols]
 * added in split order starting from 0.0f and rounded once (:27-35). */
EXPORT void or_add_rms_norm(const uint16_t* residual, const void* branch, int32_t splits,
                            const uint16_t* w, int64_t rows, int64_t cols, float eps,
                            float* scratch, uint16_t* total, uint16_t* normed) {
  const int64_t n = rows * cols;
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t i = r * cols + c;
      float y;
      if (splits == 0) {
        y = or_f32(((const uint16_t*)branch)[i]);
      } else {
        const float* p = (const float*)branch;
        y = 0.0f;
        for (int32_t s = 0; s < splits; ++s) y += p[(int64_t)s * n + i];
        y = rbf(y);
      }
      /* "total = (x + y).to(S.dtype.element_ty)" (:37) */
      const uint16_t t = or_bf16(or_f32(residual[i]) + y);
      total[i] = t;
      scratch[c] = or_f32(t);
    }
    norm_gain(scratch, cols, inv_rms(scratch, cols, eps), w, normed + r * cols);
  }
}

/* ------------------------------------------------------------- SiLU * up */

/* engine/kernels/decode_fused.py:47-56: act = bf16(g / (1 + exp(-g)));
 * out = bf16(act * up).  gate_up is [rows, 2*cols], gate first. */
EXPORT void or_silu_mul(const uint16_t* gate_up, int64_t rows, int64_t cols, uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* g = gate_up + r * 2 * cols;
    const uint16_t* u = g + cols;
    for (int64_t c = 0; c < cols; ++c) {
      const float gv = or_f32(g[c]);
      const float act = rbf(gv / (1.0f + expf(-gv)));
      out[r * cols + c] = or_bf16(act * or_f32(u[c]));
    }
  }
}

/* --------------------------------------------------- Q/K norm + RoPE row */

#define HEAD 128
#define HALF 64

/* One head row of f32 values x (bf16-representable):
 *   inv = 1/sqrt(sum(x^2)/128 + eps); n = bf16(bf16(x*inv) * w)
 *   rot = [-n[64:], n[:64]];  out = bf16(bf16(n*cos) + bf16(rot*sin))
 * engine/kernels/qk_norm_rope.py:27-44 (the partner element is the +-64 one,
 * :30 "partner = (cols + D // 2) % D"; rotate_half negates the second half
 * and moves it first).  round_products = 0 plants the "no product rounding"
 * mistake used as a negative control by the tests. */
static void norm_rope_row(const float* x, const uint16_t* w, const uint16_t* cs,
                          const uint16_t* sn, float eps, int round_products, uint16_t* out) {
  float n[HEAD];
  const float inv = inv_rms(x, HEAD, eps);
  for (int j = 0; j < HEAD; ++j) n[j] = rbf(rbf(x[j] * inv) * or_f32(w[j]));
  for (int j = 0; j < HEAD; ++j) {
    const float rot = j < HALF ? -n[j + HALF] : n[j - HALF];
    float left = n[j] * or_f32(cs[j]);
    float right = rot * or_f32(sn[j]);
    if (round_products) {
      left = rbf(left);
      right = rbf(right);
    }
    out[j] = or_bf16(left + right);
  }
}

static void load_row(const uint16_t* src, float* x) {
  for (int j = 0; j < HEAD; ++j) x[j] = or_f32(src[j]);
}

/* engine/kernels/qk_norm_rope.py:47-73 (qk_norm_rope): q head h of sequence b
 * at q + b*q_bs + h*q_hs; cos/sin row of sequence b at cos + b*cs_bs. */
EXPORT void or_qk_norm_rope(const uint16_t* q, const uint16_t* k, int64_t batch, int32_t nq,
                            int32_t nk, int64_t q_bs, int64_t q_hs, int64_t k_bs, int64_t k_hs,
                            const uint16_t* qw, const uint16_t* kw, const uint16_t* cos,
                            const uint16_t* sin, int64_t cs_bs, float q_eps, float k_eps,
                            int32_t round_products, uint16_t* oq, uint16_t* ok) {
  float x[HEAD];
  for (int64_t b = 0; b < batch; ++b) {
    const uint16_t* c = cos + b * cs_bs;
    const uint16_t* s = sin + b * cs_bs;
    for (int32_t h = 0; h < nq; ++h) {
      load_row(q + b * q_bs + h * q_hs, x);
      norm_rope_row(x, qw, c, s, q_eps, round_products, oq + (b * nq + h) * HEAD);
    }
    for (int32_t h = 0; h < nk; ++h) {
      load_row(k + b * k_bs + h * k_hs, x);
      norm_rope_row(x, kw, c, s, k_eps, round_products, ok + (b * nk + h) * HEAD);
    }
  }
}

/* engine/kernels/decode_fused.py:59-118 (_qkv_norm_rope_cache_kernel).
 * qkv: bf16 [batch, W] (splits == 0) or f32 [splits, batch, W], W = (nq+2nk)*128,
 * summed in split order from 0 and rounded once (:82-93, :111-117).
 * position: the slot (host value here).  K/V rows go to cache[b, h, position].
 * Matches the kernel's documented guard: a position outside [0, capacity)
 * writes no cache row and fills q_out with bf16 NaN. */
EXPORT void or_qkv_norm_rope_cache(const void* qkv, int32_t splits, int64_t batch, int32_t nq,
                                   int32_t nk, const uint16_t* qw, const uint16_t* kw,
                                   float q_eps, float k_eps, const uint16_t* cos,
                                   const uint16_t* sin, int64_t position, int64_t capacity,
                                   int32_t round_products, uint16_t* q_out, uint16_t* kc,
                                   uint16_t* vc) {
  const int64_t heads = (int64_t)nq + 2 * (int64_t)nk;
  const int64_t width = heads * HEAD;
  const int ok_pos = position >= 0 && position < capacity;
  float x[HEAD];
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t h = 0; h < heads; ++h) {
      const int64_t off = b * width + h * HEAD;
      if (splits == 0) {
        load_row((const uint16_t*)qkv + off, x);
      } else {
        const float* p = (const float*)qkv;
        for (int j = 0; j < HEAD; ++j) {
          float acc = 0.0f;
          for (int32_t s = 0; s < splits; ++s) acc += p[(int64_t)s * batch * width + off + j];
          x[j] = rbf(acc);
        }
      }
      if (h < nq) {
        uint16_t* dst = q_out + (b * nq + h) * HEAD;
        if (!ok_pos) {
          for (int j = 0; j < HEAD; ++j) dst[j] = 0x7FC0;
          continue;
        }
        norm_rope_row(x, qw, cos + position * HEAD, sin + position * HEAD, q_eps,
                      round_products, dst);
      } else if (ok_pos) {
        const int is_k = h < nq + nk;
        const int64_t kvh = is_k ? h - nq : h - nq - nk;
        uint16_t* dst = (is_k ? kc : vc) + ((b * nk + kvh) * capacity + position) * HEAD;
        if (is_k) {
          norm_rope_row(x, kw, cos + position * HEAD, sin + position * HEAD, k_eps,
                        round_products, dst);
        } else if (splits == 0) {
          memcpy(dst, (const uint16_t*)qkv + off, HEAD * sizeof(uint16_t)); /* raw copy */
        } else {
          for (int j = 0; j < HEAD; ++j) dst[j] = or_bf16(x[j]);
        }
      }
    }
  }
}

/* engine/kernels/prefill.py:19-63 (_prefill_qkv): token t of sequence b uses
 * rotary row t and cache slot t (":239 batch, pos = token // T, token % T"). */
EXPORT void or_prefill_qkv(const uint16_t* qkv, int64_t batch, int64_t length, int32_t nq,
                           int32_t nk, const uint16_t* qw, const uint16_t* kw, float q_eps,
                           float k_eps, const uint16_t* cos, const uint16_t* sin,
                           int64_t capacity, int32_t round_products, uint16_t* q_out,
                           uint16_t* kc, uint16_t* vc) {
  const int64_t heads = (int64_t)nq + 2 * (int64_t)nk;
  const int64_t width = heads * HEAD;
  float x[HEAD];
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t t = 0; t < length; ++t) {
      const int64_t token = b * length + t;
      const uint16_t* c = cos + t * HEAD;
      const uint16_t* s = sin + t * HEAD;
      for (int64_t h = 0; h < heads; ++h) {
        const uint16_t* src = qkv + token * width + h * HEAD;
        if (h < nq) {
          load_row(src, x);
          norm_rope_row(x, qw, c, s, q_eps, round_products, q_out + (token * nq + h) * HEAD);
        } else if (h < nq + nk) {
          load_row(src, x);
          norm_rope_row(x, kw, c, s, k_eps, round_products,
                        kc + ((b * nk + (h - nq)) * capacity + t) * HEAD);
        } else {
          memcpy(vc + ((b * nk + (h - nq - nk)) * capacity + t) * HEAD, src,
                 HEAD * sizeof(uint16_t));
        }
      }
    }
  }
}

/* ------------------------------------------------------------- embedding */

/* nn.Embedding lookup (engine/decode_step.py:38): out[i] = table[ids[i]].
 * Out-of-range ids give zero rows, the kernel's documented guard. */
EXPORT void or_embedding(const int64_t* ids, int64_t n_ids, const uint16_t* table,
                         int64_t vocab, int64_t cols, uint16_t* out) {
  for (int64_t i = 0; i < n_ids; ++i) {
    const int64_t id = ids[i];
    if (id >= 0 && id < vocab)
      memcpy(out + i * cols, table + id * cols, (size_t)cols * sizeof(uint16_t));
    else
      memset(out + i * cols, 0, (size_t)cols * sizeof(uint16_t));
  }
}

/* ---------------------------------------------------------- rotary table */

/* engine/decode.py:52-59 evaluating Qwen3RotaryEmbedding.forward:
 *   freqs = inv_freq (x) float(pos)  (one f32 product per entry)
 *   emb = cat(freqs, freqs); cos/sin in f32, cast to bf16.
 * cos/sin here are the correctly rounded f32 values (evaluated in double). */
EXPORT void or_rope_table(const float* inv_freq, int32_t half, const int64_t* positions,
                          int64_t start, int64_t n_pos, uint16_t* cos_out, uint16_t* sin_out) {
  for (int64_t p = 0; p < n_pos; ++p) {
    const int64_t pos = positions ? positions[p] : start + p;
    for (int32_t j = 0; j < half; ++j) {
      const float ang = inv_freq[j] * (float)pos;
      const uint16_t c = or_bf16((float)cos((double)ang));
      const uint16_t s = or_bf16((float)sin((double)ang));
      cos_out[p * 2 * half + j] = c;
      cos_out[p * 2 * half + j + half] = c;
      sin_out[p * 2 * half + j] = s;
      sin_out[p * 2 * half + j + half] = s;
    }
  }
}

/* ---------------------------------------------------- decode projections */

/* Exactly rounded f32 value of sum_c x[c] * w[c] over [c0, c1): the bf16
 * products are exact in double and so is their sum up to a relative 2^-40
 * for any realistic length, so rounding the double sum once to f32 gives
 * the correctly rounded dot product.  A hardware f32 accumulation (tensor or
 * matrix cores) differs from it by f32 rounding error only. */
static float dot_f32(const uint16_t* x, const uint16_t* w, int64_t c0, int64_t c1) {
  double acc = 0.0;
  for (int64_t c = c0; c < c1; ++c) acc += (double)or_f32(x[c]) * (double)or_f32(w[c]);
  return (float)acc;
}

/* engine/kernels/skinny_gemm.py:28-46 (_partials_kernel) and :100-109:
 * partial s of x @ W^T over k in [s*k/S, (s+1)*k/S) with f32 accumulation
 * (tl.dot on bf16 operands).  x is [m, k], W is [n, k], out is f32
 * [splits, m, n]. */
EXPORT void or_linear_partials(const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                               int64_t n, int32_t splits, float* out) {
  const int64_t per = k / splits;
  for (int32_t s = 0; s < splits; ++s)
    for (int64_t i = 0; i < m; ++i)
      for (int64_t j = 0; j < n; ++j)
        out[((int64_t)s * m + i) * n + j] = dot_f32(x + i * k, w + j * k, s * per, (s + 1) * per);
}

/* engine/kernels/skinny_gemm.py:49-72 (_silu_mul_kernel) and :112-121:
 *   g = bf16(x @ gate^T), u = bf16(x @ up^T)     (each projection a bf16 tensor)
 *   out = bf16(bf16(g / (1 + exp(-g))) * u)      (as or_silu_mul)
 * gate_up is the packed [2n, k] weight, gate rows first; out is [m, n]. */
EXPORT void or_linear_silu_mul(const uint16_t* x, int64_t m, int64_t k, const uint16_t* gate_up,
                               int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      const float g = rbf(dot_f32(x + i * k, gate_up + j * k, 0, k));
      const float u = rbf(dot_f32(x + i * k, gate_up + (n + j) * k, 0, k));
      const float act = rbf(g / (1.0f + expf(-g)));
      out[i * n + j] = or_bf16(act * u);
    }
}

/* ------------------------------------------------------ decode attention */

/* engine/kernels/small_query_attention.py:113-158 (the function it computes;
 * its tests' float64 restatement is tests/test_small_query_attention.py:
 * 151-163): for query head h of sequence b, kv head h / G (G = hq / hk),
 *   out = bf16( softmax((q . k_j) * scale over j < used) @ v )
 * in double; no valid key -> zeros.  q [b*hq, 128], k/v [b*hk*capacity, 128],
 * used [b*hk], out [b*hq, 128].  Keys at or beyond used are not read. */
EXPORT void or_decode_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const int32_t* used, int64_t batch, int32_t hq, int32_t hk,
                                int64_t capacity, double scale, double* scratch, uint16_t* out) {
  const int32_t groups = hq / hk;
  for (int64_t b = 0; b < batch; ++b)
    for (int32_t h = 0; h < hq; ++h) {
      const int64_t vh = b * hk + h / groups;
      int64_t n = used[vh];
      if (n < 0) n = 0;
      if (n > capacity) n = capacity;
      const uint16_t* qr = q + (b * hq + h) * HEAD;
      uint16_t* o = out + (b * hq + h) * HEAD;
      double mx = -INFINITY;
      for (int64_t j = 0; j < n; ++j) {
        const uint16_t* kr = k + (vh * capacity + j) * HEAD;
        double dot = 0.0;
        for (int d = 0; d < HEAD; ++d) dot += (double)or_f32(qr[d]) * (double)or_f32(kr[d]);
        scratch[j] = dot * scale;
        if (scratch[j] > mx) mx = scratch[j];
      }
      double acc[HEAD] = {0};
      double den = 0.0;
      for (int64_t j = 0; j < n; ++j) {
        const double p = exp(scratch[j] - mx);
        den += p;
        const uint16_t* vr = v + (vh * capacity + j) * HEAD;
        for (int d = 0; d < HEAD; ++d) acc[d] += p * (double)or_f32(vr[d]);
      }
      for (int d = 0; d < HEAD; ++d) o[d] = n ? or_bf16((float)(acc[d] / den)) : 0;
    }
}

/* Causal prefill attention (engine/prefill.py:13-23, the reference's
 * aten._flash_attention_forward(..., is_causal=True) over the first `length`
 * cache slots):
 *   out[b, t, h] = bf16( softmax_j<=t((q[b,t,h] . k[b,h/G,j]) * scale) @ v[b,h/G,j] )
 * in double.  q [b, length, hq, 128] (the prefill_qkv layout), k/v
 * [b, hk, capacity, 128] head-major caches, out like q.  Slots at or beyond
 * `length` are not read. */
EXPORT void or_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 int64_t batch, int64_t length, int32_t hq, int32_t hk,
                                 int64_t capacity, double scale, double* scratch, uint16_t* out) {
  const int32_t groups = hq / hk;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t t = 0; t < length; ++t)
      for (int32_t h = 0; h < hq; ++h) {
        const int64_t vh = b * hk + h / groups;
        const uint16_t* qr = q + ((b * length + t) * hq + h) * HEAD;
        uint16_t* o = out + ((b * length + t) * hq + h) * HEAD;
        double mx = -INFINITY;
        for (int64_t j = 0; j <= t; ++j) {
          const uint16_t* kr = k + (vh * capacity + j) * HEAD;
          double dot = 0.0;
          for (int d = 0; d < HEAD; ++d) dot += (double)or_f32(qr[d]) * (double)or_f32(kr[d]);
          scratch[j] = dot * scale;
          if (scratch[j] > mx) mx = scratch[j];
        }
        double acc[HEAD] = {0};
        double den = 0.0;
        for (int64_t j = 0; j <= t; ++j) {
          const double p = exp(scratch[j] - mx);
          den += p;
          const uint16_t* vr = v + (vh * capacity + j) * HEAD;
          for (int d = 0; d < HEAD; ++d) acc[d] += p * (double)or_f32(vr[d]);
        }
        for (int d = 0; d < HEAD; ++d) o[d] = or_bf16((float)(acc[d] / den));
      }
}

/* ------------------------------------------------ LM head + token choice */

/* engine/decode_step.py:64 and engine/decode.py:93: logits = bf16(x @ W^T)
 * (exactly rounded here), token = argmax with the lowest index among equal
 * maxima (torch.argmax returns the first maximum; NaN counts as maximal).
 * x [m, k], W [vocab, k], tokens [m], logits [m, vocab] (may be NULL). */
EXPORT void or_lm_head_argmax(const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                              int64_t vocab, int64_t* tokens, uint16_t* logits) {
  for (int64_t i = 0; i < m; ++i) {
    float best = 0.0f;
    int64_t besti = -1;
    for (int64_t j = 0; j < vocab; ++j) {
      const uint16_t b = or_bf16(dot_f32(x + i * k, w + j * k, 0, k));
      if (logits) logits[i * vocab + j] = b;
      const float v = or_f32(b);
      const int vn = isnan(v), bn = besti >= 0 && isnan(best);
      if (besti < 0 || (vn && !bn) || (!vn && !bn && v > best)) {
        best = v;
        besti = j;
      }
    }
    tokens[i] = besti;
  }
}
