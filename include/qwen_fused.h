/*
 * qwen_fused.h - C ABI of the MI355X (gfx950) fused layer kernels of the
 * Qwen3-4B decode engine: residual-add + RMSNorm, per-head Q/K RMSNorm fused
 * with NeoX rotary embedding (three layouts), SiLU(gate)*up, the token
 * embedding gather, the rotary cos/sin table builder, the split-K decode
 * projections that feed the fused consumers, grouped-query decode attention
 * over the K/V cache, and the LM head fused with greedy token selection.
 *
 * Conventions shared by every entry point:
 *   - Tensors are plain device pointers.  "bf16" buffers hold IEEE bfloat16
 *     bit patterns (uint16_t); "f32" buffers hold IEEE binary32.
 *   - Sizes and strides are in ELEMENTS, never bytes.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is
 *     only enqueued: no entry point synchronises, allocates, frees or reads a
 *     device value on the host, so every call may be captured into a HIP graph.
 *   - Return value: 0 on success; a negative QF_E* code for an argument error
 *     detected on the host before anything is launched; otherwise the positive
 *     hipError_t reported for the launch.  qf_error_string() names a code.
 *   - The library keeps no mutable global state, with one exception:
 *     qf_lm_head_argmax_static's per-GPU static scratch array (and the host
 *     cache of its device addresses, guarded by a mutex).  Every other call
 *     is reentrant.
 *   - Inputs are read-only.  Outputs must not alias inputs.
 *
 * Each entry point cites the reference (jadenpxrk/starter) Python/Triton
 * function whose semantics it replaces.
 */
#ifndef QWEN_FUSED_H
#define QWEN_FUSED_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QF_OK 0
#define QF_E_ARG (-1)     /* null pointer, negative size, bad stride */
#define QF_E_SHAPE (-2)   /* unsupported shape (e.g. head width != 128) */
#define QF_E_ALIGN (-3)   /* pointer alignment the selected path needs */
#define QF_E_CAPACITY (-4) /* input larger than a static scratch buffer holds */

/* Library version: major*10000 + minor*100 + patch. */
int qf_version(void);

/* Static text for a status code returned by any qf_* call. */
const char* qf_error_string(int status);

/*
 * RMSNorm over the last dimension, rounding to bf16 BEFORE the gain multiply:
 *   var = sum(float(x)^2) / cols;  n = bf16(float(x) * (1 / sqrt(var + eps)))
 *   out = bf16(float(n) * float(weight))
 * Replaces engine/kernels/rmsnorm.py:39-62 (rms_norm + _rms_norm_kernel:12-36).
 * Row r of x starts at x + (r / inner) * outer_stride + (r % inner) * inner_stride
 * (a two-level row walk, so transposed 3-D inputs need no copy); the last
 * dimension is contiguous.  out is contiguous [rows, cols].
 */
int qf_rms_norm(const void* x, int64_t rows, int64_t cols, int64_t inner,
                int64_t outer_stride, int64_t inner_stride,
                const void* weight, float eps, void* out, void* stream);

/*
 * Residual add folded into the following RMSNorm:
 *   branch = splits == 0 ? bf16 branch[r, c]
 *                        : bf16(((0 + p[0][r,c]) + p[1][r,c]) + ...)  (f32 partials)
 *   total  = bf16(float(residual) + float(branch))        (stored)
 *   normed = RMSNorm(total) with the cast placement of qf_rms_norm.
 * Replaces engine/kernels/decode_fused.py:140-158 (add_rms_norm +
 * _add_rms_norm_kernel:19-44).  residual/branch/total/normed are contiguous
 * [rows, cols]; f32 partials are contiguous [splits, rows, cols].
 */
int qf_add_rms_norm(const void* residual, const void* branch, int32_t splits,
                    const void* weight, int64_t rows, int64_t cols, float eps,
                    void* total, void* normed, void* stream);

/*
 * SiLU(gate) * up on a packed [rows, 2*cols] projection (gate = first half):
 *   a = bf16(g / (1 + exp(-g)));  out = bf16(float(a) * float(up))
 * Replaces engine/kernels/decode_fused.py:161-169 (silu_mul +
 * _silu_mul_kernel:47-56).  out is contiguous [rows, cols].
 */
int qf_silu_mul(const void* gate_up, int64_t rows, int64_t cols, void* out,
                void* stream);

/*
 * Per-head Q/K RMSNorm + NeoX rotate-half RoPE for one decode token
 * (head width 128):
 *   n = bf16(bf16(x * inv) * w);  rot = [-n[64:], n[:64]]
 *   out = bf16(bf16(n * cos) + bf16(rot * sin))
 * Replaces engine/kernels/qk_norm_rope.py:47-73 (qk_norm_rope +
 * _qk_norm_rope_kernel:8-44).  Head h of sequence b of q starts at
 * q + b*q_bstride + h*q_hstride (likewise k); cos/sin rows of sequence b
 * start at cos + b*cs_bstride (0 = one row shared by the batch).
 * out_q is contiguous [batch, nq, 128], out_k [batch, nk, 128].
 */
int qf_qk_norm_rope(const void* q, const void* k, int64_t batch, int32_t nq,
                    int32_t nk, int64_t q_bstride, int64_t q_hstride,
                    int64_t k_bstride, int64_t k_hstride,
                    const void* q_weight, const void* k_weight,
                    const void* cos, const void* sin, int64_t cs_bstride,
                    float q_eps, float k_eps, void* out_q, void* out_k,
                    void* stream);

/*
 * Packed decode Q/K/V: per-head norm + RoPE of the q and k heads of one
 * packed [q | k | v] row per sequence, at the slot `*position` read on the
 * device; K and V rows go straight into cache slot `position`.
 * Replaces engine/kernels/decode_fused.py:172-210 (qkv_norm_rope_cache +
 * _qkv_norm_rope_cache_kernel:59-118).
 *   qkv: bf16 [batch, (nq + 2 nk) * 128] when splits == 0, else f32 split-K
 *        partials [splits, batch, (nq + 2 nk) * 128], summed in order from 0
 *        and rounded once to bf16.
 *   cos, sin: bf16 [capacity, 128] tables; position: one int64 on the device.
 *   q_out: bf16 [batch, nq, 128]; key_cache, value_cache: bf16
 *        [batch, nk, capacity, 128], only slot `position` is written.
 * A position outside [0, capacity) writes no cache row and fills q_out with
 * bf16 NaN (0x7FC0) instead of reading or writing out of bounds.
 */
int qf_qkv_norm_rope_cache(const void* qkv, int32_t splits, int64_t batch,
                           int32_t nq, int32_t nk, const void* q_weight,
                           const void* k_weight, float q_eps, float k_eps,
                           const void* cos, const void* sin,
                           const int64_t* position, int64_t capacity,
                           void* q_out, void* key_cache, void* value_cache,
                           void* stream);

/*
 * Packed prefill Q/K/V for a fresh prompt of `length` tokens per sequence:
 * token t of sequence b sits at slot t.  Same arithmetic as
 * qf_qkv_norm_rope_cache.  Replaces engine/kernels/prefill.py:66-96
 * (prefill_qkv + _prefill_qkv:19-63).
 *   qkv: bf16 [batch*length, (nq + 2 nk) * 128]; cos/sin bf16 [capacity, 128]
 *   q_out: bf16 [batch, length, nq, 128]
 *   key_cache/value_cache: bf16 [batch, nk, capacity, 128], only slots
 *   [0, length) are written.
 */
int qf_prefill_qkv(const void* qkv, int64_t batch, int64_t length, int32_t nq,
                   int32_t nk, const void* q_weight, const void* k_weight,
                   float q_eps, float k_eps, const void* cos, const void* sin,
                   int64_t capacity, void* q_out, void* key_cache,
                   void* value_cache, void* stream);

/*
 * Causal attention of a fresh prompt over its own K/V cache slots, grouped
 * query heads (G = q_heads / kv_heads query heads per KV head).  Replaces the
 * prefill's call of torch's dense causal flash attention,
 * engine/prefill.py:13-23 (_native_attention: aten._flash_attention_forward
 * with is_causal on q and the cache views k/v[:, :, :length]):
 *   out[b, t, h] = bf16( softmax_{j <= t}((q[b,t,h] . k[b, h/G, j]) * scale)
 *                        @ v[b, h/G, j] )
 * with f32 scores and running softmax statistics, the probabilities rounded
 * to bf16 before they multiply V, and the f32 result divided by its f32
 * denominator once.
 *   q:   bf16 [batch, length, q_heads, 128] (the layout qf_prefill_qkv writes)
 *   key_cache/value_cache: bf16 [batch, kv_heads, capacity, 128]; slots
 *        [0, length) are read, nothing at or past `length` is attended.
 *   out: bf16 [batch, length, q_heads, 128]
 * G must be 1, 2, 4 or 8 (QF_E_SHAPE otherwise); every pointer 16-byte
 * aligned.  One launch (matrix-core scores and P V, keys staged in LDS).
 */
int qf_prefill_attention(const void* q, const void* key_cache, const void* value_cache,
                         int64_t batch, int64_t length, int32_t q_heads, int32_t kv_heads,
                         int64_t capacity, float scale, void* out, void* stream);

/*
 * Token embedding gather, bit-exact: out[i, :] = table[ids[i], :].
 * Replaces the nn.Embedding call base.embed_tokens(ids) at
 * engine/decode_step.py:38, engine/prefill.py:34, engine/decode.py:19.
 * An id outside [0, vocab) yields a zero row (never an out-of-bounds read).
 */
int qf_embedding(const int64_t* ids, int64_t n_ids, const void* table,
                 int64_t vocab, int64_t cols, void* out, void* stream);

/*
 * Rotary cos/sin tables (Qwen3 default RoPE):
 *   ang[p, j] = inv_freq[j] * float(pos_p)  (one f32 product),  j < half
 *   cos[p, j] = cos[p, j + half] = bf16(cos(ang)),  sin likewise.
 * pos_p = positions[p] when positions != NULL, else start + p.
 * Replaces the table build of engine/decode.py:52-59, which evaluates
 * Qwen3RotaryEmbedding.forward (transformers models/qwen3/modeling_qwen3.py)
 * for every cache slot.  cos/sin are contiguous bf16 [n_pos, 2*half].
 */
int qf_rope_table(const float* inv_freq, int32_t half, const int64_t* positions,
                  int64_t start, int64_t n_pos, void* cos, void* sin,
                  void* stream);

/*
 * Decode projections for at most 64 rows (the shape rule of
 * engine/kernels/skinny_gemm.py:75-83 supports()): x bf16 [rows, k] and
 * W bf16 [n, k], both contiguous; 1 <= rows <= 64, k % 64 == 0, n % 32 == 0;
 * x, W and partials 16-byte aligned.  Otherwise QF_E_SHAPE / QF_E_ALIGN.
 *
 * qf_linear_splits: the number of K splits qf_linear_partials is meant to be
 * called with for this shape (>= 1, a power of two dividing k / 64), or a
 * negative status.  Replaces split_count (engine/kernels/skinny_gemm.py:86-91);
 * unlike the reference's it also depends on rows.
 */
int qf_linear_splits(int64_t rows, int64_t k, int64_t n);

/*
 * f32 split-K partials of y = x @ W^T:
 *   partials[s, m, j] = sum over c in [s*k/splits, (s+1)*k/splits) of
 *                       float(x[m, c]) * float(W[j, c])
 * accumulated in f32 (products exact; addition order fixed by the matrix
 * cores, deterministic).  partials is contiguous f32 [splits, rows, n];
 * splits >= 1 must divide k / 64 (QF_E_ARG otherwise).  qf_add_rms_norm and
 * qf_qkv_norm_rope_cache take the result directly.
 * Replaces linear_partials + _partials_kernel (engine/kernels/skinny_gemm.py:
 * 28-46, 100-109).
 */
int qf_linear_partials(const void* x, int64_t rows, int64_t k, const void* weight,
                       int64_t n, int32_t splits, void* partials, void* stream);

/*
 * qf_linear_partials of the attention output, taken from the unmerged
 * segments of qf_decode_attention / qf_decode_attention_qkv (called with
 * out = NULL): x = the merge those calls would have written, bf16
 * [batch, q_heads * 128], k = q_heads * 128.  Each projection workgroup
 * merges the heads of its own K range into LDS while its first weight
 * chunks are in flight, so the attention needs no merge launch and x never
 * goes to memory.  seg_partials / seg_stats / seg_splits (>= 2) are the
 * attention's scratch and splits; 1 <= batch <= 16; splits must divide
 * k / 64 into an even number of chunks (whole heads per split), and
 * batch * (k / splits * 2 + 16) bytes must fit 64 KiB (QF_E_ARG /
 * QF_E_SHAPE otherwise).  Bit-identical to the attention's merge followed
 * by qf_linear_partials with the same splits.
 * Replaces the hand-off engine/decode_step.py:48-52 makes from the
 * attention's merged output (the _merge kernel of
 * engine/kernels/small_query_attention.py:88-110) to linear_partials for
 * o_proj (engine/kernels/skinny_gemm.py:100-109).
 */
int qf_linear_partials_merged(const float* seg_partials, const float* seg_stats,
                              int32_t seg_splits, int64_t batch, int32_t q_heads,
                              int32_t kv_heads, const void* weight, int64_t n, int32_t splits,
                              void* partials, void* stream);

/*
 * Decode gate/up projection with the SiLU * up epilogue, for a packed
 * weight gate_up bf16 [2n, k] (gate rows first):
 *   g = bf16(x @ gate^T),  u = bf16(x @ up^T)     (f32 accumulation, as above)
 *   out[m, j] = bf16(float(bf16(silu(g))) * float(u)),  silu(g) = g / (1 + exp(-g))
 * out is contiguous bf16 [rows, n], 8-byte aligned.
 * Replaces linear_silu_mul + _silu_mul_kernel (engine/kernels/skinny_gemm.py:
 * 49-72, 112-121).
 */
int qf_linear_silu_mul(const void* x, int64_t rows, int64_t k, const void* gate_up,
                       int64_t n, void* out, void* stream);

/*
 * Decode projections at 1..4 rows as QF_ROW_GROUPS workgroups (one per
 * compute unit), each over the whole K range of n / QF_ROW_GROUPS columns,
 * so that the residual add and the RMSNorm of the decode step's add + norm
 * launch move into the projections on either side of it.  They replace the
 * down projection + add + norm of engine/decode_step.py:56-59,
 * linear_partials (engine/kernels/skinny_gemm.py:100-109) then add_rms_norm
 * (engine/kernels/decode_fused.py:140-160), and the next layer's qkv
 * projection of the normalised row (engine/decode_step.py:43-44).
 *
 * Shapes: x / total bf16 [rows, k], weight bf16 [n, k], all contiguous and
 * 16-byte aligned; k % 8 == 0; n = QF_ROW_GROUPS * c with
 * c in {2, 4, 8, 10, 16, 24, 32} and (rows <= 2 ? rows : 4) * c <= 128;
 * qf_row_supported answers for a shape, others get QF_E_SHAPE.  sq is
 * f64 [rows, QF_ROW_GROUPS], 8-byte aligned.
 *
 * qf_linear_rows:     out = bf16(x W^T)  (f32 accumulation).
 * qf_linear_residual: y = bf16(x W^T);  total = bf16(residual + y) (total
 *                     may alias residual) and sq[r][g] = the f64 sum of
 *                     total[r][j]^2 over workgroup g's columns j.
 * qf_linear_normed:   x = bf16(bf16(total * inv) * gain) with
 *                     inv = 1 / sqrt(f32(sum_g sq[r][g]) / k + eps), the
 *                     rounding steps of qf_add_rms_norm (so x equals the row
 *                     it would write); out = bf16(x W^T).
 */
#define QF_ROW_GROUPS 256
int qf_row_supported(int32_t rows, int64_t k, int64_t n);
int qf_linear_rows(const void* x, int32_t rows, int64_t k, const void* weight, int64_t n,
                   void* out, void* stream);
int qf_linear_residual(const void* x, int32_t rows, int64_t k, const void* weight, int64_t n,
                       const void* residual, void* total, double* sq, void* stream);
int qf_linear_normed(const void* total, const double* sq, const void* gain, float eps,
                     int32_t rows, int64_t k, const void* weight, int64_t n, void* out,
                     void* stream);

/*
 * The other half of a decoder layer in the same form: the attention's output
 * projection with the residual add (replacing engine/decode_step.py:48-52,
 * o_proj then add_rms_norm), and the gate/up projection of the normalised
 * row with the SiLU * up epilogue (engine/decode_step.py:53,
 * linear_silu_mul of add_rms_norm's output; engine/kernels/skinny_gemm.py:
 * 112-121).
 *
 * qf_linear_residual_merged: x = the merge of the decode attention's key
 *   segments, exactly as qf_linear_partials_merged takes them (seg_partials
 *   f32 [rows * kv_heads, segments, G, 128], seg_stats f32
 *   [rows * kv_heads, segments, 2, G], 2 <= segments <= 32; the bits of the
 *   attention's own merge), k = q_heads * 128; then as qf_linear_residual.
 *   qf_row_merged_supported answers for a shape (the merged rows are staged
 *   in LDS: (rows <= 2 ? rows : 4) * k <= 32768).
 * qf_linear_silu_mul_normed: x = the normalised row as qf_linear_normed;
 *   g = bf16(x @ gate^T), u = bf16(x @ up^T) for the packed gate_up bf16
 *   [2n, k] (gate rows first); out bf16 [rows, n] =
 *   bf16(float(bf16(silu(g))) * float(u)), the SiLU of qf_linear_silu_mul.
 *   2n = QF_ROW_GROUPS * c with c in {4, 8, 16, 32, 76} and
 *   (rows <= 2 ? rows : 4) * c <= 128 (qf_row_silu_supported).
 */
int qf_row_merged_supported(int32_t rows, int32_t segments, int32_t q_heads, int32_t kv_heads,
                            int64_t n);
int qf_linear_residual_merged(const float* seg_partials, const float* seg_stats,
                              int32_t segments, int32_t rows, int32_t q_heads, int32_t kv_heads,
                              const void* weight, int64_t n, const void* residual, void* total,
                              double* sq, void* stream);
int qf_row_silu_supported(int32_t rows, int64_t k, int64_t n);
int qf_linear_silu_mul_normed(const void* total, const double* sq, const void* gain, float eps,
                              int32_t rows, int64_t k, const void* gate_up, int64_t n, void* out,
                              void* stream);

/*
 * The same normalisation on the matrix-core projections instead of the row
 * kernels: the consumers of a qf_linear_residual producer (its total and sq)
 * at 1..4 rows, as many workgroups as qf_linear_partials /
 * qf_linear_silu_mul launch.  Each workgroup first normalises the rows'
 * slice of its own K range into LDS (x = bf16(bf16(total * inv) * gain) with
 * inv = 1 / sqrt(f32(sum_g sq[r][g]) / k + eps), the rounding steps of
 * qf_add_rms_norm) while its first weight chunks are in flight, then runs
 * the tiles of the plain entry point, so the result is bit-identical to
 * qf_linear_partials / qf_linear_silu_mul called on the row qf_add_rms_norm
 * writes.  They replace, like qf_linear_normed
 * and qf_linear_silu_mul_normed, add_rms_norm (engine/kernels/
 * decode_fused.py:140-160) followed by linear_partials / linear_silu_mul
 * (engine/kernels/skinny_gemm.py:100-121) at engine/decode_step.py:43-44
 * and :53.
 *
 * total bf16 [rows, k], gain bf16 [k] and the weight 16-byte aligned, sq f64
 * [rows, QF_ROW_GROUPS] 8-byte aligned; 1 <= rows <= 4; k % 64 == 0 and
 * n % 32 == 0 as qf_linear_partials (splits as there); the slice,
 * rows * k / splits values (qf_linear_silu_mul_normed_tiled: rows * k), at
 * most 10,240.  Otherwise QF_E_SHAPE / QF_E_ARG / QF_E_ALIGN as the plain
 * entry points.
 */
int qf_linear_partials_normed(const void* total, const double* sq, const void* gain, float eps,
                              int64_t rows, int64_t k, const void* weight, int64_t n,
                              int32_t splits, void* partials, void* stream);
int qf_linear_silu_mul_normed_tiled(const void* total, const double* sq, const void* gain,
                                    float eps, int64_t rows, int64_t k, const void* gate_up,
                                    int64_t n, void* out, void* stream);

/*
 * Key-segment plan of qf_decode_attention for virtual_heads = batch * Hkv
 * heads of a cache with `capacity` slots on a GPU with compute_units CUs:
 * at most one workgroup per CU, segments of whole 64-key tiles, at most 32.
 * Writes *splits >= 1 and *span (keys per segment, a multiple of 64) with
 * (splits - 1) * span < capacity <= splits * span.
 * Replaces partition_keys (engine/kernels/small_query_attention.py:24-38).
 */
int qf_attention_partition(int64_t virtual_heads, int64_t capacity, int32_t compute_units,
                           int32_t* splits, int64_t* span);

/*
 * The plan qf_attention_partition aims for (at most one workgroup per CU,
 * at most 32 segments, at least one 64-key tile each) with the segment
 * lengths balanced to `align` (16, 32 or 64) keys instead of whole 64-key
 * tiles, so the aimed-for count is kept where 64-key rounding drops a
 * segment (4 x 2081 keys: 8 x 272 instead of 7 x 320): span a multiple of
 * align, (splits - 1) * span < capacity <= splits * span.  No counterpart in
 * the reference, whose partition_keys contract fixes 64-key tiles; the
 * Engine's decode step uses align 16 (qf_decode_attention accepts any span
 * that is a multiple of 16).
 */
int qf_attention_partition_aligned(int64_t virtual_heads, int64_t capacity, int32_t compute_units,
                                   int32_t align, int32_t* splits, int64_t* span);

/*
 * Decode attention, one query token per sequence, grouped-query heads:
 *   q bf16 [batch, q_heads, 1, 128]; k, v bf16 [batch, kv_heads, capacity, 128]
 *   (all contiguous); used int32 [batch * kv_heads] on the device: keys
 *   0 .. used-1 of each (sequence, kv head) are attended (clamped to
 *   [0, capacity]); slots at or beyond used are never read.
 *   Query head h of sequence b reads kv head h / (q_heads / kv_heads).
 *   s = (q . k) * scale; out = softmax(s) @ v with f32 statistics, the
 *   probabilities rounded to bf16 before they multiply v, the result rounded
 *   once to bf16; no valid key -> zeros.  out bf16 [batch, 1, q_heads, 128].
 * q_heads / kv_heads <= 16.  (splits, span) as qf_attention_partition gives
 * (any split of the capacity into whole 16-key multiples works).  splits > 1
 * needs scratch: partials f32 [batch*kv_heads, splits, G, 128] and stats f32
 * [batch*kv_heads, splits, 2, G] (G = q_heads / kv_heads); calls sharing it
 * must be ordered on one stream.  One launch per 8 query rows of a group
 * (one for Qwen3's G = 4), plus a merge launch when splits > 1.  With
 * splits > 1, out may be NULL: the merge launch is skipped and the unmerged
 * segments stay in partials/stats for qf_linear_partials_merged.
 * Replaces SmallQueryAttention.run + _segments + _merge
 * (engine/kernels/small_query_attention.py:41-110, 135-158).
 */
int qf_decode_attention(const void* q, const void* k, const void* v, const int32_t* used,
                        int64_t batch, int32_t q_heads, int32_t kv_heads, int64_t capacity,
                        float scale, int32_t splits, int64_t span, float* partials,
                        float* stats, void* out, void* stream);

/*
 * qf_qkv_norm_rope_cache followed by qf_decode_attention on its Q, in the
 * attention launches (Q never goes to memory):
 *   qkv (bf16 [batch, (q_heads + 2 kv_heads) * 128], qkv_splits == 0, or f32
 *   partials [qkv_splits, batch, ...]), q/k gains, eps, cos/sin [capacity, 128]
 *   and the int64 device position as qf_qkv_norm_rope_cache takes them; the
 *   caches are the attention's k and v and get the new K/V row at slot
 *   position (a position outside [0, capacity) writes nothing and gives NaN
 *   queries, as there); used, scale, (splits, span), scratch and out as
 *   qf_decode_attention.  Bit-identical to the two calls in sequence.
 * Replaces the pair engine/decode_step.py:43-47 issues back to back:
 * qkv_norm_rope_cache (engine/kernels/decode_fused.py:59-118, 172-210) then
 * SmallQueryAttention.run (engine/kernels/small_query_attention.py:135-158),
 * saving the Q round trip and one launch per layer.
 */
int qf_decode_attention_qkv(const void* qkv, int32_t qkv_splits, const void* q_weight,
                            const void* k_weight, float q_eps, float k_eps, const void* cos,
                            const void* sin, const int64_t* position, void* key_cache,
                            void* value_cache, const int32_t* used, int64_t batch,
                            int32_t q_heads, int32_t kv_heads, int64_t capacity, float scale,
                            int32_t splits, int64_t span, float* partials, float* stats,
                            void* out, void* stream);

/*
 * Candidate slots per row that qf_lm_head_argmax needs (vocab / 16), or a
 * negative status when vocab is not a positive multiple of 16.
 */
int64_t qf_lm_head_blocks(int64_t vocab);

/*
 * LM head + greedy token selection (the final step of engine/decode.py:93,106
 * and engine/decode_step.py:64, `logits.argmax(-1)` of F.linear(normed, W)):
 *   logits[m, j] = bf16(x[m] . W[j])   (f32 accumulation on the matrix cores)
 *   tokens[m]    = argmax_j logits[m, j], the LOWEST j among equal maxima
 *                  (NaN counts as the maximum), as torch.argmax picks.
 * x bf16 [rows, k], W bf16 [vocab, k] (the tied embedding), both contiguous
 * and 16-byte aligned; 1 <= rows <= 64, k % 64 == 0, vocab % 16 == 0.
 * candidates: scratch of rows * qf_lm_head_blocks(vocab) 8-byte slots
 * (8-byte aligned; no initialisation needed).  tokens: int64 [rows].
 * logits: optional bf16 [rows, vocab] copy of the logits (NULL to skip).
 * Two launches (vocabulary tiles, then one workgroup per row).  No
 * counterpart kernel in the reference, whose engine calls F.linear and
 * torch.argmax (the fusion OPTIMIZATION_GUIDE.md:213 describes).
 */
int qf_lm_head_argmax(const void* x, int64_t rows, int64_t k, const void* weight, int64_t vocab,
                      void* candidates, int64_t* tokens, void* logits, void* stream);

/*
 * qf_lm_head_argmax whose second launch also advances the decode state by one
 * step, replacing the step's trailing `self.position.add_(1)`
 * (engine/decode.py:107) and the attention lengths' increment:
 *   position[0] += 1;  lengths[i] += 1 for i < length_count.
 * position: int64 (8-byte aligned); lengths: int32 [length_count] (4-byte
 * aligned; NULL when length_count is 0).  Nothing else in the call reads
 * them.  Same errors as qf_lm_head_argmax, plus QF_E_ARG / QF_E_ALIGN for
 * these two.
 */
int qf_lm_head_argmax_advance(const void* x, int64_t rows, int64_t k, const void* weight,
                              int64_t vocab, void* candidates, int64_t* tokens, void* logits,
                              int64_t* position, int32_t* lengths, int64_t length_count,
                              void* stream);

/* 8-byte candidate slots in qf_lm_head_argmax_static's scratch (8 MiB per GPU). */
#define QF_LM_HEAD_STATIC_SLOTS (1 << 20)

/*
 * qf_lm_head_argmax without the caller's candidate buffer and without any
 * allocation: the candidates live in a static device array of
 * QF_LM_HEAD_STATIC_SLOTS slots, one per GPU, held until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, results and status codes as
 * qf_lm_head_argmax minus `candidates`; QF_E_CAPACITY when
 * rows * qf_lm_head_blocks(vocab) exceeds QF_LM_HEAD_STATIC_SLOTS (64 rows
 * of a vocabulary up to 262,144).  Calls that overlap on one GPU (other
 * streams or threads) share the array and race: order them on one stream.
 * The array used is the one on the device `stream` belongs to (the current
 * device for the null stream).  The first call on a device looks its address
 * up (a host call, no allocation; briefly making that device current if it
 * is not) and keeps it, so a call under graph capture that is the first on
 * its device still captures only kernel launches.
 */
int qf_lm_head_argmax_static(const void* x, int64_t rows, int64_t k, const void* weight,
                             int64_t vocab, int64_t* tokens, void* logits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_FUSED_H */
