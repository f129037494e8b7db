// Causal prefill attention for gfx950 (the prompt's queries against the first
// `length` slots of the head-major K/V caches, grouped query heads).
//
// Reference: engine/prefill.py:13-23, which calls torch's dense causal flash
// attention (aten._flash_attention_forward, is_causal) on the packed
// prefill's Q [B, T, Hq, 128] and the cache views k/v[:, :, :T]:
//   out[b, t, h] = softmax_{j <= t}((q[b,t,h] . k[b,h/G,j]) * scale) @ v[b,h/G,j]
// evaluated online (flash attention): per query row a running maximum m,
// f32 denominator l and f32 numerator O, rescaled by 2^(m_old - m_new) as m
// grows; the probabilities are rounded to bf16 before they multiply V (as
// the flash kernel feeds them to its bf16 P V product) while l sums them in
// f32; only O / l is rounded to bf16.
//
// Work split: a workgroup (W = 4 or 8 waves) takes one (sequence, KV head)
// and QB consecutive query positions for all G query heads of that KV head,
// i.e. G QB / 16 tiles of 16 query rows (one head, 16 positions); wave w
// takes tiles w, w + W, ...  Workgroups run longest first (the last query
// blocks attend the most keys).  Keys stream in blocks of 64, staged once per
// workgroup in LDS (cooperative 16-byte loads into one of two buffers, the
// next block's loads in flight during this block's arithmetic) and shared by
// every tile, so the K/V bytes a CU pulls from L2 per flop shrink with the
// workgroup's query rows (the per-CU L2 request rate, not the matrix cores,
// bounded the 4-wave form).
//
// Both products are on the matrix cores (v_mfma_f32_16x16x32_bf16):
// * Scores, transposed: S^T = K Q^T for a 16-key tile is a chain of four
//   MFMAs (A = 16 keys x 32 dims from LDS, lane l reading key l % 16, dims
//   8 (l / 16) + 32 s; B = the tile's 16 query rows, kept in registers),
//   leaving lane l with S[query l % 16][keys 4 (l / 16) + i].
// * P V: two 16-key tiles form one 32-wide k step.  Lane l's eight A values
//   are its own probabilities: keys 4 (l / 16) + i of the first tile and of
//   the second, in that k-slot order; the B operand must list V in the same
//   order, which two ds_read_b64_tr_b16 per k step give: lane i of each
//   16-lane group receives element i % 4 of the 8 bytes lanes 4q + i / 4
//   address, so lane 4q + t addressing dims 16 db + 4t of key 4 (l / 16) + q
//   yields keys 4 (l / 16) + 0..3 of dim 16 db + l % 16.  Eight dim tiles of
//   16 cover the head; lane l accumulates O[query 4 (l / 16) + i][16 db + l % 16].
// Each lane keeps the running maximum and denominator of its own query
// (l % 16) over its own keys; the accumulators of query row r are rescaled
// with the factor of the lanes that own query r (fetched by shuffles) when
// some maximum of the tile moved.  K rows in LDS are 272 bytes (the score
// reads, 16 keys at one column per 16-lane group, fall on distinct banks),
// V rows 288 bytes (the transposing reads, 4 keys x 4 column groups per
// 16-lane group, on distinct banks).  Keys at or past `length` are never
// attended (causality); their loads read slot length - 1 instead, so stale
// or NaN cache contents past the prompt never reach a product.
#include "qf_device.h"

#include <type_traits>

namespace qf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

constexpr int kD = 128;
constexpr int kKB = 64;                 // keys per staged block
constexpr int kKRow = 272;              // LDS bytes per staged K row
constexpr int kVRow = 288;              // LDS bytes per staged V row
constexpr int kORow = 272;              // LDS bytes per row of the output staging tile
constexpr float kNegInf = -__builtin_inff();
constexpr float kLog2e = 1.4426950408889634f;
// A row's exponent offset (its reference maximum, log2 units) is raised only
// when a block's row maximum exceeds it by more than this, so unnormalised
// probabilities stay below 2^8 and the accumulators are rarely rescaled.
constexpr float kLazy = 8.0f;

struct PrefillArgs {
  const uint16_t* q;   // [B, T, Hq, 128]
  const uint16_t* k;   // [B, Hkv, C, 128]
  const uint16_t* v;
  uint16_t* out;       // [B, T, Hq, 128]
  int64_t length, capacity;
  int32_t q_heads, kv_heads;
  int32_t qblocks;     // ceil(T / query positions per workgroup)
  int32_t pairs;       // B * Hkv
  float scale_log2;    // |scale| * log2(e)
  uint32_t qsign;      // 0x80008000 when scale < 0: Q enters negated (exact in bf16)
};

// Work split per group size G (query heads per KV head): QB query positions
// per workgroup (a divisor of the key block, so a workgroup's queries share
// one diagonal block), W waves per workgroup and TPW 16-row tiles per wave,
// G * QB / 16 = W * TPW.  Each staged key block serves all of a workgroup's
// G * QB query rows, so its K/V traffic from L2 per flop falls as that grows:
// at G = 4, 8 waves of 64 positions (256 rows) need half the block loads of
// two 4-wave workgroups of 32 (the same two waves per SIMD).
// WIDE (8 waves) is taken when the grid still has two workgroups per CU;
// smaller prompts keep the 4-wave form's twice as many workgroups.
template <int G, bool WIDE> struct Split;
template <bool WIDE> struct Split<1, WIDE> { static constexpr int QB = 64, TPW = 1, W = 4; };
template <bool WIDE> struct Split<2, WIDE> { static constexpr int QB = 64, TPW = 2, W = 4; };
template <> struct Split<4, false> { static constexpr int QB = 32, TPW = 2, W = 4; };
template <> struct Split<4, true> { static constexpr int QB = 64, TPW = 2, W = 8; };
template <> struct Split<8, false> { static constexpr int QB = 16, TPW = 2, W = 4; };
template <> struct Split<8, true> { static constexpr int QB = 32, TPW = 2, W = 8; };
constexpr int64_t kWideWorkgroups = 2 * kCUs;

__device__ __forceinline__ f32x4 mfma32(const uint4& a, const uint4& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ v4i16 read_tr(const uint8_t* base, int off) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)((__attribute__((address_space(3))) uint8_t*)base + off));
}

template <int G, bool WIDE>
__global__ __launch_bounds__((Split<G, WIDE>::W * kWave)) void prefill_attn_kernel(PrefillArgs a) {
  constexpr int QB = Split<G, WIDE>::QB;
  constexpr int TPW = Split<G, WIDE>::TPW;
  constexpr int W = Split<G, WIDE>::W;
  constexpr int kThreads = W * kWave;
  constexpr int kSubs = QB / 16;  // position tiles per head
  constexpr int kLoadsPerThread = kKB * kD * 2 / 16 / kThreads;  // 16-byte loads per operand
  static_assert(G * kSubs == W * TPW, "every wave holds TPW tiles");
  static_assert(W % kSubs == 0, "a wave's tiles share their positions");
  static_assert(W * 16 * kORow <= 2 * kKB * kKRow, "output staging fits the K buffers");
  // Two K/V block buffers: block j + 1 is staged into one while block j is
  // read from the other, so one barrier per block separates the two.
  __shared__ __attribute__((aligned(16))) uint8_t klds[2][kKB * kKRow];
  __shared__ __attribute__((aligned(16))) uint8_t vlds[2][kKB * kVRow];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int r = lane % 16;
  const int g4 = lane / 16;
  // Longest workgroups first: the block index runs over (query block
  // descending, then sequence x KV head).
  const int qb = a.qblocks - 1 - (int)(blockIdx.x / a.pairs);
  const int pair = (int)(blockIdx.x % a.pairs);
  const int b = pair / a.kv_heads;
  const int kvh = pair % a.kv_heads;
  const int64_t p0 = (int64_t)qb * QB;
  const int64_t last = a.length - 1;
  const int nkb = (int)(p0 / kKB) + 1;  // key blocks: all below the diagonal one, and it
  const uint16_t* kbase = a.k + (int64_t)pair * a.capacity * kD;
  const uint16_t* vbase = a.v + (int64_t)pair * a.capacity * kD;

  // This wave's tiles: tile tau = wave + W u -> head kvh G + tau / kSubs,
  // positions p0 + 16 (tau % kSubs) .. +16 (the same positions for every
  // tile of a wave, since kSubs divides W).
  const int64_t pt = p0 + 16 * (wave % kSubs);
  int head[TPW];
  uint4 qf[TPW][4];
  const int64_t qpos = pt + r < a.length ? pt + r : last;
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    head[u] = kvh * G + (wave + W * u) / kSubs;
    const uint16_t* qr = a.q + (((int64_t)b * a.length + qpos) * a.q_heads + head[u]) * kD;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint4 x = load16<false>(qr + 8 * g4 + 32 * s);
      qf[u][s] = make_uint4(x.x ^ a.qsign, x.y ^ a.qsign, x.z ^ a.qsign, x.w ^ a.qsign);
    }
  }

  float mq[TPW], lq[TPW];
  f32x4 o[TPW][8];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    mq[u] = kNegInf;
    lq[u] = 0.0f;
#pragma unroll
    for (int db = 0; db < 8; ++db) o[u][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Cooperative block loads: thread tid moves 16-byte chunk tid % 16 of keys
  // tid / 16 + (kThreads / 16) i of the block, for K and for V.
  uint4 kreg[kLoadsPerThread], vreg[kLoadsPerThread];
  const int chunk = tid % 16;
  auto fetch = [&](int j) {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      int64_t key = (int64_t)j * kKB + tid / 16 + (kThreads / 16) * i;
      key = key < a.length ? key : last;
      kreg[i] = load16<true>(kbase + key * kD + 8 * chunk);
      vreg[i] = load16<true>(vbase + key * kD + 8 * chunk);
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kLoadsPerThread; ++i) {
      const int key = tid / 16 + (kThreads / 16) * i;
      *reinterpret_cast<uint4*>(klds[buf] + key * kKRow + 16 * chunk) = kreg[i];
      *reinterpret_cast<uint4*>(vlds[buf] + key * kVRow + 16 * chunk) = vreg[i];
    }
  };

  const int vrd = (4 * g4 + (r >> 2)) * kVRow + 8 * (r & 3);
  // One staged key block against this wave's tiles.  On the diagonal block
  // (the last) keys past a row's position are masked and 16-key tiles that
  // start past the wave's last position are skipped; every other block is
  // entirely visible to every row.
  auto attend = [&](const uint8_t* kb, const uint8_t* vb, int64_t key0, auto diag_tag) {
    constexpr bool kDiag = decltype(diag_tag)::value;
    const int ktn = kDiag ? (int)((pt + 15 - key0) >> 4) + 1 : 4;  // wave-uniform, 1..4
    // S^T for the attended 16-key tiles of the block, every query tile.
    f32x4 c[TPW][4];
#pragma unroll
    for (int u = 0; u < TPW; ++u)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) c[u][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      if (kDiag && kt >= ktn) break;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 kf = *reinterpret_cast<const uint4*>(kb + (16 * kt + r) * kKRow + 16 * (g4 + 4 * s));
#pragma unroll
        for (int u = 0; u < TPW; ++u) c[u][kt] = mfma32(kf, qf[u][s], c[u][kt]);
      }
    }
    uint4 pa[TPW][2];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      // Lane: query pt + r, keys key0 + 16 kt + 4 g4 + i (raw dot products).
      bool live[4][4];
      float bm = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          live[kt][i] = !kDiag || key0 + 16 * kt + 4 * g4 + i <= pt + r;
          bm = fmaxf(bm, live[kt][i] ? c[u][kt][i] : kNegInf);
        }
      bm = fmaxf(bm, __shfl_xor(bm, 16));
      bm = fmaxf(bm, __shfl_xor(bm, 32));
      bm *= a.scale_log2;  // the row's scaled maximum (rounding is monotonic)
      if (__builtin_amdgcn_ballot_w64(bm > mq[u] + kLazy) != 0) {  // wave-uniform
        // Raise the offsets to the block maxima; O row 4 g4 + i belongs to
        // query 4 g4 + i, whose factor lane 4 g4 + i holds.
        const float mn = fmaxf(mq[u], bm);
        const float corr = exp2_hw(mq[u] - mn);
        lq[u] *= corr;
        mq[u] = mn;
        float cr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) cr[i] = __shfl(corr, 4 * g4 + i);
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[u][db][i] *= cr[i];
      }
      const float nm = -mq[u];
      float p[4][4], ps = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[kt][i] = live[kt][i] ? exp2_hw(fmaf(c[u][kt][i], a.scale_log2, nm)) : 0.0f;
          ps += p[kt][i];
        }
      lq[u] += ps;
      // The probabilities, rounded to bf16, as the A operand of the two k steps.
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        pa[u][ks] = make_uint4(pack2(p[2 * ks][0], p[2 * ks][1]), pack2(p[2 * ks][2], p[2 * ks][3]),
                               pack2(p[2 * ks + 1][0], p[2 * ks + 1][1]),
                               pack2(p[2 * ks + 1][2], p[2 * ks + 1][3]));
    }
    const int ksn = ktn > 2 ? 2 : 1;  // 32-key steps with an attended tile
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (kDiag && ks >= ksn) break;
        const v4i16 lo = read_tr(vb, vrd + 32 * ks * kVRow + 32 * db);
        const v4i16 hi = read_tr(vb, vrd + (32 * ks + 16) * kVRow + 32 * db);
        const uint4 vt = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                    __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
#pragma unroll
        for (int u = 0; u < TPW; ++u) o[u][db] = mfma32(pa[u][ks], vt, o[u][db]);
      }
  };

  fetch(0);
  stage(0);
  __syncthreads();
  for (int j = 0; j + 1 < nkb; ++j) {
    // Block j is in buffer j % 2; block j + 1's loads fly during its
    // arithmetic and land in the other buffer, last read during block j - 1
    // (before the previous barrier).
    fetch(j + 1);
    attend(klds[j & 1], vlds[j & 1], (int64_t)j * kKB, std::false_type{});
    stage((j + 1) & 1);
    __syncthreads();
  }
  attend(klds[(nkb - 1) & 1], vlds[(nkb - 1) & 1], (int64_t)(nkb - 1) * kKB, std::true_type{});

  // O / l in bf16, through LDS (this wave's 16 x 128 tile, one tile at a
  // time) so that every lane stores 16 contiguous bytes of one output row.
  __syncthreads();  // every wave is done with the K/V blocks
  uint8_t* ot = reinterpret_cast<uint8_t*>(klds) + wave * 16 * kORow;  // both K buffers
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    float lt = lq[u] + __shfl_xor(lq[u], 16);
    lt += __shfl_xor(lt, 32);  // lanes of query r: its denominator
    float inv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float den = __shfl(lt, 4 * g4 + i);
      inv[i] = 1.0f / den;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint16_t*>(ot + (4 * g4 + i) * kORow + 2 * (16 * db + r)) =
            to_bf16(o[u][db][i] * inv[i]);
    wave_lds_fence();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int row = g4 + 4 * k;
      const int64_t pos = pt + row;
      const uint4 val = *reinterpret_cast<const uint4*>(ot + row * kORow + 16 * r);
      if (pos < a.length)
        store16<false>(a.out + (((int64_t)b * a.length + pos) * a.q_heads + head[u]) * kD + 8 * r, val);
    }
    wave_lds_fence();  // reads done before the next tile's writes
  }
}

template <int G, bool WIDE>
int launch_prefill_as(PrefillArgs a, hipStream_t s) {
  constexpr int QB = Split<G, WIDE>::QB;
  a.qblocks = (int32_t)((a.length + QB - 1) / QB);
  const int64_t blocks = (int64_t)a.qblocks * a.pairs;
  if (blocks > (int64_t)INT32_MAX) return QF_E_SHAPE;
  hipLaunchKernelGGL((prefill_attn_kernel<G, WIDE>), dim3((unsigned)blocks),
                     dim3(Split<G, WIDE>::W * kWave), 0, s, a);
  return launch_status();
}

template <int G>
int launch_prefill(PrefillArgs a, hipStream_t s) {
  const int64_t wide_blocks = (a.length + Split<G, true>::QB - 1) / Split<G, true>::QB * a.pairs;
  return wide_blocks >= kWideWorkgroups ? launch_prefill_as<G, true>(a, s)
                                        : launch_prefill_as<G, false>(a, s);
}

}  // namespace
}  // namespace qf

using namespace qf;

extern "C" int qf_prefill_attention(const void* q, const void* key_cache, const void* value_cache,
                                    int64_t batch, int64_t length, int32_t q_heads,
                                    int32_t kv_heads, int64_t capacity, float scale, void* out,
                                    void* stream) {
  if (batch < 1 || length < 1 || capacity < length || q_heads < 1 || kv_heads < 1) return QF_E_ARG;
  if (!q || !key_cache || !value_cache || !out) return QF_E_ARG;
  if (!(scale == scale) || scale == __builtin_inff() || scale == -__builtin_inff()) return QF_E_ARG;
  if (q_heads % kv_heads != 0) return QF_E_SHAPE;
  const int32_t groups = q_heads / kv_heads;
  if (groups != 1 && groups != 2 && groups != 4 && groups != 8) return QF_E_SHAPE;
  if (!aligned16(q) || !aligned16(key_cache) || !aligned16(value_cache) || !aligned16(out))
    return QF_E_ALIGN;
  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(key_cache);
  a.v = static_cast<const uint16_t*>(value_cache);
  a.out = static_cast<uint16_t*>(out);
  a.length = length;
  a.capacity = capacity;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  if (batch * kv_heads > INT32_MAX) return QF_E_SHAPE;
  a.qblocks = 0;
  a.pairs = (int32_t)(batch * kv_heads);
  a.scale_log2 = (scale < 0.0f ? -scale : scale) * kLog2e;
  a.qsign = scale < 0.0f ? 0x80008000u : 0u;
  hipStream_t s = as_stream(stream);
  switch (groups) {
    case 1: return launch_prefill<1>(a, s);
    case 2: return launch_prefill<2>(a, s);
    case 4: return launch_prefill<4>(a, s);
    default: return launch_prefill<8>(a, s);
  }
}
