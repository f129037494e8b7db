// Grouped-query decode attention for gfx950: one query token per sequence
// against the head-major K/V cache, split over key segments with an f32
// merge (engine/kernels/small_query_attention.py:41-110 is the reference:
// _segments :41-86, _merge :89-110).
//
// A virtual head vh = batch * Hkv + kv_head owns G = Hq / Hkv query rows
// (flattened query row vh * G + g) and the first used[vh] keys of its cache
// rows [vh * capacity, ...).  Per query row, with s = (q . k) * scale * log2 e:
//   out = sum_k bf16(2^(s_k - m)) * v_k / sum_k 2^(s_k - m),  m = max_k s_k
// evaluated online: each key segment keeps a running maximum m, f32
// denominator l and f32 numerator, rescaled by 2^(m_old - m_new) as the
// maximum grows; the probabilities that multiply V are rounded to bf16 first
// (as the reference feeds them to a bf16 dot) while l sums them in f32.
// Segments are merged with weights 2^(m_s - M), in segment order, by a
// second small kernel; only the merged result is rounded to bf16.  Keys at
// or beyond used[vh] are never loaded, so stale values (NaN poison included)
// in unused cache slots stay invisible.
//
// Groups of up to 4 query rows (Qwen3-4B's 4) take attn_mfma_kernel, which
// computes both the scores and P V on the matrix cores (see there); wider
// groups take attn_kernel, all on the VALU, described next.
//
// Layout (HBM-bound: every K/V byte of the used prefix is read once, ~4
// flops per byte): a wave reads 4 consecutive keys per 16-byte load - 16
// lanes per 256-byte key row, lane r holding d = 8r .. 8r+8 - so every load
// is one contiguous KiB.  Scores use v_dot2c_f32_bf16 on the packed bf16
// pairs and a 16-lane DPP sum; the numerator update is f32 FMAs.  The 16
// lane groups of a workgroup (4 per wave x 4 waves) take interleaved keys of
// the segment, each with its own running state, and are merged in lane-group
// then wave order at the end.
#include "qf_device.h"
#include "qf_merge.h"
#include "qf_rope.h"

namespace qf {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kD = 128;
constexpr int kKeysPerWave = 4;                       // one 1 KiB load = 4 key rows
constexpr int kSpanAlign = 16;                        // segment lengths are multiples of 16
constexpr int kMaxGroups = 16;
constexpr int kMaxSplits = kMaxSegments;
constexpr float kNegInf = -__builtin_inff();

struct AttnArgs {
  const uint16_t* q;     // [vh * G, 128]
  const uint16_t* k;     // [vh * capacity, 128]
  const uint16_t* v;
  const int32_t* used;   // [vh]
  float* partials;       // [vh, S, G, 128]
  float* stats;          // [vh, S, 2, G]: maxima then denominators
  uint16_t* out;         // [vh * G, 128]
  int64_t capacity;
  int32_t groups;        // G
  int32_t g0;            // first query row of the group this launch handles
  int32_t splits;
  int32_t span;          // keys per segment
  float scale_log2;      // scale * log2(e)
  // Fused Q/K/V prologue (qf_decode_attention_qkv only): Q comes from the
  // packed projection row instead of `q`, and the new K/V row goes to slot
  // *position of the caches (`k` / `v` viewed writable).
  const void* qkv;       // bf16 [batch, W] or f32 partials [qkv_splits, batch, W]
  int32_t qkv_splits;    // 0: bf16 rows
  int32_t kv_heads;
  int64_t qkv_stride;    // batch * W: f32 elements between partials
  const uint16_t* qw;
  const uint16_t* kw;
  float q_eps, k_eps;
  const uint16_t* cos;   // [capacity, 128]
  const uint16_t* sin;
  const int64_t* position;
  uint16_t* kc;
  uint16_t* vc;
  // Phase timestamps (the instrumented build only; see kPhases).
  uint64_t* stamps;
};

// Phase boundaries an instrumented attention workgroup records
// (s_memrealtime: the constant clock, one time base for every CU).  Wave 0:
//   0 entry; 1 `used` and the position have arrived; 2 the fused prologue's
//   loads (and the first key blocks behind them) are issued; 3 the queries
//   are normalised, rotated and in every wave (after the barrier); 4 the
//   wave's first key block is consumed (its loads landed, scores, softmax
//   and P V done); 5 the key loop is done; 6 the four waves are merged;
//   7 the output or partials are stored and acknowledged; 12 every wave has
//   passed the barrier before the merge.
// Wave w: 8 + w its key loop done; 12 + w (w > 0) its first block consumed.
// The merge kernel records 0 entry, 3 its first loads landed, 1 merged,
// 2 stored and acknowledged.
constexpr int kPhases = 16;
constexpr int kMergePhases = 4;

__device__ __forceinline__ uint64_t phase_clock() { return __builtin_amdgcn_s_memrealtime(); }

__device__ __forceinline__ float dpp_f32_sum16(float x) {
  // All-reduce over aligned 16-lane rows (every lane ends with the sum).
  x += __uint_as_float(dpp_u32<kQuadXor1>(__float_as_uint(x)));
  x += __uint_as_float(dpp_u32<kQuadXor2>(__float_as_uint(x)));
  x += __uint_as_float(dpp_u32<kRowHalfMirror>(__float_as_uint(x)));
  x += __uint_as_float(dpp_u32<kRowMirror>(__float_as_uint(x)));
  return x;
}

__device__ __forceinline__ float dot8(const uint4& a, const uint4& b) {
  float s = 0.0f;
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.x), __builtin_bit_cast(bf16x2, b.x), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.y), __builtin_bit_cast(bf16x2, b.y), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.z), __builtin_bit_cast(bf16x2, b.z), s, false);
  s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.w), __builtin_bit_cast(bf16x2, b.w), s, false);
  return s;
}

// Running softmax state of one lane group for GT query rows; the lane holds
// the numerator for d = 8r .. 8r+8.
template <int GT>
struct State {
  float m[GT], l[GT], acc[GT][8];
};

// Merge one row's state (om, ol, oacc) into row g of `s` (disjoint key sets).
template <int GT>
__device__ __forceinline__ void merge_row(State<GT>& s, int g, float om, float ol, const float* oacc) {
  const float mt = fmaxf(s.m[g], om);
  if (mt == kNegInf) return;  // both empty
  const float c1 = exp2_hw(s.m[g] - mt), c2 = exp2_hw(om - mt);
  s.l[g] = s.l[g] * c1 + ol * c2;
#pragma unroll
  for (int j = 0; j < 8; ++j) s.acc[g][j] = s.acc[g][j] * c1 + oacc[j] * c2;
  s.m[g] = mt;
}

// Merge the state of lane (lane ^ mask) into this lane's.
template <int GT>
__device__ __forceinline__ void merge_lanes(State<GT>& s, int mask) {
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    float oacc[8];
    const float om = __shfl_xor(s.m[g], mask);
    const float ol = __shfl_xor(s.l[g], mask);
#pragma unroll
    for (int j = 0; j < 8; ++j) oacc[j] = __shfl_xor(s.acc[g][j], mask);
    merge_row<GT>(s, g, om, ol, oacc);
  }
}

// The bf16-row form of fused_prologue in two halves, so a caller can issue
// other loads between the prologue's loads and their use.
struct PrologueLoads {
  uint4 wv, cv, sv, xv;
};

__device__ __forceinline__ PrologueLoads prologue_issue(const AttnArgs& a, int vh, int lg, int r,
                                                        int rows, int64_t pos) {
  const int G = a.groups;
  const int64_t hkv = a.kv_heads;
  const int64_t b = vh / hkv, h = vh - b * hkv;
  const int64_t hq = hkv * G;
  const int64_t width = (hq + 2 * hkv) * kD;
  const int64_t slot = pos >= 0 && pos < a.capacity ? pos : 0;
  const bool is_q = lg < rows, is_k = lg == 8;
  const int64_t head = is_q ? h * G + a.g0 + lg : is_k ? hq + h : hq + hkv + h;
  PrologueLoads L;
  L.wv = load16<false>((is_q ? a.qw : a.kw) + 8 * r);
  L.cv = load16<false>(a.cos + slot * kD + 8 * r);
  L.sv = load16<false>(a.sin + slot * kD + 8 * r);
  // every lane group loads a row of its virtual head (the value row when it
  // holds none), so the load count is fixed
  L.xv = load16<false>(static_cast<const uint16_t*>(a.qkv) + b * width + head * kD + 8 * r);
  return L;
}

// The split-K form for up to kPrologueSplits partials: every lane loads a
// partial of its row for each of the kPrologueSplits slots (slots past the
// split count re-read the last split and are not added), so the count is
// fixed; the sum runs in split order as sum_partials8's does.
constexpr int kPrologueSplits = 8;
struct PartialLoads {
  uint4 wv, cv, sv;
  float4 lo[kPrologueSplits], hi[kPrologueSplits];
};

__device__ __forceinline__ PartialLoads partials_issue(const AttnArgs& a, int vh, int lg, int r,
                                                       int rows, int64_t pos) {
  const int G = a.groups;
  const int64_t hkv = a.kv_heads;
  const int64_t b = vh / hkv, h = vh - b * hkv;
  const int64_t hq = hkv * G;
  const int64_t width = (hq + 2 * hkv) * kD;
  const int64_t slot = pos >= 0 && pos < a.capacity ? pos : 0;
  const bool is_q = lg < rows, is_k = lg == 8;
  const int64_t head = is_q ? h * G + a.g0 + lg : is_k ? hq + h : hq + hkv + h;
  PartialLoads L;
  L.wv = load16<false>((is_q ? a.qw : a.kw) + 8 * r);
  L.cv = load16<false>(a.cos + slot * kD + 8 * r);
  L.sv = load16<false>(a.sin + slot * kD + 8 * r);
  const float* p = static_cast<const float*>(a.qkv) + b * width + head * kD + 8 * r;
#pragma unroll
  for (int i = 0; i < kPrologueSplits; ++i) {
    const int s = i < a.qkv_splits ? i : a.qkv_splits - 1;
    const float4* q = reinterpret_cast<const float4*>(p + (int64_t)s * a.qkv_stride);
    L.lo[i] = q[0];
    L.hi[i] = q[1];
  }
  return L;
}

__device__ __forceinline__ uint4 partials_sum(const AttnArgs& a, const PartialLoads& L) {
  float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kPrologueSplits; ++i) {
    const bool on = i < a.qkv_splits;
    y[0] = on ? y[0] + L.lo[i].x : y[0];
    y[1] = on ? y[1] + L.lo[i].y : y[1];
    y[2] = on ? y[2] + L.lo[i].z : y[2];
    y[3] = on ? y[3] + L.lo[i].w : y[3];
    y[4] = on ? y[4] + L.hi[i].x : y[4];
    y[5] = on ? y[5] + L.hi[i].y : y[5];
    y[6] = on ? y[6] + L.hi[i].z : y[6];
    y[7] = on ? y[7] + L.hi[i].w : y[7];
  }
  return pack8(y);  // one rounding of the f32 sum
}

__device__ __forceinline__ bool prologue_finish(const AttnArgs& a, const PrologueLoads& L, int vh,
                                                int lg, int r, int rows, int64_t start, int64_t pos,
                                                uint4 (*qs)[16], uint4 (*kvs)[16]) {
  const bool pos_ok = pos >= 0 && pos < a.capacity;
  const bool is_q = lg < rows, is_k = lg == 8, is_v = lg == 9;
  // Lane groups without a row of their own work on the value row they
  // loaded (nothing of theirs is stored), so the load is used by every lane
  // and the compiler cannot sink it under a branch.
  const uint4 xv = L.xv;
  float x[8];
  unpack8(xv, x);
  const uint4 o = norm_rope(x, L.wv, L.cv, L.sv, is_q ? a.q_eps : a.k_eps, r);  // every lane: DPP
  const uint4 nan4 = make_uint4(0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u);
  if (is_q) qs[lg][r] = select4(pos_ok, o, nan4);
  if (is_k) kvs[0][r] = o;
  if (is_v) kvs[1][r] = xv;
  const bool owns_slot = pos_ok && pos >= start && pos < start + a.span;
  if (owns_slot && a.g0 == 0 && (is_k || is_v))
    store16<false>((is_k ? a.kc : a.vc) + ((int64_t)vh * a.capacity + pos) * kD + 8 * r,
                   select4(is_k, o, xv));
  return owns_slot;
}

// Fused Q/K/V prologue (qf_decode_attention_qkv), run by every lane of the
// workgroup before the key loop: lane group lg (16 lanes = one DPP row, lane
// r holding elements 8r..8r+8) folds or loads one packed row of virtual head
// vh - query rows g0 + lg for lg < rows, the new key row for lg == 8, the new
// value row for lg == 9 - and writes the normalised, rotated queries to
// qs[lg] and the new K / V rows to kvs[0] / kvs[1] (LDS; the caller
// synchronises before reading them).  The segment starting at `start` that
// owns slot `pos` also stores the new K / V row into the caches (first
// launch of a wide group only).  A position outside the cache gives NaN
// queries and writes nothing, as qf_qkv_norm_rope_cache does.  Returns
// whether this segment owns the slot.
__device__ __forceinline__ bool fused_prologue(const AttnArgs& a, int vh, int lg, int r, int rows,
                                               int64_t start, int64_t pos, uint4 (*qs)[16],
                                               uint4 (*kvs)[16]) {
  const int G = a.groups;
  const int64_t hkv = a.kv_heads;
  const int64_t b = vh / hkv, h = vh - b * hkv;
  const int64_t hq = hkv * G;
  const int64_t width = (hq + 2 * hkv) * kD;
  const bool pos_ok = pos >= 0 && pos < a.capacity;
  const int64_t slot = pos_ok ? pos : 0;
  const bool is_q = lg < rows, is_k = lg == 8, is_v = lg == 9;
  const bool live = is_q || is_k || is_v;
  const int64_t head = is_q ? h * G + a.g0 + lg : is_k ? hq + h : hq + hkv + h;
  const int64_t off = b * width + head * kD + 8 * r;
  // Gains and rotary rows first: the fold below waits for its loads, and
  // these should already be in flight by then.
  const uint4 wv = load16<false>((is_q ? a.qw : a.kw) + 8 * r);
  const uint4 cv = load16<false>(a.cos + slot * kD + 8 * r);
  const uint4 sv = load16<false>(a.sin + slot * kD + 8 * r);
  float x[8];
  uint4 xv;
  if (a.qkv_splits == 0) {
    xv = live ? load16<false>(static_cast<const uint16_t*>(a.qkv) + off) : make_uint4(0, 0, 0, 0);
  } else {
    sum_partials8<8>(static_cast<const float*>(a.qkv) + off, a.qkv_stride, a.qkv_splits, live, x);
    xv = pack8(x);  // one rounding of the f32 sum
  }
  unpack8(xv, x);
  const uint4 o = norm_rope(x, wv, cv, sv, is_q ? a.q_eps : a.k_eps, r);  // every lane: DPP
  const uint4 nan4 = make_uint4(0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u);
  if (is_q) qs[lg][r] = select4(pos_ok, o, nan4);
  if (is_k) kvs[0][r] = o;
  if (is_v) kvs[1][r] = xv;
  const bool owns_slot = pos_ok && pos >= start && pos < start + a.span;
  if (owns_slot && a.g0 == 0 && (is_k || is_v))
    store16<false>((is_k ? a.kc : a.vc) + ((int64_t)vh * a.capacity + pos) * kD + 8 * r,
                   select4(is_k, o, xv));
  return owns_slot;
}

// One workgroup per (virtual head, key segment), for query rows g0 .. g0+GT-1
// of the group (those below G); each lane group keeps NS sets of U key
// blocks (4 keys per wave each) in flight.  With one segment the workgroup
// writes the output; otherwise it writes its f32 partials and statistics for
// attn_merge_kernel.
//
// FUSED: the workgroup first does qf_qkv_norm_rope_cache's work for its
// virtual head: lane groups 0..rows-1 fold (or load) and normalise + rotate
// its query rows, lane groups 8 and 9 its new key and value row, all while the
// first key blocks are in flight.  Queries reach the other lane groups
// through LDS.  The segment that owns slot `position` writes the new K/V
// there (first launch of a wide group only) and uses the new rows in place
// of whatever the slot held when its loads were issued, so no workgroup
// reads back its own store.
template <int GT, int U, int W, bool FUSED, int NS = 2>
__global__ __launch_bounds__(W * kWave) void attn_kernel(AttnArgs a) {
  static_assert(NS >= 2, "at least two sets in flight");
  constexpr int kWavesA = W;
  constexpr int kKeysPerIter = kKeysPerWave * W;  // keys per workgroup step
  static_assert(!FUSED || (W == 4 && GT <= 8), "fused prologue: 16 lane groups, <= 8 query rows");
  __shared__ float xm[kWavesA - 1][GT], xl[kWavesA - 1][GT];
  __shared__ float xacc[kWavesA - 1][GT][kD];
  __shared__ uint4 qs[FUSED ? GT : 1][16], kvs[2][16];
  const int vh = blockIdx.x;
  const int seg = blockIdx.y;
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int r = lane % 16;   // d slice 8r .. 8r+8
  const int q4 = lane / 16;  // key within the wave's 4
  const int G = a.groups;
  const int rows = G - a.g0 < GT ? G - a.g0 : GT;  // query rows of this launch

  uint4 qv[GT];
  if constexpr (!FUSED) {
#pragma unroll
    for (int g = 0; g < GT; ++g)
      qv[g] = g < rows ? load16<false>(a.q + ((int64_t)vh * G + a.g0 + g) * kD + 8 * r)
                       : make_uint4(0, 0, 0, 0);
  }

  const int32_t used_in = a.used[vh];
  // Fused: the new key's slot, read alongside `used` so that the rotary-row
  // loads it addresses issue as early as the first key blocks (the empty asm
  // pins both scalar loads here instead of next to their first uses).
  const int64_t pos_in = FUSED ? *a.position : 0;
  if constexpr (FUSED) asm volatile("" ::"s"(used_in), "s"(pos_in));
  int64_t used = used_in;
  used = used < 0 ? 0 : (used > a.capacity ? a.capacity : used);
  const int64_t start = (int64_t)seg * a.span;
  int64_t end = start + a.span;
  if (end > used) end = used;
  const uint16_t* kb = a.k + (int64_t)vh * a.capacity * kD + 8 * r;
  const uint16_t* vb = a.v + (int64_t)vh * a.capacity * kD + 8 * r;

  State<GT> st;
#pragma unroll
  for (int g = 0; g < GT; ++g) {
    st.m[g] = kNegInf;
    st.l[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) st.acc[g][j] = 0.0f;
  }

  // Block set i of this wave: keys base0 + i*step + q4 + 16u, u < U.
  constexpr int64_t step = (int64_t)kKeysPerIter * U;
  const int64_t base0 = start + kKeysPerWave * wave;
  const int n = base0 < end ? (int)((end - base0 + step - 1) / step) : 0;
  const int64_t last_key = end - 1;  // a valid slot whenever n > 0
  uint4 kv[NS][U], vv[NS][U];
  // Fused: subst marks the segment that attends slot pos, whose new K/V row
  // (this lane's slice) is knew / vnew.
  int64_t pos = 0;
  bool subst = false;
  uint4 knew = make_uint4(0, 0, 0, 0), vnew = knew;
  // Loads are issued unconditionally (keys past the segment re-read its last
  // valid key, an L2 hit, and are masked out), so the compiler's wait counts
  // stay exact and the next set's loads overlap this set's arithmetic.
  auto issue = [&](int d, int i) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t key = base0 + i * step + q4 + (int64_t)kKeysPerIter * u;
      const int64_t kc = key < end ? key : last_key;
      kv[d][u] = load16<false>(kb + kc * kD);
      vv[d][u] = load16<false>(vb + kc * kD);
    }
  };
  auto consume = [&](int d, int i) {
    if constexpr (FUSED) {
      if (subst) {  // the new K/V row replaces slot pos wherever it was loaded
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t key = base0 + i * step + q4 + (int64_t)kKeysPerIter * u;
          if ((key < end ? key : last_key) == pos) {
            kv[d][u] = knew;
            vv[d][u] = vnew;
          }
        }
      }
    }
    float s[U][GT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool on = base0 + i * step + q4 + (int64_t)kKeysPerIter * u < end;
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        const float dot = dpp_f32_sum16(dot8(qv[g], kv[d][u]));  // all 64 lanes take part
        s[u][g] = on ? dot * a.scale_log2 : kNegInf;
      }
    }
    float vf[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) unpack8(vv[d][u], vf[u]);
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      float mb = s[0][g];
#pragma unroll
      for (int u = 1; u < U; ++u) mb = fmaxf(mb, s[u][g]);
      const float mn = fmaxf(st.m[g], mb);
      if (mn == kNegInf) continue;  // no valid key yet in this lane group
      const float corr = exp2_hw(st.m[g] - mn);
      float lsum = st.l[g] * corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) st.acc[g][j] *= corr;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2_hw(s[u][g] - mn);  // 0 for a masked key
        lsum += p;
        const float pb = from_bf16(to_bf16(p));
#pragma unroll
        for (int j = 0; j < 8; ++j) st.acc[g][j] = __builtin_fmaf(pb, vf[u][j], st.acc[g][j]);
      }
      st.l[g] = lsum;
      st.m[g] = mn;
    }
  };
  if (n > 0) {
#pragma unroll
    for (int d = 0; d + 1 < NS; ++d) issue(d, d);
  }

  // Fused prologue (see above).
  if constexpr (FUSED) {
    pos = pos_in;
    const bool owns_slot = fused_prologue(a, vh, wave * 4 + q4, r, rows, start, pos, qs, kvs);
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GT; ++g) qv[g] = g < rows ? qs[g][r] : make_uint4(0, 0, 0, 0);
    subst = owns_slot && pos < end;
    if (subst) {
      knew = kvs[0][r];
      vnew = kvs[1][r];
    }
  }

  // NS sets in flight: set t lives in buffer t % NS; before consuming it the
  // wave issues set t + NS - 1 into the buffer set t - 1 just freed.
  if (n > 0) {
    for (int i = 0;; i += NS) {
      bool done = false;
#pragma unroll
      for (int d = 0; d < NS; ++d) {
        if (!done) {
          issue((d + NS - 1) % NS, i + d + NS - 1);
          consume(d, i + d);
          done = i + d + 1 >= n;
        }
      }
      if (done) break;
    }
  }

  // Lane groups of a wave (lanes r, r+16, r+32, r+48 hold the same d slice).
  merge_lanes<GT>(st, 16);
  merge_lanes<GT>(st, 32);
  // Waves 1..3 hand over to wave 0 (lanes 0..15 carry the 128-wide slices).
  if (wave > 0 && lane < 16) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (lane == 0) {
        xm[wave - 1][g] = st.m[g];
        xl[wave - 1][g] = st.l[g];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) xacc[wave - 1][g][8 * r + j] = st.acc[g][j];
    }
  }
  __syncthreads();
  const bool owner = wave == 0 && lane < 16;
  if (owner) {
#pragma unroll
    for (int w = 0; w < kWavesA - 1; ++w)
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        float oacc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) oacc[j] = xacc[w][g][8 * r + j];
        merge_row<GT>(st, g, xm[w][g], xl[w][g], oacc);
      }
  }

  if (a.splits == 1) {
    if (!owner) return;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (g >= rows) break;
      const float den = st.l[g] > 0.0f ? st.l[g] : 1.0f;
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = st.acc[g][j] / den;
      store16<false>(a.out + ((int64_t)vh * G + a.g0 + g) * kD + 8 * r, pack8(o));
    }
    return;
  }

  if (owner) {
    const int64_t slot = (int64_t)vh * a.splits + seg;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (g >= rows) break;
      const int row = a.g0 + g;
      float* dst = a.partials + (slot * G + row) * kD + 8 * r;
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[j] = st.acc[g][j];
      if (r == 0) {
        a.stats[slot * 2 * G + row] = st.m[g];
        a.stats[slot * 2 * G + G + row] = st.l[g];
      }
    }
  }
}

// Matrix-core variant for groups of at most 4 query rows (Qwen3: 4), the
// same contract and results within the kernels' bf16 rounding of the
// probabilities and f32 accumulation order.  Each wave takes 16-key blocks
// w, w+4, ... of the segment, and both products run on the matrix cores:
//
// * Scores, transposed: S^T = K Q^T of a block is one chain of four
//   v_mfma_f32_16x16x32_bf16 (A = the 16 keys, lane l reading key l % 16,
//   dims 8 (l / 16) + 32 s straight from the cache; B = the query rows,
//   zero-padded to 16).  That leaves lane l holding S[query l % 16][keys
//   4 (l / 16) + i], i < 4: exactly the A operand of
//   v_mfma_f32_16x16x16_bf16 for P V with the keys along k, so the bf16
//   probabilities need no cross-lane moves.
// * P V: the block's V rows go to the wave's LDS buffer in their own
//   key-major layout (288-byte rows: at most two-way bank conflicts for the
//   reads below), and ds_read_b64_tr_b16 - lane i of each 16-lane group
//   receives element i % 4 of the 8 bytes that lanes 4q + i / 4 address,
//   q = 0..3 - turns lane 4q + t's address of dims 16 db + 4t .. +4 of key
//   4 (l / 16) + q into the B operand (key 4 (l / 16) + q, dim 16 db + l % 16).
//   Eight MFMAs cover the 128 dims; lanes 0..15 accumulate O[query i][16 db + l].
//
// Each lane keeps the running maximum and the f32 denominator of its own
// query over its own keys (the four lanes of a query share the maximum, a
// two-step shuffle reduction per block); the accumulators of a query are
// rescaled when its maximum moves (a wave-uniform test of the four
// queries' factors).  The four waves' totals are merged through LDS.
// Measured against the earlier form of this kernel (scores Q K^T on the
// matrix cores, P V on the VALU as packed bf16 dot products after
// ds_bpermute moves of the probabilities) on the engine's shapes: batch 1 x
// 545 keys 9.58 -> 8.67 us, 4 x 2081 14.35 -> 13.50, 16 x 641 15.36 ->
// 14.61, 64 x 1024 47.40 -> 45.89 us.  Three or four sets in flight are
// 5-25% slower than two.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
constexpr int kVRow = 288;  // LDS bytes per staged V key row (256 + 32 pad)

// Where the query rows come from (attn_mfma_kernel's PRO): q in memory, or
// the fused Q/K/V prologue over bf16 rows, over at most kPrologueSplits f32
// split-K partials, or over more partials.  One kernel per source keeps each
// prologue straight-line code, so the compiler's wait counts see exactly the
// loads of one path.
constexpr int kProNone = 0, kProRows = 1, kProPartials = 2, kProMany = 3;

template <int GT, int PRO, bool NTL = false, int NS = 2, bool STAMP = false>
__global__ __launch_bounds__(kBlock) void attn_mfma_kernel(AttnArgs a) {
  static_assert(GT == 1 || GT == 2 || GT == 4, "query rows per kv head");
  constexpr bool FUSED = PRO != kProNone;
  uint64_t ts[kPhases] = {};
  if constexpr (STAMP) ts[0] = phase_clock();
  constexpr int kW = kBlock / kWave;
  __shared__ float xm[kW][GT], xl[kW][GT];
  __shared__ float xacc[kW][GT][kD];
  __shared__ __attribute__((aligned(16))) uint8_t vlds[kW][16 * kVRow];
  __shared__ uint4 qs[FUSED ? GT : 1][16], kvs[2][16];
  const int vh = blockIdx.x;
  const int seg = blockIdx.y;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: scalar branches
  const int r = lane % 16;
  const int q4 = lane / 16;
  const int G = a.groups;  // <= GT
  const int rows = G;

  const int32_t used_in = a.used[vh];
  const int64_t pos_in = FUSED ? *a.position : 0;
  if constexpr (FUSED) asm volatile("" ::"s"(used_in), "s"(pos_in));
  if constexpr (STAMP) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::"s"(used_in), "s"(pos_in) : "memory");
    ts[1] = phase_clock();
  }
  int64_t used = used_in;
  used = used < 0 ? 0 : (used > a.capacity ? a.capacity : used);
  const int64_t start = (int64_t)seg * a.span;
  int64_t end = start + a.span;
  if (end > used) end = used;
  // The fused paths with bf16 rows or up to kPrologueSplits partials issue
  // their first key blocks whether or not the wave has keys (the loads are
  // then discarded); a head with no valid key at all reads them from the
  // query gain (128 values, in bounds for every lane's offsets), so no cache
  // slot at or beyond used is ever read.
  const bool dummy = FUSED && used == 0;
  const uint16_t* kbase = dummy ? a.qw : a.k + (int64_t)vh * a.capacity * kD;
  const uint16_t* vbase = dummy ? a.qw : a.v + (int64_t)vh * a.capacity * kD;
  const int64_t nb = end > start ? (end - start + 15) / 16 : 0;  // 16-key blocks of the segment
  const int n = nb > wave ? (int)((nb - wave + kW - 1) / kW) : 0;
  const int64_t last_key = end > 0 ? end - 1 : 0;  // below used whenever used > 0

  // Query rows as the scores' B operand: column = lane % 16 (< G), k = dims
  // 8*(lane/16) + 32 s.
  uint4 qa[4];
  if constexpr (!FUSED) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qa[s] = r < rows ? load16<false>(a.q + ((int64_t)vh * G + r) * kD + 8 * q4 + 32 * s)
                       : make_uint4(0, 0, 0, 0);
  }

  uint4 kf[NS][4], vf[NS][4];
  int64_t pos = 0;
  bool subst = false;
  uint4 knew[4], vnew = make_uint4(0, 0, 0, 0);
  auto issue = [&](int d, int j) {
    const int64_t b0 = start + (int64_t)(wave + kW * j) * 16;
    const int64_t kk = b0 + r < end ? b0 + r : last_key;
#pragma unroll
    for (int s = 0; s < 4; ++s) kf[d][s] = load16<NTL>(kbase + kk * kD + 8 * q4 + 32 * s);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t vk = b0 + q4 + 4 * u < end ? b0 + q4 + 4 * u : last_key;
      vf[d][u] = load16<NTL>(vbase + vk * kD + 8 * r);
    }
  };
  if constexpr (FUSED) {
    pos = pos_in;
    // Only waves 0 and 1 hold a prologue row: wave 0's lane groups the query
    // rows (lane group q4 < rows), wave 1's lane groups 8 (the new key) and
    // 9 (the new value); waves 2 and 3 issue nothing but their key blocks
    // (the prologue's loads from all four waves took 1.8 us to issue with
    // eight split-K partials, measured with the phase stamps).
    const bool pro = wave < 2;
    const int plg = wave == 0 ? q4 : 8 + q4;
    const bool owns_slot = pos >= 0 && pos < a.capacity && pos >= start && pos < start + a.span;
    if constexpr (PRO == kProRows) {
      // bf16 rows: the prologue's loads, then the first key blocks (issued
      // unconditionally, so the prologue waits for its own loads only and
      // its arithmetic overlaps the key loads).
      PrologueLoads pl;
      if (pro) pl = prologue_issue(a, vh, plg, r, rows, pos);
#pragma unroll
      for (int d = 0; d + 1 < NS; ++d) issue(d, d);
      if constexpr (STAMP) ts[2] = phase_clock();
      if (pro) prologue_finish(a, pl, vh, plg, r, rows, start, pos, qs, kvs);
    } else if constexpr (PRO == kProPartials) {
      // split-K partials, likewise
      PartialLoads pp;
      if (pro) pp = partials_issue(a, vh, plg, r, rows, pos);
#pragma unroll
      for (int d = 0; d + 1 < NS; ++d) issue(d, d);
      __builtin_amdgcn_sched_barrier(0);  // every key load issued before the sum waits
      if constexpr (STAMP) ts[2] = phase_clock();
      if (pro) {
        PrologueLoads pl;
        pl.wv = pp.wv;
        pl.cv = pp.cv;
        pl.sv = pp.sv;
        pl.xv = partials_sum(a, pp);
        prologue_finish(a, pl, vh, plg, r, rows, start, pos, qs, kvs);
      }
    } else {
      if (n > 0) {
#pragma unroll
        for (int d = 0; d + 1 < NS; ++d) issue(d, d);
      }
      if (pro) fused_prologue(a, vh, plg, r, rows, start, pos, qs, kvs);
    }
    __syncthreads();
    if constexpr (STAMP) ts[3] = phase_clock();
#pragma unroll
    for (int s = 0; s < 4; ++s) qa[s] = r < rows ? qs[r][q4 + 4 * s] : make_uint4(0, 0, 0, 0);
    subst = owns_slot && pos < end;
    if (subst) {
#pragma unroll
      for (int s = 0; s < 4; ++s) knew[s] = kvs[0][q4 + 4 * s];
      vnew = kvs[1][r];
    }
  } else {
    if (n > 0) {
#pragma unroll
      for (int d = 0; d + 1 < NS; ++d) issue(d, d);
    }
    if constexpr (STAMP) ts[2] = ts[3] = phase_clock();
  }

  // This lane's query r: running maximum and partial denominator over the
  // lane's keys; O in tiles of 16 dims (lanes 0..15: O[query i][16 db + r]).
  float mq = kNegInf, lq = 0.0f;
  f32x4 oacc[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint8_t* vb = vlds[wave];
  const int rd = (4 * q4 + (r >> 2)) * kVRow + 8 * (r & 3);  // transpose-read address
  auto consume = [&](int d, int j) {
    const int64_t b0 = start + (int64_t)(wave + kW * j) * 16;
    if constexpr (FUSED) {
      if (subst) {  // the new K/V row replaces slot pos wherever it was loaded
        if ((b0 + r < end ? b0 + r : last_key) == pos) {
#pragma unroll
          for (int s = 0; s < 4; ++s) kf[d][s] = knew[s];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if ((b0 + q4 + 4 * u < end ? b0 + q4 + 4 * u : last_key) == pos) vf[d][u] = vnew;
      }
    }
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[d][s]),
                                                   __builtin_bit_cast(bf16x8, qa[s]), c, 0, 0, 0);
    float sc[4], bm = kNegInf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool on = r < rows && b0 + 4 * q4 + i < end;
      sc[i] = on ? c[i] * a.scale_log2 : kNegInf;
      bm = fmaxf(bm, sc[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16));
    bm = fmaxf(bm, __shfl_xor(bm, 32));
    const float mn = fmaxf(mq, bm);
    const float corr = mn == kNegInf ? 1.0f : exp2_hw(mq - mn);
    float p[4], ps = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = mn == kNegInf ? 0.0f : exp2_hw(sc[i] - mn);  // 0 for a masked key or row
      ps += p[i];
    }
    lq = lq * corr + ps;
    mq = mn;
    float cq[GT];
    bool rescale = false;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      cq[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), g));
      rescale |= cq[g] != 1.0f;
    }
    if (rescale) {  // wave-uniform
#pragma unroll
      for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int g = 0; g < GT; ++g) oacc[db][g] *= cq[g];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      *reinterpret_cast<uint4*>(vb + (q4 + 4 * u) * kVRow + 16 * r) = vf[d][u];
    wave_lds_fence();
    // The probabilities are rounded to bf16 before they multiply V.
    const v4i16 pa = __builtin_bit_cast(v4i16, make_uint2(pack2(p[0], p[1]), pack2(p[2], p[3])));
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const v4i16 vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4i16*)((__attribute__((address_space(3))) uint8_t*)vb + rd + 32 * db));
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, vt, oacc[db], 0, 0, 0);
    }
    wave_lds_fence();  // the reads complete before the next block's writes
  };
  if (n > 0) {
    for (int i = 0;; i += NS) {
      bool done = false;
#pragma unroll
      for (int d = 0; d < NS; ++d) {
        if (!done) {
          issue((d + NS - 1) % NS, i + d + NS - 1);
          consume(d, i + d);
          if constexpr (STAMP) {
            if (i + d == 0) ts[4] = phase_clock();
          }
          done = i + d + 1 >= n;
        }
      }
      if (done) break;
    }
  }
  if constexpr (STAMP) {
    if (n == 0) ts[4] = phase_clock();
    ts[5] = phase_clock();
  }

  // Wave totals through LDS: query g's maximum and denominator (summed over
  // its four key lanes) from lane g, O rows from lanes 0..15.  Then every
  // thread merges at once: wave g takes query row g (g < rows), lane l its
  // dims 2l and 2l + 1, each wave's share weighted by 2^(m_w - M) against
  // the row's overall maximum M.  (Wave 0 merging the waves one after
  // another - rescaling its running state per wave, four rows of 8 dims per
  // lane - took 1.7 us per workgroup, measured with the phase stamps; this
  // takes a few hundred nanoseconds.)
  float lt = lq + __shfl_xor(lq, 16);
  lt += __shfl_xor(lt, 32);
  if (lane < GT) {
    xm[wave][lane] = mq;
    xl[wave][lane] = lt;
  }
  if (q4 == 0) {
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int g = 0; g < GT; ++g) xacc[wave][g][16 * db + r] = oacc[db][g];
  }
  __syncthreads();
  if constexpr (STAMP) ts[12] = phase_clock();
  const int gq = wave;  // this wave's query row
  const bool owner = gq < rows;
  float rm = kNegInf, rl = 0.0f, r0 = 0.0f, r1 = 0.0f;
  if (owner) {
    float mw[kW], lw[kW];
    float2 ow[kW];
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      mw[w] = xm[w][gq];
      lw[w] = xl[w][gq];
      ow[w] = *reinterpret_cast<const float2*>(&xacc[w][gq][2 * lane]);
    }
#pragma unroll
    for (int w = 0; w < kW; ++w) rm = fmaxf(rm, mw[w]);
    const float base = rm == kNegInf ? 0.0f : rm;  // no valid key: every weight 0
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const float c = exp2_hw(mw[w] - base);
      rl = __builtin_fmaf(lw[w], c, rl);
      r0 = __builtin_fmaf(ow[w].x, c, r0);
      r1 = __builtin_fmaf(ow[w].y, c, r1);
    }
  }
  // Instrumented build: every wave stores its own stamps (lane 0, ordinary
  // vector stores); thread 0 waits for the output stores, takes the last
  // stamp and stores wave 0's.
  uint64_t* const stamp_row = STAMP ? a.stamps + ((int64_t)seg * gridDim.x + vh) * kPhases : nullptr;
  if constexpr (STAMP) {
    ts[6] = phase_clock();
    if (lane == 0) {
      stamp_row[8 + wave] = ts[5];
      if (wave > 0) stamp_row[12 + wave] = ts[4];
    }
  }
  auto record = [&]() {
    if constexpr (STAMP) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      ts[7] = phase_clock();
      if (threadIdx.x == 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) stamp_row[i] = ts[i];
        stamp_row[12] = ts[12];
      }
    }
  };
  if (a.splits == 1) {
    if (!owner) return;  // wave 0 always owns row 0
    const float den = rl > 0.0f ? rl : 1.0f;
    reinterpret_cast<uint32_t*>(a.out + ((int64_t)vh * G + gq) * kD)[lane] = pack2(r0 / den, r1 / den);
    record();
    return;
  }
  if (owner) {
    const int64_t slot = (int64_t)vh * a.splits + seg;
    *reinterpret_cast<float2*>(a.partials + (slot * G + gq) * kD + 2 * lane) = make_float2(r0, r1);
    if (lane == 0) {
      a.stats[slot * 2 * G + gq] = rm;
      a.stats[slot * 2 * G + G + gq] = rl;
    }
  }
  record();
}

// One wave per query row, four rows per workgroup.
constexpr int kMergeRows = kBlock / kWave;
template <int NB, bool STAMP = false>
__global__ __launch_bounds__(kBlock) void attn_merge_kernel(AttnArgs a, int64_t rows) {
  uint64_t ts[kMergePhases] = {};
  if constexpr (STAMP) ts[0] = phase_clock();
  const int64_t row = (int64_t)blockIdx.x * kMergeRows + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const int G = a.groups;
  const int64_t vh = row / G;
  const int g = (int)(row - vh * G);
  SegmentLoads<NB> L;
  merge_issue(L, a.partials, a.stats, vh, a.splits, G, g, lane);
  if constexpr (STAMP) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ts[3] = phase_clock();
  }
  const uint32_t merged = merge_finish(L, a.partials, vh, a.splits, G, g, lane);
  if constexpr (STAMP) {
    asm volatile("" ::"v"(merged));
    ts[1] = phase_clock();
  }
  reinterpret_cast<uint32_t*>(a.out + row * kD)[lane] = merged;
  if constexpr (STAMP) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ts[2] = phase_clock();
    if (threadIdx.x == 0) {
      uint64_t* dst = a.stamps + kMergePhases * (int64_t)blockIdx.x;
#pragma unroll
      for (int i = 0; i < kMergePhases; ++i) dst[i] = ts[i];
    }
  }
}

template <int GT, bool FUSED, bool STAMP = false>
int launch_attn(const AttnArgs& args, int64_t vheads, hipStream_t s) {
  // Two sets of U = 2 key blocks in flight per wave.  Measured on the engine's
  // workloads (batch x keys = 1 x 545, 4 x 2081, 16 x 641, 64 x 1024): U = 4
  // is up to 6% slower, U = 8 and three or four sets in flight 10-45%
  // slower (they only lengthen each wave's chain; the grid already has the
  // bytes in flight).  Groups wider than GT (9..16 rows) take two launches
  // of 8 rows each.
  constexpr int U = 2;
  AttnArgs a = args;
  int st = QF_OK;
  if constexpr (GT <= 4) {  // one launch: Q.K^T on the matrix cores
    // K/V stream once per step: nontemporal loads (measured 2-15% faster from
    // batch 1 x 545 to 64 x 1024 keys; the bandwidth of a plain read of this
    // access pattern rises from 5.6 to 6.1-6.7 TB/s).
    const dim3 grid((unsigned)vheads, (unsigned)a.splits);
    if constexpr (!FUSED) {
      static_assert(!STAMP, "the instrumented build times the fused entry point");
      hipLaunchKernelGGL((attn_mfma_kernel<GT, kProNone, true>), grid, dim3(kBlock), 0, s, a);
    } else if (a.qkv_splits == 0) {
      hipLaunchKernelGGL((attn_mfma_kernel<GT, kProRows, true, 2, STAMP>), grid, dim3(kBlock), 0, s, a);
    } else if (a.qkv_splits <= kPrologueSplits) {
      hipLaunchKernelGGL((attn_mfma_kernel<GT, kProPartials, true, 2, STAMP>), grid, dim3(kBlock), 0, s,
                         a);
    } else {
      hipLaunchKernelGGL((attn_mfma_kernel<GT, kProMany, true, 2, STAMP>), grid, dim3(kBlock), 0, s, a);
    }
    st = launch_status();
  } else {
    static_assert(!STAMP, "the instrumented build times the matrix-core kernel");
    for (a.g0 = 0; a.g0 < a.groups && st == QF_OK; a.g0 += GT) {
      hipLaunchKernelGGL((attn_kernel<GT, U, 4, FUSED>), dim3((unsigned)vheads, (unsigned)a.splits),
                         dim3(kBlock), 0, s, a);
      st = launch_status();
    }
  }
  if (st != QF_OK || a.splits == 1 || !a.out) return st;  // no out: segments stay unmerged
  const int64_t rows = vheads * a.groups;
  if constexpr (STAMP) a.stamps += (int64_t)vheads * a.splits * kPhases;  // after the attention's
  // Segment loads per batch: the fewest of 2, 4, 8, 12, 16 that cover the
  // split count (one batch up to 16 segments, two for 17-32).
  const dim3 grid((unsigned)((rows + kMergeRows - 1) / kMergeRows));
  if (a.splits <= 2)
    hipLaunchKernelGGL((attn_merge_kernel<2, STAMP>), grid, dim3(kBlock), 0, s, a, rows);
  else if (a.splits <= 4)
    hipLaunchKernelGGL((attn_merge_kernel<4, STAMP>), grid, dim3(kBlock), 0, s, a, rows);
  else if (a.splits <= 8)
    hipLaunchKernelGGL((attn_merge_kernel<8, STAMP>), grid, dim3(kBlock), 0, s, a, rows);
  else if (a.splits <= 12)
    hipLaunchKernelGGL((attn_merge_kernel<12, STAMP>), grid, dim3(kBlock), 0, s, a, rows);
  else
    hipLaunchKernelGGL((attn_merge_kernel<16, STAMP>), grid, dim3(kBlock), 0, s, a, rows);
  return launch_status();
}

}  // namespace
}  // namespace qf

using namespace qf;

namespace {
// Segments per (sequence, KV head): at most one workgroup per compute unit
// (measured with the matrix-core kernel at batch x keys from 1 x 545 to
// 64 x 1024 against every split count: a CU that runs two segments finishes
// last, so 1.25 per CU - the earlier plan - cost 4-17% at batch 4 x 545, 16
// and 32; fewer segments lengthen each workgroup's chain), at least one
// 64-key tile per segment, at most 32 segments.
int64_t segment_count(int64_t virtual_heads, int64_t capacity, int32_t compute_units) {
  const int64_t tiles = (capacity + 63) / 64;
  const int64_t desired = (int64_t)compute_units / virtual_heads;
  int64_t s = desired < 1 ? 1 : desired;
  if (s > tiles) s = tiles;
  if (s > kMaxSplits) s = kMaxSplits;
  return s;
}

// s segments of whole `unit`-key multiples covering capacity, as balanced as
// that granularity allows.
void segment_plan(int64_t capacity, int64_t s, int64_t unit, int32_t* splits, int64_t* span) {
  const int64_t units = (capacity + unit - 1) / unit;
  const int64_t per = (units + s - 1) / s;
  *splits = (int32_t)((units + per - 1) / per);
  *span = per * unit;
}
}  // namespace

extern "C" int qf_attention_partition(int64_t virtual_heads, int64_t capacity,
                                      int32_t compute_units, int32_t* splits, int64_t* span) {
  if (virtual_heads < 1 || capacity < 1 || compute_units < 1 || !splits || !span) return QF_E_ARG;
  segment_plan(capacity, segment_count(virtual_heads, capacity, compute_units), 64, splits, span);
  return QF_OK;
}

extern "C" int qf_attention_partition_aligned(int64_t virtual_heads, int64_t capacity,
                                              int32_t compute_units, int32_t align,
                                              int32_t* splits, int64_t* span) {
  if (virtual_heads < 1 || capacity < 1 || compute_units < 1 || !splits || !span) return QF_E_ARG;
  if (align != 16 && align != 32 && align != 64) return QF_E_ARG;
  // The same segment count with lengths balanced to `align` keys (at 4 x
  // 2081 keys: 8 x 272 instead of 7 x 320, one workgroup per CU instead of
  // 224 of 256).
  segment_plan(capacity, segment_count(virtual_heads, capacity, compute_units), align, splits, span);
  return QF_OK;
}

namespace {

// Checks shared by both entry points (query source `qsrc`: q, or the packed
// projection row of the fused entry) and the attention half of the arguments.
int attention_setup(const void* qsrc, const void* k, const void* v, const int32_t* used,
                    int64_t batch, int32_t q_heads, int32_t kv_heads, int64_t capacity,
                    float scale, int32_t splits, int64_t span, float* partials, float* stats,
                    void* out, AttnArgs& a, int64_t& vheads) {
  if (batch < 1 || q_heads < 1 || kv_heads < 1 || capacity < 1) return QF_E_ARG;
  if (q_heads % kv_heads != 0 || q_heads / kv_heads > kMaxGroups) return QF_E_SHAPE;
  if (!qsrc || !k || !v || !used || (!out && splits == 1)) return QF_E_ARG;
  if (splits < 1 || splits > kMaxSplits || span < 1 || span % kSpanAlign != 0 ||
      (int64_t)splits * span < capacity || (int64_t)(splits - 1) * span >= capacity)
    return QF_E_ARG;
  if (splits > 1 && (!partials || !stats)) return QF_E_ARG;
  if (!(scale == scale) || scale == __builtin_inff() || scale == kNegInf) return QF_E_ARG;
  if (!aligned16(qsrc) || !aligned16(k) || !aligned16(v) || !aligned16(out)) return QF_E_ALIGN;
  vheads = batch * kv_heads;
  if (vheads > INT32_MAX) return QF_E_SHAPE;
  a = AttnArgs{};
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.used = used;
  a.partials = partials;
  a.stats = stats;
  a.out = static_cast<uint16_t*>(out);
  a.capacity = capacity;
  a.groups = q_heads / kv_heads;
  a.g0 = 0;
  a.splits = splits;
  a.span = (int32_t)span;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.kv_heads = kv_heads;
  return QF_OK;
}

template <bool FUSED>
int dispatch_attn(const AttnArgs& a, int64_t vheads, hipStream_t s) {
  switch (a.groups) {
    case 1: return launch_attn<1, FUSED>(a, vheads, s);
    case 2: return launch_attn<2, FUSED>(a, vheads, s);
    case 3: case 4: return launch_attn<4, FUSED>(a, vheads, s);
    default: return launch_attn<8, FUSED>(a, vheads, s);
  }
}

// Fills the attention half of `a` for the fused entry points.
int fused_setup(AttnArgs& a, const void* qkv, int32_t qkv_splits, const void* q_weight,
                const void* k_weight, float q_eps, float k_eps, const void* cos, const void* sin,
                const int64_t* position, void* key_cache, void* value_cache, int64_t batch,
                int32_t q_heads, int32_t kv_heads) {
  if (qkv_splits < 0 || !q_weight || !k_weight || !cos || !sin || !position) return QF_E_ARG;
  if (!aligned16(q_weight) || !aligned16(k_weight) || !aligned16(cos) || !aligned16(sin) ||
      (reinterpret_cast<uintptr_t>(position) & 7u))
    return QF_E_ALIGN;
  a.qkv = qkv;
  a.qkv_splits = qkv_splits;
  a.qkv_stride = batch * ((int64_t)q_heads + 2 * (int64_t)kv_heads) * kD;
  a.qw = static_cast<const uint16_t*>(q_weight);
  a.kw = static_cast<const uint16_t*>(k_weight);
  a.q_eps = q_eps;
  a.k_eps = k_eps;
  a.cos = static_cast<const uint16_t*>(cos);
  a.sin = static_cast<const uint16_t*>(sin);
  a.position = position;
  a.kc = static_cast<uint16_t*>(key_cache);
  a.vc = static_cast<uint16_t*>(value_cache);
  return QF_OK;
}

}  // namespace

extern "C" int qf_decode_attention(const void* q, const void* k, const void* v,
                                   const int32_t* used, int64_t batch, int32_t q_heads,
                                   int32_t kv_heads, int64_t capacity, float scale,
                                   int32_t splits, int64_t span, float* partials, float* stats,
                                   void* out, void* stream) {
  AttnArgs a;
  int64_t vheads = 0;
  const int st = attention_setup(q, k, v, used, batch, q_heads, kv_heads, capacity, scale, splits,
                                 span, partials, stats, out, a, vheads);
  if (st != QF_OK) return st;
  a.q = static_cast<const uint16_t*>(q);
  return dispatch_attn<false>(a, vheads, as_stream(stream));
}

extern "C" int qf_decode_attention_qkv(const void* qkv, int32_t qkv_splits, const void* q_weight,
                                       const void* k_weight, float q_eps, float k_eps,
                                       const void* cos, const void* sin, const int64_t* position,
                                       void* key_cache, void* value_cache, const int32_t* used,
                                       int64_t batch, int32_t q_heads, int32_t kv_heads,
                                       int64_t capacity, float scale, int32_t splits, int64_t span,
                                       float* partials, float* stats, void* out, void* stream) {
  AttnArgs a;
  int64_t vheads = 0;
  const int st = attention_setup(qkv, key_cache, value_cache, used, batch, q_heads, kv_heads,
                                 capacity, scale, splits, span, partials, stats, out, a, vheads);
  if (st != QF_OK) return st;
  const int fs = fused_setup(a, qkv, qkv_splits, q_weight, k_weight, q_eps, k_eps, cos, sin,
                            position, key_cache, value_cache, batch, q_heads, kv_heads);
  if (fs != QF_OK) return fs;
  return dispatch_attn<true>(a, vheads, as_stream(stream));
}

#ifdef QF_PHASE_STAMPS
// Instrumented qf_decode_attention_qkv for phase timing (built only into the
// measurement library, never into libqwen_fused.so): same arguments and
// results, query groups of at most 4 rows (the matrix-core kernel), plus
// `stamps`, u64 [virtual heads * splits * kPhases] for the attention's
// workgroups (index (split * virtual heads + vh) * kPhases + phase) followed,
// when splits > 1, by [merge workgroups * kMergePhases] for the merge.
extern "C" int qf_decode_attention_qkv_phases(
    const void* qkv, int32_t qkv_splits, const void* q_weight, const void* k_weight, float q_eps,
    float k_eps, const void* cos, const void* sin, const int64_t* position, void* key_cache,
    void* value_cache, const int32_t* used, int64_t batch, int32_t q_heads, int32_t kv_heads,
    int64_t capacity, float scale, int32_t splits, int64_t span, float* partials, float* stats,
    void* out, uint64_t* stamps, void* stream) {
  AttnArgs a;
  int64_t vheads = 0;
  const int st = attention_setup(qkv, key_cache, value_cache, used, batch, q_heads, kv_heads,
                                 capacity, scale, splits, span, partials, stats, out, a, vheads);
  if (st != QF_OK) return st;
  if (!stamps) return QF_E_ARG;
  if (a.groups > 4) return QF_E_SHAPE;
  const int fs = fused_setup(a, qkv, qkv_splits, q_weight, k_weight, q_eps, k_eps, cos, sin,
                            position, key_cache, value_cache, batch, q_heads, kv_heads);
  if (fs != QF_OK) return fs;
  a.stamps = stamps;
  hipStream_t s = as_stream(stream);
  switch (a.groups) {
    case 1: return launch_attn<1, true, true>(a, vheads, s);
    case 2: return launch_attn<2, true, true>(a, vheads, s);
    default: return launch_attn<4, true, true>(a, vheads, s);
  }
}
#endif
