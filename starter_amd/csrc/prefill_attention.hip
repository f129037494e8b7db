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
// blocks attend the most keys), on grids of at least one workgroup per CU
// per group of pairs on each XCD (see work order below).  Keys stream in blocks of 64, staged once per
// workgroup in LDS and shared by every tile, so the K/V bytes a CU pulls from
// L2 per flop shrink with the workgroup's query rows (the per-CU L2 request
// rate, not the matrix cores, bounded the 4-wave form).  The blocks go from
// the cache straight into LDS (global_load_lds_dwordx4), K one block ahead
// of V, so no registers hold them in flight.
//
// Schedules.  A matrix-core product and VALU work issued by the same wave
// overlap only about two VALU instructions per product, while VALU work of
// the SIMD's other wave overlaps the products almost fully (timing probes on
// gfx950), and the softmax (an exp2, an FMA, a sum and half a conversion per
// score) is about as much VALU work as the block's products.  So the 8-wave
// form ping-pongs: waves 0-3 and 4-7 (one of each per SIMD) run the same
// steps, the second set one step behind; in step M j a wave issues block j -
// 1's P V and block j's scores (the LDS reads kept 6-8 ahead of the
// products), in step V j the softmax of block j, and a barrier ends every
// step.  The 4-wave form issues block j + 1's scores beside block j's
// softmax, then block j's P V; at G = 4 its waves hold one 16-row tile each,
// which leaves room for two workgroups per CU.
//
// Both products are on the matrix cores (v_mfma_f32_16x16x32_bf16):
// * Scores, transposed: S^T = K Q^T for a 16-key tile is a chain of four
//   MFMAs (A = 16 keys x 32 dims from LDS, lane l reading key l % 16, dims
//   8 (l / 16) + 32 s; B = the tile's 16 query rows, kept in registers),
//   leaving lane l with S[query l % 16][keys 4 (l / 16) + i].
// * O^T = V^T P^T: two 16-key tiles form one 32-wide k step.  Lane l's
//   eight B values are its own probabilities: keys 4 (l / 16) + i of the
//   first tile and of the second, in that k-slot order; the A operand must
//   list V in the same order, which two ds_read_b64_tr_b16 per k step give:
//   lane i of each 16-lane group receives element i % 4 of the 8 bytes lanes
//   4q + i / 4 address, so lane 4q + t addressing dims 16 db + 4t of key
//   4 (l / 16) + q yields keys 4 (l / 16) + 0..3 of dim 16 db + l % 16.
//   Eight dim tiles of 16 cover the head; lane l accumulates dims
//   16 db + 4 (l / 16) + i of its own query l % 16, so its rescale factor and
//   denominator are its own and its output is 8 contiguous bytes per db.
// Each query row keeps a reference maximum (log2 units, the same on the
// row's four lanes) and each lane its part of the denominator.  The first
// block sets the references to its row maxima; later blocks take their
// probabilities against the reference directly, and the reference is
// raised (the accumulators rescaled) only when a lane's sum of its 16
// probabilities of a block exceeds 2^kLazy, which any probability above
// 2^kLazy forces.  K rows in LDS are 272 bytes (the score
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
// when a lane's 16 probabilities of a block sum past 2^kLazy, so
// unnormalised probabilities stay below 2^8 and the accumulators are rarely
// rescaled.
constexpr float kLazy = 8.0f;
constexpr float kLazyBound = 256.0f;  // 2^kLazy

struct PrefillArgs {
  const uint16_t* q;   // [B, T, Hq, 128]
  const uint16_t* k;   // [B, Hkv, C, 128]
  const uint16_t* v;
  uint16_t* out;       // [B, T, Hq, 128]
  int64_t length, capacity;
  int32_t q_heads, kv_heads;
  int32_t qblocks;     // ceil(T / query positions per workgroup)
  int32_t pairs;       // B * Hkv
  int32_t group;       // pairs per XCD and group of the work order (0: query-block major)
  float scale_log2;    // |scale| * log2(e)
  uint32_t qsign;      // 0x80008000 when scale < 0: Q enters negated (exact in bf16)
};

// Work split per group size G (query heads per KV head): QB query positions
// per workgroup (a divisor of the key block, so a workgroup's queries share
// one diagonal block), W waves per workgroup and TPW 16-row tiles per wave,
// G * QB / 16 = W * TPW.  Each staged key block serves all of a workgroup's
// G * QB query rows, so its K/V traffic from L2 per flop falls as that grows:
// at G = 4, 8 waves of 64 positions (256 rows) need a quarter of the block
// loads of four 4-wave workgroups of 16.
// WIDE (8 waves, the ping-pong schedule) is taken when the grid has at least
// one workgroup per CU (1 x 2048, 4 x 512 and up at Qwen3-4B's heads).
// Smaller prompts take the 4-wave form, which at G = 4 holds 16 positions
// per workgroup (one tile per wave, 157 VGPRs: two workgroups per CU; with
// 32 positions and two tiles per wave it needed 312 registers, one
// workgroup per CU) - four times the 8-wave form's workgroups, each with a
// shorter chain per key block.  Measured (Qwen3-4B heads, bit-identical
// outputs): 1 x 512 18.7 -> 13.4 us, 2 x 512 19.3 -> 15.5, 3 x 512 20.5 ->
// 18.7, 1 x 1024 32.3 -> 24.4, 1 x 1536 45.7 -> 34.6 against 32 positions;
// the 8-wave form stays ahead from one workgroup per CU (1 x 2048 53.9
// against 57.1 us, 4 x 512 21.2 against 21.9) and behind below it (1 x 1024
// 30.8, 3 x 512 20.5 at 128 and 192 workgroups).
template <int G, bool WIDE> struct Split;
template <bool WIDE> struct Split<1, WIDE> { static constexpr int QB = 64, TPW = 1, W = 4; };
template <bool WIDE> struct Split<2, WIDE> { static constexpr int QB = 64, TPW = 2, W = 4; };
template <> struct Split<4, false> { static constexpr int QB = 16, TPW = 1, W = 4; };
template <> struct Split<4, true> { static constexpr int QB = 64, TPW = 2, W = 8; };
template <> struct Split<8, false> { static constexpr int QB = 16, TPW = 2, W = 4; };
template <> struct Split<8, true> { static constexpr int QB = 32, TPW = 2, W = 8; };
constexpr int64_t kWideWorkgroups = kCUs;

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
  constexpr int kSubs = QB / 16;  // position tiles per head
  constexpr int kKLoads = kKB * kKRow / 1024;  // 1 KB direct loads per staged K block (17)
  constexpr int kVLoads = kKB * kVRow / 1024;  // ... per V block (18)
  constexpr int kKPerWave = (kKLoads + W - 1) / W;
  constexpr int kVPerWave = (kVLoads + W - 1) / W;
  static_assert(G * kSubs == W * TPW, "every wave holds TPW tiles");
  static_assert(W % kSubs == 0, "a wave's tiles share their positions");
  static_assert(W * 16 * kORow <= 2 * kKB * kKRow, "output staging fits the K buffers");
  static_assert(kKB * kKRow % 1024 == 0 && kKB * kVRow % 1024 == 0, "whole 1 KB loads");
  __shared__ __attribute__((aligned(1024))) uint8_t klds[2][kKB * kKRow];
  __shared__ __attribute__((aligned(1024))) uint8_t vlds[2][kKB * kVRow];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int r = lane % 16;
  const int g4 = lane / 16;
  // Work order.  Workgroup i runs on XCD i % kXCDs, and a (sequence, KV
  // head) pair's workgroups share its K/V through that XCD's L2 only when
  // they run there at the same time.  Query-block-major order (group 0)
  // runs the longest blocks of every pair first; with `group` > 0 (pairs a
  // multiple of kXCDs, pairs / kXCDs a multiple of group) each XCD takes its
  // pairs xcd, xcd + kXCDs, ... `group` at a time, longest first within the
  // group, so fewer pairs' keys are live in its L2 at once.
  int qb, pair;
  if (a.group > 0) {
    const int i = (int)blockIdx.x, k = i / kXCDs;
    const int per = a.group * a.qblocks;
    qb = a.qblocks - 1 - (k % per) / a.group;
    pair = i % kXCDs + kXCDs * ((k / per) * a.group + (k % per) % a.group);
  } else {
    qb = a.qblocks - 1 - (int)(blockIdx.x / a.pairs);
    pair = (int)(blockIdx.x % a.pairs);
  }
  const int b = pair / a.kv_heads;
  const int kvh = pair % a.kv_heads;
  const int64_t p0 = (int64_t)qb * QB;
  const int64_t last = a.length - 1;
  const int nkb = (int)(p0 / kKB) + 1;
  const uint16_t* kbase = a.k + (int64_t)pair * a.capacity * kD;
  const uint16_t* vbase = a.v + (int64_t)pair * a.capacity * kD;

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

  // Blocks move from the cache straight into LDS (global_load_lds_dwordx4:
  // lane l of a load writes 16 bytes at the load's 1 KB segment + 16 l), so no
  // registers hold them in flight.  Staged rows keep their padding (K 272,
  // V 288 bytes): linear 16-byte slot L of a buffer is slot L % (row / 16) of
  // row L / (row / 16); lanes on a padding slot re-read the row's first chunk
  // (the bytes land in the padding, never read).  Load i of a block is
  // issued by wave i % W.  Per lane the (row, chunk) of each of its loads is
  // fixed, so its byte offset inside a block is computed once.
  int koff[kKPerWave], voff[kVPerWave];
#pragma unroll
  for (int i = 0; i < kKPerWave; ++i) {
    const int L = 64 * (wave + W * i) + lane;
    const int row = L / (kKRow / 16), slot = L % (kKRow / 16);
    koff[i] = row * (kD * 2) + (slot < 16 ? 16 * slot : 0);
  }
#pragma unroll
  for (int i = 0; i < kVPerWave; ++i) {
    const int L = 64 * (wave + W * i) + lane;
    const int row = L / (kVRow / 16), slot = L % (kVRow / 16);
    voff[i] = row * (kD * 2) + (slot < 16 ? 16 * slot : 0);
  }
  // Rows at or past `length` (the last block only) re-read row length - 1.
  auto load_block = [&](const uint16_t* base, uint8_t* dst, const int* off, int count, int loads,
                        int j, bool clamp) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(base) + (int64_t)j * kKB * kD * 2;
#pragma unroll
    for (int i = 0; i < count; ++i) {
      const int li = wave + W * i;
      if (li < loads) {  // wave-uniform
        int o_ = off[i];
        if (clamp) {
          const int64_t row = (int64_t)j * kKB + o_ / (kD * 2);
          if (row > last) o_ = (int)(last - (int64_t)j * kKB) * (kD * 2) + o_ % (kD * 2);
        }
        // Issued as inline assembly: the compiler's wait counting would
        // otherwise order every later LDS read after these loads, though
        // they fill a buffer no read of this block touches.  The block's
        // loads are waited for explicitly (vmcnt(0)) before its barrier.
        const uint32_t m0 = (uint32_t)(uintptr_t)(
            const __attribute__((address_space(3))) uint8_t*)(dst + 1024 * li);
        uint32_t saved;
        asm volatile(
            "s_mov_b32 %0, m0\n\t"
            "s_mov_b32 m0, %1\n\t"
            "s_nop 0\n\t"
            "global_load_lds_dwordx4 %2, off\n\t"
            "s_mov_b32 m0, %0"
            : "=&s"(saved) : "s"(m0), "v"(src + o_) : "memory");
      }
    }
  };
  auto load_k = [&](int j, int buf) {
    load_block(kbase, klds[buf], koff, kKPerWave, kKLoads, j, j == nkb - 1);
  };
  auto load_v = [&](int j, int buf) {
    load_block(vbase, vlds[buf], voff, kVPerWave, kVLoads, j, j == nkb - 1);
  };

  // S^T of the block staged in klds[buf] against every query tile of this
  // wave (on the diagonal block only the 16-key tiles that some row attends).
  auto scores = [&](int buf, int ktn, auto diag_tag, f32x4 (&c)[TPW][4]) {
    constexpr bool kDiag = decltype(diag_tag)::value;
    const uint8_t* kb = klds[buf];
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
  };

  uint4 pa[TPW][2];
  // Online softmax of one block's scores: the bf16 probabilities go to pa.
  // The first block sets each row's reference maximum mq to its row maximum;
  // later blocks take the probabilities against mq directly and raise it
  // (rescaling the accumulators) only when some lane's sum of its 16
  // probabilities exceeds 2^kLazy, which any probability above 2^kLazy (a
  // row maximum more than kLazy above the reference) forces.  The common
  // case is therefore straight-line code without a row maximum; the rare
  // raise computes the block's row maxima and recomputes that tile.
  auto softmax = [&](f32x4 (&c)[TPW][4], int64_t key0, auto diag_tag, auto hint_tag,
                     auto first_tag) {
    constexpr bool kDiag = decltype(diag_tag)::value;
    constexpr bool HINT = decltype(hint_tag)::value;
    constexpr bool kFirst = decltype(first_tag)::value;
    float ps[TPW];
    auto probabilities = [&](int u) {
      const float nm = -mq[u];
      float p[4][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool live = !kDiag || key0 + 16 * kt + 4 * g4 + i <= pt + r;
          p[kt][i] = live ? exp2_hw(fmaf(c[u][kt][i], a.scale_log2, nm)) : 0.0f;
        }
      float s4[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s4[kt] = (p[kt][0] + p[kt][1]) + (p[kt][2] + p[kt][3]);
      ps[u] = (s4[0] + s4[1]) + (s4[2] + s4[3]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        pa[u][ks] = make_uint4(pack2(p[2 * ks][0], p[2 * ks][1]), pack2(p[2 * ks][2], p[2 * ks][3]),
                               pack2(p[2 * ks + 1][0], p[2 * ks + 1][1]),
                               pack2(p[2 * ks + 1][2], p[2 * ks + 1][3]));
    };
    // The row maximum of this block's live scores, over the four lanes of
    // each query.
    auto row_max = [&](int u) {
      float m = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool live = !kDiag || key0 + 16 * kt + 4 * g4 + i <= pt + r;
          m = fmaxf(m, live ? c[u][kt][i] : kNegInf);
        }
      const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m),
                                                        false, false);
      m = fmaxf(__uint_as_float(s16[0]), __uint_as_float(s16[1]));
      const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m),
                                                        false, false);
      return fmaxf(__uint_as_float(s32[0]), __uint_as_float(s32[1]));
    };
    if constexpr (kFirst) {  // the first block: the references start at its row maxima
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        mq[u] = row_max(u) * a.scale_log2;
        probabilities(u);
        lq[u] = ps[u];
      }
    } else {
    bool grow = false;
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      probabilities(u);
      grow |= !(ps[u] <= kLazyBound);  // also a NaN or infinite sum
    }
    if constexpr (HINT) {  // beside the next block's scores: interleave
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // the key tile's reads
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one product
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // four VALU
        }
      }
    }
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform, rare
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        if (__builtin_amdgcn_ballot_w64(!(ps[u] <= kLazyBound)) == 0) continue;
        const float m = row_max(u);
        // Raise the references to the block maxima (a row whose maximum did
        // not grow keeps its reference: factor 1); this lane's accumulators
        // all belong to its own query.
        const float mn = fmaxf(mq[u], m * a.scale_log2);
        const float corr = exp2_hw(mq[u] - mn);
        lq[u] *= corr;
        mq[u] = mn;
#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[u][db][i] *= corr;
        probabilities(u);
      }
    }
#pragma unroll
    for (int u = 0; u < TPW; ++u) lq[u] += ps[u];
    }
  };

  const int vrd = (4 * g4 + (r >> 2)) * kVRow + 8 * (r & 3);
  auto pv = [&](int buf, int ksn, auto diag_tag) {
    constexpr bool kDiag = decltype(diag_tag)::value;
    const uint8_t* vb = vlds[buf];
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
        for (int u = 0; u < TPW; ++u) o[u][db] = mfma32(vt, pa[u][ks], o[u][db]);
      }
  };

  const int dtn = (int)((pt + 15 - (int64_t)(nkb - 1) * kKB) >> 4) + 1;  // diagonal tiles, 1..4
  const int dks = dtn > 2 ? 2 : 1;
  if constexpr (W == 8) {
    // Ping-pong between the two waves of each SIMD: waves 0-3 and 4-7 run
    // the same steps, the second set one step behind, so that while one wave
    // of a SIMD issues matrix-core products (step M j: block j - 1's P V,
    // then block j's scores) the other runs the VALU softmax of its block
    // (step V j), and the matrix core is fed from two instruction streams.
    // A barrier ends every step.  Loads of K j + 1 and V j are issued in
    // global step 2 j (by every wave) and waited for by the end of step
    // 2 j + 1; K j and V j - 1 are read in steps 2 j and 2 j + 1.
    const bool late = wave >= 4;
    f32x4 cc[TPW][4];
    auto bar = [] {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    auto vmwait = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
    auto issue = [&](int jk, int jv) {
      if (jk < nkb) load_k(jk, jk & 1);
      if (jv < nkb) load_v(jv, jv & 1);
    };
    auto block = [&](int j, auto diag_tag, auto first_tag) {
      constexpr bool kDiag = decltype(diag_tag)::value;
      if (!late) issue(j + 1, j);
      if (j > 0) {
        pv((j - 1) & 1, 2, std::false_type{});
        scores(j & 1, kDiag ? dtn : 4, diag_tag, cc);
        if constexpr (!kDiag) {
          // Keep LDS reads in flight ahead of the products: 8 reads first,
          // then P V's products one read each, then the scores' products
          // (two per K fragment) one read per two.
          __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
          for (int i = 0; i < 24; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        }
      } else {
        scores(j & 1, kDiag ? dtn : 4, diag_tag, cc);
      }
      if (late) vmwait();
      bar();
      if (late) issue(j + 2, j + 1);
      softmax(cc, (int64_t)j * kKB, diag_tag, std::false_type{}, first_tag);
      if (!late) vmwait();
      bar();
    };
    load_k(0, 0);
    vmwait();
    bar();
    if (late) {
      issue(1, 0);
      bar();
    }
    if (nkb == 1) {
      block(0, std::true_type{}, std::true_type{});
    } else {
      block(0, std::false_type{}, std::true_type{});
      for (int j = 1; j + 1 < nkb; ++j) block(j, std::false_type{}, std::false_type{});
      block(nkb - 1, std::true_type{}, std::false_type{});
    }
    pv((nkb - 1) & 1, dks, std::true_type{});
    if (!late) bar();  // the same barrier count for both sets
  } else {
    // Pipeline: block j + 1's scores (matrix cores) are issued beside block
    // j's softmax (VALU), then block j's P V.  K blocks run one ahead of V:
    // during block j the loads of K j + 2 (into K j's buffer) and V j + 1 (into
    // V j - 1's) fly; one barrier per block.
    f32x4 cc[TPW][4], cn[TPW][4];
    load_k(0, 0);
    if (nkb > 1) load_k(1, 1);
    load_v(0, 0);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) (every counter)
    __syncthreads();
    if (nkb == 1) {
      scores(0, dtn, std::true_type{}, cc);
      softmax(cc, 0, std::true_type{}, std::false_type{}, std::true_type{});
      pv(0, dks, std::true_type{});
    } else {
      scores(0, 4, std::false_type{}, cc);
      __syncthreads();  // every wave has read K 0: its buffer takes K 2
      int j = 0;
      for (; j + 2 < nkb; ++j) {  // block j + 1 is not the diagonal one
        load_k(j + 2, j & 1);
        load_v(j + 1, (j + 1) & 1);
        scores((j + 1) & 1, 4, std::false_type{}, cn);
        if (j == 0) softmax(cc, 0, std::false_type{}, std::false_type{}, std::true_type{});
        else softmax(cc, (int64_t)j * kKB, std::false_type{}, std::true_type{}, std::false_type{});
        pv(j & 1, 2, std::false_type{});
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < TPW; ++u)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) cc[u][kt] = cn[u][kt];
      }
      // j = nkb - 2: the next block is the diagonal one
      load_v(j + 1, (j + 1) & 1);
      scores((j + 1) & 1, dtn, std::true_type{}, cn);
      if (j == 0) softmax(cc, 0, std::false_type{}, std::false_type{}, std::true_type{});
      else softmax(cc, (int64_t)j * kKB, std::false_type{}, std::false_type{}, std::false_type{});
      pv(j & 1, 2, std::false_type{});
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      ++j;
      softmax(cn, (int64_t)j * kKB, std::true_type{}, std::false_type{}, std::false_type{});
      pv(j & 1, dks, std::true_type{});
    }
  }

  // O / l in bf16 through LDS (this wave's 16 x 128 tile; lane l writes the
  // 8 bytes of dims 16 db + 4 g4 .. + 3 of its own query), read back so that
  // every lane stores 16 contiguous bytes of one output row.
  if constexpr (W != 8) __syncthreads();  // every wave is done with the K blocks
  uint8_t* ot = reinterpret_cast<uint8_t*>(klds) + wave * 16 * kORow;  // both K buffers
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    float lt = lq[u] + __shfl_xor(lq[u], 16);
    lt += __shfl_xor(lt, 32);  // the four lanes of query r: its denominator
    const float inv = 1.0f / lt;
#pragma unroll
    for (int db = 0; db < 8; ++db)
      *reinterpret_cast<uint2*>(ot + r * kORow + 2 * (16 * db + 4 * g4)) =
          make_uint2(pack2(o[u][db][0] * inv, o[u][db][1] * inv),
                     pack2(o[u][db][2] * inv, o[u][db][3] * inv));
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

// Pairs per XCD and group of the wide grids' work order: at least 4, and
// at least 16 / qblocks, a divisor of the pairs each XCD holds (0 where
// that is one group, i.e. the plain order, or the pairs do not divide among
// the XCDs).  Measured on Qwen3-4B heads (8 calls per graph, the same
// tensors): 16 x 512 61.3 -> 56.7 us, 32 x 256 49.2 -> 44.2, 64 x 128 (8 per
// group) 42.9 -> 39.8, 8 x 1024 83.1 -> 81.6; 4 x 2048 holds 4 pairs per
// XCD, its plain order.  Grids under one workgroup per CU measured the
// same in either order.
int32_t work_group(int32_t pairs, int32_t qblocks) {
  if (pairs % kXCDs != 0) return 0;
  const int32_t per_xcd = pairs / kXCDs;
  int32_t g = 16 / qblocks > 4 ? (16 + qblocks - 1) / qblocks : 4;
  if (g > per_xcd) g = per_xcd;
  while (per_xcd % g != 0) --g;
  return g < per_xcd ? g : 0;
}

template <int G, bool WIDE>
int launch_prefill_as(PrefillArgs a, hipStream_t s) {
  constexpr int QB = Split<G, WIDE>::QB;
  a.qblocks = (int32_t)((a.length + QB - 1) / QB);
  const int64_t blocks = (int64_t)a.qblocks * a.pairs;
  if (blocks > (int64_t)INT32_MAX) return QF_E_SHAPE;
  a.group = WIDE ? work_group(a.pairs, a.qblocks) : 0;
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
  a.group = 0;
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
