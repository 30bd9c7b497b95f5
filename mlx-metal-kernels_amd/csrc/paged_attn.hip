// Paged GQA/MQA/MHA decode attention over fp16/bf16 or symmetric q8/q4 paged
// KV caches, for gfx950.
//
// Semantics: for each sequence b and query head h (kv head h / (Hq/Hkv)),
//   out[b,h] = softmax_j(q[b,h].K[j] * scale) . V[j]   over positions
//   j < min(lengths[b], max_blocks*P), position j living in physical page
//   block_table[b, j/P], slot j%P  (ops/gqa_ops.py:278-342,
//   ops/paged_kv_ops.py:258-304, ops/paged_quantized_kv_ops.py:469-515 with
//   per-sequence lengths).  Pages with an id outside [0, num_pages) are
//   skipped (kernels/q8_paged_gqa_decode_attention.metal:52-57).  A sequence
//   with no position yields zeros.  Quantized K/V dequantize as
//   (code - 128|8) * scale rounded to fp16, as dequantize_kv_pages does.
//
// Fast path (D in {64,128}, fp16 q for quantized caches): the 32-position
// blocks of all sequences are cut into equal "pairs" (see the stream plan);
// one wave per (pair, kv head[, block of 16 query heads]) streams its pair's
// blocks, crossing sequence boundaries.
//   QK^T : v_mfma_f32_16x16x32  A = K tile (16 positions x 32 d), loaded
//          straight from the page (lane = position, 4 lanes cover one row),
//          B = q^T (32 d x 16 heads; the GQA group fills the columns, so one
//          K read serves all Hq/Hkv heads).
//   P.V  : v_mfma_f32_16x16x32  A = P (16 heads x 32 positions) -- exactly
//          the accumulator layout QK^T leaves behind, B = V tile regrouped
//          per output column.
// The online softmax runs in base 2 on 32-position blocks; a sequence split
// over several pairs gets (m, l, O) partials that a second kernel merges
// (LSE merge, ops/attention_ops.py:534-550); one inside a single pair is
// finished in place.
// Short total contexts (few or short block-table rows, pages of a multiple
// of 16 positions) take a one-kernel plan instead (paged_attn_sp_kernel):
// splits laid out from the table width, merged in LDS within a workgroup and
// across workgroups by the last one to arrive at a per-(sequence, kv head)
// counter in the workspace.
#include <mutex>

#include "common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBlockPos = 32;         // positions per softmax block (two MFMA tiles)
constexpr int kMaxSplitPages = 512;   // page ids one split may touch (LDS)

// Fewest 32-position blocks per pair: below it a wave's fixed start-up cost
// outweighs the extra parallelism.  Measured (config 3 fp16 / config 4):
// 8 for fp16 and q4 pages (config 3 56.7 -> 54.0 us), 4 for q8 (8 cost it 2 %).
constexpr int kMinSplitBlocks16 = 8;
constexpr int kMinSplitBlocksQ8 = 4;
// A short total context shortens the pairs, down to kMinSplitFloor blocks, so
// that kMinPairs of them run at once: a short pair's time is mostly the
// dependent lengths -> table -> page latency at its start, not its bytes
// (one 2048-position sequence: 8 pairs 17.3 us, 32 pairs 13.3 us per call).
constexpr int kMinPairs = 32;
constexpr int kMinSplitFloor = 2;
// Segments per pair whose q is staged in LDS at start-up (a pair crossing
// more sequences loads the rest when it reaches them).
#ifndef MK_ATTN_QSLOTS
#define MK_ATTN_QSLOTS 3
#endif
constexpr int kQSlots = MK_ATTN_QSLOTS;
// Segments one pair may touch (one per block at most; the plan keeps a pair
// within 64 blocks).
constexpr int kMaxSegs = 64;
// Size of the fixed scratch of mk_paged_decode_attention_noalloc (16 MiB:
// split partials for about 1000 (pair or sequence) slots at Hq = 32, D = 128).
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;

// One segment of a pair: sequence, first and end position, page-list index
// of its first page (bit 30: the segment is the whole sequence).  (Verify
// kernels keep each segment's sequence length in a parallel LDS array.)
struct SegDesc {
  int b, t0, t1, po;
};
// MK_ATTN_NT 1 reads K/V pages with nontemporal loads (measured: no gain on
// balance -- slightly faster for fp16 pages, slower for q8 -- so off).
#ifndef MK_ATTN_NT
#define MK_ATTN_NT 0
#endif

struct PagedArgs {
  const void* q;       // [B, Hq, D]
  const void* K;       // pages (fp16/bf16 or uint8 codes)
  const void* V;
  const uint16_t* Ks;  // quantized: fp16 scales [NP, P, Hkv, G]
  const uint16_t* Vs;
  const int32_t* bt;   // [B, MB]
  const int32_t* lengths;
  void* out;           // [B, Hq, D]
  float* ws;           // partials O: [slots][Hq][D] fp32, slots = max_pairs + B
  float* ws_ml;        // partials (m, l): [slots][Hq][2] fp32
  int B, Hq, Hkv, G, HB;
  int NP, P, MB, lgP;  // fast path: P = 1 << lgP
  int gs, ngroups;     // quantization group size and groups per head
  int lg_gs;           // fast path: gs = 1 << lg_gs
  // fast-path stream plan (see stream_plan): pairs per round of resident
  // waves, the most blocks one pair may hold, and the pair count bound the
  // workspace and the grid are sized for
  int T_pairs, cap_blk, max_pairs;
  int min_split;       // fewest blocks per pair
  int units;           // (kv head, block of 16 query heads) waves per pair
  int wg_units;        // units per workgroup (a divisor of units, <= 8)
  // short-context plan (paged_attn_sp_kernel): blocks per split, waves
  // (splits) per workgroup, workgroups per (sequence, unit); sp_nw == 0
  // selects the stream plan
  int sp_blk, sp_nw, sp_nwg;
  int* cnt;            // arrival counters [B][units], zero between calls
  float scale_log2;
  // verify width: query rows per sequence (1 for decode).  With vw = W the
  // kernels see W * Hq "virtual heads" v = h * W + w per sequence (so a kv
  // head's W * G rows are consecutive, like its GQA group in decode), row w
  // seeing positions < length - (W - 1 - w); q and out stay [B, W, Hq, D]
  int vw;
  int vw_magic;        // ceil(2^16 / vw), see vsplit
};

// Row of q / out that holds virtual head v of sequence b: [B, Hq, D] in
// decode; [B, W, Hq / W, D] with v = h * W + w for verify rows.  (The merge
// and generic kernels use this; the attention kernels use qo_row_j below.)
__device__ __forceinline__ size_t qo_row(const PagedArgs& a, int b, int v) {
  if (a.vw <= 1) return (size_t)b * a.Hq + v;
  const int h = v / a.vw, w = v - h * a.vw;
  return ((size_t)b * a.vw + w) * (size_t)(a.Hq / a.vw) + h;
}

// Verify kernels: the virtual heads a wave touches are h0 + j, j < 16, for
// its wave-uniform h0 = hq0 * W + hr0.  (h0 + j) / W = hq0 + x / W with
// x = hr0 + j < W + 16 <= 80, and x / W = (x * vw_magic) >> 16 exactly for
// vw_magic = ceil(2^16 / W), W <= 64 (the rounding error x (W - 1) / 2^16 W
// stays below the 1 / W gap to the next integer) -- no division per lane.
struct VRows {
  int hq0, hr0;
};
__device__ __forceinline__ VRows vrows(const PagedArgs& a, int h0) {
  const int q = h0 / a.vw;  // wave-uniform, once per wave
  return VRows{q, h0 - q * a.vw};
}
// row w of virtual head h0 + j and its head index h
__device__ __forceinline__ void vsplit(const PagedArgs& a, VRows r, int j, int* h, int* w) {
  const int x = r.hr0 + j;
  const int qd = (x * a.vw_magic) >> 16;
  *w = x - qd * a.vw;
  *h = r.hq0 + qd;
}
// row of q / out for virtual head h0 + j of sequence b (verify: 32-bit
// arithmetic, the host keeps B * W * Hq below 2^31)
template <bool VW>
__device__ __forceinline__ size_t qo_row_j(const PagedArgs& a, VRows r, int b, int h0, int j) {
  if constexpr (!VW) {
    return (size_t)b * a.Hq + h0 + j;
  } else {
    int h, w;
    vsplit(a, r, j, &h, &w);
    return (size_t)(uint32_t)((b * a.vw + w) * (a.Hq / a.vw) + h);
  }
}

// Positions before a sequence's end that virtual head v may not see: W - 1 - w
// for verify row w, 0 in decode.
__device__ __forceinline__ int causal_offset(const PagedArgs& a, int v) {
  return a.vw <= 1 ? 0 : a.vw - 1 - v % a.vw;
}

// --------------------------------------------------------------- MFMA wrappers
template <typename AT>
__device__ __forceinline__ f32x4 mfma_k32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_k32<f16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_k32<bf16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0,
                                                 0);
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return (uint32_t)bitcast<uint16_t>((f16)lo) | ((uint32_t)bitcast<uint16_t>((f16)hi) << 16);
}
template <typename AT>
__device__ __forceinline__ uint32_t pack_act2(float lo, float hi) {
  return (uint32_t)bitcast<uint16_t>(from_f32<AT>(lo)) |
         ((uint32_t)bitcast<uint16_t>(from_f32<AT>(hi)) << 16);
}

// ------------------------------------------------------------ KV dequant
// Exact symmetric dequant into fp16 pairs: the code sits in the mantissa of
// 1024.0h, subtracting (1024 + offset) leaves (code - offset) exactly, and one
// packed multiply rounds (code - offset) * s once -- the same value as the
// fp32 product rounded to fp16.
__device__ __forceinline__ uint32_t q8_pair(uint32_t u, int shift, f16x2 s2) {
  const f16x2 k = {(f16)1152.0f, (f16)1152.0f};  // 1024 + 128
  // bytes (b0|b1, 0x64, b2|b3, 0x64) of {0x64646464, u}: one v_perm_b32
  const uint32_t t = perm_b32(0x64646464u, u, shift == 0 ? 0x04020400u : 0x04030401u);
  f16x2 v = bitcast<f16x2>(t) - k;
  return bitcast<uint32_t>(v * s2);
}
__device__ __forceinline__ uint32_t q4_pair(uint32_t u, int shift, f16x2 s2) {
  const f16x2 k = {(f16)1032.0f, (f16)1032.0f};  // 1024 + 8
  f16x2 v = bitcast<f16x2>(((u >> shift) & 0x000F000Fu) | 0x64006400u) - k;
  return bitcast<uint32_t>(v * s2);
}

// 8 q8 codes (two words) -> 8 fp16, order [0,2,1,3,4,6,5,7]
__device__ __forceinline__ u32x4 deq8x8(uint32_t u0, uint32_t u1, f16x2 s2) {
  u32x4 r;
  r[0] = q8_pair(u0, 0, s2);
  r[1] = q8_pair(u0, 8, s2);
  r[2] = q8_pair(u1, 0, s2);
  r[3] = q8_pair(u1, 8, s2);
  return r;
}
// 8 q4 codes (one word) -> 8 fp16, order [0,4,1,5,2,6,3,7].  Even nibbles
// sit at mantissa bits 0..3 of 1024.0h (ulp 1): 1024 + c.  Odd nibbles stay
// in place at bits 4..7 under the exponent of 64.0h (ulp 1/16): 64 + c.  So
// both halves give (c - 8) exactly after one subtraction and share the same
// scale multiply, which rounds (c - 8) * s once -- one shift per word.
__device__ __forceinline__ u32x4 deq4x8(uint32_t u, f16x2 s2) {
  const f16x2 k_lo = {(f16)1032.0f, (f16)1032.0f};  // 1024 + 8
  const f16x2 k_hi = {(f16)72.0f, (f16)72.0f};      // 64 + 8
  const uint32_t magic_lo = 0x64006400u;            // 1024.0h
  const uint32_t magic_hi = 0x54005400u;            // 64.0h
  const uint32_t v = u >> 8;
  u32x4 r;
  r[0] = bitcast<uint32_t>((bitcast<f16x2>((u & 0x000F000Fu) | magic_lo) - k_lo) * s2);
  r[1] = bitcast<uint32_t>((bitcast<f16x2>((u & 0x00F000F0u) | magic_hi) - k_hi) * s2);
  r[2] = bitcast<uint32_t>((bitcast<f16x2>((v & 0x000F000Fu) | magic_lo) - k_lo) * s2);
  r[3] = bitcast<uint32_t>((bitcast<f16x2>((v & 0x00F000F0u) | magic_hi) - k_hi) * s2);
  return r;
}

// --------------------------------------------------------------- fast path
// One wave per ((sequence, split) pair, kv head [, block of 16 query heads]);
// the split plan is below.  Lane l is (r16 = l % 16, kb = l / 16).
//
//   QK^T : v_mfma_f32_16x16x32, A = K tile (16 positions x 32 d; lane = row
//          r16, d run kb), B = q^T (32 d x 16 query heads; the GQA group fills
//          the columns, so one K read serves every head of the group).
//          Result: lane holds S[position 4kb+i][head r16].
//   P.V  : v_mfma_f32_16x16x32, A = P (16 heads x 32 positions) -- the two
//          QK tiles' accumulators as they lie (k = 8kb+i <-> position 4kb+i,
//          k = 8kb+4+i <-> position 16+4kb+i), B = V (32 positions x 16 d
//          columns) with the same k <-> position map, one MFMA per d slot.
//
// The context of a split streams in blocks of 32 positions, double-buffered
// in registers: the loads of block i+1 are issued before block i is
// consumed.  Loads are branch-free -- positions past the split's end or on
// an unmapped page read a clamped in-bounds row and are masked out of the
// softmax (their V is zeroed) -- so the compiler's wait counts stay exact.
// Page ids of the split are read once (see SplitCtx).  Splits that do not
// finish their sequence write (m, l, O) partials that paged_attn_merge_kernel
// combines.

__device__ __forceinline__ u32x4 kv_ld128(const void* p) {
  if constexpr (MK_ATTN_NT) return ldg128_stream(p);
  else return ldg128(p);
}
__device__ __forceinline__ u32x2 kv_ld64(const void* p) {
  if constexpr (MK_ATTN_NT) return ldg64_stream(p);
  else return ldg64(p);
}

template <int KVF, int D>
struct Fmt {
  static constexpr int KSTEPS = D / 32;  // QK MFMAs per 16-position tile
  static constexpr int DPL = D / 16;     // d's per V lane = PV MFMAs per block
  // 8-d K chunks one lane loads per instruction (16 B for every format but
  // q4 at D = 64, 8 B)
  static constexpr int KRUN_RAW = KVF == 0 ? 1 : (KVF == 8 ? 2 : 4);
  static constexpr int KRUN = KRUN_RAW < KSTEPS ? KRUN_RAW : KSTEPS;
  static constexpr int NRUN = KSTEPS / KRUN;
  static constexpr int BITS = KVF == 0 ? 16 : KVF;  // stored bits per element
  static constexpr int KBYTES_RUN = KRUN * 8 * BITS / 8;
  static constexpr int VBYTES = DPL * BITS / 8;
  static constexpr int ROW_BYTES = D * BITS / 8;
  // first d of step j for lane column kb
  static __device__ __forceinline__ int dbase(int j, int kb) {
    return (j / KRUN) * (32 * KRUN) + kb * (8 * KRUN) + (j % KRUN) * 8;
  }
  // d (within a lane's V chunk) of the half in slot j after dequant
  static __device__ __forceinline__ constexpr int vslot(int j) {
    if constexpr (KVF == 0) {
      return j;
    } else if constexpr (DPL == 4) {
      constexpr int p[4] = {0, 2, 1, 3};
      return p[j];
    } else if constexpr (KVF == 8) {
      constexpr int p[8] = {0, 2, 1, 3, 4, 6, 5, 7};
      return p[j];
    } else {
      constexpr int p[8] = {0, 4, 1, 5, 2, 6, 3, 7};
      return p[j];
    }
  }
};

// q regrouped into the order the K dequant produces (natural for fp16/bf16)
template <int KVF>
__device__ __forceinline__ u32x4 qperm(u32x4 X) {
  if constexpr (KVF == 8) {  // [0,2,1,3,4,6,5,7]
    return (u32x4){pack_lo16(X[0], X[1]), pack_hi16(X[0], X[1]), pack_lo16(X[2], X[3]),
                   pack_hi16(X[2], X[3])};
  } else if constexpr (KVF == 4) {  // [0,4,1,5,2,6,3,7]
    return (u32x4){pack_lo16(X[0], X[2]), pack_hi16(X[0], X[2]), pack_lo16(X[1], X[3]),
                   pack_hi16(X[1], X[3])};
  } else {
    return X;
  }
}

// 4 q8 codes (one word) -> 4 fp16, order [0,2,1,3]; 4 q4 codes (low 16 bits) likewise
__device__ __forceinline__ u32x2 deq8x4(uint32_t u, f16x2 s2) {
  return (u32x2){q8_pair(u, 0, s2), q8_pair(u, 8, s2)};
}
__device__ __forceinline__ u32x2 deq4x4(uint32_t u, f16x2 s2) {
  // bytes (b0, 0, b1, 0): n0 n1 @ bits 0..7, n2 n3 @ 16..23, one v_perm_b32;
  // the odd nibbles stay in place under 64.0h as in deq4x8
  const uint32_t t = perm_b32(0u, u, 0x04010400u);
  const f16x2 k_lo = {(f16)1032.0f, (f16)1032.0f};
  const f16x2 k_hi = {(f16)72.0f, (f16)72.0f};
  return (u32x2){bitcast<uint32_t>((bitcast<f16x2>((t & 0x000F000Fu) | 0x64006400u) - k_lo) * s2),
                 bitcast<uint32_t>((bitcast<f16x2>((t & 0x00F000F0u) | 0x54005400u) - k_hi) * s2)};
}

__device__ __forceinline__ f16x2 splat_h(uint32_t s) {
  return bitcast<f16x2>(s | (s << 16));
}

template <int KVF, int D, bool SB>
struct KVBlock {
  using F = Fmt<KVF, D>;
  static constexpr int NKS = KVF == 0 ? 0 : (SB ? F::NRUN : F::KSTEPS);  // K scales per tile
  u32x4 k[2][F::NRUN];
  uint32_t ks[2][NKS > 0 ? NKS : 1];  // fp16 scale bits (32-bit slots keep the block in registers)
  u32x4 v[8];
  uint32_t vs[8];
  uint32_t mask;  // bit p: position p of the block is valid (wave-uniform)
  // positions from the block's first to its sequence's end (wave-uniform):
  // verify row w may see block positions p < rel_end - (W - 1 - w)
  int rel_end;
};

// ------------------------------------------------------------ stream plan
// The context of sequence b is cut into nblk_b = ceil(len_b / 32) blocks of
// 32 positions.  The blocks of all sequences, in sequence order, form one
// list of TB blocks, cut into N pairs of Q or Q + 1 consecutive blocks (the
// first R = TB mod N pairs take Q + 1), so every pair -- one wave per unit
// (kv head, block of 16 query heads) -- carries the same work whatever the
// lengths; a CU's time is the bytes of the waves it holds, so equal pairs
// keep every CU busy to the end.  N is one round of resident waves
// (T_pairs), fewer when the pairs would hold less than
// min_split blocks (by KV format; less on a short total context, down to
// kMinSplitFloor, while fewer than kMinPairs pairs would run), more when they
// would exceed cap_blk (the
// blocks whose pages one wave can address).  A pair that crosses a sequence
// boundary works on one segment per sequence it touches.  A segment that
// covers its whole sequence writes the output; any other writes a partial
// (m, l, O) to slot pair + b -- unique, and consecutive over the pairs of one
// sequence -- which the merge kernel combines (LSE merge,
// ops/attention_ops.py:534-550).  Every wave derives the same plan from the
// lengths on the device.
__device__ __forceinline__ int clamp_len(int len, int max_s) {
  return len < 0 ? 0 : (len > max_s ? max_s : len);
}

__device__ __forceinline__ int nblk_of(int len) { return (len + kBlockPos - 1) / kBlockPos; }

__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int64_t wave_incl_scan_i64(int64_t v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

struct StreamPlan {
  int64_t TB;  // blocks over all sequences
  int64_t N;   // pairs in use (0 when every sequence is empty)
  int64_t Q;   // blocks per pair; the first R pairs take one more
  int64_t R;
  int len0;    // lane b < 64: positions of sequence b
  int start0;  // lane b < 64: global index of sequence b's first block
};

__device__ __forceinline__ int64_t pair_start(const StreamPlan& sp, int64_t p) {
  return p * sp.Q + (p < sp.R ? p : sp.R);
}

// pair holding global block g (g < TB)
__device__ __forceinline__ int64_t pair_of(const StreamPlan& sp, int64_t g) {
  const int64_t big = sp.R * (sp.Q + 1);
  return g < big ? g / (sp.Q + 1) : sp.R + (g - big) / sp.Q;
}

__device__ StreamPlan stream_plan(const PagedArgs& a, int lane) {
  const int max_s = a.MB << a.lgP;
  StreamPlan sp;
  sp.len0 = lane < a.B ? clamp_len(a.lengths[lane], max_s) : 0;
  const int nb0 = nblk_of(sp.len0);
  int64_t tb = nb0;
  for (int c = 64; c < a.B; c += 64) {
    const int b = c + lane;
    tb += b < a.B ? nblk_of(clamp_len(a.lengths[b], max_s)) : 0;
  }
  sp.TB = wave_sum_i64(tb);
  sp.start0 = (int)(wave_incl_scan_i64(nb0, lane) - nb0);
  int64_t N = a.T_pairs;
  int64_t minb = a.min_split < a.cap_blk ? a.min_split : a.cap_blk;
  const int64_t want = sp.TB / kMinPairs;  // blocks per pair at kMinPairs pairs
  if (want < minb) minb = want > kMinSplitFloor ? want : kMinSplitFloor;
  if (minb > a.cap_blk) minb = a.cap_blk;
  if (sp.TB < N * minb) N = (sp.TB + minb - 1) / minb;
  if (N > 0 && (sp.TB + N - 1) / N > a.cap_blk) N = (sp.TB + a.cap_blk - 1) / a.cap_blk;
  if (N > sp.TB) N = sp.TB;
  sp.N = N;
  sp.Q = N > 0 ? sp.TB / N : 0;
  sp.R = N > 0 ? sp.TB - sp.Q * N : 0;
  return sp;
}

// Length and first global block of sequence b (wave-uniform b < B).
__device__ void seq_info(const PagedArgs& a, const StreamPlan& sp, int b, int lane, int* len,
                         int64_t* start) {
  if (b < 64) {
    *len = __builtin_amdgcn_readlane(sp.len0, b);
    *start = __builtin_amdgcn_readlane(sp.start0, b);
    return;
  }
  const int max_s = a.MB << a.lgP;
  int64_t carry = wave_sum_i64(nblk_of(sp.len0));
  for (int c = 64; c < a.B; c += 64) {
    const int bb = c + lane;
    const int l = bb < a.B ? clamp_len(a.lengths[bb], max_s) : 0;
    const int64_t incl = wave_incl_scan_i64(nblk_of(l), lane) + carry;
    if (b < c + 64) {
      *len = __shfl(l, b - c, 64);
      *start = __shfl(incl, b - c, 64) - nblk_of(*len);
      return;
    }
    carry = __shfl(incl, 63, 64);
  }
  *len = 0;
  *start = carry;
}

// The sequence holding global block g (g < TB) and its first global block.
__device__ int seq_of_block(const PagedArgs& a, const StreamPlan& sp, int64_t g, int lane, int64_t* start) {
  const int max_s = a.MB << a.lgP;
  int64_t carry = 0;
  for (int c = 0; c < a.B; c += 64) {
    const int bb = c + lane;
    const int nb = c == 0 ? nblk_of(sp.len0) : (bb < a.B ? nblk_of(clamp_len(a.lengths[bb], max_s)) : 0);
    const int64_t incl = wave_incl_scan_i64(nb, lane) + carry;
    // sequences ending at or before g come first (ends never decrease)
    const uint64_t before = __ballot(bb < a.B && incl <= g);
    const int k = __popcll(before);
    if (k < 64 && c + k < a.B) {
      *start = __shfl(incl, k, 64) - __shfl(nb, k, 64);
      return c + k;
    }
    carry = __shfl(incl, 63, 64);
  }
  *start = carry;
  return a.B - 1;
}

// Merge the split partials of query heads [h0, h0 + hcount) of sequence b
// (LSE merge, ops/attention_ops.py:534-550): one wave, lanes over d.
template <typename AT, int D>
__device__ void merge_heads(const PagedArgs& a, int b, int h0, int hcount, int first, int nsplit,
                            int lane) {
  constexpr int DPT = D / 64;  // d's per lane
  const size_t sstride = (size_t)a.Hq;  // slots between consecutive splits of one head
  for (int hh = 0; hh < hcount; ++hh) {
    const int h = h0 + hh;
    const float* ml = a.ws_ml + ((size_t)first * a.Hq + h) * 2;
    const float* po = a.ws + ((size_t)first * a.Hq + h) * D + lane * DPT;
    if (nsplit <= 64) {
      // one round trip: lane s holds split s's (m, l); the O partials go out
      // in batches of 32 that do not wait for (m, l).  Indices past the last
      // split re-read it and get weight exp2(-inf) = 0.
      constexpr int BATCH = 32;
      const f32x2 v = lane < nsplit ? *reinterpret_cast<const f32x2*>(ml + (size_t)lane * sstride * 2)
                                    : (f32x2){-INFINITY, 0.0f};
      float acc[DPT];
#pragma unroll
      for (int e = 0; e < DPT; ++e) acc[e] = 0.0f;
      float x[BATCH][DPT];
#pragma unroll
      for (int k = 0; k < BATCH; ++k) {
        const float* p = po + (size_t)(k < nsplit ? k : nsplit - 1) * sstride * D;
        if constexpr (DPT == 2) {
          const f32x2 y = *reinterpret_cast<const f32x2*>(p);
          x[k][0] = y[0];
          x[k][1] = y[1];
        } else {
          x[k][0] = p[0];
        }
      }
      const float M = wave_max(v[0]);
      const float Mu = M == -INFINITY ? 0.0f : M;
      const float w = __builtin_amdgcn_exp2f(v[0] - Mu);
      const float L = wave_sum(v[1] * w);
#pragma unroll
      for (int k = 0; k < BATCH; ++k) {
        const float wk = __shfl(w, k, 64);
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[e] += wk * x[k][e];
      }
      if (nsplit > BATCH) {  // wave-uniform
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
          const int sk = BATCH + k;
          const float* p = po + (size_t)(sk < nsplit ? sk : nsplit - 1) * sstride * D;
          if constexpr (DPT == 2) {
            const f32x2 y = *reinterpret_cast<const f32x2*>(p);
            x[k][0] = y[0];
            x[k][1] = y[1];
          } else {
            x[k][0] = p[0];
          }
        }
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
          const float wk = __shfl(w, BATCH + k, 64);
#pragma unroll
          for (int e = 0; e < DPT; ++e) acc[e] += wk * x[k][e];
        }
      }
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      AT* op = reinterpret_cast<AT*>(a.out) + qo_row(a, b, h) * D + lane * DPT;
      if constexpr (DPT == 2) {
        *reinterpret_cast<uint32_t*>(op) = pack_act2<AT>(acc[0] * inv, acc[1] * inv);
      } else {
        op[0] = from_f32<AT>(acc[0] * inv);
      }
      continue;
    }
    float M = -INFINITY;
    for (int s0 = 0; s0 < nsplit; s0 += 64) {
      const int s = s0 + lane;
      M = fmaxf(M, s < nsplit ? ml[(size_t)s * sstride * 2] : -INFINITY);
    }
    M = wave_max(M);
    const float Mu = M == -INFINITY ? 0.0f : M;
    float acc[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[e] = 0.0f;
    float L = 0.0f;
    for (int s0 = 0; s0 < nsplit; s0 += 64) {
      const int s = s0 + lane;
      const f32x2 v = s < nsplit ? *reinterpret_cast<const f32x2*>(ml + (size_t)s * sstride * 2)
                                 : (f32x2){-INFINITY, 0.0f};
      const float w = __builtin_amdgcn_exp2f(v[0] - Mu);
      L += v[1] * w;
      const int n = min(64, nsplit - s0);
      int t = 0;
      for (; t + 4 <= n; t += 4) {
        float x[4][DPT], ws[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          ws[k] = __shfl(w, t + k, 64);
          const float* p = po + (size_t)(s0 + t + k) * sstride * D;
          if constexpr (DPT == 2) {
            const f32x2 y = *reinterpret_cast<const f32x2*>(p);
            x[k][0] = y[0];
            x[k][1] = y[1];
          } else {
            x[k][0] = p[0];
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int e = 0; e < DPT; ++e) acc[e] += ws[k] * x[k][e];
      }
      for (; t < n; ++t) {
        const float wt = __shfl(w, t, 64);
        const float* p = po + (size_t)(s0 + t) * sstride * D;
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[e] += wt * p[e];
      }
    }
    L = wave_sum(L);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    AT* op = reinterpret_cast<AT*>(a.out) + qo_row(a, b, h) * D + lane * DPT;
    if constexpr (DPT == 2) {
      *reinterpret_cast<uint32_t*>(op) = pack_act2<AT>(acc[0] * inv, acc[1] * inv);
    } else {
      op[0] = from_f32<AT>(acc[0] * inv);
    }
  }
}

// One wave per (sequence, query head): merges the partials of the pairs the
// sequence spans (a sequence inside one pair was written by the attention
// kernel) and writes zeros for a sequence with no position.
template <typename AT, int D>
__global__ __launch_bounds__(64) void paged_attn_merge_kernel(const PagedArgs a) {
  const int lane = threadIdx.x;
  const int b = (int)blockIdx.x / a.Hq;
  const int h = (int)blockIdx.x - b * a.Hq;
  const StreamPlan sp = stream_plan(a, lane);
  int len;
  int64_t start;
  seq_info(a, sp, b, lane, &len, &start);
  if (len == 0) {
    AT* op = reinterpret_cast<AT*>(a.out) + qo_row(a, b, h) * D;
    for (int d = lane; d < D; d += 64) op[d] = from_f32<AT>(0.0f);
    return;
  }
  const int64_t p0 = pair_of(sp, start), p1 = pair_of(sp, start + nblk_of(len) - 1);
  if (p0 == p1) return;
  merge_heads<AT, D>(a, b, h, 1, (int)(p0 + b), (int)(p1 - p0 + 1), lane);
}

// Where one segment's positions live.  The page ids of all segments of a
// pair sit in one list, segment by segment (a segment's first page at index
// po).  Two addressing modes:
//  * PT (page size a multiple of 16): a 16-position tile never crosses a
//    page, so each tile needs one page id -- read from a register that holds
//    the list (lane i: entry i, at most 64) -- and the tile's row base is
//    wave-uniform; lanes add fixed offsets.
//  * otherwise: every position looks its page up in an LDS copy of the list.
struct SplitCtx {
  const int* spage;  // !PT: LDS page list (invalid as -1)
  int my_page;       // PT: page list entry `lane` (invalid as -1)
  int blk0;          // logical page of the segment's first position
  int po;            // list index of that page
  int t_begin, t_end, lgP, Pm, Hkv, hkv;
  int seq_len;       // length of the segment's sequence
  // !PT: row index (page, slot, kv head) of position t, clamped into the
  // segment; *ok says whether t is a real, mapped position
  __device__ __forceinline__ uint32_t row(int t, bool* ok) const {
    const bool in = t < t_end;
    const int tc = in ? t : t_end - 1;
    const int pg = spage[po + (tc >> lgP) - blk0];
    *ok = in && pg >= 0;
    const uint32_t p = pg < 0 ? 0u : (uint32_t)pg;
    return (((p << lgP) + (uint32_t)(tc & Pm)) * (uint32_t)Hkv) + (uint32_t)hkv;
  }
  // PT: row index of the first position of the 16-position tile at tu
  // (clamped to the split's last tile) and the tile's validity bits
  __device__ __forceinline__ uint32_t tile_row(int tu, uint32_t* bits) const {
    const int last = (t_end - 1) & ~15;
    const int tc = tu < last ? tu : last;
    const int pg = __builtin_amdgcn_readlane(my_page, po + (tc >> lgP) - blk0);
    int n = t_end - tu;
    n = n < 0 ? 0 : (n > 16 ? 16 : n);
    *bits = pg < 0 ? 0u : (n == 16 ? 0xFFFFu : ((1u << n) - 1u));
    const uint32_t p = pg < 0 ? 0u : (uint32_t)pg;
    return (((p << lgP) + (uint32_t)(tc & Pm)) * (uint32_t)Hkv) + (uint32_t)hkv;
  }
};

// Lane-constant byte offsets of the PT addressing mode.  The K run r of row
// r16 sits at k0 + r * KRUN_STRIDE and the V chunk of row 4kb + i at
// v0 + i * rs (rs, the bytes between positions of a page, is wave-uniform and
// goes into the scalar base), so two offsets stay live across the block loop.
template <int KVF, int D, bool SB>
struct LaneOffsets {
  using F = Fmt<KVF, D>;
  static constexpr int NKS = KVF == 0 ? 0 : (SB ? F::NRUN : F::KSTEPS);
  static constexpr uint32_t KRUN_STRIDE = 32 * F::KRUN * F::BITS / 8;  // dbase(j + KRUN) - dbase(j), bytes
  uint32_t k0;                     // K codes of run 0 of row r16
  uint32_t v0;                     // V chunk of row 4kb
  uint32_t rs;                     // bytes between positions of a page (wave-uniform)
  uint32_t ks[NKS > 0 ? NKS : 1];  // K scale (elements) of the lane's chunks
  uint32_t vs[4];                  // V scale (elements)
};

// The lane offsets of the PT addressing mode for lane (r16, kb).
template <int KVF, int D, bool SB>
__device__ __forceinline__ LaneOffsets<KVF, D, SB> pt_lane_offsets(const PagedArgs& a, int r16, int kb) {
  using F = Fmt<KVF, D>;
  LaneOffsets<KVF, D, SB> lo;
  const uint32_t rs = (uint32_t)a.Hkv * F::ROW_BYTES;  // bytes between positions of a page
  lo.rs = rs;
  lo.k0 = (uint32_t)r16 * rs + (uint32_t)(F::dbase(0, kb) * F::BITS / 8);
  lo.v0 = (uint32_t)(4 * kb) * rs + (uint32_t)(r16 * F::VBYTES);
  if constexpr (KVF != 0) {
    const uint32_t ss = (uint32_t)a.Hkv * a.ngroups;  // scale elements between positions
#pragma unroll
    for (int e = 0; e < KVBlock<KVF, D, SB>::NKS; ++e) {
      const int j = SB ? e * F::KRUN : e;
      lo.ks[e] = (uint32_t)r16 * ss + (uint32_t)(F::dbase(j, kb) >> a.lg_gs);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) lo.vs[i] = (uint32_t)(4 * kb + i) * ss + (uint32_t)((r16 * F::DPL) >> a.lg_gs);
  }
  return lo;
}

template <typename AT, int D, int KVF, bool SB, bool PT>
__device__ __forceinline__ void load_block(KVBlock<KVF, D, SB>& blk, const PagedArgs& a,
                                           const SplitCtx& c, const LaneOffsets<KVF, D, SB>& lo,
                                           int tb, int r16, int kb) {
  using F = Fmt<KVF, D>;
  constexpr int NKS = KVBlock<KVF, D, SB>::NKS;
  const uint8_t* Kb = reinterpret_cast<const uint8_t*>(a.K);
  const uint8_t* Vb = reinterpret_cast<const uint8_t*>(a.V);
  if constexpr (PT) {
    uint32_t m = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      uint32_t bits;
      const uint32_t row0 = c.tile_row(tb + 16 * u, &bits);
      m |= bits << (16 * u);
      const uint8_t* kt = Kb + (uint64_t)row0 * F::ROW_BYTES;
      const uint8_t* vt = Vb + (uint64_t)row0 * F::ROW_BYTES;
#pragma unroll
      for (int r = 0; r < F::NRUN; ++r) {
        if constexpr (F::KBYTES_RUN == 16) {
          blk.k[u][r] = kv_ld128(kt + lo.k0 + r * LaneOffsets<KVF, D, SB>::KRUN_STRIDE);
        } else {
          const u32x2 x = kv_ld64(kt + lo.k0 + r * LaneOffsets<KVF, D, SB>::KRUN_STRIDE);
          blk.k[u][r] = (u32x4){x[0], x[1], 0u, 0u};
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint8_t* vr = (vt + (uint64_t)i * lo.rs) + lo.v0;
        u32x4 x;
        if constexpr (F::VBYTES == 16) {
          x = kv_ld128(vr);
        } else if constexpr (F::VBYTES == 8) {
          const u32x2 y = kv_ld64(vr);
          x = (u32x4){y[0], y[1], 0u, 0u};
        } else if constexpr (F::VBYTES == 4) {
          x = (u32x4){*reinterpret_cast<const uint32_t*>(vr), 0u, 0u, 0u};
        } else {
          x = (u32x4){(uint32_t)*reinterpret_cast<const uint16_t*>(vr), 0u, 0u, 0u};
        }
        blk.v[4 * u + i] = x;
      }
      if constexpr (KVF != 0) {
        const uint16_t* kst = a.Ks + (uint64_t)row0 * a.ngroups;
        const uint16_t* vst = a.Vs + (uint64_t)row0 * a.ngroups;
#pragma unroll
        for (int e = 0; e < NKS; ++e) blk.ks[u][e] = kst[lo.ks[e]];
#pragma unroll
        for (int i = 0; i < 4; ++i) blk.vs[4 * u + i] = vst[lo.vs[i]];
      }
    }
    blk.mask = m;
    blk.rel_end = c.seq_len - tb;
  } else {
    uint32_t m = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bool ok;
      const uint32_t row = c.row(tb + 16 * u + r16, &ok);
      const uint8_t* kr = Kb + (uint64_t)row * F::ROW_BYTES;
#pragma unroll
      for (int r = 0; r < F::NRUN; ++r) {
        const int off = F::dbase(r * F::KRUN, kb) * F::BITS / 8;
        if constexpr (F::KBYTES_RUN == 16) {
          blk.k[u][r] = kv_ld128(kr + off);
        } else {
          const u32x2 x = kv_ld64(kr + off);
          blk.k[u][r] = (u32x4){x[0], x[1], 0u, 0u};
        }
      }
      if constexpr (KVF != 0) {
        const uint16_t* sr = a.Ks + (uint64_t)row * a.ngroups;
#pragma unroll
        for (int e = 0; e < NKS; ++e) {
          const int j = SB ? e * F::KRUN : e;
          blk.ks[u][e] = sr[F::dbase(j, kb) >> a.lg_gs];
        }
      }
      const uint64_t bal = __ballot(ok);
      m |= ((uint32_t)bal & 0xFFFFu) << (16 * u);
    }
    blk.mask = m;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      bool ok;
      const int pos = (p < 4 ? 4 * kb + p : 16 + 4 * kb + (p - 4));
      const uint32_t row = c.row(tb + pos, &ok);
      const uint8_t* vr = Vb + (uint64_t)row * F::ROW_BYTES + r16 * F::VBYTES;
      if constexpr (F::VBYTES == 16) {
        blk.v[p] = kv_ld128(vr);
      } else if constexpr (F::VBYTES == 8) {
        const u32x2 x = kv_ld64(vr);
        blk.v[p] = (u32x4){x[0], x[1], 0u, 0u};
      } else if constexpr (F::VBYTES == 4) {
        blk.v[p] = (u32x4){*reinterpret_cast<const uint32_t*>(vr), 0u, 0u, 0u};
      } else {
        blk.v[p] = (u32x4){(uint32_t)*reinterpret_cast<const uint16_t*>(vr), 0u, 0u, 0u};
      }
      if constexpr (KVF != 0)
        blk.vs[p] = a.Vs[(uint64_t)row * a.ngroups + ((r16 * F::DPL) >> a.lg_gs)];
    }
    blk.rel_end = c.seq_len - tb;
  }
}

// 8 act-type values of K step j (order as qperm<KVF>)
template <typename AT, int D, int KVF, bool SB>
__device__ __forceinline__ u32x4 k_operand(const KVBlock<KVF, D, SB>& blk, int u, int j) {
  using F = Fmt<KVF, D>;
  const int r = j / F::KRUN, e = j % F::KRUN;
  if constexpr (KVF == 0) {
    return blk.k[u][r];
  } else {
    const f16x2 s2 = splat_h(blk.ks[u][SB ? r : j]);
    if constexpr (KVF == 8) return deq8x8(blk.k[u][r][2 * e], blk.k[u][r][2 * e + 1], s2);
    else return deq4x8(blk.k[u][r][e], s2);
  }
}

// V chunk of position p as DPL act-type values in slot order (Fmt::vslot)
template <int D, int KVF, bool SB>
__device__ __forceinline__ u32x4 v_chunk(const KVBlock<KVF, D, SB>& blk, int p) {
  if constexpr (KVF == 0) {
    return blk.v[p];
  } else {
    const f16x2 s2 = splat_h(blk.vs[p]);
    if constexpr (D == 128) {
      if constexpr (KVF == 8) return deq8x8(blk.v[p][0], blk.v[p][1], s2);
      else return deq4x8(blk.v[p][0], s2);
    } else {
      const u32x2 x = KVF == 8 ? deq8x4(blk.v[p][0], s2) : deq4x4(blk.v[p][0], s2);
      return (u32x4){x[0], x[1], 0u, 0u};
    }
  }
}

// Segment s of the list, as wave-uniform (scalar) values.
__device__ __forceinline__ SegDesc seg_at(const SegDesc* sd, int s) {
  const SegDesc d = sd[s];
  return SegDesc{__builtin_amdgcn_readfirstlane(d.b), __builtin_amdgcn_readfirstlane(d.t0),
                 __builtin_amdgcn_readfirstlane(d.t1), __builtin_amdgcn_readfirstlane(d.po)};
}

// Page-list entry i of a pair: the page of logical block
// (t0_s >> lgP) + (i - po_s) of sequence b_s, s the last segment with
// po_s <= i; -1 for an id outside [0, NP).
__device__ __forceinline__ int page_entry(const PagedArgs& a, int i, int nseg, const SegDesc* sd) {
  int b = 0, pg = 0;
  for (int s = 0; s < nseg; ++s) {
    const SegDesc d = seg_at(sd, s);
    const int po = d.po & ((1 << 30) - 1);
    if (i >= po) {
      b = d.b;
      pg = (d.t0 >> a.lgP) + (i - po);
    }
  }
  const int p = a.bt[(size_t)b * a.MB + pg];
  return (p >= 0 && p < a.NP) ? p : -1;
}

// Point the addressing context at a segment.
__device__ __forceinline__ void set_segment(SplitCtx& c, const SegDesc d) {
  c.t_begin = d.t0;
  c.t_end = d.t1;
  c.po = d.po & ((1 << 30) - 1);
  c.blk0 = c.t_begin >> c.lgP;
}

// Dynamic LDS bytes per wave: the staged q operands of segments
// 1 .. kQSlots-1, then the segment list.
template <int D>
__host__ __device__ constexpr size_t attn_wave_lds() {
  return (size_t)(kQSlots - 1) * (D / 32) * 64 * 16 + kMaxSegs * (sizeof(SegDesc) + sizeof(int));
}

// q^T operand of sequence b: lane (head r16, kb) gets q[b, h0 + r16][dbase(j, kb) .. +8]
// (zeros for heads past hcount), in the K dequant order.
template <typename AT, int D, int KVF, bool VW>
__device__ __forceinline__ void load_q(const PagedArgs& a, VRows vr, int b, int h0, int hcount, int r16, int kb,
                                       u32x4* qv) {
  using F = Fmt<KVF, D>;
  const bool hv = r16 < hcount;
  const AT* qp = reinterpret_cast<const AT*>(a.q) + qo_row_j<VW>(a, vr, b, h0, hv ? r16 : 0) * D;
#pragma unroll
  for (int j = 0; j < F::KSTEPS; ++j) {
    const u32x4 x = ldg128(qp + F::dbase(j, kb));
    qv[j] = hv ? qperm<KVF>(x) : (u32x4){0u, 0u, 0u, 0u};
  }
}

// q of segment s >= 1: from its LDS slot, or (past kQSlots) from global memory.
template <typename AT, int D, int KVF, bool VW>
__device__ __forceinline__ void begin_segment(const PagedArgs& a, VRows vr, u32x4* qv, const u32x4* qslots, int s,
                                              const SegDesc* sd, int h0, int hcount, int lane, int r16, int kb) {
  constexpr int KSTEPS = Fmt<KVF, D>::KSTEPS;
  if (s < kQSlots) {
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) qv[j] = qslots[((s - 1) * KSTEPS + j) * 64 + lane];
  } else {
    load_q<AT, D, KVF, VW>(a, vr, seg_at(sd, s).b, h0, hcount, r16, kb, qv);
  }
}

// Write segment s's result: the output when the segment is its whole
// sequence, else the partial (O unnormalised, m, l) in slot pair + b.
// Lane holds O[head 4kb + i][d = r16*DPL + vslot(j)].
template <typename AT, int D, int KVF, bool VW>
__device__ __forceinline__ void write_segment(const PagedArgs& a, VRows vr, const f32x4* o, float m_run,
                                              float l_run, const SegDesc d, int pair, int h0, int hcount) {
  using F = Fmt<KVF, D>;
  constexpr int DPL = F::DPL;
  // lane-derived values are recomputed here so they need not stay live
  // across the block loop (verify kernels: an opaque lane index, so the
  // compiler cannot hoist the rows' address arithmetic out of the loop)
  int lane = (int)__lane_id();
  if constexpr (VW) asm volatile("" : "+v"(lane));
  const int r16 = lane & 15, kb = lane >> 4;
  const int b = d.b;
  const bool whole = (d.po >> 30) & 1;
  float lv[4], mv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lv[i] = __shfl(l_run, 4 * kb + i, 64);
    mv[i] = __shfl(m_run, 4 * kb + i, 64);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * kb + i;
    if (h >= hcount) continue;
    float nat[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) nat[F::vslot(j)] = o[j][i];
    if (whole) {
      const float inv = lv[i] > 0.0f ? 1.0f / lv[i] : 0.0f;
      uint32_t w[DPL / 2];
#pragma unroll
      for (int e = 0; e < DPL / 2; ++e) w[e] = pack_act2<AT>(nat[2 * e] * inv, nat[2 * e + 1] * inv);
      AT* op = reinterpret_cast<AT*>(a.out) + qo_row_j<VW>(a, vr, b, h0, h) * D + r16 * DPL;
      if constexpr (DPL == 8) *reinterpret_cast<u32x4*>(op) = (u32x4){w[0], w[1], w[2], w[3]};
      else *reinterpret_cast<u32x2*>(op) = (u32x2){w[0], w[1]};
    } else {
      const size_t slot = (size_t)(pair + b) * a.Hq + h0 + h;
      float* po = a.ws + slot * D + r16 * DPL;
#pragma unroll
      for (int e = 0; e < DPL / 4; ++e)
        reinterpret_cast<f32x4*>(po)[e] = (f32x4){nat[4 * e], nat[4 * e + 1], nat[4 * e + 2], nat[4 * e + 3]};
      if (r16 == 0) *reinterpret_cast<f32x2*>(a.ws_ml + slot * 2) = (f32x2){mv[i], lv[i]};
    }
  }
}

// Softmax scores are kept in base 2.  The running max of a head is only
// raised when a block's max exceeds it by more than kLazyMax (so p <= 2^8,
// exact in fp16/bf16 exponent range); the O rescale runs only then.
constexpr float kLazyMax = 8.0f;

// One 32-position block of the online softmax: S = K q^T for its two
// 16-position tiles, the (lazy) running max and sum, O += P V.  Lane
// (r16, kb) holds m_run / l_run of head r16 and O[head 4kb + i][d slot j] in
// o[j][i]; masked positions get p = 0 and a zeroed V row.
template <typename AT, int D, int KVF, bool SB, bool VW>
__device__ __forceinline__ void consume_block(const KVBlock<KVF, D, SB> blk,
                                              const u32x4 (&qv)[Fmt<KVF, D>::KSTEPS], float scale_log2,
                                              int kb, const PagedArgs& a, VRows vr, float& m_run,
                                              float& l_run, f32x4 (&o)[Fmt<KVF, D>::DPL]) {
  constexpr int KSTEPS = Fmt<KVF, D>::KSTEPS;
  constexpr int DPL = Fmt<KVF, D>::DPL;
  // ---- S^T = K q^T for the two 16-position tiles
  f32x4 sc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) acc = mfma_k32<AT>(k_operand<AT, D, KVF, SB>(blk, u, j), qv[j], acc);
    sc[u] = acc;
  }
  // ---- scores (base 2); lane holds S[16u + 4kb + i][head r16]
  float sv[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[u][i] = sc[u][i] * scale_log2;
  const bool full = blk.mask == 0xFFFFFFFFu;  // wave-uniform
  // verify rows: a row's causal limit inside this block (wave-uniform test)
  const bool climit = VW && blk.rel_end - (a.vw - 1) < kBlockPos;
  if (!full || climit) {
    uint32_t mk = blk.mask;
    if (climit) {
      // lane column r16 is virtual head h0 + r16 = h * W + w, which sees
      // block positions < rel_end - (W - 1 - w); folded into the mask here,
      // in the few blocks that need it, so nothing stays live across the loop
      int hh, w;
      vsplit(a, vr, (int)__lane_id() & 15, &hh, &w);
      const int lim = blk.rel_end - (a.vw - 1 - w);
      mk &= lim >= kBlockPos ? 0xFFFFFFFFu : (lim <= 0 ? 0u : (1u << lim) - 1u);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!((mk >> (16 * u + 4 * kb + i)) & 1u)) sv[u][i] = -INFINITY;
  }
  float bmax = fmaxf(fmaxf(fmaxf(sv[0][0], sv[0][1]), fmaxf(sv[0][2], sv[0][3])),
                     fmaxf(fmaxf(sv[1][0], sv[1][1]), fmaxf(sv[1][2], sv[1][3])));
  bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
  // lazy max: raise m only when the block exceeds it by more than kLazyMax
  const bool raise = bmax > m_run + kLazyMax;
  const float m_new = raise ? bmax : m_run;
  const float m_use = m_new == -INFINITY ? 0.0f : m_new;  // an all-masked head keeps p = 0
  float psum = 0.0f;
  float p[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[u][i] = __builtin_amdgcn_exp2f(sv[u][i] - m_use);
      psum += p[u][i];
    }
  }
  psum += __shfl_xor(psum, 16, 64);
  psum += __shfl_xor(psum, 32, 64);
  if (__builtin_amdgcn_ballot_w64(raise) != 0) {  // wave-uniform: some head's max moved
    const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;
    l_run *= alpha;
    // O lane holds O[head 4kb + i][column r16]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float al = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[j][i] *= al;
    }
  }
  l_run += psum;
  m_run = m_new;
  const u32x4 pa = {pack_act2<AT>(p[0][0], p[0][1]), pack_act2<AT>(p[0][2], p[0][3]),
                    pack_act2<AT>(p[1][0], p[1][1]), pack_act2<AT>(p[1][2], p[1][3])};

  // ---- V operand chunks; masked positions are zeroed so stale or non-finite
  // cache contents cannot reach the output through p = 0
  u32x4 vc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) vc[q] = v_chunk<D, KVF, SB>(blk, q);
  if (!full) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int pos = q < 4 ? 4 * kb + q : 16 + 4 * kb + (q - 4);
      if (!((blk.mask >> pos) & 1u)) vc[q] = (u32x4){0u, 0u, 0u, 0u};
    }
  }
  // ---- O += P V, one MFMA per d slot
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int w = j >> 1;
    u32x4 bop;
    if (j & 1) {
      bop = (u32x4){pack_hi16(vc[0][w], vc[1][w]), pack_hi16(vc[2][w], vc[3][w]),
                    pack_hi16(vc[4][w], vc[5][w]), pack_hi16(vc[6][w], vc[7][w])};
    } else {
      bop = (u32x4){pack_lo16(vc[0][w], vc[1][w]), pack_lo16(vc[2][w], vc[3][w]),
                    pack_lo16(vc[4][w], vc[5][w]), pack_lo16(vc[6][w], vc[7][w])};
    }
    o[j] = mfma_k32<AT>(pa, bop, o[j]);
  }
}

template <typename AT, int D, int KVF, bool SB, bool PT, bool VW>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void paged_attn_kernel(
    const PagedArgs a) {
  using F = Fmt<KVF, D>;
  using Blk = KVBlock<KVF, D, SB>;
  constexpr int KSTEPS = F::KSTEPS;
  constexpr int DPL = F::DPL;

  const int lane = threadIdx.x & 63;
  const int r16 = lane & 15;
  const int kb = lane >> 4;
  // workgroup -> (pair, group of wg_units units); wave -> unit = (kv head,
  // block of 16 query heads).  The units of a pair read the same pages (one
  // kv head's slice of every position each), so they share a workgroup: the
  // CU then streams whole pages instead of every XCD fetching a strided
  // slice of the same page.
  // With one unit per workgroup the dispatcher's round-robin over XCDs
  // would give each XCD one kv head; rotating the units by the pair index
  // spreads every head over all XCDs.
  const int groups = a.units / a.wg_units;
  const int pair = (int)blockIdx.x / groups;
  const int unit = (((int)blockIdx.x - pair * groups) * a.wg_units + (int)(threadIdx.x >> 6) +
                    (a.wg_units == 1 ? pair : 0)) % a.units;
  const int hkv = unit / a.HB;
  const int hb = unit - hkv * a.HB;
  const StreamPlan sp = stream_plan(a, lane);
  if (pair >= sp.N) return;  // workgroup-uniform: a pair the plan leaves unused
  const int64_t g0 = pair_start(sp, pair), g1 = pair_start(sp, pair + 1);
  const int h0 = hkv * a.G + hb * 16;
  const int hcount = min(16, a.G - hb * 16);

  // ---- the pair's segments, in this wave's LDS after its staged q operands
  // (segments 1 .. kQSlots-1): kMaxSegs descriptors (a pair holds at most
  // cap_blk <= 64 blocks, so at most 64 segments)
  extern __shared__ __align__(16) uint8_t attn_dyn[];
  u32x4* qslots = reinterpret_cast<u32x4*>(attn_dyn + (size_t)(threadIdx.x >> 6) * attn_wave_lds<D>());
  SegDesc* sd = reinterpret_cast<SegDesc*>(qslots + (kQSlots - 1) * KSTEPS * 64);
  int* slen = reinterpret_cast<int*>(sd + kMaxSegs);  // verify: segment s's sequence length
  const VRows vr = VW ? vrows(a, h0) : VRows{0, 0};
  int nseg = 0, npg = 0;
  {
    int64_t st;
    int b = seq_of_block(a, sp, g0, lane, &st);
    for (int64_t g = g0; g < g1 && b < a.B; ++b) {
      int len;
      seq_info(a, sp, b, lane, &len, &st);
      const int nb = nblk_of(len);
      if (nb == 0) continue;
      const int lbb = (int)(g - st);
      const int lbe = (int)((int64_t)nb < g1 - st ? (int64_t)nb : g1 - st);
      const int t0 = lbb * kBlockPos;
      const int t1 = min(lbe * kBlockPos, len);
      if (lane == 0) {
        sd[nseg] = SegDesc{b, t0, t1, npg | ((lbb == 0 && lbe == nb) ? (1 << 30) : 0)};
        if constexpr (VW) slen[nseg] = len;
      }
      npg += ((t1 - 1) >> a.lgP) - (t0 >> a.lgP) + 1;
      ++nseg;
      g = st + lbe;
    }
  }

  // q^T operands: segment 0's into registers; segments 1 .. kQSlots-1 into
  // this wave's LDS slots.  They are requested before the page list, so
  // their latency overlaps the block-table reads the first K/V loads wait on.
  // Lane (head r16, kb) holds q[h0 + r16][dbase(j, kb) .. +8] for step j.
  u32x4 qv[KSTEPS];
  u32x4 qx[kQSlots > 1 ? kQSlots - 1 : 1][KSTEPS];
  load_q<AT, D, KVF, VW>(a, vr, seg_at(sd, 0).b, h0, hcount, r16, kb, qv);
#pragma unroll
  for (int s = 1; s < kQSlots; ++s)
    load_q<AT, D, KVF, VW>(a, vr, seg_at(sd, s < nseg ? s : 0).b, h0, hcount, r16, kb, qx[s - 1]);

  __shared__ int spage[PT ? 1 : kMaxSplitPages];
  SplitCtx c;
  c.spage = spage;
  c.my_page = -1;
  c.lgP = a.lgP;
  c.Pm = (1 << a.lgP) - 1;
  c.Hkv = a.Hkv;
  c.hkv = hkv;
  // the host keeps a pair within 64 (PT) / kMaxSplitPages page-list entries
  if constexpr (PT) {
    if (lane < npg) c.my_page = page_entry(a, lane, nseg, sd);
  } else {
    for (int i = threadIdx.x; i < npg; i += blockDim.x) spage[i] = page_entry(a, i, nseg, sd);
  }

#pragma unroll
  for (int s = 1; s < kQSlots; ++s)
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) qslots[((s - 1) * KSTEPS + j) * 64 + lane] = qx[s - 1][j];
  LaneOffsets<KVF, D, SB> lo;
  if constexpr (PT) lo = pt_lane_offsets<KVF, D, SB>(a, r16, kb);

  if constexpr (!PT) __syncthreads();

  float m_run = -INFINITY;  // per head r16 (replicated over kb)
  float l_run = 0.0f;
  f32x4 o[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto consume = [&](const Blk& blk) {
    consume_block<AT, D, KVF, SB, VW>(blk, qv, a.scale_log2, kb, a, vr, m_run, l_run, o);
  };

  // Blocks 2k and 2k+1 of the pair stream through buffers A and B.  Each
  // buffer has one load site, so its registers are the same on every trip; B
  // starts empty (mask 0: consuming it changes nothing) and a block index past
  // the end reloads the last block, masked off.  Loads run one block ahead of
  // the consumes and cross segment boundaries: the load side (c, segL) and the
  // consume side (segC) each step to the next segment when they reach it.
  const int nbt = (int)(g1 - g0);
  Blk A, Bq;
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < F::NRUN; ++r) Bq.k[u][r] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
  for (int q = 0; q < 8; ++q) Bq.v[q] = (u32x4){0u, 0u, 0u, 0u};
  if constexpr (KVF != 0) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int e = 0; e < Blk::NKS; ++e) Bq.ks[u][e] = 0u;
#pragma unroll
    for (int q = 0; q < 8; ++q) Bq.vs[q] = 0u;
  }
  Bq.mask = 0u;
  Bq.rel_end = 1 << 30;

  int segL = 0, jL0 = 0, jL1 = 0;  // load side: segment, its first and end pair-local block
  auto seg_len = [&](int sgi) {
    if constexpr (VW) c.seq_len = __builtin_amdgcn_readfirstlane(slen[sgi]);
  };
  set_segment(c, seg_at(sd, 0));
  seg_len(0);
  jL1 = nblk_of(c.t_end - c.t_begin);
  int segC = 0, jC1 = jL1;         // consume side: segment and its end block

  for (int i = 0; i < nbt; i += 2) {
    if (i >= jL1) {  // wave-uniform
      ++segL;
      jL0 = jL1;
      set_segment(c, seg_at(sd, segL));
      seg_len(segL);
      jL1 = jL0 + nblk_of(c.t_end - c.t_begin);
    }
    load_block<AT, D, KVF, SB, PT>(A, a, c, lo, c.t_begin + kBlockPos * (i - jL0), r16, kb);
    __builtin_amdgcn_sched_barrier(0);
    consume(Bq);  // block i-1 (empty on the first trip)
    const bool has1 = i + 1 < nbt;
    if (has1 && i + 1 >= jL1) {  // wave-uniform
      ++segL;
      jL0 = jL1;
      set_segment(c, seg_at(sd, segL));
      seg_len(segL);
      jL1 = jL0 + nblk_of(c.t_end - c.t_begin);
    }
    load_block<AT, D, KVF, SB, PT>(Bq, a, c, lo, c.t_begin + kBlockPos * ((has1 ? i + 1 : i) - jL0), r16, kb);
    if (!has1) Bq.mask = 0u;
    __builtin_amdgcn_sched_barrier(0);
    if (i >= jC1) {  // wave-uniform: block i opens the next segment
      write_segment<AT, D, KVF, VW>(a, vr, o, m_run, l_run, seg_at(sd, segC), pair, h0, hcount);
      ++segC;
      {
        const SegDesc d = seg_at(sd, segC);
        jC1 += nblk_of(d.t1 - d.t0);
      }
      begin_segment<AT, D, KVF, VW>(a, vr, qv, qslots, segC, sd, h0, hcount, lane, r16, kb);
      m_run = -INFINITY;
      l_run = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    consume(A);
    if (has1 && i + 1 >= jC1) {  // wave-uniform: block i + 1 (consumed next trip) opens the next segment
      write_segment<AT, D, KVF, VW>(a, vr, o, m_run, l_run, seg_at(sd, segC), pair, h0, hcount);
      ++segC;
      {
        const SegDesc d = seg_at(sd, segC);
        jC1 += nblk_of(d.t1 - d.t0);
      }
      begin_segment<AT, D, KVF, VW>(a, vr, qv, qslots, segC, sd, h0, hcount, lane, r16, kb);
      m_run = -INFINITY;
      l_run = 0.0f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
  }
  consume(Bq);  // the last odd block (or an empty one)
  write_segment<AT, D, KVF, VW>(a, vr, o, m_run, l_run, seg_at(sd, segC), pair, h0, hcount);
}

// ------------------------------------------------------- short-context plan
// A small total context (B x blocks per block-table row x units at most
// kSpMaxWaveBlocks, see sp_plan) runs on a grid laid out from the block-table width
// instead of the lengths.  Sequence b's 32-position blocks are cut into splits
// of sp_blk blocks, one wave per (split, unit), and sp_nw consecutive splits
// of one (sequence, unit) share a workgroup.  So nothing on the way to the
// first K/V load waits for the lengths: the length, q and the split's page
// ids are requested together.  The waves of a workgroup merge their (m, l, O)
// in LDS.  A sequence covered by one workgroup is written final; otherwise
// each workgroup stores one partial and counts itself in at the (sequence,
// unit) arrival counter, and the workgroup that arrives last merges the
// partials (LSE merge, ops/attention_ops.py:534-550), writes the output and
// sets the counter back to zero -- the call is one kernel, and its counters
// are zero again when it ends.  Workgroups past a sequence's last split exit
// at once (the first of them writes zeros for an empty sequence).
// Device-coherent (agent-scope) relaxed store of one float: it writes
// through the per-XCD L2, so a partial written on one XCD reaches memory
// without an L2 write-back.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ordering of the partials before the arrival count.  By default the
// count is a relaxed fetch_add after s_waitcnt vmcnt(0): under the HIP/C++
// memory model the partial stores and the last workgroup's reads then race,
// and the merge is correct only because of how this toolchain (ROCm 7.x
// clang) lowers agent-scope relaxed stores on gfx950: write-through to
// memory (sc1), complete once vmcnt reaches zero, so the last workgroup's
// acquire (L1/L2 invalidate) sees them.  A compiler or ISA that lowered them
// otherwise would break the merge silently and leave counters non-zero.
// Building with -DMK_SP_MERGE_RELEASE=1 (make MKDEFS=-DMK_SP_MERGE_RELEASE=1)
// makes the count a release fetch_add, which the memory model guarantees,
// at the cost of an L2 write-back per workgroup; run the split-plan parity
// tests under both builds when the toolchain changes.
#ifndef MK_SP_MERGE_RELEASE
#define MK_SP_MERGE_RELEASE 0
#endif

// Experiments: a fixed number of waves per workgroup (0: the plan's rule).
#ifndef MK_ATTN_SP_NW
#define MK_ATTN_SP_NW 0
#endif
#ifndef MK_ATTN_SP_MAXWB
#define MK_ATTN_SP_MAXWB 16384
#endif
#ifndef MK_ATTN_SP_WAVES
#define MK_ATTN_SP_WAVES 2048
#endif
constexpr int64_t kSpMaxWaveBlocks = MK_ATTN_SP_MAXWB;  // B x blocks x units on the short-context plan
// ... or up to twice that when no table row exceeds kSpShortRowBlocks blocks
// (4096 positions), so a sequence shorter than its row leaves few idle splits
// (measured: 32 sequences of 2112 positions 53.4 -> 49.4 us per call; config 3,
// rows of 256 blocks, stays on the stream plan)
constexpr int64_t kSpMaxWaveBlocksShort = 2 * kSpMaxWaveBlocks;
constexpr int64_t kSpShortRowBlocks = 128;
constexpr int64_t kSpWaves = MK_ATTN_SP_WAVES;          // waves it aims for (one round on 256 CUs)
constexpr int kSpMergeTrip = 16;                        // partials the final merge reads per trip

template <typename AT, int D, int KVF, bool SB, bool VW>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void paged_attn_sp_kernel(
    const PagedArgs a) {
  using F = Fmt<KVF, D>;
  using Blk = KVBlock<KVF, D, SB>;
  constexpr int KSTEPS = F::KSTEPS;
  constexpr int DPL = F::DPL;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = a.sp_nw;
  const int r16 = lane & 15;
  const int kb = lane >> 4;
  // workgroup -> (its index within the sequence, sequence, unit); neighbouring
  // workgroups take different units
  const int unit = (int)blockIdx.x % a.units;
  const int rest = (int)blockIdx.x / a.units;
  const int b = rest % a.B;
  const int wgi = rest / a.B;
  const int hkv = unit / a.HB;
  const int hb = unit - hkv * a.HB;
  const int h0 = hkv * a.G + hb * 16;
  const int hcount = min(16, a.G - hb * 16);
  const int max_s = a.MB << a.lgP;
  const int span = a.sp_blk * kBlockPos;     // positions per split
  const int t0 = (wgi * nw + wave) * span;  // this wave's first position
  const VRows vr = VW ? vrows(a, h0) : VRows{0, 0};

  // ---- requested together: the length, q and the split's page ids
  const int len = clamp_len(a.lengths[b], max_s);
  u32x4 qv[KSTEPS];
  load_q<AT, D, KVF, VW>(a, vr, b, h0, hcount, r16, kb, qv);
  const int pg0 = t0 >> a.lgP;
  int my_page = -1;
  {
    const int npg = ((t0 + span - 1) >> a.lgP) - pg0 + 1;  // <= 64 (host: span <= 63 P)
    if (lane < npg && pg0 + lane < a.MB) {
      const int p = a.bt[(size_t)b * a.MB + pg0 + lane];
      my_page = (p >= 0 && p < a.NP) ? p : -1;
    }
  }
  const int nsplit = (nblk_of(len) + a.sp_blk - 1) / a.sp_blk;  // splits holding positions
  const int nwg = (nsplit + nw - 1) / nw;                       // workgroups holding positions
  if (wgi >= nwg) {  // workgroup-uniform
    if (wgi == 0) {  // empty sequence
      for (int i = threadIdx.x; i < hcount * D; i += blockDim.x)
        reinterpret_cast<AT*>(a.out)[qo_row_j<VW>(a, vr, b, h0, i / D) * D + i % D] = from_f32<AT>(0.0f);
    }
    return;
  }
  const int t1 = min(t0 + span, len);
  const int nbt = t0 < t1 ? nblk_of(t1 - t0) : 0;  // wave-uniform

  SplitCtx c;
  c.spage = nullptr;
  c.my_page = my_page;
  c.blk0 = pg0;
  c.po = 0;
  c.t_begin = t0;
  c.t_end = t1;
  c.lgP = a.lgP;
  c.Pm = (1 << a.lgP) - 1;
  c.Hkv = a.Hkv;
  c.hkv = hkv;
  c.seq_len = len;
  const LaneOffsets<KVF, D, SB> lo = pt_lane_offsets<KVF, D, SB>(a, r16, kb);

  float m_run = -INFINITY;  // per head r16 (replicated over kb)
  float l_run = 0.0f;
  f32x4 o[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  auto consume = [&](const Blk& blk) {
    consume_block<AT, D, KVF, SB, VW>(blk, qv, a.scale_log2, kb, a, vr, m_run, l_run, o);
  };

  // Blocks stream through buffers A and B, each refilled right after it is
  // consumed; every load is issued on a path whose later waits are exact
  // (no load sits under a branch that rejoins before its data is used).
  if (nbt == 1) {  // wave-uniform
    Blk A;
    load_block<AT, D, KVF, SB, true>(A, a, c, lo, t0, r16, kb);
    consume(A);
  } else if (nbt > 1) {
    // as in paged_attn_kernel: B starts empty, and a block index past the
    // end reloads the last block, masked off
    Blk A, Bq;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < F::NRUN; ++r) Bq.k[u][r] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int q = 0; q < 8; ++q) Bq.v[q] = (u32x4){0u, 0u, 0u, 0u};
    if constexpr (KVF != 0) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < Blk::NKS; ++e) Bq.ks[u][e] = 0u;
#pragma unroll
      for (int q = 0; q < 8; ++q) Bq.vs[q] = 0u;
    }
    Bq.mask = 0u;
    Bq.rel_end = 1 << 30;
    for (int i = 0; i < nbt; i += 2) {
      load_block<AT, D, KVF, SB, true>(A, a, c, lo, t0 + kBlockPos * i, r16, kb);
      __builtin_amdgcn_sched_barrier(0);
      consume(Bq);
      const bool has1 = i + 1 < nbt;
      load_block<AT, D, KVF, SB, true>(Bq, a, c, lo, t0 + kBlockPos * (has1 ? i + 1 : i), r16, kb);
      if (!has1) Bq.mask = 0u;
      __builtin_amdgcn_sched_barrier(0);
      consume(A);
    }
    consume(Bq);
  }

  // ---- the workgroup's splits, merged in LDS: wave w's O row of head h at
  // so[(w * hcount + h) * D], its (m, l) at sm[(w * hcount + h) * 2]
  extern __shared__ __align__(16) uint8_t attn_dyn[];
  float* so = reinterpret_cast<float*>(attn_dyn);
  float* sm = so + (size_t)nw * hcount * D;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * kb + i;
    if (h >= hcount) continue;
    float nat[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) nat[F::vslot(j)] = o[j][i];
    float* dst = so + (size_t)(wave * hcount + h) * D + r16 * DPL;
#pragma unroll
    for (int e = 0; e < DPL / 4; ++e)
      reinterpret_cast<f32x4*>(dst)[e] = (f32x4){nat[4 * e], nat[4 * e + 1], nat[4 * e + 2], nat[4 * e + 3]};
  }
  if (kb == 0 && r16 < hcount)
    *reinterpret_cast<f32x2*>(sm + (size_t)(wave * hcount + r16) * 2) = (f32x2){m_run, l_run};
  __syncthreads();

  const bool single = nwg == 1;  // workgroup-uniform
  // partial (g) of head h0 + h: row ((b * Hq + h0 + h) * sp_nwg + g)
  const size_t prow = ((size_t)b * a.Hq + h0) * a.sp_nwg;
  AT* const outp = reinterpret_cast<AT*>(a.out);
  for (int it = threadIdx.x; it < hcount * D; it += blockDim.x) {
    const int h = it / D;
    const int d = it - h * D;
    float M = -INFINITY;
    for (int w = 0; w < nw; ++w) M = fmaxf(M, sm[(w * hcount + h) * 2]);
    const float Mu = M == -INFINITY ? 0.0f : M;
    float L = 0.0f, O = 0.0f;
    for (int w = 0; w < nw; ++w) {
      const float e = __builtin_amdgcn_exp2f(sm[(w * hcount + h) * 2] - Mu);
      L += sm[(w * hcount + h) * 2 + 1] * e;
      O += so[(size_t)(w * hcount + h) * D + d] * e;
    }
    if (single) {
      outp[qo_row_j<VW>(a, vr, b, h0, h) * D + d] = from_f32<AT>(O * (L > 0.0f ? 1.0f / L : 0.0f));
    } else {
      const size_t row = prow + (size_t)h * a.sp_nwg + wgi;
      store_agent(a.ws + row * D + d, O);
      if (d == 0) {
        store_agent(a.ws_ml + row * 2, M);
        store_agent(a.ws_ml + row * 2 + 1, L);
      }
    }
  }
  if (single) return;

  // ---- arrival.  The partials went out as device-coherent stores (they
  // write through this XCD's L2); once every thread has seen them complete,
  // one thread counts the workgroup in.  The last to arrive drops its
  // cached lines (acquire: L1/L2 invalidate), reads the partials, merges them
  // and clears the counter.  (A release fence would order the stores too,
  // but its L2 write-back costs each workgroup more than the whole merge.)
  __shared__ int is_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  lds_barrier();
  if (threadIdx.x == 0) {
    int* ctr = a.cnt + (size_t)b * a.units + unit;
    const int prev = __hip_atomic_fetch_add(ctr, 1, MK_SP_MERGE_RELEASE ? __ATOMIC_RELEASE : __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == nwg - 1;
    if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = last;
  }
  lds_barrier();
  if (!is_last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // tp consecutive threads share an output chunk (4 floats of one head),
  // each taking every tp-th partial, 16 per trip, all requested before any is
  // used; a trip that raises a thread's max rescales its running (M, L, O),
  // and the tp running states are combined by lane shuffles at the end
  constexpr int DV = D / 4;  // 4-float chunks per head row
  constexpr int CH = kSpMergeTrip;
  const int items = hcount * DV;
  int tp = 1;
  while (tp < 8 && items * tp * 2 <= (int)blockDim.x && nwg > CH * tp) tp *= 2;
  const int sub = (int)threadIdx.x & (tp - 1);
  for (int it = (int)threadIdx.x / tp; it < items; it += (int)blockDim.x / tp) {
    const int h = it / DV;
    const int dv = it - h * DV;
    const size_t row0 = prow + (size_t)h * a.sp_nwg;
    const f32x2* ml = reinterpret_cast<const f32x2*>(a.ws_ml) + row0;
    const f32x4* po = reinterpret_cast<const f32x4*>(a.ws + row0 * D) + dv;  // partial g at po[g * DV]
    float M = -INFINITY, L = 0.0f;
    float O[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g0 = sub; g0 < nwg; g0 += CH * tp) {
      f32x2 v[CH];
      f32x4 x[CH];
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const int gk = g0 + k * tp;
        const int g = gk < nwg ? gk : nwg - 1;  // past the end: re-read, weight 0
        v[k] = ml[g];
        x[k] = po[(size_t)g * DV];
      }
      float Mc = M;
#pragma unroll
      for (int k = 0; k < CH; ++k) Mc = fmaxf(Mc, g0 + k * tp < nwg ? v[k][0] : -INFINITY);
      const float Mu = Mc == -INFINITY ? 0.0f : Mc;
      const float r = __builtin_amdgcn_exp2f(M - Mu);  // 0 while M is -inf
      L *= r;
#pragma unroll
      for (int e = 0; e < 4; ++e) O[e] *= r;
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        const float w = g0 + k * tp < nwg ? __builtin_amdgcn_exp2f(v[k][0] - Mu) : 0.0f;
        L += v[k][1] * w;
#pragma unroll
        for (int e = 0; e < 4; ++e) O[e] += x[k][e] * w;
      }
      M = Mc;
    }
    for (int off = tp >> 1; off > 0; off >>= 1) {  // tp is uniform
      const float Mo = __shfl_xor(M, off, 64);
      const float Lo = __shfl_xor(L, off, 64);
      float Oo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) Oo[e] = __shfl_xor(O[e], off, 64);
      const float Mn = fmaxf(M, Mo);
      const float Mu = Mn == -INFINITY ? 0.0f : Mn;
      const float r0 = __builtin_amdgcn_exp2f(M - Mu), r1 = __builtin_amdgcn_exp2f(Mo - Mu);
      L = L * r0 + Lo * r1;
#pragma unroll
      for (int e = 0; e < 4; ++e) O[e] = O[e] * r0 + Oo[e] * r1;
      M = Mn;
    }
    if (sub == 0) {
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      *reinterpret_cast<u32x2*>(outp + qo_row_j<VW>(a, vr, b, h0, h) * D + 4 * dv) =
          (u32x2){pack_act2<AT>(O[0] * inv, O[1] * inv), pack_act2<AT>(O[2] * inv, O[3] * inv)};
    }
  }
}

// --------------------------------------------------------------- generic path
// Any D / group / dtype: one wave per (sequence, query head), lanes over d,
// fp32 online softmax over positions.
template <typename AT, int KVF>
__global__ __launch_bounds__(64) void paged_attn_generic_kernel(const PagedArgs a, int D) {
  const int bh = blockIdx.x;
  const int b = bh / a.Hq;
  const int h = bh - b * a.Hq;
  const int hkv = h / a.G;
  int len = a.lengths[b];
  const int max_s = a.MB * a.P;
  len = len < 0 ? 0 : (len > max_s ? max_s : len);
  len -= causal_offset(a, h);  // a verify row's causal limit
  const size_t qrow = qo_row(a, b, h);
  const AT* qp = reinterpret_cast<const AT*>(a.q) + qrow * D;
  constexpr int MAXPL = 4;  // D <= 256
  float qr[MAXPL], acc[MAXPL];
#pragma unroll
  for (int k = 0; k < MAXPL; ++k) {
    const int d = threadIdx.x + 64 * k;
    qr[k] = d < D ? to_f32(qp[d]) : 0.0f;
    acc[k] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  const float scale = a.scale_log2;
  for (int t = 0; t < len; ++t) {
    const int page = a.bt[(size_t)b * a.MB + t / a.P];
    if (page < 0 || page >= a.NP) continue;
    const size_t row = ((size_t)page * a.P + t % a.P) * a.Hkv + hkv;
    float kk[MAXPL], vv[MAXPL];
#pragma unroll
    for (int k = 0; k < MAXPL; ++k) {
      const int d = threadIdx.x + 64 * k;
      kk[k] = vv[k] = 0.0f;
      if (d >= D) continue;
      if constexpr (KVF == 0) {
        kk[k] = to_f32(reinterpret_cast<const AT*>(a.K)[row * D + d]);
        vv[k] = to_f32(reinterpret_cast<const AT*>(a.V)[row * D + d]);
      } else {
        const float ks = (float)bitcast<f16>(a.Ks[row * a.ngroups + d / a.gs]);
        const float vs = (float)bitcast<f16>(a.Vs[row * a.ngroups + d / a.gs]);
        uint32_t kc, vc;
        float off;
        if constexpr (KVF == 8) {
          kc = reinterpret_cast<const uint8_t*>(a.K)[row * D + d];
          vc = reinterpret_cast<const uint8_t*>(a.V)[row * D + d];
          off = 128.0f;
        } else {
          const size_t dp = (D + 1) / 2;
          const uint8_t kb8 = reinterpret_cast<const uint8_t*>(a.K)[row * dp + d / 2];
          const uint8_t vb8 = reinterpret_cast<const uint8_t*>(a.V)[row * dp + d / 2];
          kc = (d & 1) ? (kb8 >> 4) : (kb8 & 15u);
          vc = (d & 1) ? (vb8 >> 4) : (vb8 & 15u);
          off = 8.0f;
        }
        kk[k] = (float)(f16)(((float)kc - off) * ks);
        vv[k] = (float)(f16)(((float)vc - off) * vs);
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXPL; ++k) dot += qr[k] * kk[k];
    dot = wave_sum(dot) * scale;
    const float m_new = fmaxf(m, dot);
    const float alpha = (m == -INFINITY) ? 0.0f : exp2f(m - m_new);
    const float p = exp2f(dot - m_new);
    l = l * alpha + p;
    m = m_new;
#pragma unroll
    for (int k = 0; k < MAXPL; ++k) acc[k] = acc[k] * alpha + p * vv[k];
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  AT* op = reinterpret_cast<AT*>(a.out) + qrow * D;
#pragma unroll
  for (int k = 0; k < MAXPL; ++k) {
    const int d = threadIdx.x + 64 * k;
    if (d < D) op[d] = from_f32<AT>(acc[k] * inv);
  }
}

// --------------------------------------------------------------- host side
inline int ilog2(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}
inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// Streaming multiprocessors (CUs) of the current device, cached per device.
inline int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

inline bool fast_ok(int64_t D, int kvf, int dtype, int64_t gs, int64_t P, int64_t NP, int64_t Hkv) {
  if (!(D == 64 || D == 128)) return false;
  if (!is_pow2(P) || (kMaxSplitPages - 1) * P < kBlockPos) return false;
  if (NP * P * Hkv >= (int64_t(1) << 31)) return false;  // 32-bit row index
  if (kvf != 0) {
    if (dtype != MK_DT_F16) return false;
    // one scale per 8-d chunk: the group must be a power of two >= 8
    if (gs < 8 || !is_pow2(gs)) return false;
  }
  return true;
}

// Host half of the stream plan: workgroup shape, pairs per round (one per
// resident wave slot: two waves per SIMD, four SIMDs per CU), the most
// blocks one pair may hold, and the pair count bound.
inline void split_plan(PagedArgs& a, int kvf) {
  a.units = a.Hkv * a.HB;
  const int64_t cus = device_cus();
  int64_t T = cus * 8 / a.units;
  if (T < 1) T = 1;
  a.T_pairs = (int)T;
  // Segments start at 32-position block boundaries, so a pair of n blocks
  // touches at most 2n pages for P >= 16 (32/P pages per block below): its
  // page list must fit 64 lanes (P % 16 == 0) or the LDS table, and its
  // segments the 64 lanes that describe them.
  int64_t cap;
  if (a.P % 16 == 0) cap = 32;
  else cap = (int64_t)kMaxSplitPages * a.P / kBlockPos;
  if (cap > 64) cap = 64;
  if (cap < 1) cap = 1;
  a.cap_blk = (int)cap;
  const int64_t blk_per_seq = ((int64_t)a.MB * a.P + kBlockPos - 1) / kBlockPos;
  const int64_t by_cap = ((int64_t)a.B * blk_per_seq + cap - 1) / cap;
  a.max_pairs = (int)(T > by_cap ? T : by_cap);
  // The units of a pair share a workgroup (up to 8 waves, one CU) when the
  // block table allows enough pairs for a workgroup per CU; with fewer pairs
  // (short total context) one-wave workgroups spread them over all CUs.
  a.min_split = kvf == 8 ? kMinSplitBlocksQ8 : kMinSplitBlocks16;
  const int64_t minb = a.min_split < cap ? a.min_split : cap;
  int64_t pairs = (a.B * blk_per_seq + minb - 1) / minb;
  if (pairs > T) pairs = T;
  int wg = 1;
  for (int d = 8; d >= 1; --d)
    if (a.units % d == 0) {
      wg = d;
      break;
    }
  a.wg_units = pairs * (a.units / wg) >= cus ? wg : 1;
}

// Short-context plan (paged_attn_sp_kernel), taken when the block-table
// width keeps B x blocks x units within kSpMaxWaveBlocks (twice that for rows
// of at most kSpShortRowBlocks blocks) and pages hold a multiple of 16
// positions: blocks per split sized for about kSpWaves
// waves, then the widest workgroup (8, 4 or 2 splits) that still gives every
// CU a workgroup, no wider than the splits of a sequence, and with its LDS
// merge buffer within 64 KiB.
inline size_t sp_lds_bytes(const PagedArgs& a, int nw, int64_t D) {
  return (size_t)nw * (a.G < 16 ? a.G : 16) * (D + 2) * sizeof(float);
}
inline void sp_plan(PagedArgs& a, int64_t D) {
  a.sp_nw = 0;
  if (a.P % 16 != 0) return;
  const int64_t blk = ((int64_t)a.MB * a.P + kBlockPos - 1) / kBlockPos;
  const int64_t wb = (int64_t)a.B * blk * a.units;
  if (wb > kSpMaxWaveBlocks && !(wb <= kSpMaxWaveBlocksShort && blk <= kSpShortRowBlocks)) return;
  const int64_t c = (wb + kSpWaves - 1) / kSpWaves;
  if (c * kBlockPos / a.P + 1 > 64) return;  // a split's page ids must fit the 64 lanes
  const int64_t S = (blk + c - 1) / c;       // splits per sequence
  // the narrowest workgroup (most workgroups, spread over the most CUs)
  // whose sequence still leaves at most kSpMergeTrip partials, which the
  // last workgroup reads in one trip
  int nw = 2;
  while (nw < 8 && (S + nw - 1) / nw > kSpMergeTrip) nw *= 2;
  if (MK_ATTN_SP_NW) nw = MK_ATTN_SP_NW;
  while (nw > 1 && nw / 2 >= S) nw /= 2;
  while (nw > 1 && sp_lds_bytes(a, nw, D) > 65536) nw /= 2;
  a.sp_blk = (int)c;
  a.sp_nw = nw;
  a.sp_nwg = (int)((S + nw - 1) / nw);
}

// Partial slots of the stream plan: pair + sequence < max_pairs + B.
inline int64_t workspace_slots(const PagedArgs& a) { return (int64_t)a.max_pairs + a.B; }

// Workspace: [arrival counters, kCounterBytes][O partials fp32][(m, l) fp32].
// The counters sit at the same place for every shape (the short-context
// plan has at most kSpMaxWaveBlocksShort of them); the partials are
// slots * Hq * (D + 2) floats for the stream plan and B * Hq * sp_nwg * (D + 2)
// for the short-context plan.
constexpr size_t kCounterBytes = (size_t)kSpMaxWaveBlocksShort * sizeof(int);
inline size_t workspace_need(const PagedArgs& a, int64_t D) {
  const int64_t stream_rows = workspace_slots(a) * a.Hq;
  const int64_t sp_rows = a.sp_nw ? (int64_t)a.B * a.Hq * a.sp_nwg : 0;
  const int64_t rows = stream_rows > sp_rows ? stream_rows : sp_rows;
  return kCounterBytes + (size_t)rows * (D + 2) * sizeof(float);
}

int attention_launch(PagedArgs a, int64_t D, int kvf, int dtype, size_t ws_bytes,
                     hipStream_t st) {
  const bool fast = fast_ok(D, kvf, dtype, a.gs, a.P, a.NP, a.Hkv);
  if (fast) {
    a.lgP = ilog2(a.P);
    a.lg_gs = kvf ? ilog2(a.gs) : 0;
    split_plan(a, kvf);
    sp_plan(a, D);
    const size_t need = workspace_need(a, D);
    if (!a.ws || ws_bytes < need || !mk_aligned(a.ws, 16)) return MK_ERR_INVALID;
    a.cnt = reinterpret_cast<int*>(a.ws);
    a.ws = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(a.ws) + kCounterBytes);
    if (a.sp_nw) {
      a.ws_ml = a.ws + (size_t)a.B * a.Hq * a.sp_nwg * D;
      const dim3 grid((unsigned)((int64_t)a.sp_nwg * a.B * a.units));
      const dim3 block(64u * (unsigned)a.sp_nw);
      const size_t lds = sp_lds_bytes(a, a.sp_nw, D);
#define MK_SP(AT, DD, KF, SB)                                                        \
  do {                                                                               \
    if (a.vw > 1) paged_attn_sp_kernel<AT, DD, KF, SB, true><<<grid, block, lds, st>>>(a);   \
    else paged_attn_sp_kernel<AT, DD, KF, SB, false><<<grid, block, lds, st>>>(a);           \
  } while (0)
      if (kvf == 0) {
        if (dtype == MK_DT_F16) {
          if (D == 128) MK_SP(f16, 128, 0, false); else MK_SP(f16, 64, 0, false);
        } else {
          if (D == 128) MK_SP(bf16, 128, 0, false); else MK_SP(bf16, 64, 0, false);
        }
      } else if (kvf == 8) {
        if (D == 128) {
          if (a.gs >= 16) MK_SP(f16, 128, 8, true); else MK_SP(f16, 128, 8, false);
        } else {
          if (a.gs >= 16) MK_SP(f16, 64, 8, true); else MK_SP(f16, 64, 8, false);
        }
      } else {
        if (D == 128) {
          if (a.gs >= 32) MK_SP(f16, 128, 4, true); else MK_SP(f16, 128, 4, false);
        } else {
          if (a.gs >= 16) MK_SP(f16, 64, 4, true); else MK_SP(f16, 64, 4, false);
        }
      }
#undef MK_SP
      MK_CHECK_LAUNCH();
      return MK_OK;
    }
    a.ws_ml = a.ws + (size_t)workspace_slots(a) * a.Hq * D;
    const dim3 grid((unsigned)((int64_t)a.max_pairs * (a.units / a.wg_units)));
    const dim3 block(64u * (unsigned)a.wg_units);
    const size_t qlds = (size_t)a.wg_units * (D == 128 ? attn_wave_lds<128>() : attn_wave_lds<64>());
#define MK_PA2(AT, DD, KF, SB)                                                               \
  do {                                                                                      \
    if (a.vw > 1) {                                                                         \
      if (a.P % 16 == 0) paged_attn_kernel<AT, DD, KF, SB, true, true><<<grid, block, qlds, st>>>(a); \
      else paged_attn_kernel<AT, DD, KF, SB, false, true><<<grid, block, qlds, st>>>(a);            \
    } else {                                                                                \
      if (a.P % 16 == 0) paged_attn_kernel<AT, DD, KF, SB, true, false><<<grid, block, qlds, st>>>(a); \
      else paged_attn_kernel<AT, DD, KF, SB, false, false><<<grid, block, qlds, st>>>(a);            \
    }                                                                                       \
  } while (0)
#define MK_PA(AT, DD, KF, SB) MK_PA2(AT, DD, KF, SB)
    if (kvf == 0) {
      if (dtype == MK_DT_F16) {
        if (D == 128) MK_PA(f16, 128, 0, false); else MK_PA(f16, 64, 0, false);
      } else {
        if (D == 128) MK_PA(bf16, 128, 0, false); else MK_PA(bf16, 64, 0, false);
      }
    } else if (kvf == 8) {
      // SB: one K scale per 16-code run (group >= 16)
      if (D == 128) {
        if (a.gs >= 16) MK_PA(f16, 128, 8, true); else MK_PA(f16, 128, 8, false);
      } else {
        if (a.gs >= 16) MK_PA(f16, 64, 8, true); else MK_PA(f16, 64, 8, false);
      }
    } else {
      // SB: one K scale per 32-code (D=128) / 16-code (D=64) run
      if (D == 128) {
        if (a.gs >= 32) MK_PA(f16, 128, 4, true); else MK_PA(f16, 128, 4, false);
      } else {
        if (a.gs >= 16) MK_PA(f16, 64, 4, true); else MK_PA(f16, 64, 4, false);
      }
    }
#undef MK_PA
#undef MK_PA2
    MK_CHECK_LAUNCH();
    const dim3 mgrid((unsigned)((int64_t)a.B * a.Hq));
    if (dtype == MK_DT_F16) {
      if (D == 128) paged_attn_merge_kernel<f16, 128><<<mgrid, 64, 0, st>>>(a);
      else paged_attn_merge_kernel<f16, 64><<<mgrid, 64, 0, st>>>(a);
    } else {
      if (D == 128) paged_attn_merge_kernel<bf16, 128><<<mgrid, 64, 0, st>>>(a);
      else paged_attn_merge_kernel<bf16, 64><<<mgrid, 64, 0, st>>>(a);
    }
    MK_CHECK_LAUNCH();
    return MK_OK;
  }
  if (D > 256) return MK_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)(a.B * a.Hq));
#define MK_PG(AT, KF) paged_attn_generic_kernel<AT, KF><<<grid, 64, 0, st>>>(a, (int)D)
  if (kvf == 0) {
    if (dtype == MK_DT_F16) MK_PG(f16, 0); else MK_PG(bf16, 0);
  } else if (kvf == 8) {
    if (dtype == MK_DT_F16) MK_PG(f16, 8); else MK_PG(bf16, 8);
  } else {
    if (dtype == MK_DT_F16) MK_PG(f16, 4); else MK_PG(bf16, 4);
  }
#undef MK_PG
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// Argument checks and PagedArgs set-up shared by the fp16/bf16 entry points.
int fp16_args(PagedArgs& a, const void* q, const void* K_pages, const void* V_pages,
              const int32_t* block_table, const int32_t* lengths, void* out, int64_t B,
              int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size, int64_t max_blocks,
              int64_t num_pages, float scale, int dtype) {
  MK_REQUIRE(q && K_pages && V_pages && block_table && lengths && out);
  MK_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && (Hq % Hkv) == 0 && D > 0 && page_size > 0);
  MK_REQUIRE(max_blocks > 0 && num_pages > 0 && num_pages < (1LL << 31));
  MK_REQUIRE(B < 65536 && max_blocks * page_size < (1LL << 31));
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  a.q = q;
  a.K = K_pages;
  a.V = V_pages;
  a.bt = block_table;
  a.lengths = lengths;
  a.out = out;
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.HB = (a.G + 15) / 16;
  a.NP = (int)num_pages;
  a.P = (int)page_size;
  a.MB = (int)max_blocks;
  a.gs = 1;
  a.ngroups = 1;
  a.scale_log2 = scale * kLog2e;
  a.vw = 1;
  return MK_OK;
}

// Argument checks and PagedArgs set-up shared by the q8/q4 entry points.
int quant_args(PagedArgs& a, const void* q, const uint8_t* K_q, const uint8_t* V_q, const f16_storage_t* K_s,
               const f16_storage_t* V_s, const int32_t* block_table, const int32_t* lengths, void* out,
               int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size, int64_t max_blocks,
               int64_t num_pages, int64_t group_size, int bits, float scale, int dtype) {
  MK_REQUIRE(q && K_q && V_q && K_s && V_s && block_table && lengths && out);
  MK_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && (Hq % Hkv) == 0 && D > 0 && page_size > 0);
  MK_REQUIRE(max_blocks > 0 && num_pages > 0 && num_pages < (1LL << 31) && group_size > 0);
  MK_REQUIRE(B < 65536 && max_blocks * page_size < (1LL << 31));
  MK_REQUIRE(bits == 4 || bits == 8);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  a.q = q;
  a.K = K_q;
  a.V = V_q;
  a.Ks = K_s;
  a.Vs = V_s;
  a.bt = block_table;
  a.lengths = lengths;
  a.out = out;
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.HB = (a.G + 15) / 16;
  a.NP = (int)num_pages;
  a.P = (int)page_size;
  a.MB = (int)max_blocks;
  a.gs = (int)group_size;
  a.ngroups = (int)((D + group_size - 1) / group_size);
  a.scale_log2 = scale * kLog2e;
  a.vw = 1;
  return MK_OK;
}

// ------------------------------------------------- no-allocation scratch
// mk_paged_decode_attention_noalloc keeps its split partials in this
// file-scope array instead of a caller workspace.  Each device that runs the
// library holds its own copy for the life of the process.  In host code the
// array's name is only a host-side handle: the device address of a device's
// copy comes from hipGetSymbolAddress with that device current, cached per
// device below, and only that address is ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch (looked up once per device).
int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -(int)e - 1000;
  if (dev < 0 || dev >= kMaxDevices) return MK_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return -(int)e - 1000;
    if (!p || !mk_aligned(p, 256)) return MK_ERR_UNSUPPORTED;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MK_OK;
}

}  // namespace

extern "C" {

size_t mk_paged_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                          int64_t max_blocks, int64_t page_size) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_blocks <= 0 || page_size <= 0) return 0;
  if (max_blocks * page_size >= (int64_t(1) << 31) || B >= 65536 || Hq >= (int64_t(1) << 24))
    return 0;
  PagedArgs a = {};
  a.B = (int)B;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.HB = (a.G + 15) / 16;
  a.P = (int)page_size;
  a.MB = (int)max_blocks;
  split_plan(a, 0);  // the workspace does not depend on the format
  sp_plan(a, D);
  return workspace_need(a, D);
}

int mk_paged_decode_attention(const void* q, const void* K_pages, const void* V_pages,
                              const int32_t* block_table, const int32_t* lengths, void* out,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                              int64_t max_blocks, int64_t num_pages, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  PagedArgs a = {};
  const int rc = fp16_args(a, q, K_pages, V_pages, block_table, lengths, out, B, Hq, Hkv, D,
                           page_size, max_blocks, num_pages, scale, dtype);
  if (rc != MK_OK || B == 0) return rc;
  a.ws = reinterpret_cast<float*>(workspace);
  return attention_launch(a, D, 0, dtype, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int mk_paged_decode_attention_noalloc(const void* q, const void* K_pages, const void* V_pages,
                                      const int32_t* block_table, const int32_t* lengths,
                                      void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                      float scale, int dtype, void* stream) {
  PagedArgs a = {};
  const int rc = fp16_args(a, q, K_pages, V_pages, block_table, lengths, out, B, Hq, Hkv, D,
                           page_size, max_blocks, num_pages, scale, dtype);
  if (rc != MK_OK || B == 0) return rc;
  // The split plan is a pure function of the shape and the device's CU
  // count; reject a call whose partials would not fit before touching the GPU.
  if (fast_ok(D, 0, dtype, a.gs, a.P, a.NP, a.Hkv)) {
    PagedArgs plan = a;
    split_plan(plan, 0);
    sp_plan(plan, D);
    if (workspace_need(plan, D) > kNoAllocScratchBytes) return MK_ERR_SCRATCH;
  }
  void* ws = nullptr;
  const int src = noalloc_scratch(&ws);
  if (src != MK_OK) return src;
  a.ws = reinterpret_cast<float*>(ws);
  return attention_launch(a, D, 0, dtype, kNoAllocScratchBytes,
                          reinterpret_cast<hipStream_t>(stream));
}

int mk_paged_quantized_decode_attention(const void* q, const uint8_t* K_q, const uint8_t* V_q,
                                        const f16_storage_t* K_s, const f16_storage_t* V_s,
                                        const int32_t* block_table, const int32_t* lengths,
                                        void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                        int64_t group_size, int bits, float scale, int dtype,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  PagedArgs a = {};
  const int rc = quant_args(a, q, K_q, V_q, K_s, V_s, block_table, lengths, out, B, Hq, Hkv, D, page_size,
                            max_blocks, num_pages, group_size, bits, scale, dtype);
  if (rc != MK_OK || B == 0) return rc;
  a.ws = reinterpret_cast<float*>(workspace);
  return attention_launch(a, D, bits, dtype, workspace_bytes,
                          reinterpret_cast<hipStream_t>(stream));
}

int mk_paged_verify_attention(const void* q, const void* K_pages, const void* V_pages,
                              const int32_t* block_table, const int32_t* lengths, void* out,
                              int64_t B, int64_t W, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                              int64_t max_blocks, int64_t num_pages, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  MK_REQUIRE(W >= 1 && W <= 64 && Hq > 0 && W * Hq < (int64_t(1) << 24) && B * W * Hq < (int64_t(1) << 31));
  PagedArgs a = {};
  const int rc = fp16_args(a, q, K_pages, V_pages, block_table, lengths, out, B, W * Hq, Hkv, D, page_size,
                           max_blocks, num_pages, scale, dtype);
  if (rc != MK_OK || B == 0) return rc;
  a.vw = (int)W;  // W * Hq virtual heads, see PagedArgs::vw
  a.vw_magic = (int)((65536 + W - 1) / W);
  a.ws = reinterpret_cast<float*>(workspace);
  return attention_launch(a, D, 0, dtype, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int mk_paged_quantized_verify_attention(const void* q, const uint8_t* K_q, const uint8_t* V_q,
                                        const f16_storage_t* K_s, const f16_storage_t* V_s,
                                        const int32_t* block_table, const int32_t* lengths, void* out,
                                        int64_t B, int64_t W, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                        int64_t group_size, int bits, float scale, int dtype,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  MK_REQUIRE(W >= 1 && W <= 64 && Hq > 0 && W * Hq < (int64_t(1) << 24) && B * W * Hq < (int64_t(1) << 31));
  PagedArgs a = {};
  const int rc = quant_args(a, q, K_q, V_q, K_s, V_s, block_table, lengths, out, B, W * Hq, Hkv, D, page_size,
                            max_blocks, num_pages, group_size, bits, scale, dtype);
  if (rc != MK_OK || B == 0) return rc;
  a.vw = (int)W;
  a.vw_magic = (int)((65536 + W - 1) / W);
  a.ws = reinterpret_cast<float*>(workspace);
  return attention_launch(a, D, bits, dtype, workspace_bytes,
                          reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
