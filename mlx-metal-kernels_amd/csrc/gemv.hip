// Groupwise-affine q4/q8 decode matvec family for gfx950.
//
// Semantics (ops/quant_ops.py:509-526, 574-588, 634-738):
//   y[m,n] = clip(sum_k x[m,k] * W[n,k], +-max(act)) rounded to the activation
//   type, W[n,k] = (q[n,k] - z[n,k/g]) * s[n,k/g].
// q4 codes are packed two per byte (low nibble = even k), so on little-endian
// hardware a 32-bit word holds 8 consecutive codes, nibble i at bits 4i.
//
// Decode batches of at most 4 rows (q8: 2) with fp16 activations and scales
// take the v_dot2 kernel below, 17-32 rows the two-column-tile kernel;
// the rest, bf16 and fp32 scales the MFMA path:
// Fast path (M <= 16 per launch, K % 64 == 0 for q4 / % 32 for q8, power-of-two
// group size >= 16 (q4) / >= 8 (q8)):
//   * one workgroup owns a 16-row output tile; its KW waves split K;
//   * lane (n = l%16, kb = l/16) streams 32 contiguous code bytes of row n per
//     chunk with two 128-bit loads, dequantizes them in registers and feeds
//     v_mfma_f32_16x16x32_{f16,bf16} with A = W tile (16 n x 32 k) and
//     B = x^T tile (32 k x 16 m); decode batches M < 16 pad B with zeros;
//   * the waves' partial 16x16 tiles are summed through LDS; the epilogue
//     saturates, and optionally fuses SwiGLU (gate/up) or a residual add.
// fp16 activations with fp16 scales use an exponent-magic dequant: a code c
// OR'ed into the mantissa of 1024.0h gives 1024+c exactly, so with zi the
// rounded zero point
//   w = fma((1024 + c) - (1024 + zi), s, -(z - zi) s)  (two packed-f16 ops
// per pair of weights; one rounding for integer zero points).
// The MFMA contraction is order-free in k, so the activation operand is built
// in the same permuted k order the magic unpack produces.
#include "common.h"
#include "norm_chunks.h"
#include "paged_common.h"

namespace {

constexpr int EPI_NONE = 0;
constexpr int EPI_RESIDUAL = 1;
constexpr int EPI_GATE_UP = 2;
constexpr int EPI_ROPE_KV = 3;  // qkv rows -> split + interleaved RoPE + paged K/V write

template <int BITS>
struct QFmt {
  static constexpr int KL = BITS == 4 ? 64 : 32;     // k per lane chunk (32 code bytes)
  static constexpr int KC = 4 * KL;                  // k per wave chunk
  static constexpr int STEPS = BITS == 4 ? 8 : 4;    // MFMA k32 steps per chunk
  static constexpr int ROW_BYTES_NUM = BITS;         // row bytes = K * BITS / 8
};

// --------------------------------------------------------------------------
// activation operand: 8 halves of x for one MFMA step, in the k order the
// weight unpack produces.
// --------------------------------------------------------------------------
template <int BITS, bool MAGIC>
__device__ __forceinline__ u32x4 xperm(u32x4 X) {
  if constexpr (!MAGIC) {
    return X;  // natural order
  } else if constexpr (BITS == 4) {
    // weight order [0,4,1,5,2,6,3,7]
    u32x4 r;
    r[0] = pack_lo16(X[0], X[2]);
    r[1] = pack_hi16(X[0], X[2]);
    r[2] = pack_lo16(X[1], X[3]);
    r[3] = pack_hi16(X[1], X[3]);
    return r;
  } else {
    // weight order [0,2,1,3,4,6,5,7]
    u32x4 r;
    r[0] = pack_lo16(X[0], X[1]);
    r[1] = pack_hi16(X[0], X[1]);
    r[2] = pack_lo16(X[2], X[3]);
    r[3] = pack_hi16(X[2], X[3]);
    return r;
  }
}

// Per-group dequant parameters.  The integer part zi of the zero point is
// subtracted exactly from the magic-biased codes: (1024 + c) - (1024 + zi)
// for codes at mantissa bits 0..3 (q8: 0..7) of 1024.0h, (64 + c) - (64 + zi)
// for q4 codes left in place at bits 4..7 under 64.0h (ulp 1/16) -- c - zi
// exactly in fp16 for |zi| < 1024 -- so w = fma(c - zi, s, corr) with
// corr = -(z - zi) s rounds once, to the fp16 of (c - z) s whenever z is an
// integer (the rounding of the reference's fp32 dequant, for any fp16 scale),
// and keeps a fractional z exact to ulp(corr).
struct GpMagic {
  f16x2 s;     // (s, s)
  f16x2 kz;    // (1024 + zi)
  f16x2 kz64;  // (64 + zi)
  f16x2 corr;  // -(z - zi) * s
};
struct GpExact {
  float s;
  float z;
};

__device__ __forceinline__ f16x2 h2(f16 v) { return (f16x2){v, v}; }

__device__ __forceinline__ GpMagic make_gp_magic(f16 s, f16 z) {
  GpMagic g;
  const float zf = (float)z;
  const float zi = rintf(zf);
  g.s = h2(s);
  g.kz = h2((f16)(1024.0f + zi));
  g.kz64 = h2((f16)(64.0f + zi));
  g.corr = h2((f16)(-(zf - zi) * (float)s));
  return g;
}

// q4 word (8 codes) -> 8 fp16 weights in order [0,4,1,5,2,6,3,7].
// `magic` = 0x64006400 (1024.0h pair) and `magic_hi` = 0x54005400 (64.0h
// pair) held in VGPRs so each unpack is one v_and_or_b32.
__device__ __forceinline__ u32x4 dq4_magic(uint32_t u, const GpMagic& g, uint32_t magic, uint32_t magic_hi) {
  const uint32_t v = u >> 8;
  f16x2 a = bitcast<f16x2>((u & 0x000F000Fu) | magic) - g.kz;       // c0 - zi, c4 - zi
  f16x2 b = bitcast<f16x2>((u & 0x00F000F0u) | magic_hi) - g.kz64;  // c1 - zi, c5 - zi
  f16x2 c = bitcast<f16x2>((v & 0x000F000Fu) | magic) - g.kz;       // c2, c6
  f16x2 d = bitcast<f16x2>((v & 0x00F000F0u) | magic_hi) - g.kz64;  // c3, c7
  a = __builtin_elementwise_fma(a, g.s, g.corr);
  b = __builtin_elementwise_fma(b, g.s, g.corr);
  c = __builtin_elementwise_fma(c, g.s, g.corr);
  d = __builtin_elementwise_fma(d, g.s, g.corr);
  u32x4 r;
  r[0] = bitcast<uint32_t>(a);
  r[1] = bitcast<uint32_t>(b);
  r[2] = bitcast<uint32_t>(c);
  r[3] = bitcast<uint32_t>(d);
  return r;
}

// byte-pair unpack of q8 codes with v_perm_b32: bytes (b0, 0x64, b2, 0x64)
// and (b1, 0x64, b3, 0x64) of {magic8 = 0x64646464, u} are 1024+b0 / 1024+b2
// and 1024+b1 / 1024+b3 as fp16 pairs.
__device__ __forceinline__ uint32_t q8_lo_pair(uint32_t u, uint32_t magic8) {
  return perm_b32(magic8, u, 0x04020400u);
}
__device__ __forceinline__ uint32_t q8_hi_pair(uint32_t u, uint32_t magic8) {
  return perm_b32(magic8, u, 0x04030401u);
}

// two q8 words (8 codes) -> 8 fp16 weights in order [0,2,1,3,4,6,5,7].
__device__ __forceinline__ u32x4 dq8_magic(uint32_t u0, uint32_t u1, const GpMagic& g,
                                           uint32_t magic8) {
  f16x2 a0 = bitcast<f16x2>(q8_lo_pair(u0, magic8)) - g.kz;
  f16x2 b0 = bitcast<f16x2>(q8_hi_pair(u0, magic8)) - g.kz;
  f16x2 a1 = bitcast<f16x2>(q8_lo_pair(u1, magic8)) - g.kz;
  f16x2 b1 = bitcast<f16x2>(q8_hi_pair(u1, magic8)) - g.kz;
  a0 = __builtin_elementwise_fma(a0, g.s, g.corr);
  b0 = __builtin_elementwise_fma(b0, g.s, g.corr);
  a1 = __builtin_elementwise_fma(a1, g.s, g.corr);
  b1 = __builtin_elementwise_fma(b1, g.s, g.corr);
  u32x4 r;
  r[0] = bitcast<uint32_t>(a0);
  r[1] = bitcast<uint32_t>(b0);
  r[2] = bitcast<uint32_t>(a1);
  r[3] = bitcast<uint32_t>(b1);
  return r;
}

// Exact path: w = AT((q - z) * s) computed in fp32, natural k order.
template <typename AT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  AT a = from_f32<AT>(lo), b = from_f32<AT>(hi);
  return (uint32_t)bitcast<uint16_t>(a) | ((uint32_t)bitcast<uint16_t>(b) << 16);
}

template <typename AT>
__device__ __forceinline__ u32x4 dq4_exact(uint32_t u, const GpExact& g) {
  float w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = ((float)((u >> (4 * e)) & 15u) - g.z) * g.s;
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = pack2<AT>(w[2 * p], w[2 * p + 1]);
  return r;
}

template <typename AT>
__device__ __forceinline__ u32x4 dq8_exact(uint32_t u0, uint32_t u1, const GpExact& g) {
  float w[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = ((float)((u0 >> (8 * e)) & 255u) - g.z) * g.s;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[4 + e] = ((float)((u1 >> (8 * e)) & 255u) - g.z) * g.s;
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = pack2<AT>(w[2 * p], w[2 * p + 1]);
  return r;
}

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

template <typename ST>
__device__ __forceinline__ float ld_scalar_f32(const ST* p) {
  return to_f32(*p);
}

// The decode token's cache write fused into the qkv projection's epilogue
// (EPI_ROPE_KV): the operands of qkv_rope_update_kernel.
struct RopeKV {
  const float* cos_t;   // [cos_rows, D/2]
  const float* sin_t;
  const int32_t* pos;   // [M]
  const int32_t* bt;    // [M, max_blocks]
  void* kp;             // [num_pages, P, Hkv, D] f16
  void* vp;
  void* q_out;          // [M, Hq, D] f16
  int Hq, Hkv, D, P, max_blocks, num_pages, cos_rows;
};

struct GemvArgs {
  const void* x;         // [M, K]
  const uint8_t* w[2];   // [N, row_bytes]
  const void* s[2];      // [N, G]
  const void* z[2];      // [N, G] or null
  const void* residual;  // [M, N] or null
  void* y0;              // EPI_NONE: y; EPI_RESIDUAL: y_mm (nullable); GATE_UP: gate (nullable)
  void* y1;              // EPI_RESIDUAL: out;  GATE_UP: up (nullable)
  void* y2;              // GATE_UP: mlp (nullable)
  int M, N, K;
  int row_bytes;
  int G;
  int lg;                // log2(group size)
  int kw;                // waves per row group (K split)
  int rg;                // dot kernel: row groups per workgroup
  // residual + RMSNorm prologue (NORM dot kernels, M = 1): the product is
  // taken against n = fp16(z * rsqrt(mean(z^2) + eps) * nw), z = fp16(x +
  // nres) (z = x when nres is null); workgroup 0 writes z and n when zout /
  // nout are given
  const void* nres;      // [K] or null
  const void* nw;        // [K] fp16
  void* zout;            // [K]
  void* nout;            // [K] or null
  float eps;
  RopeKV rk;             // EPI_ROPE_KV only
};

// --------------------------------------------------------------------------
// shared epilogue: value(s) of output row n for activation row m
// --------------------------------------------------------------------------
template <typename AT, int EPI>
__device__ __forceinline__ void store_out(const GemvArgs& args, size_t o, float v0, float v1) {
  if constexpr (EPI == EPI_NONE) {
    reinterpret_cast<AT*>(args.y0)[o] = saturate_cast<AT>(v0);
  } else if constexpr (EPI == EPI_RESIDUAL) {
    const AT d = saturate_cast<AT>(v0);
    if (args.y0) reinterpret_cast<AT*>(args.y0)[o] = d;
    const float r = to_f32(reinterpret_cast<const AT*>(args.residual)[o]);
    reinterpret_cast<AT*>(args.y1)[o] = from_f32<AT>(r + to_f32(d));
  } else {
    const AT g = saturate_cast<AT>(v0);
    const AT u = saturate_cast<AT>(v1);
    if (args.y0) reinterpret_cast<AT*>(args.y0)[o] = g;
    if (args.y1) reinterpret_cast<AT*>(args.y1)[o] = u;
    if (args.y2) {
      const float gf = to_f32(g);
      const float sil = gf / (1.0f + expf(-gf));
      reinterpret_cast<AT*>(args.y2)[o] = from_f32<AT>(sil * to_f32(u));
    }
  }
}

// EPI_ROPE_KV: the launch's rows' cache slots (page * P + offset, -1 when
// skipped), looked up once per workgroup before its reduction barrier, so the
// later-row-wins rule reads LDS in the epilogue (rows <= 32 per launch).
constexpr int kRopeRows = 32;
__device__ __forceinline__ void rope_fill_slots(const GemvArgs& a, int* slots) {
  const int t = threadIdx.x;
  if (t < a.M && t < kRopeRows) {
    const RopeKV& r = a.rk;
    int off;
    const int pg = slot_page(r.bt, r.pos, t, r.max_blocks, r.P, r.num_pages, &off);
    slots[t] = pg < 0 ? -1 : pg * r.P + off;
  }
}
// this row's slot, or -1 when skipped or taken by a later row of the launch
__device__ __forceinline__ int rope_slot(const GemvArgs& a, const int* slots, int m) {
  const int sl = slots[m];
  if (sl < 0) return -1;
  for (int b2 = m + 1; b2 < a.M; ++b2)
    if (slots[b2] == sl) return -1;
  return sl;
}

// EPI_ROPE_KV: qkv output n of row m, rounded as the projection stores it,
// then the arithmetic of qkv_rope_update_kernel -- q and k pairs (n, n ^ 1)
// rotated in fp32 and rounded, v copied; q to q_out, k and v to the token's
// cache slot unless its position is out of range or a later row takes the
// slot.  Called by every lane of the pair (the partner value comes by
// shuffle), whether or not (m, n) is in range.
__device__ __forceinline__ void rope_kv_store(const GemvArgs& a, const int* slots, int m, int n, float v) {
  const f16 hv = saturate_cast<f16>(v);
  const float xv = to_f32(hv);
  const float xo = __shfl_xor(xv, 1, 64);
  if (n >= a.N || m >= a.M) return;
  const RopeKV& r = a.rk;
  const int p = r.pos[m];
  if (p < 0 || p >= r.cos_rows) return;
  const int D = r.D, QD = r.Hq * D, KD = r.Hkv * D;
  const int d = n % D;
  f16 out = hv;
  f16* dst = reinterpret_cast<f16*>(r.vp);
  int h;
  if (n < QD + KD) {
    const bool even = (d & 1) == 0;
    const size_t ci = (size_t)p * (D / 2) + (d >> 1);
    float ye, yo;
    rope_pair(even ? xv : xo, even ? xo : xv, r.cos_t[ci], r.sin_t[ci], &ye, &yo);
    out = from_f32<f16>(even ? ye : yo);
    if (n < QD) {
      reinterpret_cast<f16*>(r.q_out)[(size_t)m * QD + n] = out;
      return;
    }
    dst = reinterpret_cast<f16*>(r.kp);
    h = (n - QD) / D;
  } else {
    h = (n - QD - KD) / D;
  }
  const int sl = rope_slot(a, slots, m);
  if (sl < 0) return;
  dst[(size_t)sl * KD + (size_t)h * D + d] = out;
}

// EPI_ROPE_KV with both values of an (even n, n + 1) pair in one lane (the
// MFMA kernels' output layout): the same arithmetic as rope_kv_store.  RES:
// slots[m] already holds the row's final slot (-1 when skipped or taken by a
// later row) and pos_l[m] its position, both in LDS.
template <bool RES = false>
__device__ __forceinline__ void rope_kv_pair(const GemvArgs& a, const int* slots, int m, int n, float v0,
                                             float v1, const int* pos_l = nullptr) {
  if (n >= a.N || m >= a.M) return;
  const RopeKV& r = a.rk;
  const int p = RES ? pos_l[m] : r.pos[m];
  if (p < 0 || p >= r.cos_rows) return;
  const int D = r.D, QD = r.Hq * D, KD = r.Hkv * D;
  const int d = n % D;
  const f16 h0 = saturate_cast<f16>(v0), h1 = saturate_cast<f16>(v1);
  f16 o0 = h0, o1 = h1;
  f16* dst = reinterpret_cast<f16*>(r.vp);
  int h;
  if (n < QD + KD) {
    const size_t ci = (size_t)p * (D / 2) + (d >> 1);
    float ye, yo;
    rope_pair(to_f32(h0), to_f32(h1), r.cos_t[ci], r.sin_t[ci], &ye, &yo);
    o0 = from_f32<f16>(ye);
    o1 = from_f32<f16>(yo);
    if (n < QD) {
      f16* q = reinterpret_cast<f16*>(r.q_out) + (size_t)m * QD + n;
      q[0] = o0;
      q[1] = o1;
      return;
    }
    dst = reinterpret_cast<f16*>(r.kp);
    h = (n - QD) / D;
  } else {
    h = (n - QD - KD) / D;
  }
  const int sl = RES ? slots[m] : rope_slot(a, slots, m);
  if (sl < 0) return;
  f16* o = dst + (size_t)sl * KD + (size_t)h * D + d;
  o[0] = o0;
  o[1] = o1;
}

// The rows' final slots (the later-row-wins rule applied) and positions into
// LDS: call after rope_fill_slots(a, raw) and a barrier; the values are
// visible after the next barrier.
__device__ __forceinline__ void rope_resolve_slots(const GemvArgs& a, const int* raw, int* res, int* pos_l) {
  const int t = threadIdx.x;
  if (t < a.M && t < kRopeRows) {
    int sl = raw[t];
    for (int b2 = t + 1; b2 < a.M; ++b2)
      if (raw[b2] == sl) sl = -1;
    res[t] = sl;
    pos_l[t] = a.rk.pos[t];
  }
}

// --------------------------------------------------------------------------
// fast MFMA kernel (any M <= 16)
// --------------------------------------------------------------------------
template <int BITS, typename ST, int NMAT, int GPC>
struct WFrag {
  u32x4 w[NMAT][2];
  ST s[NMAT][GPC];
  ST z[NMAT][GPC];
};

template <int BITS, typename AT, typename ST, bool MAGIC, int GPC, int NMAT, int EPI>
__global__ __launch_bounds__(512) void gemv_mfma_kernel(const GemvArgs args) {
  using F = QFmt<BITS>;
  constexpr int STEPS = F::STEPS;
  constexpr int SPG = STEPS / GPC;  // MFMA steps per quantization group

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kw = args.kw;
  const int M = args.M, N = args.N, K = args.K;

  const int n0 = blockIdx.x * 16;
  const int nl = lane & 15;
  const int kb = lane >> 4;
  const int n = n0 + nl;
  const int n_ld = n < N ? n : N - 1;  // rows past N load a valid row; results discarded
  const int m = lane & 15;
  const bool x_active = m < M;
  const uint32_t magic = in_vgpr(BITS == 4 ? 0x64006400u : 0x64646464u);
  const uint32_t magic_hi = in_vgpr(0x54005400u);  // q4 odd nibbles under 64.0h

  // this wave's chunk range
  const int chunks = (K + F::KC - 1) / F::KC;
  const int c_begin = (chunks * wave) / kw;
  const int c_end = (chunks * (wave + 1)) / kw;

  const uint8_t* wrow[NMAT];
  const ST* srow[NMAT];
  const ST* zrow[NMAT];
#pragma unroll
  for (int t = 0; t < NMAT; ++t) {
    wrow[t] = args.w[t] + (size_t)n_ld * args.row_bytes + kb * 32;
    srow[t] = reinterpret_cast<const ST*>(args.s[t]) + (size_t)n_ld * args.G;
    zrow[t] = args.z[t] ? reinterpret_cast<const ST*>(args.z[t]) + (size_t)n_ld * args.G : nullptr;
  }
  const AT* xrow = reinterpret_cast<const AT*>(args.x) + (size_t)(x_active ? m : 0) * K + kb * F::KL;

  // weights and scales of chunk c (the HBM streams); zero past K
  auto load_w = [&](int c, WFrag<BITS, ST, NMAT, GPC>& f) {
    const int k0 = c * F::KC + kb * F::KL;
    if (c < c_end && k0 < K) {
      const size_t boff = (size_t)c * (F::KC * BITS / 8);
      const int g0 = k0 >> args.lg;
#pragma unroll
      for (int t = 0; t < NMAT; ++t) {
        f.w[t][0] = ldg128_stream(wrow[t] + boff);
        f.w[t][1] = ldg128_stream(wrow[t] + boff + 16);
#pragma unroll
        for (int j = 0; j < GPC; ++j) {
          f.s[t][j] = srow[t][g0 + j];
          f.z[t][j] = zrow[t] ? zrow[t][g0 + j] : (ST)0.0f;
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < NMAT; ++t) {
        f.w[t][0] = (u32x4){0u, 0u, 0u, 0u};
        f.w[t][1] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < GPC; ++j) {
          f.s[t][j] = (ST)0.0f;
          f.z[t][j] = (ST)0.0f;
        }
      }
    }
  };

  f32x4 acc[NMAT];
#pragma unroll
  for (int t = 0; t < NMAT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  WFrag<BITS, ST, NMAT, GPC> cur, nxt;
  load_w(c_begin, cur);
  for (int c = c_begin; c < c_end; ++c) {
    load_w(c + 1, nxt);  // prefetch: next chunk's weights are in flight while this one computes
    const int k0 = c * F::KC + kb * F::KL;
    u32x4 xv[STEPS];
    if (x_active && k0 < K) {
#pragma unroll
      for (int s = 0; s < STEPS; ++s) xv[s] = ldg128(xrow + (size_t)c * F::KC + 8 * s);
    } else {
#pragma unroll
      for (int s = 0; s < STEPS; ++s) xv[s] = (u32x4){0u, 0u, 0u, 0u};
    }

#pragma unroll
    for (int t = 0; t < NMAT; ++t) {
#pragma unroll
      for (int j = 0; j < GPC; ++j) {
        if constexpr (MAGIC) {
          const GpMagic gp = make_gp_magic((f16)cur.s[t][j], (f16)cur.z[t][j]);
#pragma unroll
          for (int s = j * SPG; s < (j + 1) * SPG; ++s) {
            u32x4 a;
            if constexpr (BITS == 4) a = dq4_magic(cur.w[t][s >> 2][s & 3], gp, magic, magic_hi);
            else a = dq8_magic(cur.w[t][s >> 1][(2 * s) & 3], cur.w[t][s >> 1][(2 * s + 1) & 3], gp, magic);
            acc[t] = mfma_k32<AT>(a, xperm<BITS, MAGIC>(xv[s]), acc[t]);
          }
        } else {
          GpExact gp;
          gp.s = to_f32(cur.s[t][j]);
          gp.z = to_f32(cur.z[t][j]);
#pragma unroll
          for (int s = j * SPG; s < (j + 1) * SPG; ++s) {
            u32x4 a;
            if constexpr (BITS == 4) a = dq4_exact<AT>(cur.w[t][s >> 2][s & 3], gp);
            else a = dq8_exact<AT>(cur.w[t][s >> 1][(2 * s) & 3], cur.w[t][s >> 1][(2 * s + 1) & 3], gp);
            acc[t] = mfma_k32<AT>(a, xv[s], acc[t]);
          }
        }
      }
    }
    cur = nxt;
  }

  // ---- cross-wave reduction through LDS
  __shared__ f32x4 red[NMAT][8][64];
  __shared__ int rk_slots[EPI == EPI_ROPE_KV ? kRopeRows : 1];
  if constexpr (EPI == EPI_ROPE_KV) rope_fill_slots(args, rk_slots);
#pragma unroll
  for (int t = 0; t < NMAT; ++t) red[t][wave][lane] = acc[t];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int t = 0; t < NMAT; ++t) {
    f32x4 v = red[t][0][lane];
    for (int w = 1; w < kw; ++w) v += red[t][w][lane];
    acc[t] = v;
  }

  // ---- epilogue: lane holds D[n = nb + i][m], i = 0..3
  if (!x_active) return;
  const int nb = n0 + 4 * kb;
  if constexpr (EPI == EPI_ROPE_KV) {  // fp16 rows; nb is even, the pairs are (nb, nb+1), (nb+2, nb+3)
    rope_kv_pair(args, rk_slots, m, nb, acc[0][0], acc[0][1]);
    rope_kv_pair(args, rk_slots, m, nb + 2, acc[0][2], acc[0][3]);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = nb + i;
    if (nn >= N) break;
    store_out<AT, EPI>(args, (size_t)m * N + nn, acc[0][i], acc[NMAT - 1][i]);
  }
}

// --------------------------------------------------------------------------
// Batched decode tile kernel: fp16 activations and fp16 scales, M <= 16 * MT
// rows per launch, power-of-two group size >= 32, K % 128 == 0.  Used with
// MT = 2 for 17-32 rows (a batch-32 decode step): one pass over the weights
// instead of two 16-row MFMA passes.
//
// A workgroup owns 16 output rows of NMAT matrices; its kw waves split K
// into 128-k chunks.  Per chunk, lane (r = l % 16, kb = l / 16) takes the 32
// consecutive k at 32 * kb: 16 code bytes (q4) or 32 (q8) of row r, the
// (s, z) of the one group they lie in, and x over the same k for column r of
// each of the MT activation tiles -- four v_mfma_f32_16x16x32_f16 steps, the
// dequantized weight operand shared by the MT column tiles.
// The loads run NB chunks ahead in a ring of register buffers refilled in
// place (the loop is unrolled by NB, so no buffer is copied and every buffer
// keeps its registers): a chunk's x, codes and scales were issued NB - 1
// chunks before it is computed, and vmcnt retires in issue order, so computing
// a chunk waits for its own loads only.  Columns past M read row M - 1 (their
// results are dropped); the chunks past a wave's range in its last ring
// re-read its first chunk and are computed with x and s zeroed.
// --------------------------------------------------------------------------
template <int BITS, int NMAT, int MT>
struct TileBuf {
  u32x4 x[MT][4];                     // 4 steps x 8 halves per column tile
  u32x4 w[NMAT][BITS == 4 ? 1 : 2];   // 16 / 32 code bytes
  f16 s[NMAT];
  f16 z[NMAT];
  bool live;
};

template <int BITS, int NMAT, int MT, int NB, int EPI>
__global__ __launch_bounds__(NMAT == 1 && BITS == 4 ? 1024 : 512) void gemv_tile_kernel(const GemvArgs args) {
  constexpr int WB = BITS == 4 ? 1 : 2;  // 16-byte code vectors per lane per chunk
  constexpr int CB = 16 * WB;            // code bytes per lane per chunk
  using Buf = TileBuf<BITS, NMAT, MT>;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar loop control
  const int kw = args.kw;
  const int M = args.M, N = args.N, K = args.K;
  const int n0 = blockIdx.x * 16;
  const int r = lane & 15;
  const int kb = lane >> 4;
  const int n_ld = n0 + r < N ? n0 + r : N - 1;  // rows past N load a valid row; results dropped
  const uint32_t magic = in_vgpr(BITS == 4 ? 0x64006400u : 0x64646464u);
  const uint32_t magic_hi = in_vgpr(0x54005400u);  // q4 odd nibbles under 64.0h
  const bool has_z = args.z[0] != nullptr;

  const int chunks = K >> 7;
  const int c_begin = (chunks * wave) / kw;
  const int c_end = (chunks * (wave + 1)) / kw;

  const uint8_t* wrow[NMAT];
  const f16* srow[NMAT];
  const f16* zrow[NMAT];
#pragma unroll
  for (int t = 0; t < NMAT; ++t) {
    wrow[t] = args.w[t] + (size_t)n_ld * args.row_bytes + kb * CB;
    srow[t] = reinterpret_cast<const f16*>(args.s[t]) + (size_t)n_ld * args.G;
    zrow[t] = has_z ? reinterpret_cast<const f16*>(args.z[t]) + (size_t)n_ld * args.G : srow[t];
  }
  const f16* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r;
    xrow[mt] = reinterpret_cast<const f16*>(args.x) + (size_t)(m < M ? m : M - 1) * K + 32 * kb;
  }

  // x first, then the codes and scales: the order the chunk is consumed in
  auto issue = [&](int c, Buf& b) {
    b.live = c < c_end;
    const int cc = b.live ? c : c_begin;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 4; ++s) b.x[mt][s] = ldg128(xrow[mt] + cc * 128 + 8 * s);
    const int g = (cc * 128 + 32 * kb) >> args.lg;
#pragma unroll
    for (int t = 0; t < NMAT; ++t) {
      const uint8_t* p = wrow[t] + (size_t)cc * (4 * CB);
#pragma unroll
      for (int v = 0; v < WB; ++v) b.w[t][v] = ldg128_stream(p + 16 * v);
      b.s[t] = srow[t][g];
      b.z[t] = zrow[t][g];
    }
  };

  f32x4 acc[NMAT][MT];
#pragma unroll
  for (int t = 0; t < NMAT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Buf& b, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    u32x4 xp[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        xp[mt][s] = xperm<BITS, true>(b.x[mt][s]);
        if constexpr (MASKED)
          if (!b.live) xp[mt][s] = (u32x4){0u, 0u, 0u, 0u};
      }
#pragma unroll
    for (int t = 0; t < NMAT; ++t) {
      f16 sc = b.s[t];
      if constexpr (MASKED)
        if (!b.live) sc = (f16)0.0f;
      const GpMagic gp = make_gp_magic(sc, has_z ? b.z[t] : (f16)0.0f);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        u32x4 a;
        if constexpr (BITS == 4) a = dq4_magic(b.w[t][0][s], gp, magic, magic_hi);
        else a = dq8_magic(b.w[t][s >> 1][(2 * s) & 3], b.w[t][s >> 1][(2 * s + 1) & 3], gp, magic);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma_k32<f16>(a, xp[mt][s], acc[t][mt]);
      }
    }
  };

  // scheduling barriers keep each buffer's loads together and in ring order,
  // so the wait before a chunk's compute leaves NB - 1 buffers in flight
  Buf b[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    issue(c_begin + i, b[i]);
    __builtin_amdgcn_sched_barrier(0);
  }
  int c = c_begin;
  for (; c + NB < c_end; c += NB) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      compute(b[i], std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
      issue(c + NB + i, b[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int i = 0; i < NB; ++i) compute(b[i], std::true_type{});

  // ---- cross-wave reduction through LDS: [kw][NMAT * MT][64] partial tiles
  extern __shared__ __align__(16) uint8_t tile_red_raw[];
  f32x4* red = reinterpret_cast<f32x4*>(tile_red_raw);
  __shared__ int rk_slots[EPI == EPI_ROPE_KV ? kRopeRows : 1];
  if constexpr (EPI == EPI_ROPE_KV) rope_fill_slots(args, rk_slots);
#pragma unroll
  for (int t = 0; t < NMAT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[(wave * NMAT * MT + t * MT + mt) * 64 + lane] = acc[t][mt];
  __syncthreads();
  // wave j finishes column tile j (j < MT): lane holds D[n = 4 kb + i][m = 16 j + r]
  if (wave >= MT) return;
  const int mt = wave;
  const int m = 16 * mt + r;
  f32x4 v[NMAT];
#pragma unroll
  for (int t = 0; t < NMAT; ++t) {
    v[t] = red[(t * MT + mt) * 64 + lane];
    for (int w = 1; w < kw; ++w) v[t] += red[(w * NMAT * MT + t * MT + mt) * 64 + lane];
  }
  if (m >= M) return;
  const int nb = n0 + 4 * kb;
  if constexpr (EPI == EPI_ROPE_KV) {
    rope_kv_pair(args, rk_slots, m, nb, v[0][0], v[0][1]);
    rope_kv_pair(args, rk_slots, m, nb + 2, v[0][2], v[0][3]);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int nn = nb + i;
    if (nn >= N) break;
    store_out<f16, EPI>(args, (size_t)m * N + nn, v[0][i], v[NMAT - 1][i]);
  }
}

// --------------------------------------------------------------------------
// Activation-stationary batched kernel (q4, fp16 activations and scales,
// 5..32 rows, K % 256 == 0, K <= 4096): the MFMA kernels above re-read each
// activation row from L2 for every 16-row weight tile, so at 32 rows the
// activation reads (M x K x 2 bytes per tile) outweigh the 16 x K / 2 code
// bytes they multiply.  Here a workgroup of K / 256 waves keeps the whole
// activation block in registers -- wave w holds k in [256 w, 256 w + 256) of
// every row, lane (r = l % 16, kb = l / 16) two 32-k runs, pre-permuted to
// the order the weight unpack produces (64 VGPRs at 32 rows) -- and walks a
// contiguous run of 16-row tiles: per tile each lane loads the 2 x 16 code
// bytes of row r over its runs, the dequantized operand feeds the MT
// column tiles' v_mfma_f32_16x16x32_f16 steps, and the K / 256 partial tiles
// are summed through LDS (double buffered) by MT waves that take turns.  The
// tile's scales and zero points (16 rows x G, contiguous) are staged in LDS
// by the whole workgroup, one 16-byte vector per thread, instead of one
// 2-byte gather per lane and group from every wave (which cost 30.5 against
// 23.9 us with the gathers replaced by constants, gate/up at 8 rows).  One
// barrier per tile publishes both the tile's partials and the next tile's
// (s, z).  Measured, 2 x 14336 x 4096 gate/up + SwiGLU: 19.4 / 21.3 / 27.4 us
// at 8 / 16 / 32 rows against 31.0 / 36.1 / 57.4 for the kernels above.
// --------------------------------------------------------------------------
template <int NMAT>
struct XsBuf {
  u32x4 w[NMAT][2];  // 32 code bytes: 64 k of row r
  u32x4 sz;          // this thread's 16-byte vector of the tile's (s, z) block
};

// The runs: RUN = 128 puts them at 32 kb and 128 + 32 kb, so each load
// instruction reads the 16 rows' aligned 64-byte half lines whole (used for
// one column tile, where it measured 2 % faster); RUN = 32 makes them one
// 64-k span at 64 kb, whose simpler addressing keeps the two-column-tile
// kernel within 128 VGPRs.
template <int NMAT, int MT, int EPI, int RUN>
__global__ __launch_bounds__(1024) void gemv_xs_kernel(const GemvArgs args) {
  constexpr int STEPS = 8;  // k32 MFMA steps per lane's 64 k (4 per run)
  using Buf = XsBuf<NMAT>;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = args.kw;  // waves = K / 256
  const int M = args.M, N = args.N, K = args.K, G = args.G;
  const int r = lane & 15, kb = lane >> 4;
  const int tiles = (N + 15) >> 4;
  const int t_begin = blockIdx.x * args.rg;  // rg: tiles per workgroup
  const int t_end = min(t_begin + args.rg, tiles);
  const int ka = wave * 256 + kb * (RUN == 128 ? 32 : 64);  // run a: steps 0-3; run b = ka + RUN: 4-7
  const uint32_t magic = in_vgpr(0x64006400u);
  const uint32_t magic_hi = in_vgpr(0x54005400u);  // odd nibbles under 64.0h
  const bool has_z = args.z[0] != nullptr;
  const int ga = ka >> args.lg, gb = (ka + RUN) >> args.lg;  // g >= 32: one group per run

  // LDS: [2][nw][NMAT * MT][64] f32x4 partial tiles, then [2][2 NMAT][16][G + 2]
  // fp16 (s, z) slots (rows padded by 4 bytes: the 16 rows a read touches
  // fall in 16 banks)
  extern __shared__ __align__(16) uint8_t xs_lds[];
  f32x4* red = reinterpret_cast<f32x4*>(xs_lds);
  const int slab = nw * NMAT * MT * 64;  // f32x4 per partial buffer
  const int gp = G + 2;
  f16* szs = reinterpret_cast<f16*>(xs_lds + (size_t)2 * slab * sizeof(f32x4));
  const int slot_len = 2 * NMAT * 16 * gp;

  // this thread's (s, z) vector: piece p (s0, z0, s1, z1), row, 8 groups at c8
  const int vec_per_piece = 2 * G;  // 16 rows x G / 8
  const int nvec = 2 * NMAT * vec_per_piece;
  const bool sz_live = tid < nvec;
  const int vt = sz_live ? tid : 0;
  const int sp = vt / vec_per_piece;
  const int se = vt - sp * vec_per_piece;
  const int srow = se / (G >> 3);
  const int sc8 = se - srow * (G >> 3);
  const bool s_zero = (sp & 1) && !has_z;  // zero points absent: z = 0
  const f16* sbase = reinterpret_cast<const f16*>((sp & 1) && has_z ? args.z[sp >> 1] : args.s[sp >> 1]) +
                     (size_t)srow * G + 8 * sc8;
  const uint32_t code_off = (uint32_t)r * (uint32_t)args.row_bytes + (uint32_t)(ka >> 1);
  // EPI_ROPE_KV: the rows' cache slots as looked up, then with the
  // later-row-wins rule applied, and the rows' positions
  __shared__ int rk_slots[EPI == EPI_ROPE_KV ? kRopeRows : 1];
  __shared__ int rk_res[EPI == EPI_ROPE_KV ? kRopeRows : 1];
  __shared__ int rk_pos[EPI == EPI_ROPE_KV ? kRopeRows : 1];

  // the activation block: column 16 mt + r (rows past M repeat row M - 1;
  // their results are dropped)
  u32x4 xp[MT][STEPS];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(16 * mt + r, M - 1);
    const f16* xr = reinterpret_cast<const f16*>(args.x) + (size_t)m * K + ka;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) xp[mt][st] = xperm<4, true>(ldg128(xr + (st >> 2) * RUN + 8 * (st & 3)));
  }
  __builtin_amdgcn_sched_barrier(0);

  // tile t's codes for row r and this thread's (s, z) vector (N % 16 == 0:
  // every row of a tile exists); tiles past the run re-read its first
  auto tile_of = [&](int t) { return __builtin_amdgcn_readfirstlane(t < t_end ? t : t_begin); };
  auto issue_codes = [&](int t, int q, Buf& b) {
    const uint8_t* p = args.w[q] + (size_t)tile_of(t) * 16 * args.row_bytes + code_off;
    b.w[q][0] = ldg128_stream(p);
    b.w[q][1] = ldg128_stream(p + RUN / 2);
  };
  auto issue_sz = [&](int t, u32x4& v) { v = ldg128(sbase + (size_t)tile_of(t) * 16 * G); };
  auto issue = [&](int t, Buf& b) {
#pragma unroll
    for (int q = 0; q < NMAT; ++q) issue_codes(t, q, b);
    issue_sz(t, b.sz);
  };
  auto stage_v = [&](const u32x4& v, int slot) {
    if (sz_live) {
      uint32_t* d = reinterpret_cast<uint32_t*>(szs + (size_t)(slot & 1) * slot_len + (sp * 16 + srow) * gp + 8 * sc8);
#pragma unroll
      for (int e = 0; e < 4; ++e) d[e] = s_zero ? 0u : v[e];
    }
  };
  auto stage = [&](const Buf& b, int slot) { stage_v(b.sz, slot); };

  // one tile: products against the staged (s, z), partials to LDS; the
  // barrier and the reduction follow in the loop
  auto compute_q = [&](const Buf& b, int it, int q) {
    const f16* sl = szs + (size_t)(it & 1) * slot_len + r * gp;
    f32x4* rb = red + (it & 1) * slab;
    {
      f32x4 acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int g = h ? gb : ga;
        const GpMagic gpm = make_gp_magic(sl[(2 * q) * 16 * gp + g], sl[(2 * q + 1) * 16 * gp + g]);
#pragma unroll
        for (int st = 4 * h; st < 4 * h + 4; ++st) {
          const u32x4 a = dq4_magic(b.w[q][h][st & 3], gpm, magic, magic_hi);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_k32<f16>(a, xp[mt][st], acc[mt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) rb[(wave * NMAT * MT + q * MT + mt) * 64 + lane] = acc[mt];
    }
  };
  // the reducing waves sum the nw partials of tile t and store them (lane
  // holds D[n = 4 kb + i][m = 16 mt + r])
  auto reduce = [&](int t, int it) {
    const f32x4* rb = red + (it & 1) * slab;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (wave != (it * MT + mt) % nw) continue;
      const int m = 16 * mt + r;
      f32x4 v[NMAT];
#pragma unroll
      for (int q = 0; q < NMAT; ++q) {
        v[q] = rb[(q * MT + mt) * 64 + lane];
        for (int w = 1; w < nw; ++w) v[q] += rb[(w * NMAT * MT + q * MT + mt) * 64 + lane];
      }
      const int nb = t * 16 + 4 * kb;
      if (m < M && t < t_end) {
        if constexpr (EPI == EPI_ROPE_KV) {  // NMAT == 1; the pairs are (nb, nb+1), (nb+2, nb+3)
          rope_kv_pair<true>(args, rk_res, m, nb, v[0][0], v[0][1], rk_pos);
          rope_kv_pair<true>(args, rk_res, m, nb + 2, v[0][2], v[0][3], rk_pos);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int nn = nb + i;
            if (nn < N) store_out<f16, EPI>(args, (size_t)m * N + nn, v[0][i], v[NMAT - 1][i]);
          }
        }
      }
    }
  };

  // One code buffer: each matrix's codes are refilled with the next tile's as
  // soon as its products are issued, and the (s, z) vector for tile t + 1 is
  // issued at the start of tile t -- ahead of t + 1's codes, so staging it at
  // the end of tile t waits for it alone and the barrier never waits for
  // codes.  (Measured against a ring of two or three code buffers refilled
  // after a whole tile, whose (s, z) wait also covered the next tile's codes:
  // 19.4 against 24.0 us for the 2 x 14336 x 4096 gate/up at 8 rows.)  The
  // loop refills the same registers in place every iteration, so no buffer
  // is copied across it.  The steps for a tile past the run compute on
  // re-read data and store nothing.
  // EPI_ROPE_KV: the rows' cache slots, in LDS before the first barrier,
  // resolved after it (the loop's barrier precedes the first epilogue)
  if constexpr (EPI == EPI_ROPE_KV) rope_fill_slots(args, rk_slots);

  Buf b;
  issue(t_begin, b);
  __builtin_amdgcn_sched_barrier(0);
  stage(b, 0);
  __syncthreads();
  if constexpr (EPI == EPI_ROPE_KV) rope_resolve_slots(args, rk_slots, rk_res, rk_pos);
  int it = 0;
  for (int t = t_begin; t < t_end; ++t, ++it) {
    issue_sz(t + 1, b.sz);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < NMAT; ++q) {
      compute_q(b, it, q);
      __builtin_amdgcn_sched_barrier(0);
      issue_codes(t + 1, q, b);
      __builtin_amdgcn_sched_barrier(0);
    }
    stage(b, it + 1);
    __syncthreads();
    reduce(t, it);
  }
}

// --------------------------------------------------------------------------
// K-split batched kernel (q4, fp16 activations and scales, 5..32 rows, one
// matrix, K % 128 == 0 with 2048 <= K <= 16384, N % 16 == 0): for the
// matrices the activation-stationary kernel does not take -- long rows (the
// 14336-k down projection) or too few row tiles to share one activation block
// (o-proj, qkv).  One 16-row tile per workgroup of 16 waves; wave w takes an
// equal run of the row's 128-k halves (7 at K = 14336) and requests all of its
// codes up front (one 16-byte load per half: lane (r, kb) reads k in
// [128 h + 32 kb, +32) of row r, so each instruction reads the 16 rows'
// aligned 64-byte half lines), then walks its halves with the activations of
// the next two in flight -- four v_mfma_f32_16x16x32_f16 steps per half and
// column tile.  The tile's scales and zero points are staged in LDS once; the
// 16 partial tiles meet in LDS at the end.  The earlier MFMA kernel loaded a
// chunk's activations behind the next chunk's codes (so each chunk waited for
// the whole prefetch) and gathered (s, z) per lane.
// --------------------------------------------------------------------------
constexpr int XK_WAVES = 16;
constexpr int XK_MAX_HALVES = 8;  // 128-k halves per wave: K <= 16 x 8 x 128

inline size_t xk_lds_bytes(int mt, int G) {
  return (size_t)XK_WAVES * mt * 64 * sizeof(f32x4) + (size_t)2 * 16 * (G + 2) * 2;
}

template <int MT, int EPI>
__global__ __launch_bounds__(1024) void gemv_xk_kernel(const GemvArgs args) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int M = args.M, N = args.N, K = args.K, G = args.G;
  const int r = lane & 15, kb = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int H = K >> 7;
  const int h0 = (H * wave) / XK_WAVES;
  const int nh = (H * (wave + 1)) / XK_WAVES - h0;  // 1..XK_MAX_HALVES (checked by the dispatcher)
  const uint32_t magic = in_vgpr(0x64006400u);
  const uint32_t magic_hi = in_vgpr(0x54005400u);  // odd nibbles under 64.0h
  const bool has_z = args.z[0] != nullptr;

  // LDS: [16][MT][64] f32x4 partial tiles, then [2][16][G + 2] fp16 (s, z)
  extern __shared__ __align__(16) uint8_t xk_lds[];
  f32x4* red = reinterpret_cast<f32x4*>(xk_lds);
  const int gp = G + 2;
  f16* szs = reinterpret_cast<f16*>(xk_lds + (size_t)XK_WAVES * MT * 64 * sizeof(f32x4));
  __shared__ int rk_slots[EPI == EPI_ROPE_KV ? kRopeRows : 1];

  // (s, z) of the tile: 16-byte vectors v = tid and tid + 1024 (piece, row,
  // 8 groups), requested first so staging them waits for nothing else
  const int vpp = 2 * G;  // vectors per piece: 16 rows x G / 8
  u32x4 szv[2];
  int szo[2];
  bool szl[2], szz[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int v = tid + 1024 * j;
    szl[j] = v < 2 * vpp;
    const int vv = szl[j] ? v : 0;
    const int p = vv / vpp, e = vv - p * vpp;
    const int row = e / (G >> 3), c8 = e - row * (G >> 3);
    szz[j] = p == 1 && !has_z;
    const f16* base = reinterpret_cast<const f16*>(p == 1 && has_z ? args.z[0] : args.s[0]);
    szv[j] = ldg128(base + (size_t)(n0 + row) * G + 8 * c8);
    szo[j] = (p * 16 + row) * gp + 8 * c8;
  }
  __builtin_amdgcn_sched_barrier(0);

  // activations of half i in slot i % XR (the first XR requested before the
  // codes, the rest as slots free up; a ring of four measured no faster):
  // column 16 mt + r, k = 128 h + 32 kb + 8 s.  With one column tile the
  // columns past M are zero and not loaded (half the activation traffic at
  // 5..8 rows); results past M are dropped.
  constexpr int XR = 2;
  const f16* xr[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xr[mt] = reinterpret_cast<const f16*>(args.x) + (size_t)min(16 * mt + r, M - 1) * K + 32 * kb;
  u32x4 xs[XR][MT][4];
  auto load_x = [&](int i, int slot) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (MT == 2 || r < M) {  // two column tiles: rows past M repeat row M - 1 (no branch)
#pragma unroll
        for (int st = 0; st < 4; ++st) xs[slot][mt][st] = ldg128(xr[mt] + 128 * (h0 + i) + 8 * st);
      } else {
#pragma unroll
        for (int st = 0; st < 4; ++st) xs[slot][mt][st] = (u32x4){0u, 0u, 0u, 0u};
      }
    }
  };
#pragma unroll
  for (int i = 0; i < XR; ++i)
    if (i < nh) load_x(i, i);
  __builtin_amdgcn_sched_barrier(0);

  // all of this wave's codes
  const uint8_t* wr = args.w[0] + (size_t)(n0 + r) * args.row_bytes + 16 * kb;
  u32x4 w[XK_MAX_HALVES];
#pragma unroll
  for (int i = 0; i < XK_MAX_HALVES; ++i)
    if (i < nh) w[i] = ldg128_stream(wr + 64 * (h0 + i));
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int j = 0; j < 2; ++j)
    if (szl[j]) {
      uint32_t* d = reinterpret_cast<uint32_t*>(szs + szo[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) d[e] = szz[j] ? 0u : szv[j][e];
    }
  __syncthreads();

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const f16* sl = szs + r * gp;
#pragma unroll
  for (int i = 0; i < XK_MAX_HALVES; ++i) {
    if (i < nh) {
      const int g = (128 * (h0 + i) + 32 * kb) >> args.lg;
      const GpMagic gpm = make_gp_magic(sl[g], sl[16 * gp + g]);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const u32x4 a = dq4_magic(w[i][st], gpm, magic, magic_hi);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = mfma_k32<f16>(a, xperm<4, true>(xs[i % XR][mt][st]), acc[mt]);
      }
      if (i + XR < nh) load_x(i + XR, i % XR);
    }
  }

  // the 16 partial tiles; wave j finishes column tile j (lane holds
  // D[n = 4 kb + i][m = 16 j + r])
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[(wave * MT + mt) * 64 + lane] = acc[mt];
  if constexpr (EPI == EPI_ROPE_KV) rope_fill_slots(args, rk_slots);
  __syncthreads();
  if (wave >= MT) return;
  const int mt = wave;
  const int m = 16 * mt + r;
  f32x4 v = red[mt * 64 + lane];
  for (int ww = 1; ww < XK_WAVES; ++ww) v += red[(ww * MT + mt) * 64 + lane];
  if (m >= M) return;
  const int nb = n0 + 4 * kb;
  if constexpr (EPI == EPI_ROPE_KV) {
    rope_kv_pair(args, rk_slots, m, nb, v[0], v[1]);
    rope_kv_pair(args, rk_slots, m, nb + 2, v[2], v[3]);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) store_out<f16, EPI>(args, (size_t)m * N + nb + i, v[i], v[i]);
}

// --------------------------------------------------------------------------
// M <= 4 kernel: v_dot2_f32_f16 on (nearly) raw codes.
//
// A lane handles 32-k "units" (16 code bytes for q4, 32 for q8) of R output
// rows (x NMAT matrices); the R rows share the lane's x registers, and with
// several activation rows (a small decode batch) every row's dot products
// reuse the same unpacked codes -- 4 v_dot2 per 8 codes and row against a
// 5-instruction unpack, where the MFMA path spends 13 instructions per 8
// codes on dequantization and at M <= 4 uses at most a quarter of each
// 16-column product.  The codes
// are never scaled: the exponent-magic trick turns each code pair into an
// fp16 pair, v_dot2 accumulates x . code in fp32, and the group's affine map
// is applied once per unit in fp32:
//   sum_k x_k (c_k - z) s = s * (t - B - z * X),   X = sum of x.
// q4 low nibbles become exact codes c (1024 + c, minus 1024); high nibbles
// stay 1024 + 16c against x/16, i.e. c + 64 per unit of x, so B = 64 * X_hi
// (X_hi = sum of the x's met by high nibbles).  q8 bytes are 1024 + c with
// B = 1024 * X.  Keeping the offset small next to (c - z) keeps the fp32
// cancellation in (t - B) harmless.  Scales and zero points of the
// workgroup's rows are staged in LDS.  Needs fp16 activations, fp16 scales,
// power-of-two group size >= 32, K % 32 == 0.
// --------------------------------------------------------------------------
// rows per workgroup (per matrix): 4 for gate/up (twice the workgroups of 8
// rows keep more waves queued behind the resident ones, which shortens the
// drain at the end of the launch), 8 for a single matrix (whose K-split over
// up to 8 waves already gives each workgroup enough waves).  A small q4
// single-matrix launch at M = 1 -- under 2048 waves at 8 rows, i.e. fewer
// than two per SIMD, such as 4096 x 4096 -- takes 4 rows instead (launch_dot;
// measured 4096 x 4096 4.74 -> 4.35 us per call; the 4096 x 14336 down at 4
// rows, 7168 waves, measured 9.8 against 8.8 us).
template <int BITS, int NMAT>
constexpr int dot_rows() {
  return NMAT == 2 ? 4 : 8;
}
constexpr int kDotSmallRows = 4;
constexpr int kDotSmallWaves = 2048;
constexpr int DOT_SZ_VEC = 2;  // 16-byte (s|z) vectors staged per lane
constexpr int SEG_STRIDE = 64; // fp16 entries per staged (s|z) run

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(bitcast<f16x2>(a), bitcast<f16x2>(b), c, false);
}

// Partner exchange at lane distance D for the reductions below.  D = 32 and
// 16 use the gfx950 permlane swaps: permlane32_swap(a, b) leaves a = (a.lo,
// b.lo) and b = (a.hi, b.hi) by 32-lane halves, permlane16_swap does the same
// for the odd/even 16-lane rows, so a + b holds, in lanes with bit D clear,
// the pair sum of a and, in lanes with bit D set, the pair sum of b.  Smaller
// distances pair lanes inside a 16-lane row with DPP (row_partner below).
template <int D>
__device__ __forceinline__ float swap_sum(float a, float b) {
  static_assert(D == 32 || D == 16, "permlane swaps cover D = 32, 16");
  const auto r = D == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false)
                         : __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The value of a partner lane that differs from this one in bit D (D = 8, 4,
// 2, 1), read with a DPP modifier (folded into the add that consumes it, no
// LDS round trip): D = 8 row_mirror (lane i <-> 15 - i, i.e. xor 15), D = 4
// row_half_mirror (xor 7), D = 2 / 1 quad_perm [2,3,0,1] / [1,0,3,2].  The
// masks 32, 16 (permlane swaps), 15, 7, 2, 1 are independent over GF(2), so
// the butterflies below still sum every lane of a group exactly once, and
// each pairing flips bit D, which is all the halving step's keep/send choice
// reads.  (Measured against ds_swizzle xor partners: the M = 1 down
// projection 8.8 -> 8.5 us.)
template <int D>
__device__ __forceinline__ float row_partner(float v) {
  static_assert(D == 8 || D == 4 || D == 2 || D == 1, "DPP row partners cover D < 16");
  constexpr int ctrl = D == 8 ? 0x140 : D == 4 ? 0x141 : D == 2 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}

// Butterfly that halves the live values per step: at distance d a lane keeps
// the half selected by (lane & d) and adds the partner's copy of it.  After
// log2(CNT) steps every lane holds one value, then plain butterflies finish
// the 64-lane sum.  Lane l ends with the total of value index idx(l), where
// idx adds CNT/2, CNT/4, ... for each set bit 32, 16, ... of l.
template <int CNT, int D>
__device__ __forceinline__ void reduce_scatter(float* v, int lane) {
  if constexpr (D >= 1) {
    if constexpr (CNT > 1) {
      constexpr int H = CNT / 2;
      if constexpr (D >= 16) {
#pragma unroll
        for (int j = 0; j < H; ++j) v[j] = swap_sum<D>(v[j], v[j + H]);
      } else {
        const bool upper = (lane & D) != 0;
#pragma unroll
        for (int j = 0; j < H; ++j) {
          const float keep = upper ? v[j + H] : v[j];
          const float send = upper ? v[j] : v[j + H];
          v[j] = keep + row_partner<D>(send);
        }
      }
      reduce_scatter<H, D / 2>(v, lane);
    } else {
      if constexpr (D >= 16) v[0] = swap_sum<D>(v[0], v[0]);
      else v[0] += row_partner<D>(v[0]);
      reduce_scatter<1, D / 2>(v, lane);
    }
  }
}

template <int BITS, int NMAT, int R, int MR>
struct DotFrag {
  u32x4 w[NMAT][R][BITS == 4 ? 1 : 2];
  u32x4 x[MR][4];
};

// Full 64-lane sum, in every lane.
__device__ __forceinline__ float wave_total(float v) {
  v = swap_sum<32>(v, v);
  v = swap_sum<16>(v, v);
  v += row_partner<8>(v);
  v += row_partner<4>(v);
  v += row_partner<2>(v);
  return v + row_partner<1>(v);
}

// Workgroup layout: rg row groups of R rows (per matrix) x kw waves, one
// 2048-k slice per wave.  The plain kernel has one row group and each wave
// reads its slice of x straight from memory.  With the norm prologue (NORM)
// the workgroup loads x, the residual and the norm weight once, 16 bytes per
// thread, normalises the row into LDS, and every wave reads its slice from
// there: two row groups share that work, and the activation traffic per
// code byte is what keeps the prologue cheap.
// MR activation rows (1, 2 or 4; rows past M repeat row M - 1 and are not
// stored) share each lane's code unpack: a batched decode step costs 4 MR
// v_dot2 per 8 codes on top of the 5-instruction unpack.
template <int BITS, int NMAT, int EPI, bool NORM, int MR, int R = dot_rows<BITS, NMAT>()>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void gemv_dot_kernel(
    const GemvArgs args) {
  static_assert(!NORM || MR == 1, "the norm prologue takes one activation row");
  constexpr int V = NMAT * R;  // values per activation row reduced per lane
  constexpr int VT = V * MR;   // values reduced per lane
  constexpr int NSEG = V * 2;  // (matrix, row, s|z) runs staged per wave
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kw = args.kw;
  const int grp = wave / kw;     // row group of this wave
  const int ks = wave - grp * kw;  // k slice of this wave
  const int N = args.N, K = args.K, G = args.G;
  const int n0 = ((int)blockIdx.x * args.rg + grp) * R;
  const uint32_t magic = in_vgpr(BITS == 4 ? 0x64006400u : 0x64646464u);
  const f16* x = reinterpret_cast<const f16*>(args.x);

  const uint8_t* wrow[NMAT][R];
#pragma unroll
  for (int t = 0; t < NMAT; ++t)
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[t][r] = args.w[t] + (size_t)min(n0 + r, N - 1) * args.row_bytes;

  // unit u = ks * 64 + lane: one 128-bit code load per row (two for q8) and
  // four 16-byte x vectors; a wave's 64 units are contiguous in k
  const int U = K / 32;
  const int ubase = ks * 64;

  // dynamic LDS: [normalised row, K fp16 | NORM][(s, z) stage per wave]
  extern __shared__ __align__(16) uint8_t dot_lds[];
  f16* xrow = reinterpret_cast<f16*>(dot_lds);
  uint8_t* stage = dot_lds + (NORM ? (size_t)K * 2 : 0) + wave * (NSEG * 2 * SEG_STRIDE);

  // Scales and zero points: each wave stages, in its own LDS region, the
  // (s, z) of its rows for the groups its 64 units cover -- NSEG runs of gpw
  // fp16 values (gpw <= 64), fetched with 128-bit loads and stored at a fixed
  // stride of 64 entries so a row's run sits at a compile-time offset.  They
  // are requested first, then the activations, then the codes (vmcnt retires
  // in issue order, so each later wait leaves the code loads in flight).  With
  // the norm prologue the activations go first: the prologue then waits for
  // its L2-resident operands only, not for the (s, z) vectors from HBM
  // (measured 15.3 -> 14.8 us at 2 x 14336 x 4096; the plain kernel keeps the
  // (s, z) vectors first, 12.7 against 12.9 us).
  const int lsv = 8 - args.lg;      // log2(16-byte vectors per run), gpw = 8 << lsv
  const int nvec = NSEG << lsv;     // <= 64 * DOT_SZ_VEC (checked by the dispatcher)
  u32x4 szv[DOT_SZ_VEC];
  uint32_t sz_zero[DOT_SZ_VEC];
  auto issue_sz = [&]() {
    // branch-free: lanes without a run (or a missing zero tensor) read a valid
    // vector of the same row and drop it, so every load counts in order for
    // vmcnt.  A partial last slice clamps its vectors to the row's last 8
    // groups: the units past K that would use them are dropped.
    const int g0 = (ubase * 32) >> args.lg;
    const f16* s0 = reinterpret_cast<const f16*>(args.s[0]);
    const f16* s1 = reinterpret_cast<const f16*>(args.s[NMAT - 1]);
    const f16* z0 = args.z[0] ? reinterpret_cast<const f16*>(args.z[0]) : s0;
    const f16* z1 = args.z[NMAT - 1] ? reinterpret_cast<const f16*>(args.z[NMAT - 1]) : s1;
    const uint32_t has_z = args.z[0] != nullptr ? 1u : 0u;
#pragma unroll
    for (int j = 0; j < DOT_SZ_VEC; ++j) {
      const int v = lane + 64 * j;
      const int vv = v < nvec ? v : 0;
      const int seg = vv >> lsv;
      const int e = vv & ((1 << lsv) - 1);
      const int t = seg / (2 * R), r = (seg >> 1) % R, isz = seg & 1;
      const f16* base = t == 0 ? (isz ? z0 : s0) : (isz ? z1 : s1);
      const int nr = min(n0 + r, N - 1);
      szv[j] = ldg128(base + (size_t)nr * G + min(g0 + 8 * e, G - 8));
      sz_zero[j] = (uint32_t)isz & (has_z ^ 1u);  // zero tensor absent: z = 0
    }
  };
  auto stage_sz = [&]() {
#pragma unroll
    for (int j = 0; j < DOT_SZ_VEC; ++j) {
      const int v = lane + 64 * j;
      if (v < nvec) {
        const int seg = v >> lsv, e = v & ((1 << lsv) - 1);
        *reinterpret_cast<u32x4*>(stage + seg * (2 * SEG_STRIDE) + e * 16) =
            sz_zero[j] ? (u32x4){0u, 0u, 0u, 0u} : szv[j];
      }
    }
  };
  if constexpr (!NORM) {
    issue_sz();
    __builtin_amdgcn_sched_barrier(0);  // keep the small loads ahead of the rest
  }
  // residual epilogue: the lane that stores output (m, n0 + rr) requests its
  // residual value now, with the operands, not after the reduction (which
  // would add a memory trip to the last workgroup's tail); every lane loads
  // (an in-range element where it stores nothing) so the load counts in order
  f16 res_pre = (f16)0.0f;
  if constexpr (EPI == EPI_RESIDUAL) {
    const int m = lane / R, rr = lane - (lane / R) * R;
    const bool st = lane < R * MR && n0 + rr < N && m < args.M;
    res_pre = reinterpret_cast<const f16*>(args.residual)[st ? (size_t)m * N + n0 + rr : 0];
  }

  // activations: NORM -- 16-byte chunks c = threadIdx.x (+ blockDim.x) of x,
  // the residual and the norm weight, at most two per thread (the dispatcher
  // keeps K / 8 <= 2 * blockDim.x), clamped so every load issues; otherwise
  // -- this lane's four vectors of its unit of x.
  const int nthr = blockDim.x;
  u32x4 ax[NORM ? 2 : 1], ar[NORM ? 2 : 1], aw[NORM ? 2 : 1];
  DotFrag<BITS, NMAT, R, MR> f;
  const int u = ubase + lane;
  const int k0 = (u < U ? u : 0) * 32;
  if constexpr (NORM) {
    // chunks past the row (threads beyond K / 8, which the norm below
    // leaves out) re-read a chunk inside it, so every load stays in the row
    const NormChunks nc = norm_prologue_chunks(threadIdx.x, nthr, K);
    const int c0c = nc.c0, c1c = nc.c1;
    // no residual: the loads read x again and are dropped, so every load
    // still issues in order
    const f16* rp = reinterpret_cast<const f16*>(args.nres ? args.nres : args.x);
    const f16* wp = reinterpret_cast<const f16*>(args.nw);
    ax[0] = ldg128(x + 8 * c0c);
    ax[1] = ldg128(x + 8 * c1c);
    ar[0] = ldg128(rp + 8 * c0c);
    ar[1] = ldg128(rp + 8 * c1c);
    aw[0] = ldg128(wp + 8 * c0c);
    aw[1] = ldg128(wp + 8 * c1c);
    __builtin_amdgcn_sched_barrier(0);
    issue_sz();
  } else {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const f16* xm = x + (size_t)(m < args.M ? m : args.M - 1) * K;
#pragma unroll
      for (int j = 0; j < 4; ++j) f.x[m][j] = ldg128(xm + k0 + 8 * j);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // the activation loads stay ahead of the codes
#pragma unroll
  for (int t = 0; t < NMAT; ++t)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t* p = wrow[t][r] + (uint32_t)(k0 * BITS / 8);
      f.w[t][r][0] = ldg128_stream(p);
      if constexpr (BITS == 8) f.w[t][r][BITS == 4 ? 0 : 1] = ldg128_stream(p + 16);
    }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!NORM) stage_sz();

  if constexpr (NORM) {
    const int c0 = threadIdx.x, c1 = threadIdx.x + nthr;
    const NormChunks nc = norm_prologue_chunks(threadIdx.x, nthr, K);
    const bool has0 = nc.has0, has1 = nc.has1;
    {
      // z = fp16(x + r) and the row's sum of z^2 (the packed fp16 add rounds
      // the exact sum once, as the norm kernel's fp32 add-then-round does for
      // fp16 inputs), then n = fp16((z * inv) * w) in fp32 -- the arithmetic
      // of rms_norm_vec_kernel; workgroup 0 writes z and n out.  (No
      // residual: the loads above read x again; they are dropped here, after
      // the code requests, since selecting them waits for them.)
      if (!args.nres) ar[0] = ar[1] = (u32x4){0u, 0u, 0u, 0u};
      u32x4 zz[2];
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          zz[i][e] = bitcast<uint32_t>(bitcast<f16x2>(ax[i][e]) + bitcast<f16x2>(ar[i][e]));
          const float sq = dot2(zz[i][e], zz[i][e], 0.0f);
          ss += (i == 0 ? has0 : has1) ? sq : 0.0f;
        }
      ss = wave_total(ss);
      __shared__ float norm_part[8];
      if (lane == 0) norm_part[wave] = ss;
      __syncthreads();
      float tot = 0.0f;
      for (int w = 0; w < (int)(nthr >> 6); ++w) tot += norm_part[w];
      const float inv = rsqrtf(tot / (float)K + args.eps);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (!(i == 0 ? has0 : has1)) continue;
        const int c = i == 0 ? c0 : c1;
        u32x4 nv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f16x2 zh = bitcast<f16x2>(zz[i][e]);
          const f16x2 wh = bitcast<f16x2>(aw[i][e]);
          const f16x2 nh = {(f16)(((float)zh[0] * inv) * (float)wh[0]),
                            (f16)(((float)zh[1] * inv) * (float)wh[1])};
          nv[e] = bitcast<uint32_t>(nh);
        }
        *reinterpret_cast<u32x4*>(xrow + 8 * c) = nv;
        if (blockIdx.x == 0) {
          if (args.zout) *reinterpret_cast<u32x4*>(reinterpret_cast<f16*>(args.zout) + 8 * c) = zz[i];
          if (args.nout) *reinterpret_cast<u32x4*>(reinterpret_cast<f16*>(args.nout) + 8 * c) = nv;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) f.x[0][j] = *reinterpret_cast<const u32x4*>(xrow + k0 + 8 * j);
    stage_sz();
  } else {
    __builtin_amdgcn_wave_barrier();
  }

  float acc[VT];  // index m * V + t * R + r
#pragma unroll
  for (int i = 0; i < VT; ++i) acc[i] = 0.0f;

  {  // one 64-unit slice per wave (the dispatcher guarantees U <= 64 * kw)
    // a lane past the last unit computes on x = 0: its codes, offsets and
    // zero-point terms all vanish, so its sums add nothing
    if (u >= U) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) f.x[m][j] = (u32x4){0u, 0u, 0u, 0u};
    }

    // activation operands in the unpack order, and their sums, per row m
    uint32_t xp[MR][16];
    float xsm[MR], nboff[MR];
    const uint32_t one2 = 0x3C003C00u;  // (1.0h, 1.0h)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
    float xs = 0.0f;  // X, the sum of the slice's x
    float boff;       // what the exponent-magic offsets add to the code sums
    if constexpr (BITS == 4) {
      // low nibbles decode to 1024 + c, high nibbles (in place) to
      // 1024 + 16 c against x / 16: the offsets sum to 1024 X_lo + 64 X_hi
      float xs_hi = 0.0f, xs_lo = 0.0f;
      const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // word j covers x[8j .. 8j+8): pairs (0,4) (1,5)/16 (2,6) (3,7)/16
        const uint32_t p0 = pack_lo16(f.x[m][j][0], f.x[m][j][2]);
        const uint32_t p1 = pack_hi16(f.x[m][j][0], f.x[m][j][2]);
        const uint32_t p2 = pack_lo16(f.x[m][j][1], f.x[m][j][3]);
        const uint32_t p3 = pack_hi16(f.x[m][j][1], f.x[m][j][3]);
        xs_hi = dot2(p1, one2, dot2(p3, one2, xs_hi));
        xs_lo = dot2(p0, one2, dot2(p2, one2, xs_lo));
        xp[m][4 * j + 0] = p0;
        xp[m][4 * j + 1] = bitcast<uint32_t>(bitcast<f16x2>(p1) * sixteenth);
        xp[m][4 * j + 2] = p2;
        xp[m][4 * j + 3] = bitcast<uint32_t>(bitcast<f16x2>(p3) * sixteenth);
      }
      xs = xs_lo + xs_hi;
      boff = 1024.0f * xs_lo + 64.0f * xs_hi;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // two words per 8 x's: pairs (0,2) (1,3) (4,6) (5,7)
        xp[m][4 * j + 0] = pack_lo16(f.x[m][j][0], f.x[m][j][1]);
        xp[m][4 * j + 1] = pack_hi16(f.x[m][j][0], f.x[m][j][1]);
        xp[m][4 * j + 2] = pack_lo16(f.x[m][j][2], f.x[m][j][3]);
        xp[m][4 * j + 3] = pack_hi16(f.x[m][j][2], f.x[m][j][3]);
        xs = dot2(xp[m][4 * j + 0], one2, dot2(xp[m][4 * j + 1], one2,
                  dot2(xp[m][4 * j + 2], one2, dot2(xp[m][4 * j + 3], one2, xs))));
      }
      boff = 1024.0f * xs;
    }
    xsm[m] = xs;
    nboff[m] = -boff;
    }
    // this lane's group within the wave's slice; run seg is at seg * 64
    const f16* szl = reinterpret_cast<const f16*>(stage) + ((lane * 32) >> args.lg);

#pragma unroll
    for (int t = 0; t < NMAT; ++t)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float tsum[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) tsum[m] = nboff[m];
        if constexpr (BITS == 4) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t q = f.w[t][r][0][w];
            const uint32_t v = q >> 8;
            const uint32_t c0 = (q & 0x000F000Fu) | magic, c1 = (q & 0x00F000F0u) | magic;
            const uint32_t c2 = (v & 0x000F000Fu) | magic, c3 = (v & 0x00F000F0u) | magic;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
              tsum[m] = dot2(c0, xp[m][4 * w + 0], tsum[m]);
              tsum[m] = dot2(c1, xp[m][4 * w + 1], tsum[m]);
              tsum[m] = dot2(c2, xp[m][4 * w + 2], tsum[m]);
              tsum[m] = dot2(c3, xp[m][4 * w + 3], tsum[m]);
            }
          }
        } else {
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            const uint32_t q = f.w[t][r][w >> 2][w & 3];
            const uint32_t lo = q8_lo_pair(q, magic), hi = q8_hi_pair(q, magic);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
              tsum[m] = dot2(lo, xp[m][2 * w + 0], tsum[m]);
              tsum[m] = dot2(hi, xp[m][2 * w + 1], tsum[m]);
            }
          }
        }
        const int seg = (t * R + r) * 2;
        const float sv = (float)szl[seg * SEG_STRIDE];
        const float zv = (float)szl[(seg + 1) * SEG_STRIDE];
#pragma unroll
        for (int m = 0; m < MR; ++m)
          acc[m * V + t * R + r] = fmaf(sv, fmaf(-zv, xsm[m], tsum[m]), acc[m * V + t * R + r]);
      }
  }

  // ---- 64-lane reduction (halving butterfly), then across the row group's
  // waves in LDS
  static_assert(VT <= 64 && (VT & (VT - 1)) == 0, "lane reduction shape");
  reduce_scatter<VT, 32>(acc, lane);
  const float tot = acc[0];
  int idx = 0;
#pragma unroll
  for (int d = 32, h = VT / 2; h >= 1; d >>= 1, h >>= 1)
    if (lane & d) idx += h;
  __shared__ float red[8][VT];
  __shared__ int rk_slots[EPI == EPI_ROPE_KV ? kRopeRows : 1];
  if constexpr (EPI == EPI_ROPE_KV) rope_fill_slots(args, rk_slots);
  constexpr int QUAD = 64 / VT;  // lanes holding the same index
  if ((lane & (QUAD - 1)) == 0) red[wave][idx] = tot;
  __syncthreads();
  if (ks != 0 || lane >= R * MR) return;
  const int m = lane / R, rr = lane - m * R;
  float v0 = 0.0f, v1 = 0.0f;
  for (int w = 0; w < kw; ++w) {
    v0 += red[wave + w][m * V + rr];
    if constexpr (NMAT == 2) v1 += red[wave + w][m * V + R + rr];
  }
  const int nn = n0 + rr;
  if constexpr (EPI == EPI_ROPE_KV) {
    rope_kv_store(args, rk_slots, m, nn, v0);  // lane pairs (rr even, rr + 1) never straddle a head: R and D even
    return;
  }
  if (nn < N && m < args.M) {
    if constexpr (EPI == EPI_RESIDUAL) {  // store_out's arithmetic with the prefetched residual
      const f16 d = saturate_cast<f16>(v0);
      if (args.y0) reinterpret_cast<f16*>(args.y0)[(size_t)m * N + nn] = d;
      reinterpret_cast<f16*>(args.y1)[(size_t)m * N + nn] = from_f32<f16>(to_f32(res_pre) + to_f32(d));
    } else {
      store_out<f16, EPI>(args, (size_t)m * N + nn, v0, v1);
    }
  }
}

// --------------------------------------------------------------------------
// generic kernel: any K (odd K uses ceil(K/2) packed columns), any group size,
// any M.  One wave per output row; fp32 math with the dequantized weight
// rounded to the activation type first, as the reference path does
// (ops/quant_ops.py:523-526).
// --------------------------------------------------------------------------
template <int BITS, typename AT, typename ST, int NMAT, int EPI>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const GemvArgs args, int gs) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= args.N) return;
  const int K = args.K, M = args.M, N = args.N;
  const AT* x = reinterpret_cast<const AT*>(args.x);
  for (int m = 0; m < M; ++m) {
    float dot[NMAT];
#pragma unroll
    for (int t = 0; t < NMAT; ++t) {
      const uint8_t* wr = args.w[t] + (size_t)n * args.row_bytes;
      const ST* sr = reinterpret_cast<const ST*>(args.s[t]) + (size_t)n * args.G;
      const ST* zr = args.z[t] ? reinterpret_cast<const ST*>(args.z[t]) + (size_t)n * args.G : nullptr;
      float a = 0.f;
      for (int k = lane; k < K; k += 64) {
        uint32_t q;
        if constexpr (BITS == 4) {
          const uint8_t b = wr[k >> 1];
          q = (k & 1) ? (b >> 4) : (b & 15u);
        } else {
          q = wr[k];
        }
        const int g = k / gs;
        const float s = to_f32(sr[g]);
        const float z = zr ? to_f32(zr[g]) : 0.0f;
        const float w = to_f32(from_f32<AT>(((float)q - z) * s));
        a += to_f32(x[(size_t)m * K + k]) * w;
      }
      dot[t] = wave_sum(a);
    }
    if (lane != 0) continue;
    const size_t o = (size_t)m * N + n;
    if constexpr (EPI == EPI_NONE) {
      reinterpret_cast<AT*>(args.y0)[o] = saturate_cast<AT>(dot[0]);
    } else if constexpr (EPI == EPI_RESIDUAL) {
      const AT d = saturate_cast<AT>(dot[0]);
      if (args.y0) reinterpret_cast<AT*>(args.y0)[o] = d;
      const float r = to_f32(reinterpret_cast<const AT*>(args.residual)[o]);
      reinterpret_cast<AT*>(args.y1)[o] = from_f32<AT>(r + to_f32(d));
    } else {
      const AT g = saturate_cast<AT>(dot[0]);
      const AT u = saturate_cast<AT>(dot[NMAT - 1]);
      if (args.y0) reinterpret_cast<AT*>(args.y0)[o] = g;
      if (args.y1) reinterpret_cast<AT*>(args.y1)[o] = u;
      if (args.y2) {
        const float gf = to_f32(g);
        const float sil = gf / (1.0f + expf(-gf));
        reinterpret_cast<AT*>(args.y2)[o] = from_f32<AT>(sil * to_f32(u));
      }
    }
  }
}

// --------------------------------------------------------------------------
// host dispatch
// --------------------------------------------------------------------------
inline int ilog2_exact(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int l = 0;
  while ((1LL << l) < v) ++l;
  return l;
}

template <int BITS, typename AT, typename ST, bool MAGIC, int NMAT, int EPI>
int launch_fast(const GemvArgs& a, int gpc, hipStream_t st) {
  const dim3 grid((a.N + 15) / 16);
  const dim3 block(64 * a.kw);
  switch (gpc) {
    case 1: gemv_mfma_kernel<BITS, AT, ST, MAGIC, 1, NMAT, EPI><<<grid, block, 0, st>>>(a); break;
    case 2: gemv_mfma_kernel<BITS, AT, ST, MAGIC, 2, NMAT, EPI><<<grid, block, 0, st>>>(a); break;
    case 4: gemv_mfma_kernel<BITS, AT, ST, MAGIC, 4, NMAT, EPI><<<grid, block, 0, st>>>(a); break;
    default: return MK_ERR_UNSUPPORTED;
  }
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// Tile kernel plan: ring depth NB (4 chunks for q4 at one column tile; 2
// where the x or q8 code registers double) and kw waves per 16-row tile,
// kw <= 16 for a single q4 matrix, else 8 (1024 / 512 threads), preferring a
// split that gives every wave a whole number of rings and at least one.
template <int BITS, int MT>
constexpr int tile_ring() { return BITS == 4 && MT == 1 ? 4 : 2; }

template <int BITS, int NMAT>
inline int tile_choose_kw(int64_t K, int nb) {
  const int64_t chunks = K / 128;
  const int kmax = NMAT == 1 && BITS == 4 ? 16 : 8;
  for (int kw = kmax; kw >= 1; --kw)
    if (chunks % kw == 0 && (chunks / kw) % nb == 0) return kw;
  int64_t kw = (chunks + nb - 1) / nb;  // every wave at least one ring
  return (int)(kw < 1 ? 1 : (kw > kmax ? kmax : kw));
}

template <int BITS, int NMAT, int MT, int EPI>
int launch_tile(GemvArgs a, hipStream_t st) {
  constexpr int NB = tile_ring<BITS, MT>();
  a.kw = tile_choose_kw<BITS, NMAT>(a.K, NB);
  if (a.kw < MT) a.kw = MT;  // wave j finishes column tile j
  const dim3 grid((unsigned)((a.N + 15) / 16));
  const dim3 block((unsigned)(64 * a.kw));
  const size_t lds = (size_t)a.kw * NMAT * MT * 64 * sizeof(f32x4);
  gemv_tile_kernel<BITS, NMAT, MT, NB, EPI><<<grid, block, lds, st>>>(a);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// CUs of the current device, cached per device.
inline int gemv_device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// the activation-stationary kernel takes 5..32-row batches of matrices with at
// least this many 16-row tiles, one per CU (measured against the K-split
// kernel at 8 / 16 / 32 rows, us: 4096 x 4096 7.05 / 8.2 / 12.8 against 7.5 /
// 8.65 / 13.0; 6144 x 4096 9.1 / 10.3 / 14.9 against 13.0 / 15.3 / 24.4)
constexpr int kXsMinRows = 5;
constexpr int kXsMinTiles = 256;
constexpr size_t kXsMaxLds = 160 * 1024;

// K-split launch: one 16-row tile per workgroup of 16 waves
template <int MT, int EPI>
int launch_xk(GemvArgs a, hipStream_t st) {
  const dim3 grid((unsigned)(a.N / 16));
  const dim3 block(64 * XK_WAVES);
  gemv_xk_kernel<MT, EPI><<<grid, block, xk_lds_bytes(MT, a.G), st>>>(a);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// q4, one matrix, fp16 activations and scales, power-of-two group >= 32,
// K % 128 == 0 with 16 <= K / 128 <= 16 x 8, N % 16 == 0, the tile's (s, z)
// within two 16-byte vectors per thread, 16-byte aligned operands
template <int BITS, int NMAT>
bool xk_eligible(const GemvArgs& a, int mt, int act_dt, int sc_dt) {
  const int H = a.K / 128;
  bool ok = BITS == 4 && NMAT == 1 && act_dt == MK_DT_F16 && sc_dt == MK_DT_F16 && a.lg >= 5 &&
            (a.K % 128) == 0 && H >= XK_WAVES && H <= XK_WAVES * XK_MAX_HALVES && (a.N % 16) == 0 &&
            (a.G % 8) == 0 && 4 * a.G <= 2 * 64 * XK_WAVES && xk_lds_bytes(mt, a.G) <= kXsMaxLds &&
            mk_aligned(a.x, 16) && (size_t)a.row_bytes % 16 == 0 && mk_aligned(a.w[0], 16) &&
            mk_aligned(a.s[0], 16) && (a.z[0] == nullptr || mk_aligned(a.z[0], 16));
  return ok;
}

// partial tiles (double buffered) + two (s, z) slots with 4-byte row padding
inline size_t xs_lds_bytes(int nw, int nmat, int mt, int G) {
  return (size_t)2 * nw * nmat * mt * 64 * sizeof(f32x4) + (size_t)2 * 2 * nmat * 16 * (G + 2) * 2;
}

// Activation-stationary launch: K / 256 waves per workgroup, the 16-row tiles
// dealt out in equal contiguous runs to at most one workgroup per CU (the
// 128 KB partial buffer and 16 waves of <= 128 VGPRs fill a CU).
template <int NMAT, int MT, int EPI>
int launch_xs(GemvArgs a, hipStream_t st) {
  const int tiles = (a.N + 15) / 16;
  const int cus = gemv_device_cus();
  const int tpw = (tiles + cus - 1) / cus;
  a.rg = tpw;
  a.kw = a.K / 256;
  const dim3 grid((unsigned)((tiles + tpw - 1) / tpw));
  const dim3 block((unsigned)(64 * a.kw));
  const size_t lds = xs_lds_bytes(a.kw, NMAT, MT, a.G);
  gemv_xs_kernel<NMAT, MT, EPI, MT == 1 ? 128 : 32><<<grid, block, lds, st>>>(a);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// q4 only, fp16 activations and scales, 256 <= K <= 4096 with K % 256 == 0,
// power-of-two group >= 32 (one group per lane's 32-k run), 16-byte
// aligned x and codes, and enough rows that every CU gets tiles to stream
template <int BITS, int NMAT, int EPI>
bool xs_eligible(const GemvArgs& a, int mt, int act_dt, int sc_dt) {
  bool ok = BITS == 4 && (EPI != EPI_ROPE_KV || NMAT == 1) && act_dt == MK_DT_F16 && sc_dt == MK_DT_F16 && a.lg >= 5 &&
            (a.K % 256) == 0 && a.K >= 256 && a.K <= 4096 &&
            (a.N % 16) == 0 && a.N / 16 >= kXsMinTiles && mk_aligned(a.x, 16) && (size_t)a.row_bytes % 16 == 0 &&
            (a.G % 8) == 0 && 4 * NMAT * a.G <= 64 * (a.K / 256) &&  // one (s, z) vector per thread
            xs_lds_bytes(a.K / 256, NMAT, mt, a.G) <= kXsMaxLds;
  for (int t = 0; t < NMAT; ++t)
    ok = ok && mk_aligned(a.w[t], 16) && mk_aligned(a.s[t], 16) && (a.z[0] == nullptr || mk_aligned(a.z[t], 16));
  return ok;
}

// fp16 activations and scales, power-of-two group >= 32, K % 128 == 0, 16-byte
// aligned x and codes
template <int NMAT>
bool tile_eligible(const GemvArgs& a, int act_dt, int sc_dt) {
  bool ok = act_dt == MK_DT_F16 && sc_dt == MK_DT_F16 && a.lg >= 5 && (a.K % 128) == 0 &&
            mk_aligned(a.x, 16) && (size_t)a.row_bytes % 16 == 0;
  for (int t = 0; t < NMAT; ++t) ok = ok && mk_aligned(a.w[t], 16);
  return ok;
}

// Row groups per dot workgroup: one for the plain kernel (measured: sharing
// x through LDS costs a barrier that outweighs its L2 savings); two for the
// norm prologue (four at K <= 2048), which keeps K / 8 <= 2 * blockDim.x for
// K <= 8192 and halves the activation reads per code byte.
template <bool NORM>
inline int dot_row_groups(int kw) { return NORM ? (kw >= 2 ? 2 : 4) : 1; }

template <int BITS, int NMAT, int EPI, bool NORM, int R>
int launch_dot_rows(GemvArgs a, hipStream_t st) {
  a.rg = dot_row_groups<NORM>(a.kw);
  const int rows = R * a.rg;
  const dim3 grid((unsigned)((a.N + rows - 1) / rows));
  const dim3 block((unsigned)(64 * a.kw * a.rg));
  const size_t stage_bytes = (size_t)a.kw * a.rg * NMAT * R * 2 * (2 * SEG_STRIDE);
  const size_t lds = (NORM ? (size_t)a.K * 2 : 0) + stage_bytes;
  if constexpr (NORM) {
    MK_REQUIRE(a.K / 8 <= 2 * (int)block.x);  // the prologue's two 16-byte chunks per thread cover the row
    gemv_dot_kernel<BITS, NMAT, EPI, true, 1, R><<<grid, block, lds, st>>>(a);
  } else {
    if (a.M <= 1) gemv_dot_kernel<BITS, NMAT, EPI, false, 1, R><<<grid, block, lds, st>>>(a);
    else if constexpr (R != dot_rows<BITS, NMAT>()) return MK_ERR_UNSUPPORTED;  // small-launch rows: M = 1 only
    else if (a.M == 2) gemv_dot_kernel<BITS, NMAT, EPI, false, 2, R><<<grid, block, lds, st>>>(a);
    else if constexpr (BITS == 4) gemv_dot_kernel<BITS, NMAT, EPI, false, 4, R><<<grid, block, lds, st>>>(a);
    else return MK_ERR_UNSUPPORTED;  // q8: at most two rows (four would spill)
  }
  MK_CHECK_LAUNCH();
  return MK_OK;
}

template <int BITS, int NMAT, int EPI, bool NORM = false>
int launch_dot(GemvArgs a, hipStream_t st) {
  constexpr int R = dot_rows<BITS, NMAT>();
  if constexpr (BITS == 4 && NMAT == 1 && R > kDotSmallRows) {
    // a q4 single matrix at M = 1 that would run under kDotSmallWaves waves
    const int rg = dot_row_groups<NORM>(a.kw);
    const int64_t waves = (int64_t)((a.N + R * rg - 1) / (R * rg)) * rg * a.kw;
    if (a.M <= 1 && waves < kDotSmallWaves) return launch_dot_rows<BITS, NMAT, EPI, NORM, kDotSmallRows>(a, st);
  }
  return launch_dot_rows<BITS, NMAT, EPI, NORM, R>(a, st);
}

template <int BITS, typename AT, typename ST, int NMAT, int EPI>
int launch_generic(const GemvArgs& a, int gs, hipStream_t st) {
  const dim3 grid((a.N + 3) / 4);
  gemv_generic_kernel<BITS, AT, ST, NMAT, EPI><<<grid, dim3(256), 0, st>>>(a, gs);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// Waves per workgroup: enough K-parallelism to keep >= ~4 waves per SIMD
// in flight on 256 CUs, without giving a wave less than one chunk.
inline int choose_kw(int64_t N, int64_t K, int kc) {
  const int64_t tiles = (N + 15) / 16;
  const int64_t chunks = (K + kc - 1) / kc;
  int kw = tiles >= 1024 ? 4 : 8;
  if (kw > chunks) kw = (int)chunks;
  if (kw < 1) kw = 1;
  return kw;
}

// Shape facts every launch needs: fills N, K, G, row_bytes and lg of a;
// returns the groups per 32-code lane chunk of the MFMA path (0: none) and
// whether the aligned fast layouts apply.
template <int BITS, int NMAT>
int gemv_prepare(GemvArgs& a, int64_t N, int64_t K, int64_t gs, bool* fast) {
  using F = QFmt<BITS>;
  a.N = (int)N;
  a.K = (int)K;
  a.G = (int)((K + gs - 1) / gs);
  a.row_bytes = BITS == 4 ? (int)((K + 1) / 2) : (int)K;
  const int lg = ilog2_exact(gs);
  int gpc = 0;
  if (lg >= 0) {
    if (gs >= F::KL) gpc = 1;
    else if (gs >= 8 && F::KL / gs <= 4) gpc = (int)(F::KL / gs);
  }
  bool f = gpc > 0 && (K % F::KL) == 0 && mk_aligned(a.x, 16);
  for (int t = 0; t < NMAT; ++t) f = f && mk_aligned(a.w[t], 16);
  a.lg = lg;
  *fast = f;
  return gpc;
}

// The dot kernel (M <= 4): one 64-unit (2048-k) slice per wave, <= 8 waves;
// the (s, z) runs of a slice must be whole 16-byte vectors and fit the stage.
template <int BITS, int NMAT>
bool dot_eligible(const GemvArgs& a, bool fast, int64_t mrows, int act_dt, int sc_dt) {
  const int lg = a.lg;
  const int64_t K = a.K;
  const int64_t gpw = lg >= 0 ? (2048 >> lg) : 0;
  return fast && mrows >= 1 && mrows <= (BITS == 4 ? 4 : 2) && act_dt == MK_DT_F16 && sc_dt == MK_DT_F16 &&
         lg >= 5 && lg <= 8 &&
         (K % 32) == 0 && K <= 8 * 2048 && (a.G % 8) == 0 && (gpw % 8) == 0 &&
         (int64_t)NMAT * dot_rows<BITS, NMAT>() * 2 * (gpw / 8) <= 64 * DOT_SZ_VEC &&
         mk_aligned(a.s[0], 16) && mk_aligned(a.s[NMAT - 1], 16) &&
         (a.z[0] == nullptr || (mk_aligned(a.z[0], 16) && mk_aligned(a.z[NMAT - 1], 16)));
}

// waves per dot-kernel workgroup: one per 64-unit slice
inline int dot_waves(int64_t K) {
  int64_t kwd = (K / 32 + 63) / 64;
  return (int)(kwd < 1 ? 1 : (kwd > 8 ? 8 : kwd));
}

template <int BITS, int NMAT, int EPI>
int gemv_dispatch(GemvArgs a, int64_t M, int64_t N, int64_t K, int64_t gs, int act_dt, int sc_dt,
                  hipStream_t st) {
  using F = QFmt<BITS>;
  MK_REQUIRE(M >= 0 && N > 0 && K > 0 && gs > 0);
  MK_REQUIRE(act_dt == MK_DT_F16 || act_dt == MK_DT_BF16);
  MK_REQUIRE(sc_dt == MK_DT_F16 || sc_dt == MK_DT_F32);
  MK_REQUIRE(N < (1LL << 31) && K < (1LL << 31));
  if (M == 0) return MK_OK;
  for (int t = 0; t < NMAT; ++t) MK_REQUIRE(a.w[t] && a.s[t]);
  MK_REQUIRE(a.x);

  bool fast;
  const int gpc = gemv_prepare<BITS, NMAT>(a, N, K, gs, &fast);

  const size_t xe = 2;  // activation element size
  int rc = MK_OK;
  // rows m0.. of every row-indexed operand
  auto rows_from = [&](GemvArgs& b, int64_t m0) {
    b.x = (const char*)a.x + (size_t)m0 * K * xe;
    if (a.residual) b.residual = (const char*)a.residual + (size_t)m0 * N * xe;
    if (a.y0) b.y0 = (char*)a.y0 + (size_t)m0 * N * xe;
    if (a.y1) b.y1 = (char*)a.y1 + (size_t)m0 * N * xe;
    if (a.y2) b.y2 = (char*)a.y2 + (size_t)m0 * N * xe;
    if constexpr (EPI == EPI_ROPE_KV) {
      // rows of a later pass write after this one: the later row of a
      // colliding pair still wins
      b.rk.pos = a.rk.pos + m0;
      b.rk.bt = a.rk.bt + (size_t)m0 * a.rk.max_blocks;
      b.rk.q_out = (char*)a.rk.q_out + (size_t)m0 * a.rk.Hq * a.rk.D * xe;
    }
  };
  if constexpr (EPI == EPI_ROPE_KV) {
    // fp16 projections on the fast layouts only (the caller falls back)
    if (act_dt != MK_DT_F16 || sc_dt != MK_DT_F16 || !fast) return MK_ERR_UNSUPPORTED;
  }
  int64_t m_done = 0;
  // up to 32 rows at a time through the activation-stationary kernel
  {
    if (M >= kXsMinRows && xs_eligible<BITS, NMAT, EPI>(a, 1, act_dt, sc_dt)) {
      while (M - m_done >= kXsMinRows && rc == MK_OK) {
        GemvArgs b = a;
        int64_t mrows = (M - m_done) < 32 ? (M - m_done) : 32;
        if (mrows > 16 && !xs_eligible<BITS, NMAT, EPI>(a, 2, act_dt, sc_dt)) mrows = 16;
        b.M = (int)mrows;
        rows_from(b, m_done);
        rc = mrows > 16 ? launch_xs<NMAT, 2, EPI>(b, st) : launch_xs<NMAT, 1, EPI>(b, st);
        m_done += mrows;
      }
    }
  }
  // otherwise up to 32 rows at a time through the K-split kernel
  if constexpr (NMAT == 1) {
    if (M - m_done >= kXsMinRows && xk_eligible<BITS, NMAT>(a, 1, act_dt, sc_dt)) {
      while (M - m_done >= kXsMinRows && rc == MK_OK) {
        GemvArgs b = a;
        int64_t mrows = (M - m_done) < 32 ? (M - m_done) : 32;
        if (mrows > 16 && !xk_eligible<BITS, NMAT>(a, 2, act_dt, sc_dt)) mrows = 16;
        b.M = (int)mrows;
        rows_from(b, m_done);
        rc = mrows > 16 ? launch_xk<2, EPI>(b, st) : launch_xk<1, EPI>(b, st);
        m_done += mrows;
      }
    }
  }
  // 17-32 rows at a time through the two-column-tile kernel, the rest below
  if (tile_eligible<NMAT>(a, act_dt, sc_dt)) {
    while (M - m_done >= 17 && rc == MK_OK) {
      GemvArgs b = a;
      const int64_t mrows = (M - m_done) < 32 ? (M - m_done) : 32;
      b.M = (int)mrows;
      rows_from(b, m_done);
      rc = launch_tile<BITS, NMAT, 2, EPI>(b, st);
      m_done += mrows;
    }
  }
  const int64_t mblocks = (M - m_done + 15) / 16;
  for (int64_t mb = 0; mb < mblocks && rc == MK_OK; ++mb) {
    GemvArgs b = a;
    const int64_t m0 = m_done + mb * 16;
    const int64_t mrows = (M - m0) < 16 ? (M - m0) : 16;
    b.M = (int)mrows;
    rows_from(b, m0);
    if (dot_eligible<BITS, NMAT>(b, fast && mk_aligned(b.x, 16), mrows, act_dt, sc_dt)) {
      b.kw = dot_waves(K);
      rc = launch_dot<BITS, NMAT, EPI>(b, st);
    } else if constexpr (EPI == EPI_ROPE_KV) {
      b.kw = choose_kw(N, K, F::KC);
      rc = launch_fast<BITS, f16, f16, true, NMAT, EPI>(b, gpc, st);
    } else if (fast) {
      b.kw = choose_kw(N, K, F::KC);
      if (act_dt == MK_DT_F16 && sc_dt == MK_DT_F16)
        rc = launch_fast<BITS, f16, f16, true, NMAT, EPI>(b, gpc, st);
      else if (act_dt == MK_DT_F16)
        rc = launch_fast<BITS, f16, float, false, NMAT, EPI>(b, gpc, st);
      else if (sc_dt == MK_DT_F16)
        rc = launch_fast<BITS, bf16, f16, false, NMAT, EPI>(b, gpc, st);
      else
        rc = launch_fast<BITS, bf16, float, false, NMAT, EPI>(b, gpc, st);
    } else {
      b.M = (int)mrows;
      if (act_dt == MK_DT_F16 && sc_dt == MK_DT_F16)
        rc = launch_generic<BITS, f16, f16, NMAT, EPI>(b, (int)gs, st);
      else if (act_dt == MK_DT_F16)
        rc = launch_generic<BITS, f16, float, NMAT, EPI>(b, (int)gs, st);
      else if (sc_dt == MK_DT_F16)
        rc = launch_generic<BITS, bf16, f16, NMAT, EPI>(b, (int)gs, st);
      else
        rc = launch_generic<BITS, bf16, float, NMAT, EPI>(b, (int)gs, st);
    }
  }
  return rc;
}

template <int BITS>
int matvec_entry(const void* x, const uint8_t* w, const void* s, const void* z, const void* residual,
                 void* y_mm, void* y_out, int64_t M, int64_t N, int64_t K, int64_t gs, int act_dt,
                 int sc_dt, void* stream) {
  GemvArgs a = {};
  a.x = x;
  a.w[0] = a.w[1] = w;
  a.s[0] = a.s[1] = s;
  a.z[0] = a.z[1] = z;
  a.residual = residual;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (residual) {
    MK_REQUIRE(y_out);
    a.y0 = y_mm;
    a.y1 = y_out;
    return gemv_dispatch<BITS, 1, EPI_RESIDUAL>(a, M, N, K, gs, act_dt, sc_dt, st);
  }
  void* y = y_out ? y_out : y_mm;
  MK_REQUIRE(y);
  a.y0 = y;
  int rc = gemv_dispatch<BITS, 1, EPI_NONE>(a, M, N, K, gs, act_dt, sc_dt, st);
  if (rc == MK_OK && y_mm && y_out && y_mm != y_out) {
    hipError_t e = hipMemcpyAsync(y_mm, y_out, (size_t)M * N * 2, hipMemcpyDeviceToDevice, st);
    if (e != hipSuccess) return -(int)e - 1000;
  }
  return rc;
}

template <int BITS>
int gate_up_entry(const void* x, const uint8_t* wg, const uint8_t* wu, const void* sg,
                  const void* su, const void* zg, const void* zu, void* gate_out, void* up_out,
                  void* mlp_out, int64_t M, int64_t N, int64_t K, int64_t gs, int act_dt,
                  int sc_dt, void* stream) {
  MK_REQUIRE(gate_out || up_out || mlp_out);
  GemvArgs a = {};
  a.x = x;
  a.w[0] = wg;
  a.w[1] = wu;
  a.s[0] = sg;
  a.s[1] = su;
  a.z[0] = zg;
  a.z[1] = zu;
  a.y0 = gate_out;
  a.y1 = up_out;
  a.y2 = mlp_out;
  return gemv_dispatch<BITS, 2, EPI_GATE_UP>(a, M, N, K, gs, act_dt, sc_dt,
                                             reinterpret_cast<hipStream_t>(stream));
}

// Residual add + RMSNorm + gate/up (+ SwiGLU) of one MLP block: one launch
// (the norm as the dot kernel's prologue) for an M = 1 fp16 q4 decode row the
// dot kernel takes, else the norm kernel and then the gate/up launch (q8's
// doubled code registers leave no room for the prologue's operands).
template <int BITS>
int norm_gate_up_entry(const void* x, const void* residual, const void* norm_w, float eps, const uint8_t* wg,
                       const uint8_t* wu, const void* sg, const void* su, const void* zg, const void* zu,
                       void* z_out, void* normed_out, void* gate_out, void* up_out, void* mlp_out, int64_t M,
                       int64_t N, int64_t K, int64_t gs, int act_dt, int sc_dt, int nw_dt, void* stream) {
  MK_REQUIRE(x && residual && norm_w && z_out && wg && wu && sg && su);
  MK_REQUIRE(gate_out || up_out || mlp_out);
  MK_REQUIRE(M >= 0 && N > 0 && K > 0 && gs > 0 && N < (1LL << 31) && K < (1LL << 31));
  MK_REQUIRE(act_dt == MK_DT_F16 || act_dt == MK_DT_BF16);
  MK_REQUIRE(sc_dt == MK_DT_F16 || sc_dt == MK_DT_F32);
  MK_REQUIRE(nw_dt == MK_DT_F16 || nw_dt == MK_DT_BF16 || nw_dt == MK_DT_F32);
  if (M == 0) return MK_OK;
  GemvArgs a = {};
  a.x = x;
  a.w[0] = wg;
  a.w[1] = wu;
  a.s[0] = sg;
  a.s[1] = su;
  a.z[0] = zg;
  a.z[1] = zu;
  a.y0 = gate_out;
  a.y1 = up_out;
  a.y2 = mlp_out;
  bool fast;
  gemv_prepare<BITS, 2>(a, N, K, gs, &fast);
  {
    // K <= 8192: the row fits two 16-byte chunks per thread of the workgroup
    if (nw_dt == MK_DT_F16 && K <= 4 * 2048 && M == 1 && dot_eligible<BITS, 2>(a, fast, M, act_dt, sc_dt) &&
        mk_aligned(residual, 16) &&
        mk_aligned(norm_w, 16) && mk_aligned(z_out, 16) && (!normed_out || mk_aligned(normed_out, 16))) {
      a.M = 1;
      a.kw = dot_waves(K);
      a.nres = residual;
      a.nw = norm_w;
      a.zout = z_out;
      a.nout = normed_out;
      a.eps = eps;
      return launch_dot<BITS, 2, EPI_GATE_UP, true>(a, reinterpret_cast<hipStream_t>(stream));
    }
  }
  MK_REQUIRE(normed_out);  // the two-launch path passes the normalised rows through it
  const int rc = mk_residual_rms_norm(x, residual, norm_w, z_out, normed_out, M, K, eps, act_dt, nw_dt, stream);
  if (rc != MK_OK) return rc;
  return gate_up_entry<BITS>(normed_out, wg, wu, sg, su, zg, zu, gate_out, up_out, mlp_out, M, N, K, gs, act_dt,
                             sc_dt, stream);
}

// RMSNorm + matvec: y = fp16(x * rsqrt(mean(x^2) + eps) * norm_w) . W^T.
// One launch (the norm as the dot kernel's prologue, no residual) for an
// M = 1 fp16 q4 row the dot kernel takes, else the norm kernel into
// normed_out and then the matvec.
template <int BITS>
int norm_matvec_entry(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* s,
                      const void* z, void* normed_out, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                      int act_dt, int sc_dt, int nw_dt, void* stream) {
  MK_REQUIRE(x && norm_w && w && s && y);
  MK_REQUIRE(M >= 0 && N > 0 && K > 0 && gs > 0 && N < (1LL << 31) && K < (1LL << 31));
  MK_REQUIRE(act_dt == MK_DT_F16 || act_dt == MK_DT_BF16);
  MK_REQUIRE(sc_dt == MK_DT_F16 || sc_dt == MK_DT_F32);
  MK_REQUIRE(nw_dt == MK_DT_F16 || nw_dt == MK_DT_BF16 || nw_dt == MK_DT_F32);
  if (M == 0) return MK_OK;
  GemvArgs a = {};
  a.x = x;
  a.w[0] = a.w[1] = w;
  a.s[0] = a.s[1] = s;
  a.z[0] = a.z[1] = z;
  a.y0 = y;
  bool fast;
  gemv_prepare<BITS, 1>(a, N, K, gs, &fast);
  if constexpr (BITS == 4) {
    // K <= 8192: the row fits two 16-byte chunks per thread of the workgroup
    if (nw_dt == MK_DT_F16 && K <= 4 * 2048 && M == 1 &&
        dot_eligible<BITS, 1>(a, fast && mk_aligned(x, 16), M, act_dt, sc_dt) &&
        mk_aligned(norm_w, 16) && (!normed_out || mk_aligned(normed_out, 16))) {
      a.M = 1;
      a.kw = dot_waves(K);
      a.nres = nullptr;
      a.nw = norm_w;
      a.zout = nullptr;
      a.nout = normed_out;
      a.eps = eps;
      return launch_dot<BITS, 1, EPI_NONE, true>(a, reinterpret_cast<hipStream_t>(stream));
    }
  }
  MK_REQUIRE(normed_out);  // the two-launch path passes the normalised rows through it
  const int rc = mk_rms_norm(x, norm_w, normed_out, M, K, eps, act_dt, nw_dt, stream);
  if (rc != MK_OK) return rc;
  return matvec_entry<BITS>(normed_out, w, s, z, nullptr, nullptr, y, M, N, K, gs, act_dt, sc_dt, stream);
}

// RMSNorm + qkv projection + split + RoPE + paged K/V write.  One launch
// (the NORM dot kernel with the EPI_ROPE_KV epilogue) for a q4 fp16 row with
// K <= 8192; otherwise the projection into qkv_scratch, then
// mk_qkv_rope_paged_update.
template <int BITS>
int norm_qkv_rope_entry(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* s,
                        const void* z, void* qkv_scratch, void* normed_out, const float* cos_t,
                        const float* sin_t, const int32_t* positions, const int32_t* block_table, void* K_pages,
                        void* V_pages, void* q_out, int64_t M, int64_t Hq, int64_t Hkv, int64_t D, int64_t P,
                        int64_t max_blocks, int64_t num_pages, int64_t cos_rows, int64_t K, int64_t gs,
                        int act_dt, int sc_dt, int nw_dt, void* stream) {
  MK_REQUIRE(x && norm_w && w && s && qkv_scratch && cos_t && sin_t && positions && block_table && K_pages &&
             V_pages && q_out);
  MK_REQUIRE(M >= 0 && M < 65536 && Hq > 0 && Hkv > 0 && D > 0 && (D % 2) == 0 && P > 0 && max_blocks > 0 &&
             num_pages > 0 && cos_rows > 0 && K > 0 && gs > 0);
  MK_REQUIRE((Hq + 2 * Hkv) * D < (1LL << 31) && num_pages * P < (1LL << 31) && max_blocks * P < (1LL << 31));
  MK_REQUIRE(act_dt == MK_DT_F16 || act_dt == MK_DT_BF16);
  if (M == 0) return MK_OK;
  const int64_t N = (Hq + 2 * Hkv) * D;
  if constexpr (BITS == 4) {
    GemvArgs a = {};
    a.x = x;
    a.w[0] = a.w[1] = w;
    a.s[0] = a.s[1] = s;
    a.z[0] = a.z[1] = z;
    bool fast;
    gemv_prepare<BITS, 1>(a, N, K, gs, &fast);
    if (act_dt == MK_DT_F16 && sc_dt == MK_DT_F16 && nw_dt == MK_DT_F16 && K <= 4 * 2048 && M == 1 &&
        dot_eligible<BITS, 1>(a, fast && mk_aligned(x, 16), M, act_dt, sc_dt) && mk_aligned(norm_w, 16) &&
        (!normed_out || mk_aligned(normed_out, 16))) {
      a.M = 1;
      a.kw = dot_waves(K);
      a.nres = nullptr;
      a.nw = norm_w;
      a.zout = nullptr;
      a.nout = normed_out;
      a.eps = eps;
      a.rk = RopeKV{cos_t, sin_t, positions, block_table, K_pages, V_pages, q_out, (int)Hq, (int)Hkv, (int)D,
                    (int)P, (int)max_blocks, (int)num_pages, (int)cos_rows};
      return launch_dot<BITS, 1, EPI_ROPE_KV, true>(a, reinterpret_cast<hipStream_t>(stream));
    }
  }
  MK_REQUIRE(normed_out);  // the multi-launch paths pass the normalised rows through it
  if (act_dt == MK_DT_F16 && sc_dt == MK_DT_F16 && max_blocks * P < (1LL << 31)) {
    // the norm kernel, then the projection whose epilogue rotates and writes
    GemvArgs a = {};
    a.x = normed_out;
    a.w[0] = a.w[1] = w;
    a.s[0] = a.s[1] = s;
    a.z[0] = a.z[1] = z;
    a.rk = RopeKV{cos_t, sin_t, positions, block_table, K_pages, V_pages, q_out, (int)Hq, (int)Hkv, (int)D,
                  (int)P, (int)max_blocks, (int)num_pages, (int)cos_rows};
    GemvArgs probe = a;
    bool fast;
    gemv_prepare<BITS, 1>(probe, N, K, gs, &fast);
    if (fast) {
      int rc = mk_rms_norm(x, norm_w, normed_out, M, K, eps, act_dt, nw_dt, stream);
      if (rc != MK_OK) return rc;
      return gemv_dispatch<BITS, 1, EPI_ROPE_KV>(a, M, N, K, gs, act_dt, sc_dt, reinterpret_cast<hipStream_t>(stream));
    }
  }
  const int rc = norm_matvec_entry<BITS>(x, norm_w, eps, w, s, z, normed_out, qkv_scratch, M, N, K, gs, act_dt,
                                         sc_dt, nw_dt, stream);
  if (rc != MK_OK) return rc;
  return mk_qkv_rope_paged_update(qkv_scratch, cos_t, sin_t, positions, block_table, K_pages, V_pages, q_out, M, Hq,
                                  Hkv, D, P, max_blocks, num_pages, cos_rows, act_dt, stream);
}

}  // namespace

extern "C" {

int mk_q4_rmsnorm_qkv_rope_paged(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                                 const void* zeros, void* qkv_scratch, void* normed_out, const float* cos_t,
                                 const float* sin_t, const int32_t* positions, const int32_t* block_table,
                                 void* K_pages, void* V_pages, void* q_out, int64_t M, int64_t Hq, int64_t Hkv,
                                 int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                 int64_t cos_rows, int64_t K, int64_t group_size, int act_dtype, int scale_dtype,
                                 int norm_w_dtype, void* stream) {
  return norm_qkv_rope_entry<4>(x, norm_w, eps, w, scales, zeros, qkv_scratch, normed_out, cos_t, sin_t, positions,
                                block_table, K_pages, V_pages, q_out, M, Hq, Hkv, D, page_size, max_blocks,
                                num_pages, cos_rows, K, group_size, act_dtype, scale_dtype, norm_w_dtype, stream);
}

int mk_q8_rmsnorm_qkv_rope_paged(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                                 const void* zeros, void* qkv_scratch, void* normed_out, const float* cos_t,
                                 const float* sin_t, const int32_t* positions, const int32_t* block_table,
                                 void* K_pages, void* V_pages, void* q_out, int64_t M, int64_t Hq, int64_t Hkv,
                                 int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                 int64_t cos_rows, int64_t K, int64_t group_size, int act_dtype, int scale_dtype,
                                 int norm_w_dtype, void* stream) {
  return norm_qkv_rope_entry<8>(x, norm_w, eps, w, scales, zeros, qkv_scratch, normed_out, cos_t, sin_t, positions,
                                block_table, K_pages, V_pages, q_out, M, Hq, Hkv, D, page_size, max_blocks,
                                num_pages, cos_rows, K, group_size, act_dtype, scale_dtype, norm_w_dtype, stream);
}

int mk_q4_rmsnorm_matvec(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                         const void* zeros, void* normed_out, void* y, int64_t M, int64_t N, int64_t K,
                         int64_t group_size, int act_dtype, int scale_dtype, int norm_w_dtype, void* stream) {
  return norm_matvec_entry<4>(x, norm_w, eps, w, scales, zeros, normed_out, y, M, N, K, group_size, act_dtype,
                              scale_dtype, norm_w_dtype, stream);
}

int mk_q8_rmsnorm_matvec(const void* x, const void* norm_w, float eps, const uint8_t* w, const void* scales,
                         const void* zeros, void* normed_out, void* y, int64_t M, int64_t N, int64_t K,
                         int64_t group_size, int act_dtype, int scale_dtype, int norm_w_dtype, void* stream) {
  return norm_matvec_entry<8>(x, norm_w, eps, w, scales, zeros, normed_out, y, M, N, K, group_size, act_dtype,
                              scale_dtype, norm_w_dtype, stream);
}


int mk_q4_matvec(const void* x, const uint8_t* w, const void* scales, const void* zeros,
                 const void* residual, void* y_mm, void* y_out, int64_t M, int64_t N, int64_t K,
                 int64_t group_size, int act_dtype, int scale_dtype, void* stream) {
  return matvec_entry<4>(x, w, scales, zeros, residual, y_mm, y_out, M, N, K, group_size, act_dtype,
                         scale_dtype, stream);
}

int mk_q8_matvec(const void* x, const uint8_t* w, const void* scales, const void* zeros,
                 const void* residual, void* y_mm, void* y_out, int64_t M, int64_t N, int64_t K,
                 int64_t group_size, int act_dtype, int scale_dtype, void* stream) {
  return matvec_entry<8>(x, w, scales, zeros, residual, y_mm, y_out, M, N, K, group_size, act_dtype,
                         scale_dtype, stream);
}

int mk_q4_gate_up(const void* x, const uint8_t* w_gate, const uint8_t* w_up, const void* s_gate,
                  const void* s_up, const void* z_gate, const void* z_up, void* gate_out,
                  void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K,
                  int64_t group_size, int act_dtype, int scale_dtype, void* stream) {
  return gate_up_entry<4>(x, w_gate, w_up, s_gate, s_up, z_gate, z_up, gate_out, up_out, mlp_out,
                          M, N, K, group_size, act_dtype, scale_dtype, stream);
}

int mk_q8_gate_up(const void* x, const uint8_t* w_gate, const uint8_t* w_up, const void* s_gate,
                  const void* s_up, const void* z_gate, const void* z_up, void* gate_out,
                  void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K,
                  int64_t group_size, int act_dtype, int scale_dtype, void* stream) {
  return gate_up_entry<8>(x, w_gate, w_up, s_gate, s_up, z_gate, z_up, gate_out, up_out, mlp_out,
                          M, N, K, group_size, act_dtype, scale_dtype, stream);
}

int mk_q4_rmsnorm_gate_up(const void* x, const void* residual, const void* norm_w, float eps,
                          const uint8_t* w_gate, const uint8_t* w_up, const void* s_gate, const void* s_up,
                          const void* z_gate, const void* z_up, void* z_out, void* normed_out, void* gate_out,
                          void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K, int64_t group_size,
                          int act_dtype, int scale_dtype, int norm_w_dtype, void* stream) {
  return norm_gate_up_entry<4>(x, residual, norm_w, eps, w_gate, w_up, s_gate, s_up, z_gate, z_up, z_out,
                               normed_out, gate_out, up_out, mlp_out, M, N, K, group_size, act_dtype, scale_dtype,
                               norm_w_dtype, stream);
}

int mk_q8_rmsnorm_gate_up(const void* x, const void* residual, const void* norm_w, float eps,
                          const uint8_t* w_gate, const uint8_t* w_up, const void* s_gate, const void* s_up,
                          const void* z_gate, const void* z_up, void* z_out, void* normed_out, void* gate_out,
                          void* up_out, void* mlp_out, int64_t M, int64_t N, int64_t K, int64_t group_size,
                          int act_dtype, int scale_dtype, int norm_w_dtype, void* stream) {
  return norm_gate_up_entry<8>(x, residual, norm_w, eps, w_gate, w_up, s_gate, s_up, z_gate, z_up, z_out,
                               normed_out, gate_out, up_out, mlp_out, M, N, K, group_size, act_dtype, scale_dtype,
                               norm_w_dtype, stream);
}

}  // extern "C"
