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
// Fast path (D in {64,128}, fp16 q for quantized caches): one wave per
// (split of the context, kv head, sequence[, block of 16 query heads]).
//   QK^T : v_mfma_f32_16x16x32  A = K tile (16 positions x 32 d), loaded
//          straight from the page (lane = position, 4 lanes cover one row),
//          B = q^T (32 d x 16 heads; the GQA group fills the columns, so one
//          K read serves all Hq/Hkv heads).
//   P.V  : v_mfma_f32_16x16x16  A = P (16 heads x 16 positions) -- exactly the
//          accumulator layout QK^T leaves behind, B = V tile regrouped per
//          output column.
// The online softmax runs in base 2 on 32-position blocks; splits write
// (m, l, O) partials that a second kernel merges (LSE merge,
// ops/attention_ops.py:534-550).  A sequence that fits one split is finished
// in place.
#include "common.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kTilesPerBlock = 2;  // 32 positions per softmax update

struct PagedArgs {
  const void* q;       // [B, Hq, D]
  const void* K;       // pages (fp16/bf16 or uint8 codes)
  const void* V;
  const uint16_t* Ks;  // quantized: fp16 scales [NP, P, Hkv, G]
  const uint16_t* Vs;
  const int32_t* bt;   // [B, MB]
  const int32_t* lengths;
  void* out;           // [B, Hq, D]
  float* ws;           // partials
  int B, Hq, Hkv, G, HB;
  int NP, P, MB;
  int gs, ngroups;     // quantization group size and groups per head
  int split_tok, s_max;
  float scale_log2;
};

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
template <typename AT>
__device__ __forceinline__ f32x4 mfma_k16(u32x2 a, u32x2 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma_k16<f16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(bitcast<f16x4>(a), bitcast<f16x4>(b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma_k16<bf16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bitcast<s16x4>(a), bitcast<s16x4>(b), c, 0, 0,
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
  f16x2 v = bitcast<f16x2>(((u >> shift) & 0x00FF00FFu) | 0x64006400u) - k;
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
// 8 q4 codes (one word) -> 8 fp16, order [0,4,1,5,2,6,3,7]
__device__ __forceinline__ u32x4 deq4x8(uint32_t u, f16x2 s2) {
  u32x4 r;
  r[0] = q4_pair(u, 0, s2);
  r[1] = q4_pair(u, 4, s2);
  r[2] = q4_pair(u, 8, s2);
  r[3] = q4_pair(u, 12, s2);
  return r;
}

// permutation of 8 consecutive d's produced by the dequant helpers, and the
// matching regroup of q (natural order) into that order
template <int KVF>
__device__ __forceinline__ u32x4 qperm(u32x4 X) {
  if constexpr (KVF == 8) {
    u32x4 r;
    r[0] = (X[0] & 0xFFFFu) | (X[1] << 16);
    r[1] = (X[0] >> 16) | (X[1] & 0xFFFF0000u);
    r[2] = (X[2] & 0xFFFFu) | (X[3] << 16);
    r[3] = (X[2] >> 16) | (X[3] & 0xFFFF0000u);
    return r;
  } else if constexpr (KVF == 4) {
    u32x4 r;
    r[0] = (X[0] & 0xFFFFu) | (X[2] << 16);
    r[1] = (X[0] >> 16) | (X[2] & 0xFFFF0000u);
    r[2] = (X[1] & 0xFFFFu) | (X[3] << 16);
    r[3] = (X[1] >> 16) | (X[3] & 0xFFFF0000u);
    return r;
  } else {
    return X;
  }
}
// slot (0..7) of the permuted vector -> d offset within the 8
template <int KVF>
__device__ __forceinline__ int dslot(int j) {
  if constexpr (KVF == 8) {
    constexpr int p[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    return p[j];
  } else if constexpr (KVF == 4) {
    constexpr int p[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    return p[j];
  } else {
    return j;
  }
}

__device__ __forceinline__ f16x2 scale2(const uint16_t* sp) {
  const f16 s = bitcast<f16>(*sp);
  return (f16x2){s, s};
}

// Load 8 consecutive d's [d0, d0+8) of one K or V row as 8 act-type values
// (permuted order for quantized formats).  row_elem = (page*P+off)*Hkv+hkv.
template <typename AT, int D, int KVF>
__device__ __forceinline__ u32x4 load8(const void* base, const uint16_t* sbase, size_t row_elem,
                                       int d0, int gs, int ngroups) {
  if constexpr (KVF == 0) {
    return ldg128(reinterpret_cast<const AT*>(base) + row_elem * D + d0);
  } else if constexpr (KVF == 8) {
    const u32x2 c = ldg64(reinterpret_cast<const uint8_t*>(base) + row_elem * D + d0);
    const f16x2 s2 = scale2(sbase + row_elem * ngroups + d0 / gs);
    return deq8x8(c[0], c[1], s2);
  } else {
    const uint32_t c =
        *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(base) +
                                           row_elem * (D / 2) + d0 / 2);
    const f16x2 s2 = scale2(sbase + row_elem * ngroups + d0 / gs);
    return deq4x8(c, s2);
  }
}

// --------------------------------------------------------------- main kernel
template <typename AT, int D, int KVF>
__global__ __launch_bounds__(64) void paged_attn_kernel(const PagedArgs a) {
  constexpr int DQ = D / 4;         // d's per K-load lane
  constexpr int KSTEPS = D / 32;    // QK MFMAs per tile
  constexpr int DPL = D / 16;       // d's per output column lane (PV MFMAs per tile)
  static_assert(DPL == 8 || DPL == 4, "D must be 64 or 128");

  const int lane = threadIdx.x;
  const int r16 = lane & 15;
  const int kb = lane >> 4;
  const int s = blockIdx.x;
  const int hkv = blockIdx.y / a.HB;
  const int hb = blockIdx.y - hkv * a.HB;
  const int b = blockIdx.z;

  int len = a.lengths[b];
  const int max_s = a.MB * a.P;
  len = len < 0 ? 0 : (len > max_s ? max_s : len);
  const int nsplit = len == 0 ? 1 : (len + a.split_tok - 1) / a.split_tok;
  if (s >= nsplit) return;
  const int t_begin = s * a.split_tok;
  const int t_end = min(len, t_begin + a.split_tok);

  const int h0 = hkv * a.G + hb * 16;
  const int hcount = min(16, a.G - hb * 16);

  // q^T operand: lane (h = r16, kb) holds q[h][kb*DQ + 8j .. +8] for step j
  u32x4 qv[KSTEPS];
  {
    const bool hv = r16 < hcount;
    const AT* qp = reinterpret_cast<const AT*>(a.q) + ((size_t)b * a.Hq + h0 + (hv ? r16 : 0)) * D +
                   kb * DQ;
#pragma unroll
    for (int j = 0; j < KSTEPS; ++j) {
      qv[j] = hv ? qperm<KVF>(ldg128(qp + 8 * j)) : (u32x4){0u, 0u, 0u, 0u};
    }
  }

  float m_run = -INFINITY;  // per head h = r16 (replicated over kb)
  float l_run = 0.0f;
  f32x4 o[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) o[j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int32_t* btrow = a.bt + (size_t)b * a.MB;
  const int P = a.P;

  for (int tb = t_begin; tb < t_end; tb += 16 * kTilesPerBlock) {
    f32x4 sc[kTilesPerBlock];
    int pg[kTilesPerBlock];
    uint64_t vmask[kTilesPerBlock];
    u32x4 vv[kTilesPerBlock][4];

#pragma unroll
    for (int u = 0; u < kTilesPerBlock; ++u) {
      const int tt0 = tb + 16 * u;
      // K-load lane: position tt0 + r16, d in [kb*DQ, kb*DQ + DQ)
      const int t = tt0 + r16;
      int page = -1;
      if (t < t_end) page = btrow[t / P];
      const bool valid = page >= 0 && page < a.NP;
      pg[u] = valid ? page : -1;
      vmask[u] = __ballot(valid);
      const size_t row = valid ? ((size_t)page * P + (t % P)) * a.Hkv + hkv : 0;
      f32x4 acc = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KSTEPS; ++j) {
        const u32x4 kv = valid ? load8<AT, D, KVF>(a.K, a.Ks, row, kb * DQ + 8 * j, a.gs, a.ngroups)
                               : (u32x4){0u, 0u, 0u, 0u};
        acc = mfma_k32<AT>(kv, qv[j], acc);
      }
      sc[u] = acc;
      // V-load lane (column r16, kb): positions tt0 + 4kb + i, d in [r16*DPL, +DPL)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int src = 4 * kb + i;
        const int vp = __shfl(pg[u], src, 64);
        const int tv = tt0 + src;
        if (vp >= 0) {
          const size_t vrow = ((size_t)vp * P + (tv % P)) * a.Hkv + hkv;
          if constexpr (DPL == 8) {
            vv[u][i] = load8<AT, D, KVF>(a.V, a.Vs, vrow, r16 * 8, a.gs, a.ngroups);
          } else {
            // 4 d's per lane: natural order for every format
            if constexpr (KVF == 0) {
              const u32x2 x = ldg64(reinterpret_cast<const AT*>(a.V) + vrow * D + r16 * 4);
              vv[u][i] = (u32x4){x[0], x[1], 0u, 0u};
            } else {
              const uint16_t* sp = a.Vs + vrow * a.ngroups + (r16 * 4) / a.gs;
              const float sf = (float)bitcast<f16>(*sp);
              float w[4];
              if constexpr (KVF == 8) {
                const uint32_t c = *reinterpret_cast<const uint32_t*>(
                    reinterpret_cast<const uint8_t*>(a.V) + vrow * D + r16 * 4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  w[e] = (float)(f16)(((float)((c >> (8 * e)) & 255u) - 128.0f) * sf);
              } else {
                const uint16_t c = *reinterpret_cast<const uint16_t*>(
                    reinterpret_cast<const uint8_t*>(a.V) + vrow * (D / 2) + r16 * 2);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  w[e] = (float)(f16)(((float)((c >> (4 * e)) & 15u) - 8.0f) * sf);
              }
              vv[u][i] = (u32x4){pack_h2(w[0], w[1]), pack_h2(w[2], w[3]), 0u, 0u};
            }
          }
        } else {
          vv[u][i] = (u32x4){0u, 0u, 0u, 0u};
        }
      }
    }

    // ---- online softmax (base 2) over the block; lane holds S[h=r16][pos 4kb+i]
    float sv[kTilesPerBlock][4];
    float bmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < kTilesPerBlock; ++u) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = (vmask[u] >> (4 * kb + i)) & 1ull;
        sv[u][i] = ok ? sc[u][i] * a.scale_log2 : -INFINITY;
        bmax = fmaxf(bmax, sv[u][i]);
      }
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float m_new = fmaxf(m_run, bmax);
    const float alpha = (m_run == -INFINITY) ? 0.0f : exp2f(m_run - m_new);
    float psum = 0.0f;
    u32x2 pa[kTilesPerBlock];
#pragma unroll
    for (int u = 0; u < kTilesPerBlock; ++u) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = (sv[u][i] == -INFINITY) ? 0.0f : exp2f(sv[u][i] - m_new);
        psum += p[i];
      }
      pa[u] = (u32x2){pack_act2<AT>(p[0], p[1]), pack_act2<AT>(p[2], p[3])};
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // ---- rescale O: lane holds O[h = 4kb + i][col r16]
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) al[i] = __shfl(alpha, 4 * kb + i, 64);
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) o[j][i] *= al[i];
    }

    // ---- O += P . V
#pragma unroll
    for (int u = 0; u < kTilesPerBlock; ++u) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        // B operand: V[pos 4kb+i][d slot j] for i = 0..3
        const int w = j >> 1;
        const int sh = (j & 1) * 16;
        const uint32_t v0 = (vv[u][0][w] >> sh) & 0xFFFFu;
        const uint32_t v1 = (vv[u][1][w] >> sh) & 0xFFFFu;
        const uint32_t v2 = (vv[u][2][w] >> sh) & 0xFFFFu;
        const uint32_t v3 = (vv[u][3][w] >> sh) & 0xFFFFu;
        const u32x2 bop = {v0 | (v1 << 16), v2 | (v3 << 16)};
        o[j] = mfma_k16<AT>(pa[u], bop, o[j]);
      }
    }
  }

  // ---- write: lane holds O[h = 4kb + i][d = r16*DPL + slot j]
  float lv[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lv[i] = __shfl(l_run, 4 * kb + i, 64);
  if (nsplit == 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kb + i;
      if (h >= hcount) continue;
      const float inv = lv[i] > 0.0f ? 1.0f / lv[i] : 0.0f;
      AT* op = reinterpret_cast<AT*>(a.out) + ((size_t)b * a.Hq + h0 + h) * D + r16 * DPL;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = DPL == 8 ? dslot<KVF>(j) : j;
        op[d] = from_f32<AT>(o[j][i] * inv);
      }
    }
  } else {
    float mv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) mv[i] = __shfl(m_run, 4 * kb + i, 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * kb + i;
      if (h >= hcount) continue;
      const size_t slot = ((size_t)b * a.Hq + h0 + h) * a.s_max + s;
      float* po = a.ws + slot * (D + 2);
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = DPL == 8 ? dslot<KVF>(j) : j;
        po[r16 * DPL + d] = o[j][i];
      }
      if (r16 == 0) {
        po[D] = mv[i];
        po[D + 1] = lv[i];
      }
    }
  }
}

// LSE merge of the split partials of one (sequence, head): one wave, lanes over d.
template <typename AT>
__global__ __launch_bounds__(64) void paged_attn_merge_kernel(const PagedArgs a, int D) {
  const int bh = blockIdx.x;
  const int b = bh / a.Hq;
  int len = a.lengths[b];
  const int max_s = a.MB * a.P;
  len = len < 0 ? 0 : (len > max_s ? max_s : len);
  const int nsplit = len == 0 ? 1 : (len + a.split_tok - 1) / a.split_tok;
  if (nsplit <= 1) return;
  const float* base = a.ws + (size_t)bh * a.s_max * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, base[(size_t)s * (D + 2) + D]);
  float L = 0.0f;
  for (int s = 0; s < nsplit; ++s) {
    const float* p = base + (size_t)s * (D + 2);
    const float m = p[D];
    if (m != -INFINITY) L += p[D + 1] * exp2f(m - M);
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  AT* op = reinterpret_cast<AT*>(a.out) + (size_t)bh * D;
  for (int d = threadIdx.x; d < D; d += 64) {
    float acc = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
      const float* p = base + (size_t)s * (D + 2);
      const float m = p[D];
      if (m != -INFINITY) acc += p[d] * exp2f(m - M);
    }
    op[d] = from_f32<AT>(acc * inv);
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
  const AT* qp = reinterpret_cast<const AT*>(a.q) + (size_t)bh * D;
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
  AT* op = reinterpret_cast<AT*>(a.out) + (size_t)bh * D;
#pragma unroll
  for (int k = 0; k < MAXPL; ++k) {
    const int d = threadIdx.x + 64 * k;
    if (d < D) op[d] = from_f32<AT>(acc[k] * inv);
  }
}

// --------------------------------------------------------------- host side
// Positions per split: aim for ~16 waves per CU over the worst-case context.
inline int choose_split_tokens(int64_t B, int64_t Hq, int64_t Hkv, int64_t max_ctx) {
  const int64_t hb = ((Hq / (Hkv > 0 ? Hkv : 1)) + 15) / 16;
  const int64_t units = B * Hkv * (hb > 0 ? hb : 1);
  const int64_t target_waves = 4096;
  int64_t st = (max_ctx * units + target_waves - 1) / target_waves;
  const int64_t blk = 16 * kTilesPerBlock;
  st = (st + blk - 1) / blk * blk;
  if (st < 64) st = 64;
  if (st > max_ctx) st = (max_ctx + blk - 1) / blk * blk;
  return (int)st;
}

inline bool fast_ok(int64_t D, int kvf, int dtype, int64_t gs) {
  if (!(D == 64 || D == 128)) return false;
  if (kvf != 0) {
    if (dtype != MK_DT_F16) return false;
    // one scale per 8 (K) / per lane's d-run (V): group must cover them
    if (gs < 8 || (gs & (gs - 1))) return false;
  }
  return true;
}

int attention_launch(PagedArgs a, int64_t D, int kvf, int dtype, size_t ws_bytes,
                     hipStream_t st) {
  const int64_t max_ctx = (int64_t)a.MB * a.P;
  a.split_tok = choose_split_tokens(a.B, a.Hq, a.Hkv, max_ctx);
  a.s_max = (int)((max_ctx + a.split_tok - 1) / a.split_tok);
  if (a.s_max < 1) a.s_max = 1;
  const bool fast = fast_ok(D, kvf, dtype, a.gs);
  if (fast && a.s_max > 1) {
    const size_t need = (size_t)a.B * a.Hq * a.s_max * (D + 2) * sizeof(float);
    if (!a.ws || ws_bytes < need) return MK_ERR_INVALID;
  }
  if (fast) {
    const dim3 grid((unsigned)a.s_max, (unsigned)(a.Hkv * a.HB), (unsigned)a.B);
#define MK_PA(AT, DD, KF) paged_attn_kernel<AT, DD, KF><<<grid, 64, 0, st>>>(a)
    if (kvf == 0) {
      if (dtype == MK_DT_F16) {
        if (D == 128) MK_PA(f16, 128, 0); else MK_PA(f16, 64, 0);
      } else {
        if (D == 128) MK_PA(bf16, 128, 0); else MK_PA(bf16, 64, 0);
      }
    } else if (kvf == 8) {
      if (D == 128) MK_PA(f16, 128, 8); else MK_PA(f16, 64, 8);
    } else {
      if (D == 128) MK_PA(f16, 128, 4); else MK_PA(f16, 64, 4);
    }
#undef MK_PA
    MK_CHECK_LAUNCH();
    if (a.s_max > 1) {
      const dim3 mgrid((unsigned)(a.B * a.Hq));
      if (dtype == MK_DT_F16)
        paged_attn_merge_kernel<f16><<<mgrid, 64, 0, st>>>(a, (int)D);
      else
        paged_attn_merge_kernel<bf16><<<mgrid, 64, 0, st>>>(a, (int)D);
      MK_CHECK_LAUNCH();
    }
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

}  // namespace

extern "C" {

size_t mk_paged_attention_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                          int64_t max_blocks, int64_t page_size) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || max_blocks <= 0 || page_size <= 0) return 0;
  const int64_t max_ctx = max_blocks * page_size;
  const int st = choose_split_tokens(B, Hq, Hkv, max_ctx);
  const int64_t s_max = (max_ctx + st - 1) / st;
  if (s_max <= 1) return 0;
  return (size_t)B * Hq * s_max * (D + 2) * sizeof(float);
}

int mk_paged_decode_attention(const void* q, const void* K_pages, const void* V_pages,
                              const int32_t* block_table, const int32_t* lengths, void* out,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t page_size,
                              int64_t max_blocks, int64_t num_pages, float scale, int dtype,
                              void* workspace, size_t workspace_bytes, void* stream) {
  MK_REQUIRE(q && K_pages && V_pages && block_table && lengths && out);
  MK_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && (Hq % Hkv) == 0 && D > 0 && page_size > 0);
  MK_REQUIRE(max_blocks > 0 && num_pages > 0 && num_pages < (1LL << 31));
  MK_REQUIRE(B < 65536 && max_blocks * page_size < (1LL << 31));
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  if (B == 0) return MK_OK;
  PagedArgs a = {};
  a.q = q;
  a.K = K_pages;
  a.V = V_pages;
  a.bt = block_table;
  a.lengths = lengths;
  a.out = out;
  a.ws = reinterpret_cast<float*>(workspace);
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
  return attention_launch(a, D, 0, dtype, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int mk_paged_quantized_decode_attention(const void* q, const uint8_t* K_q, const uint8_t* V_q,
                                        const f16_storage_t* K_s, const f16_storage_t* V_s,
                                        const int32_t* block_table, const int32_t* lengths,
                                        void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t page_size, int64_t max_blocks, int64_t num_pages,
                                        int64_t group_size, int bits, float scale, int dtype,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  MK_REQUIRE(q && K_q && V_q && K_s && V_s && block_table && lengths && out);
  MK_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && (Hq % Hkv) == 0 && D > 0 && page_size > 0);
  MK_REQUIRE(max_blocks > 0 && num_pages > 0 && num_pages < (1LL << 31) && group_size > 0);
  MK_REQUIRE(B < 65536 && max_blocks * page_size < (1LL << 31));
  MK_REQUIRE(bits == 4 || bits == 8);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  if (B == 0) return MK_OK;
  PagedArgs a = {};
  a.q = q;
  a.K = K_q;
  a.V = V_q;
  a.Ks = K_s;
  a.Vs = V_s;
  a.bt = block_table;
  a.lengths = lengths;
  a.out = out;
  a.ws = reinterpret_cast<float*>(workspace);
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
  return attention_launch(a, D, bits, dtype, workspace_bytes,
                          reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"
