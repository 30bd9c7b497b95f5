// q4 pack/unpack and groupwise dequant (bit-exact).
//
// pack_q4 / unpack_q4_reference: ops/quant_ops.py:166-188.
// dequant_q4 / dequant_q8:       ops/quant_ops.py:191-316 -- the product
//   (q - z) * s is formed in fp32 and rounded once (RNE) into the output type,
//   exactly as the reference's fp32 expression followed by astype().
// Every kernel walks 16-byte (q8/unpack) or 8-byte (q4) runs of codes per
// thread so HBM traffic is coalesced; rows are independent.
//
// quantize_weight_groupwise: models/quantize_weights.py:164-203 -- symmetric
//   absmax per group: scale = max(max|w| / limit, eps) in double, codes
//   clip(rint(w / float(scale)), +-limit) + 8|128 (fp32 divide correctly
//   rounded, round-half-even), the scale stored in the scale dtype after use.
#include "common.h"

namespace {

__global__ void pack_q4_kernel(const uint8_t* __restrict__ q, uint8_t* __restrict__ packed,
                               int64_t rows, int64_t K) {
  const int64_t kp = (K + 1) / 2;
  const int64_t total = rows * kp;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / kp, j = i - r * kp;
    const uint8_t* row = q + r * K;
    const uint32_t lo = row[2 * j] & 0xFFu;
    const uint32_t hi = (2 * j + 1 < K) ? row[2 * j + 1] : 0u;
    // uint8 arithmetic wraps exactly like the reference's uint8 add/shift
    packed[i] = (uint8_t)((lo + (hi << 4)) & 0xFFu);
  }
}

__global__ void unpack_q4_kernel(const uint8_t* __restrict__ packed, uint8_t* __restrict__ q,
                                 int64_t rows, int64_t kp, int64_t kout) {
  const int64_t total = rows * kout;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / kout, k = i - r * kout;
    const uint8_t b = packed[r * kp + (k >> 1)];
    q[i] = (k & 1) ? (uint8_t)((b >> 4) & 15u) : (uint8_t)(b & 15u);
  }
}

template <int BITS, typename ST, typename OT>
__global__ void dequant_kernel(const uint8_t* __restrict__ codes, const ST* __restrict__ scales,
                               const ST* __restrict__ zeros, OT* __restrict__ out, int64_t rows,
                               int64_t K, int64_t gs, int64_t G) {
  // each thread produces 8 consecutive outputs of one row (K % 8 handled by tail check)
  const int64_t per_row = (K + 7) / 8;
  const int64_t total = rows * per_row;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row;
    const int64_t k0 = (i - r * per_row) * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t k = k0 + e;
      if (k >= K) break;
      uint32_t q;
      if constexpr (BITS == 4) {
        const uint8_t b = codes[r * (K / 2) + (k >> 1)];
        q = (k & 1) ? (b >> 4) : (b & 15u);
      } else {
        q = codes[r * K + k];
      }
      const int64_t g = k / gs;
      const float s = to_f32(scales[r * G + g]);
      const float w = zeros ? ((float)q - to_f32(zeros[r * G + g])) * s : (float)q * s;
      out[r * K + k] = from_f32<OT>(w);
    }
  }
}

inline dim3 grid_for(int64_t work, int threads) {
  int64_t b = (work + threads - 1) / threads;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return dim3((unsigned)b);
}

template <int BITS>
int dequant_entry(const uint8_t* codes, const void* s, const void* z, void* out, int64_t rows,
                  int64_t K, int64_t gs, int sdt, int odt, void* stream) {
  MK_REQUIRE(codes && s && out && rows >= 0 && K >= 0 && gs > 0);
  MK_REQUIRE(sdt == MK_DT_F16 || sdt == MK_DT_F32);
  MK_REQUIRE(odt == MK_DT_F16 || odt == MK_DT_BF16);
  if (rows == 0 || K == 0) return MK_OK;
  const int64_t G = (K + gs - 1) / gs;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid = grid_for(rows * ((K + 7) / 8), 256);
#define MK_DQ(ST, OT)                                                                            \
  dequant_kernel<BITS, ST, OT><<<grid, 256, 0, st>>>(codes, (const ST*)s, (const ST*)z, (OT*)out, \
                                                     rows, K, gs, G)
  if (sdt == MK_DT_F16 && odt == MK_DT_F16) MK_DQ(f16, f16);
  else if (sdt == MK_DT_F16) MK_DQ(f16, bf16);
  else if (odt == MK_DT_F16) MK_DQ(float, f16);
  else MK_DQ(float, bf16);
#undef MK_DQ
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// One group's quantization; `put(k, code)` stores code of column k.
template <typename WT, typename PUT>
__device__ __forceinline__ float quantize_group(const WT* __restrict__ w, int64_t k0, int64_t k1,
                                                int limit, int zp, double eps, PUT put) {
  float amax = 0.0f;
  for (int64_t k = k0; k < k1; ++k) amax = fmaxf(amax, fabsf(to_f32(w[k])));
  double sd = (double)amax / (double)limit;
  if (sd < eps) sd = eps;
  const float s = (float)sd;
  const float lim = (float)limit;
  for (int64_t k = k0; k < k1; ++k) {
    float qv = rintf(to_f32(w[k]) / s);
    qv = fminf(fmaxf(qv, -lim), lim);
    put(k, (uint32_t)((int)qv + zp));
  }
  return s;
}

// Thread per (row, group).  q4 needs an even group size here, so the two
// nibbles of a byte always come from the same group (same thread).
template <typename WT, typename ST, int BITS>
__global__ void quantize_weight_kernel(const WT* __restrict__ w, uint8_t* __restrict__ codes,
                                       ST* __restrict__ scales, int64_t rows, int64_t K, int64_t gs,
                                       int64_t G, double eps) {
  constexpr int limit = BITS == 4 ? 7 : 127;
  constexpr int zp = BITS == 4 ? 8 : 128;
  const int64_t kp = BITS == 4 ? (K + 1) / 2 : K;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < rows * G;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / G, g = i - r * G;
    const int64_t k0 = g * gs, k1 = min(K, k0 + gs);
    const WT* wr = w + r * K;
    uint8_t* cr = codes + r * kp;
    uint32_t lo = 0;
    const float s = quantize_group(wr, k0, k1, limit, zp, eps, [&](int64_t k, uint32_t c) {
      if constexpr (BITS == 8) {
        cr[k] = (uint8_t)c;
      } else if ((k & 1) == 0) {
        lo = c;
        if (k + 1 == K) cr[k >> 1] = (uint8_t)lo;  // odd K: the pad nibble is 0
      } else {
        cr[k >> 1] = (uint8_t)(lo | (c << 4));
      }
    });
    scales[i] = from_f32<ST>(s);
  }
}

// q4 with an odd group size: a byte can straddle two groups, so one thread
// walks a whole row.
template <typename WT, typename ST>
__global__ void quantize_weight_q4_rows_kernel(const WT* __restrict__ w, uint8_t* __restrict__ codes,
                                               ST* __restrict__ scales, int64_t rows, int64_t K,
                                               int64_t gs, int64_t G, double eps) {
  const int64_t kp = (K + 1) / 2;
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < rows;
       r += (int64_t)gridDim.x * blockDim.x) {
    const WT* wr = w + r * K;
    uint8_t* cr = codes + r * kp;
    uint32_t lo = 0;
    for (int64_t g = 0; g < G; ++g) {
      const int64_t k0 = g * gs, k1 = min(K, k0 + gs);
      const float s = quantize_group(wr, k0, k1, 7, 8, eps, [&](int64_t k, uint32_t c) {
        if ((k & 1) == 0) {
          lo = c;
          if (k + 1 == K) cr[k >> 1] = (uint8_t)lo;
        } else {
          cr[k >> 1] = (uint8_t)(lo | (c << 4));
        }
      });
      scales[r * G + g] = from_f32<ST>(s);
    }
  }
}

template <typename WT, typename ST>
int quantize_weight_launch(const void* w, uint8_t* codes, void* scales, int64_t rows, int64_t K,
                           int64_t gs, int bits, double eps, hipStream_t st) {
  const int64_t G = (K + gs - 1) / gs;
  if (bits == 8) {
    quantize_weight_kernel<WT, ST, 8><<<grid_for(rows * G, 256), 256, 0, st>>>(
        (const WT*)w, codes, (ST*)scales, rows, K, gs, G, eps);
  } else if (gs % 2 == 0) {
    quantize_weight_kernel<WT, ST, 4><<<grid_for(rows * G, 256), 256, 0, st>>>(
        (const WT*)w, codes, (ST*)scales, rows, K, gs, G, eps);
  } else {
    quantize_weight_q4_rows_kernel<WT, ST><<<grid_for(rows, 64), 64, 0, st>>>(
        (const WT*)w, codes, (ST*)scales, rows, K, gs, G, eps);
  }
  MK_CHECK_LAUNCH();
  return MK_OK;
}

}  // namespace

extern "C" {

int mk_abi_version(void) { return 2; }

int mk_pack_q4(const uint8_t* q, uint8_t* packed, int64_t rows, int64_t K, void* stream) {
  MK_REQUIRE(q && packed && rows >= 0 && K >= 0);
  if (rows == 0 || K == 0) return MK_OK;
  const int64_t work = rows * ((K + 1) / 2);
  pack_q4_kernel<<<grid_for(work, 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      q, packed, rows, K);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_unpack_q4(const uint8_t* packed, uint8_t* q, int64_t rows, int64_t k_packed, int64_t k_out,
                 void* stream) {
  MK_REQUIRE(packed && q && rows >= 0 && k_packed >= 0 && k_out >= 0 && k_out <= 2 * k_packed);
  if (rows == 0 || k_out == 0) return MK_OK;
  unpack_q4_kernel<<<grid_for(rows * k_out, 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      packed, q, rows, k_packed, k_out);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_dequant_q4(const uint8_t* packed, const void* scales, const void* zeros, void* out,
                  int64_t rows, int64_t k_packed, int64_t group_size, int scale_dtype,
                  int out_dtype, void* stream) {
  return dequant_entry<4>(packed, scales, zeros, out, rows, 2 * k_packed, group_size, scale_dtype,
                          out_dtype, stream);
}

int mk_dequant_q8(const uint8_t* q, const void* scales, const void* zeros, void* out, int64_t rows,
                  int64_t K, int64_t group_size, int scale_dtype, int out_dtype, void* stream) {
  return dequant_entry<8>(q, scales, zeros, out, rows, K, group_size, scale_dtype, out_dtype,
                          stream);
}

int mk_quantize_weight(const void* weight, uint8_t* codes, void* scales, int64_t rows, int64_t K,
                       int64_t group_size, int bits, double eps, int w_dtype, int scale_dtype,
                       void* stream) {
  MK_REQUIRE(weight && codes && scales && rows >= 0 && K >= 0 && group_size > 0 && eps > 0.0);
  MK_REQUIRE(bits == 4 || bits == 8);
  MK_REQUIRE(w_dtype == MK_DT_F16 || w_dtype == MK_DT_BF16 || w_dtype == MK_DT_F32);
  MK_REQUIRE(scale_dtype == MK_DT_F16 || scale_dtype == MK_DT_BF16 || scale_dtype == MK_DT_F32);
  if (rows == 0 || K == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define MK_QW(WT)                                                                              \
  do {                                                                                         \
    if (scale_dtype == MK_DT_F16)                                                              \
      return quantize_weight_launch<WT, f16>(weight, codes, scales, rows, K, group_size, bits, \
                                             eps, st);                                         \
    if (scale_dtype == MK_DT_BF16)                                                             \
      return quantize_weight_launch<WT, bf16>(weight, codes, scales, rows, K, group_size,      \
                                              bits, eps, st);                                  \
    return quantize_weight_launch<WT, float>(weight, codes, scales, rows, K, group_size, bits, \
                                             eps, st);                                         \
  } while (0)
  if (w_dtype == MK_DT_F32) MK_QW(float);
  if (w_dtype == MK_DT_F16) MK_QW(f16);
  MK_QW(bf16);
#undef MK_QW
}

}  // extern "C"
