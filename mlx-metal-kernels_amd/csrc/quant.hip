// q4 pack/unpack and groupwise dequant (bit-exact).
//
// pack_q4 / unpack_q4_reference: ops/quant_ops.py:166-188.
// dequant_q4 / dequant_q8:       ops/quant_ops.py:191-316 -- the product
//   (q - z) * s is formed in fp32 and rounded once (RNE) into the output type,
//   exactly as the reference's fp32 expression followed by astype().
// Every kernel walks 16-byte (q8/unpack) or 8-byte (q4) runs of codes per
// thread so HBM traffic is coalesced; rows are independent.
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

}  // namespace

extern "C" {

int mk_abi_version(void) { return 1; }

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

}  // extern "C"
