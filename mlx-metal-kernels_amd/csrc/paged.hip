// Paged KV-cache plumbing for one decode token per sequence.
//
// block_table_lookup    ops/paged_kv_ops.py:138-182
// paged_kv_cache_update ops/paged_kv_ops.py:185-255 -- done in place: only the
//   B*H*D target elements move (O(token), not O(cache)).
// fused qkv split + interleaved RoPE + paged update -- the composition
//   paged_gqa_decode_block_from_qkv runs (ops/gqa_ops.py:493-547):
//   reference_gqa_qkv_split_rope (ops/gqa_ops.py:118-160, ops/rope_ops.py:61-75)
//   then the paged scatter; the quantized variant applies the symmetric
//   per-group quantizers of ops/paged_quantized_kv_ops.py:146-175 to the
//   rounded k_rope / v before the scatter.
// Collisions (two sequences targeting one slot) resolve to the later sequence,
// as the reference's loop over b does: a sequence skips its cache write when a
// later sequence targets the same (page, offset).
#include "common.h"
#include "paged_common.h"

namespace {

__global__ void block_table_lookup_kernel(const int32_t* __restrict__ bt,
                                          const int32_t* __restrict__ pos, int32_t* page_ids,
                                          int32_t* offsets, int B, int max_blocks, int P) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int p = pos[b];
  const int blk = p / P;
  page_ids[b] = (p >= 0 && blk < max_blocks) ? bt[(size_t)b * max_blocks + blk] : -1;
  offsets[b] = p % P;
}

// One workgroup per sequence; threads copy the H*D token vector.
template <typename T>
__global__ void paged_update_kernel(T* __restrict__ Kp, T* __restrict__ Vp,
                                    const T* __restrict__ k, const T* __restrict__ v,
                                    const int32_t* __restrict__ bt, const int32_t* __restrict__ pos,
                                    int B, int H, int D, int P, int max_blocks, int num_pages) {
  const int b = blockIdx.x;
  int off;
  const int page = slot_page(bt, pos, b, max_blocks, P, num_pages, &off);
  if (page < 0) return;
  if (superseded(bt, pos, b, B, max_blocks, P, num_pages, page, off)) return;
  const size_t dst = ((size_t)page * P + off) * H * D;
  const size_t src = (size_t)b * H * D;
  const int n = H * D;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    Kp[dst + i] = k[src + i];
    Vp[dst + i] = v[src + i];
  }
}

// qkv row layout: [Q (Hq*D) | K (Hkv*D) | V (Hkv*D)]
template <typename T>
__global__ __launch_bounds__(256) void qkv_rope_update_kernel(
    const T* __restrict__ qkv, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int32_t* __restrict__ pos, const int32_t* __restrict__ bt, T* __restrict__ Kp,
    T* __restrict__ Vp, T* __restrict__ q_out, int B, int Hq, int Hkv, int D, int P,
    int max_blocks, int num_pages, int cos_rows) {
  const int b = blockIdx.x;
  const int p = pos[b];
  if (p < 0 || p >= cos_rows) return;
  const int half = D / 2;
  const T* row = qkv + (size_t)b * (Hq + 2 * Hkv) * D;
  const float* cr = cos_t + (size_t)p * half;
  const float* sr = sin_t + (size_t)p * half;
  // q
  for (int i = threadIdx.x; i < Hq * half; i += blockDim.x) {
    const int h = i / half, j = i - h * half;
    float ye, yo;
    rope_pair(to_f32(row[h * D + 2 * j]), to_f32(row[h * D + 2 * j + 1]), cr[j], sr[j], &ye, &yo);
    T* qo = q_out + ((size_t)b * Hq + h) * D;
    qo[2 * j] = from_f32<T>(ye);
    qo[2 * j + 1] = from_f32<T>(yo);
  }
  int off;
  const int page = slot_page(bt, pos, b, max_blocks, P, num_pages, &off);
  if (page < 0) return;
  if (superseded(bt, pos, b, B, max_blocks, P, num_pages, page, off)) return;
  const size_t dst = ((size_t)page * P + off) * Hkv * D;
  const T* krow = row + (size_t)Hq * D;
  const T* vrow = krow + (size_t)Hkv * D;
  for (int i = threadIdx.x; i < Hkv * half; i += blockDim.x) {
    const int h = i / half, j = i - h * half;
    float ye, yo;
    rope_pair(to_f32(krow[h * D + 2 * j]), to_f32(krow[h * D + 2 * j + 1]), cr[j], sr[j], &ye,
              &yo);
    Kp[dst + h * D + 2 * j] = from_f32<T>(ye);
    Kp[dst + h * D + 2 * j + 1] = from_f32<T>(yo);
  }
  for (int i = threadIdx.x; i < Hkv * D; i += blockDim.x) Vp[dst + i] = vrow[i];
}

// Vectorised form of qkv_rope_update_kernel for D % 8 == 0 and 16-byte
// aligned rows: one thread per 8 elements (four RoPE pairs, one 16-byte load
// and store), the q, k and v tasks of a sequence spread over
// ceil(tasks / 128) workgroups so a small batch still fills several CUs.
// Same arithmetic and the same skip rules as the scalar kernel.
constexpr int kRopeSlotMax = 1024;  // batch rows whose slots a workgroup stages in LDS

template <typename T>
__global__ __launch_bounds__(128) void qkv_rope_update_vec_kernel(
    const T* __restrict__ qkv, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int32_t* __restrict__ pos, const int32_t* __restrict__ bt, T* __restrict__ Kp,
    T* __restrict__ Vp, T* __restrict__ q_out, int B, int Hq, int Hkv, int D, int P,
    int max_blocks, int num_pages, int cos_rows, bool stage_slots) {
  const int b = blockIdx.x;
  const int cpr = D / 8;  // 8-element chunks per head row
  const int nq = Hq * cpr, nk = Hkv * cpr;
  const int t = (int)blockIdx.y * 128 + (int)threadIdx.x;
  // every row's cache slot (page * P + offset, -1 when skipped), looked up once
  // per workgroup with independent loads: the collision rule then reads LDS
  // instead of walking the later rows' block-table entries one by one
  __shared__ int slot_lds[kRopeSlotMax];
  if (stage_slots) {  // workgroup-uniform
    for (int r = threadIdx.x; r < B; r += blockDim.x) {
      int o;
      const int pg = slot_page(bt, pos, r, max_blocks, P, num_pages, &o);
      slot_lds[r] = pg < 0 ? -1 : pg * P + o;
    }
    __syncthreads();
  }
  if (t >= nq + 2 * nk) return;
  const int p = pos[b];
  if (p < 0 || p >= cos_rows) return;
  // this row's slot unless out of range or taken by a later row
  auto my_slot = [&](int* page, int* off) {
    if (stage_slots) {
      const int sl = slot_lds[b];
      if (sl < 0) return false;
      for (int b2 = b + 1; b2 < B; ++b2)
        if (slot_lds[b2] == sl) return false;
      *page = sl / P;
      *off = sl - *page * P;
      return true;
    }
    *page = slot_page(bt, pos, b, max_blocks, P, num_pages, off);
    return *page >= 0 && !superseded(bt, pos, b, B, max_blocks, P, num_pages, *page, *off);
  };
  const T* row = qkv + (size_t)b * (Hq + 2 * Hkv) * D;
  if (t < nq + nk) {
    const bool isq = t < nq;
    const int tt = isq ? t : t - nq;
    const int h = tt / cpr, c = tt - h * cpr;
    const u32x4 xv = ldg128(row + (isq ? 0 : (size_t)Hq * D) + (size_t)h * D + 8 * c);
    const u32x4 cv = ldg128(cos_t + (size_t)p * (D / 2) + 4 * c);
    const u32x4 sv = ldg128(sin_t + (size_t)p * (D / 2) + 4 * c);
    T xe[8], ye8[8];
    float ce[4], se[4];
    __builtin_memcpy(xe, &xv, 16);
    __builtin_memcpy(ce, &cv, 16);
    __builtin_memcpy(se, &sv, 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float ye, yo;
      rope_pair(to_f32(xe[2 * e]), to_f32(xe[2 * e + 1]), ce[e], se[e], &ye, &yo);
      ye8[2 * e] = from_f32<T>(ye);
      ye8[2 * e + 1] = from_f32<T>(yo);
    }
    u32x4 yv;
    __builtin_memcpy(&yv, ye8, 16);
    if (isq) {
      *reinterpret_cast<u32x4*>(q_out + ((size_t)b * Hq + h) * D + 8 * c) = yv;
      return;
    }
    int page, off;
    if (!my_slot(&page, &off)) return;
    *reinterpret_cast<u32x4*>(Kp + ((size_t)page * P + off) * Hkv * D + (size_t)h * D + 8 * c) = yv;
    return;
  }
  const int tt = t - nq - nk;  // v chunk
  int page, off;
  if (!my_slot(&page, &off)) return;
  *reinterpret_cast<u32x4*>(Vp + ((size_t)page * P + off) * Hkv * D + 8 * (size_t)tt) =
      ldg128(row + (size_t)(Hq + Hkv) * D + 8 * (size_t)tt);
}

// Quantized variant.  LDS holds the rounded k_rope / v (as fp32) and the
// codes; one wave quantizes one (K|V, head, group) at a time.
constexpr int QUPD_MAX_ELEMS = 4096;  // Hkv * D per K or V

template <typename T, int BITS>
__global__ __launch_bounds__(256) void qkv_rope_update_quant_kernel(
    const T* __restrict__ qkv, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const int32_t* __restrict__ pos, const int32_t* __restrict__ bt, uint8_t* __restrict__ Kq,
    uint8_t* __restrict__ Vq, uint16_t* __restrict__ Ks, uint16_t* __restrict__ Vs,
    T* __restrict__ q_out, int B, int Hq, int Hkv, int D, int P, int max_blocks, int num_pages,
    int cos_rows, int gs) {
  __shared__ float vals[2][QUPD_MAX_ELEMS];
  __shared__ uint8_t codes[2][QUPD_MAX_ELEMS];
  const int b = blockIdx.x;
  const int p = pos[b];
  if (p < 0 || p >= cos_rows) return;
  const int half = D / 2;
  const T* row = qkv + (size_t)b * (Hq + 2 * Hkv) * D;
  const float* cr = cos_t + (size_t)p * half;
  const float* sr = sin_t + (size_t)p * half;
  for (int i = threadIdx.x; i < Hq * half; i += blockDim.x) {
    const int h = i / half, j = i - h * half;
    float ye, yo;
    rope_pair(to_f32(row[h * D + 2 * j]), to_f32(row[h * D + 2 * j + 1]), cr[j], sr[j], &ye, &yo);
    T* qo = q_out + ((size_t)b * Hq + h) * D;
    qo[2 * j] = from_f32<T>(ye);
    qo[2 * j + 1] = from_f32<T>(yo);
  }
  int off;
  const int page = slot_page(bt, pos, b, max_blocks, P, num_pages, &off);
  if (page < 0) return;  // uniform across the workgroup
  if (superseded(bt, pos, b, B, max_blocks, P, num_pages, page, off)) return;

  const T* krow = row + (size_t)Hq * D;
  const T* vrow = krow + (size_t)Hkv * D;
  for (int i = threadIdx.x; i < Hkv * half; i += blockDim.x) {
    const int h = i / half, j = i - h * half;
    float ye, yo;
    rope_pair(to_f32(krow[h * D + 2 * j]), to_f32(krow[h * D + 2 * j + 1]), cr[j], sr[j], &ye,
              &yo);
    vals[0][h * D + 2 * j] = to_f32(from_f32<T>(ye));
    vals[0][h * D + 2 * j + 1] = to_f32(from_f32<T>(yo));
  }
  for (int i = threadIdx.x; i < Hkv * D; i += blockDim.x) vals[1][i] = to_f32(vrow[i]);
  __syncthreads();

  const float qmax = BITS == 8 ? 127.0f : 7.0f;
  const float qoff = BITS == 8 ? 128.0f : 8.0f;
  const int G = (D + gs - 1) / gs;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const size_t sbase = ((size_t)page * P + off) * Hkv * G;
  for (int it = wave; it < 2 * Hkv * G; it += nw) {
    const int kv = it / (Hkv * G);
    const int h = (it / G) % Hkv;
    const int g = it % G;
    const int e0 = g * gs;
    const int e1 = min(e0 + gs, D);
    const float* src = &vals[kv][h * D];
    float amax = 0.0f;
    for (int e = e0 + lane; e < e1; e += 64) amax = fmaxf(amax, fabsf(src[e]));
    amax = wave_max(amax);
    amax = fmaxf(amax, 1e-8f);
    const float scale = amax / qmax;  // correctly rounded fp32 division
    for (int e = e0 + lane; e < e1; e += 64) {
      float qv = rintf(src[e] / scale);
      qv = fminf(fmaxf(qv, -qmax), qmax);
      codes[kv][h * D + e] = (uint8_t)(int)(qv + qoff);
    }
    if (lane == 0) {
      uint16_t* sdst = kv == 0 ? Ks : Vs;
      sdst[sbase + (size_t)h * G + g] = bitcast<uint16_t>((f16)scale);
    }
  }
  __syncthreads();
  if constexpr (BITS == 8) {
    const size_t dst = ((size_t)page * P + off) * Hkv * D;
    for (int i = threadIdx.x; i < Hkv * D; i += blockDim.x) {
      Kq[dst + i] = codes[0][i];
      Vq[dst + i] = codes[1][i];
    }
  } else {
    const int dp = (D + 1) / 2;
    const size_t dst = ((size_t)page * P + off) * Hkv * dp;
    for (int i = threadIdx.x; i < Hkv * dp; i += blockDim.x) {
      const int h = i / dp, j = i - h * dp;
      const int e = h * D + 2 * j;
      const bool has_hi = 2 * j + 1 < D;
      Kq[dst + i] = (uint8_t)(codes[0][e] | ((has_hi ? codes[0][e + 1] : 0) << 4));
      Vq[dst + i] = (uint8_t)(codes[1][e] | ((has_hi ? codes[1][e + 1] : 0) << 4));
    }
  }
}

// Bulk symmetric quantization of KV rows (every page, slot and kv head):
// ops/paged_quantized_kv_ops.py:194-292 applied to rows of D values.  One
// thread per row walks its groups; q4 codes are packed as they are produced,
// pairs straddling a group boundary included.
template <typename T, int BITS>
__global__ void quantize_kv_rows_kernel(const T* __restrict__ src, uint8_t* __restrict__ codes,
                                        uint16_t* __restrict__ scales, int64_t rows, int D,
                                        int gs) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float qmax = BITS == 8 ? 127.0f : 7.0f;
  const float qoff = BITS == 8 ? 128.0f : 8.0f;
  const int G = (D + gs - 1) / gs;
  const T* row = src + r * D;
  uint8_t* out = codes + r * (BITS == 8 ? D : (D + 1) / 2);
  uint16_t* srow = scales + r * G;
  uint32_t pending = 0;
  for (int g = 0; g < G; ++g) {
    const int e0 = g * gs, e1 = min(e0 + gs, D);
    float amax = 0.0f;
    for (int e = e0; e < e1; ++e) amax = fmaxf(amax, fabsf(to_f32(row[e])));
    amax = fmaxf(amax, 1e-8f);
    const float scale = amax / qmax;  // correctly rounded fp32 division
    srow[g] = bitcast<uint16_t>((f16)scale);
    for (int e = e0; e < e1; ++e) {
      float qv = rintf(to_f32(row[e]) / scale);
      qv = fminf(fmaxf(qv, -qmax), qmax);
      const uint32_t c = (uint32_t)(int)(qv + qoff);
      if constexpr (BITS == 8) {
        out[e] = (uint8_t)c;
      } else if (e & 1) {
        out[e >> 1] = (uint8_t)(pending | (c << 4));
      } else {
        pending = c;
      }
    }
  }
  if constexpr (BITS == 4) {
    if (D & 1) out[D >> 1] = (uint8_t)pending;
  }
}

}  // namespace

extern "C" {

int mk_quantize_kv(const void* src, uint8_t* codes, f16_storage_t* scales, int64_t rows, int64_t D,
                   int64_t group_size, int bits, int dtype, void* stream) {
  MK_REQUIRE(src && codes && scales && rows >= 0 && D > 0 && group_size > 0);
  MK_REQUIRE(bits == 4 || bits == 8);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  MK_REQUIRE(D < (1 << 20));
  if (rows == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((rows + 255) / 256));
#define MK_QKV(T, BB)                                                                 \
  quantize_kv_rows_kernel<T, BB><<<grid, 256, 0, st>>>((const T*)src, codes, scales, rows, \
                                                       (int)D, (int)group_size)
  if (dtype == MK_DT_F16) {
    if (bits == 8) MK_QKV(f16, 8);
    else MK_QKV(f16, 4);
  } else {
    if (bits == 8) MK_QKV(bf16, 8);
    else MK_QKV(bf16, 4);
  }
#undef MK_QKV
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_block_table_lookup(const int32_t* block_table, const int32_t* positions, int32_t* page_ids,
                          int32_t* offsets, int64_t B, int64_t max_blocks, int64_t page_size,
                          void* stream) {
  MK_REQUIRE(block_table && positions && page_ids && offsets);
  MK_REQUIRE(B >= 0 && max_blocks > 0 && page_size > 0 && B < (1 << 30));
  if (B == 0) return MK_OK;
  block_table_lookup_kernel<<<(unsigned)((B + 255) / 256), 256, 0,
                              reinterpret_cast<hipStream_t>(stream)>>>(
      block_table, positions, page_ids, offsets, (int)B, (int)max_blocks, (int)page_size);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_paged_kv_update(void* K_pages, void* V_pages, const void* k_new, const void* v_new,
                       const int32_t* block_table, const int32_t* positions, int64_t B, int64_t H,
                       int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                       int dtype, void* stream) {
  MK_REQUIRE(K_pages && V_pages && k_new && v_new && block_table && positions);
  MK_REQUIRE(B >= 0 && H > 0 && D > 0 && page_size > 0 && max_blocks > 0 && num_pages > 0);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  MK_REQUIRE(H * D < (1 << 30) && num_pages < (1LL << 31) && B < 65536);
  if (B == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // f16 and bf16 are both 16-bit: the copy is type-agnostic
  paged_update_kernel<uint16_t><<<(unsigned)B, 256, 0, st>>>(
      (uint16_t*)K_pages, (uint16_t*)V_pages, (const uint16_t*)k_new, (const uint16_t*)v_new,
      block_table, positions, (int)B, (int)H, (int)D, (int)page_size, (int)max_blocks,
      (int)num_pages);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_qkv_rope_paged_update(const void* qkv, const float* cos_t, const float* sin_t,
                             const int32_t* positions, const int32_t* block_table, void* K_pages,
                             void* V_pages, void* q_out, int64_t B, int64_t Hq, int64_t Hkv,
                             int64_t D, int64_t page_size, int64_t max_blocks, int64_t num_pages,
                             int64_t cos_rows, int dtype, void* stream) {
  MK_REQUIRE(qkv && cos_t && sin_t && positions && block_table && K_pages && V_pages && q_out);
  MK_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && D > 0 && (D % 2) == 0 && page_size > 0);
  MK_REQUIRE(max_blocks > 0 && num_pages > 0 && cos_rows > 0 && B < 65536);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  if (B == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t tasks = (Hq + 2 * Hkv) * (D / 8);
  if ((D % 8) == 0 && tasks <= 65535LL * 128 && mk_aligned(qkv, 16) && mk_aligned(q_out, 16) &&
      mk_aligned(K_pages, 16) && mk_aligned(V_pages, 16) && mk_aligned(cos_t, 16) &&
      mk_aligned(sin_t, 16)) {
    const dim3 grid((unsigned)B, (unsigned)((tasks + 127) / 128));
    const bool stage = B > 1 && B <= kRopeSlotMax && num_pages * page_size < (1LL << 31);
#define MK_QRV(T)                                                                                 \
  qkv_rope_update_vec_kernel<T><<<grid, 128, 0, st>>>(                                            \
      (const T*)qkv, cos_t, sin_t, positions, block_table, (T*)K_pages, (T*)V_pages, (T*)q_out, \
      (int)B, (int)Hq, (int)Hkv, (int)D, (int)page_size, (int)max_blocks, (int)num_pages,        \
      (int)cos_rows, stage)
    if (dtype == MK_DT_F16) MK_QRV(f16);
    else MK_QRV(bf16);
#undef MK_QRV
    MK_CHECK_LAUNCH();
    return MK_OK;
  }
#define MK_QRU(T)                                                                                 \
  qkv_rope_update_kernel<T><<<(unsigned)B, 256, 0, st>>>(                                         \
      (const T*)qkv, cos_t, sin_t, positions, block_table, (T*)K_pages, (T*)V_pages, (T*)q_out, \
      (int)B, (int)Hq, (int)Hkv, (int)D, (int)page_size, (int)max_blocks, (int)num_pages,        \
      (int)cos_rows)
  if (dtype == MK_DT_F16) MK_QRU(f16);
  else MK_QRU(bf16);
#undef MK_QRU
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_qkv_rope_paged_update_quant(const void* qkv, const float* cos_t, const float* sin_t,
                                   const int32_t* positions, const int32_t* block_table,
                                   uint8_t* K_q, uint8_t* V_q, f16_storage_t* K_s,
                                   f16_storage_t* V_s, void* q_out, int64_t B, int64_t Hq,
                                   int64_t Hkv, int64_t D, int64_t page_size, int64_t max_blocks,
                                   int64_t num_pages, int64_t cos_rows, int64_t group_size,
                                   int bits, int dtype, void* stream) {
  MK_REQUIRE(qkv && cos_t && sin_t && positions && block_table && K_q && V_q && K_s && V_s &&
             q_out);
  MK_REQUIRE(B >= 0 && Hq > 0 && Hkv > 0 && D > 0 && (D % 2) == 0 && page_size > 0);
  MK_REQUIRE(max_blocks > 0 && num_pages > 0 && cos_rows > 0 && group_size > 0 && B < 65536);
  MK_REQUIRE(bits == 4 || bits == 8);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  MK_REQUIRE(Hkv * D <= QUPD_MAX_ELEMS);
  if (B == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define MK_QRUQ(T, BITS)                                                                          \
  qkv_rope_update_quant_kernel<T, BITS><<<(unsigned)B, 256, 0, st>>>(                             \
      (const T*)qkv, cos_t, sin_t, positions, block_table, K_q, V_q, K_s, V_s, (T*)q_out, (int)B, \
      (int)Hq, (int)Hkv, (int)D, (int)page_size, (int)max_blocks, (int)num_pages, (int)cos_rows, \
      (int)group_size)
  if (dtype == MK_DT_F16) {
    if (bits == 8) MK_QRUQ(f16, 8);
    else MK_QRUQ(f16, 4);
  } else {
    if (bits == 8) MK_QRUQ(bf16, 8);
    else MK_QRUQ(bf16, 4);
  }
#undef MK_QRUQ
  MK_CHECK_LAUNCH();
  return MK_OK;
}

}  // extern "C"
