// Elementwise prologue/epilogue kernels of the quantized MLP block.
//
// swiglu / fused_swiglu  ops/activation_ops.py:83-153   out = g/(1+exp(-g))*u
// residual_add           ops/fused_ops.py:149-180        out = x + r
// rms_norm               ops/norm_ops.py:47-85           y = x*rsqrt(mean(x^2)+eps)*w
// residual + rms_norm    ops/mlp_block_ops.py:343-344    (z = x + r; y = rms_norm(z))
// All math is fp32 with one rounding into the storage type per output, as the
// reference's astype() chain does.  These are O(hidden) per token -- noise next
// to the matvecs -- so they stay simple grid-stride loops.
#include "common.h"

namespace {

template <typename T>
__device__ __forceinline__ float silu_mul(T g, T u) {
  const float gf = to_f32(g);
  return gf / (1.0f + expf(-gf)) * to_f32(u);
}

template <typename T>
__global__ void swiglu_kernel(const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ out,
                              int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = from_f32<T>(silu_mul(g[i], u[i]));
}

template <typename T>
__global__ void residual_add_kernel(const T* __restrict__ x, const T* __restrict__ r,
                                    T* __restrict__ out, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = from_f32<T>(to_f32(x[i]) + to_f32(r[i]));
}

// One workgroup (256 threads) per row.  With RES, z = x + r is rounded to T,
// stored, and the norm is taken over the rounded z (the reference normalizes
// the materialized z).
template <typename T, typename WT, bool RES>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T* __restrict__ x,
                                                       const T* __restrict__ r,
                                                       const WT* __restrict__ w,
                                                       T* __restrict__ z_out, T* __restrict__ y,
                                                       int64_t D, float eps) {
  const int64_t row = blockIdx.x;
  const T* xr = x + row * D;
  const T* rr = RES ? r + row * D : nullptr;
  T* zr = RES ? z_out + row * D : nullptr;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < D; i += blockDim.x) {
    float v = to_f32(xr[i]);
    if constexpr (RES) {
      const T zt = from_f32<T>(v + to_f32(rr[i]));
      zr[i] = zt;
      v = to_f32(zt);
    }
    ss += v * v;
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = rsqrtf(tot / (float)D + eps);
  T* yr = y + row * D;
  const T* src = RES ? zr : xr;
  for (int64_t i = threadIdx.x; i < D; i += blockDim.x) {
    // each thread re-reads the z it wrote itself, so no barrier is needed
    const float v = to_f32(src[i]);
    yr[i] = from_f32<T>(v * inv * to_f32(w[i]));
  }
}

// 8 consecutive elements through 128-bit accesses (16-byte aligned pointers).
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&o)[8]) {
  T t[8];
  if constexpr (sizeof(T) == 2) {
    const u32x4 v = ldg128(p);
    __builtin_memcpy(t, &v, 16);
  } else {
    const u32x4 a = ldg128(p), b = ldg128(p + 4);
    __builtin_memcpy(t, &a, 16);
    __builtin_memcpy(t + 4, &b, 16);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = to_f32(t[i]);
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const T (&t)[8]) {
  if constexpr (sizeof(T) == 2) {
    u32x4 v;
    __builtin_memcpy(&v, t, 16);
    *reinterpret_cast<u32x4*>(p) = v;
  } else {
    u32x4 a, b;
    __builtin_memcpy(&a, t, 16);
    __builtin_memcpy(&b, t + 4, 16);
    reinterpret_cast<u32x4*>(p)[0] = a;
    reinterpret_cast<u32x4*>(p)[1] = b;
  }
}

// Same arithmetic as rms_norm_kernel, for D % 8 == 0 and D <= 8 * 256 * CH:
// each thread owns CH chunks of 8 elements, loads x, r and w for all of them
// before the single block reduction, and keeps them in registers (one HBM
// round trip instead of D / 256 dependent ones).
template <typename T, typename WT, bool RES, int CH>
__global__ __launch_bounds__(256) void rms_norm_vec_kernel(const T* __restrict__ x,
                                                           const T* __restrict__ r,
                                                           const WT* __restrict__ w,
                                                           T* __restrict__ z_out,
                                                           T* __restrict__ y, int64_t D, float eps) {
  const int64_t row = blockIdx.x;
  const int nch = (int)(D >> 3);
  float v[CH][8], wv[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch < nch) {
      const int64_t off = row * D + 8 * ch;
      load8(x + off, v[c]);
      load8(w + 8 * ch, wv[c]);
      if constexpr (RES) {
        float rv[8];
        load8(r + off, rv);
        T zt[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          zt[i] = from_f32<T>(v[c][i] + rv[i]);
          v[c][i] = to_f32(zt[i]);
        }
        store8(z_out + off, zt);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[c][i] * v[c][i];
    }
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = rsqrtf(tot / (float)D + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = threadIdx.x + 256 * c;
    if (ch < nch) {
      T o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = from_f32<T>(v[c][i] * inv * wv[c][i]);
      store8(y + row * D + 8 * ch, o);
    }
  }
}

inline dim3 grid_for(int64_t work, int threads) {
  int64_t b = (work + threads - 1) / threads;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return dim3((unsigned)b);
}

template <bool RES>
int norm_entry(const void* x, const void* r, const void* w, void* z, void* y, int64_t rows,
               int64_t D, float eps, int xdt, int wdt, void* stream) {
  MK_REQUIRE(x && w && y && rows >= 0 && D > 0);
  MK_REQUIRE(!RES || (r && z));
  MK_REQUIRE(xdt == MK_DT_F16 || xdt == MK_DT_BF16 || (xdt == MK_DT_F32 && !RES));
  MK_REQUIRE(wdt == MK_DT_F16 || wdt == MK_DT_BF16 || wdt == MK_DT_F32);
  MK_REQUIRE(rows < (1LL << 31));
  if (rows == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)rows);
  // the vector kernel needs 16-byte aligned rows: D % 8 == 0 and aligned bases
  const bool vec = D % 8 == 0 && D <= 8 * 256 * 4 && mk_aligned(x, 16) && mk_aligned(w, 16) &&
                   mk_aligned(y, 16) && (!RES || (mk_aligned(r, 16) && mk_aligned(z, 16)));
  const int ch = (int)((D / 8 + 255) / 256);
#define MK_NORM_VEC(T, WT, CH)                                                         \
  rms_norm_vec_kernel<T, WT, RES, CH><<<grid, 256, 0, st>>>((const T*)x, (const T*)r, \
                                                            (const WT*)w, (T*)z, (T*)y, D, eps)
#define MK_NORM(T, WT)                                                                       \
  do {                                                                                       \
    if (vec && ch == 1) MK_NORM_VEC(T, WT, 1);                                               \
    else if (vec && ch == 2) MK_NORM_VEC(T, WT, 2);                                          \
    else if (vec) MK_NORM_VEC(T, WT, 4);                                                     \
    else                                                                                     \
      rms_norm_kernel<T, WT, RES><<<grid, 256, 0, st>>>((const T*)x, (const T*)r,            \
                                                        (const WT*)w, (T*)z, (T*)y, D, eps); \
  } while (0)
  if (xdt == MK_DT_F16) {
    if (wdt == MK_DT_F16) MK_NORM(f16, f16);
    else if (wdt == MK_DT_BF16) MK_NORM(f16, bf16);
    else MK_NORM(f16, float);
  } else if (xdt == MK_DT_BF16) {
    if (wdt == MK_DT_F16) MK_NORM(bf16, f16);
    else if (wdt == MK_DT_BF16) MK_NORM(bf16, bf16);
    else MK_NORM(bf16, float);
  } else {
    if (wdt == MK_DT_F16) MK_NORM(float, f16);
    else if (wdt == MK_DT_BF16) MK_NORM(float, bf16);
    else MK_NORM(float, float);
  }
#undef MK_NORM
#undef MK_NORM_VEC
  MK_CHECK_LAUNCH();
  return MK_OK;
}

// Greedy sampling, models/sampling.py:120-124: per row the index of the
// largest value, the first one on ties, a NaN counting as the largest (the
// rule np.argmax follows).  One 1024-thread workgroup per row; threads scan
// 16-byte chunks eight loads at a time, then the (value, index) pairs reduce
// across lanes and waves.
__device__ __forceinline__ bool argmax_better(float v, int64_t i, float bv, int64_t bi) {
  if (bv != bv) return v != v && i < bi;
  if (v != v) return true;
  return v > bv || (v == bv && i < bi);
}

// (value, index) of the row's best entry from every thread -> out[row]
__device__ __forceinline__ void argmax_finish(float bv, int64_t bi, int64_t n, int64_t* __restrict__ out) {
  for (int d = 32; d >= 1; d >>= 1) {
    const float ov = __shfl_xor(bv, d, 64);
    const int64_t oi = __shfl_xor(bi, d, 64);
    if (argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  __shared__ float sv[16];
  __shared__ int64_t si[16];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { sv[wave] = bv; si[wave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
      if (argmax_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    out[blockIdx.x] = bi < n ? bi : 0;
  }
}

template <typename T>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const T* __restrict__ x, int64_t* __restrict__ out,
                                                           int64_t n, bool vec) {
  const T* r = x + (size_t)blockIdx.x * n;
  float bv = -INFINITY;
  int64_t bi = n;  // no candidate yet: any real index is better on ties
  const int nt = blockDim.x;
  if (vec) {
    // eight independent 16-byte loads in flight per thread before any compare
    constexpr int EPC = 16 / sizeof(T);  // elements per 16-byte load
    constexpr int UNR = 8;
    const int64_t nc = n / EPC;
    for (int64_t c0 = 0; c0 < nc; c0 += (int64_t)nt * UNR) {
      u32x4 w[UNR];
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        const int64_t c = c0 + (int64_t)j * nt + threadIdx.x;
        w[j] = ldg128(r + EPC * (c < nc ? c : nc - 1));
      }
#pragma unroll
      for (int j = 0; j < UNR; ++j) {
        const int64_t c = c0 + (int64_t)j * nt + threadIdx.x;
        if (c >= nc) continue;
        T e[EPC];
        __builtin_memcpy(e, &w[j], 16);
#pragma unroll
        for (int k = 0; k < EPC; ++k) {
          const float v = to_f32(e[k]);
          const int64_t i = EPC * c + k;
          if (argmax_better(v, i, bv, bi)) { bv = v; bi = i; }
        }
      }
    }
  } else {
    for (int64_t i = threadIdx.x; i < n; i += nt) {
      const float v = to_f32(r[i]);
      if (argmax_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
  }
  argmax_finish(bv, bi, n, out);
}

// fp16 rows of whole 16-byte chunks (the logits of a decode step): a thread
// takes a chunk's 8 values with packed fp16 ops -- the chunk maximum
// (maxNum, so NaNs drop out of it), and a packed sum that is NaN whenever the
// chunk holds a NaN (or both infinities, which the exact check below then
// rules out) -- keeps the first chunk that raises its maximum, with its 16
// bytes, and only at the end finds the first position of that maximum inside
// it.  A chunk flagged by its sum is checked value by value for the first
// NaN, which np.argmax's rule puts above every number.  16 loads per thread in
// flight cover a 128256-entry row in one round.
__global__ __launch_bounds__(1024) void argmax_rows_f16_kernel(const f16* __restrict__ x,
                                                               int64_t* __restrict__ out, int64_t n) {
  const f16* r = x + (size_t)blockIdx.x * n;
  const int64_t nc = n / 8;
  const int nt = blockDim.x;
  f16 best = (f16)(-INFINITY);
  int64_t bc = -1;         // this thread's chunk holding its first maximum
  u32x4 bw = {0u, 0u, 0u, 0u};
  int64_t nan_i = n;       // this thread's first NaN
  constexpr int UNR = 16;
  for (int64_t c0 = 0; c0 < nc; c0 += (int64_t)nt * UNR) {
    u32x4 w[UNR];
#pragma unroll
    for (int j = 0; j < UNR; ++j) {
      const int64_t c = c0 + (int64_t)j * nt + threadIdx.x;
      w[j] = ldg128(r + 8 * (c < nc ? c : nc - 1));
    }
#pragma unroll
    for (int j = 0; j < UNR; ++j) {
      const int64_t c = c0 + (int64_t)j * nt + threadIdx.x;
      if (c >= nc) continue;
      const f16x2 a0 = bitcast<f16x2>(w[j][0]), a1 = bitcast<f16x2>(w[j][1]);
      const f16x2 a2 = bitcast<f16x2>(w[j][2]), a3 = bitcast<f16x2>(w[j][3]);
      const f16x2 m2 = __builtin_elementwise_max(__builtin_elementwise_max(a0, a1), __builtin_elementwise_max(a2, a3));
      const f16 m = __builtin_elementwise_max(m2[0], m2[1]);
      const f16x2 s2 = (a0 + a1) + (a2 + a3);
      const f16 sum = s2[0] + s2[1];
      if (sum != sum && nan_i == n) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t h = (w[j][e >> 1] >> (16 * (e & 1))) & 0x7FFFu;
          if (h > 0x7C00u && nan_i == n) nan_i = 8 * c + e;
        }
      }
      if (bc < 0 || m > best) {
        best = m;
        bc = c;
        bw = w[j];
      }
    }
  }
  float bv = -INFINITY;
  int64_t bi = n;
  if (nan_i < n) {
    bv = __builtin_nanf("");
    bi = nan_i;
  } else if (bc >= 0) {
    int first = 7;
#pragma unroll
    for (int e = 7; e >= 0; --e)
      if (bitcast<f16x2>(bw[e >> 1])[e & 1] == best) first = e;
    bv = (float)best;
    bi = 8 * bc + first;
  }
  argmax_finish(bv, bi, n, out);
}

}  // namespace

extern "C" {

int mk_argmax_rows(const void* x, int64_t* out, int64_t rows, int64_t n, int dtype, void* stream) {
  MK_REQUIRE(x && out && rows >= 0 && n > 0 && rows < (1LL << 31));
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16 || dtype == MK_DT_F32);
  if (rows == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const size_t es = dtype == MK_DT_F32 ? 4 : 2;
  // every row starts 16-byte aligned and holds whole 16-byte chunks
  const bool vec = mk_aligned(x, 16) && ((size_t)n * es) % 16 == 0;
  if (dtype == MK_DT_F16 && vec)
    argmax_rows_f16_kernel<<<(unsigned)rows, 1024, 0, st>>>((const f16*)x, out, n);
  else if (dtype == MK_DT_F16)
    argmax_rows_kernel<f16><<<(unsigned)rows, 1024, 0, st>>>((const f16*)x, out, n, vec);
  else if (dtype == MK_DT_BF16)
    argmax_rows_kernel<bf16><<<(unsigned)rows, 1024, 0, st>>>((const bf16*)x, out, n, vec);
  else
    argmax_rows_kernel<float><<<(unsigned)rows, 1024, 0, st>>>((const float*)x, out, n, vec);
  MK_CHECK_LAUNCH();
  return MK_OK;
}


int mk_swiglu(const void* gate, const void* up, void* out, int64_t n, int dtype, void* stream) {
  MK_REQUIRE(gate && up && out && n >= 0);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  if (n == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == MK_DT_F16)
    swiglu_kernel<f16><<<grid_for(n, 256), 256, 0, st>>>((const f16*)gate, (const f16*)up,
                                                         (f16*)out, n);
  else
    swiglu_kernel<bf16><<<grid_for(n, 256), 256, 0, st>>>((const bf16*)gate, (const bf16*)up,
                                                          (bf16*)out, n);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_residual_add(const void* x, const void* residual, void* out, int64_t n, int dtype,
                    void* stream) {
  MK_REQUIRE(x && residual && out && n >= 0);
  MK_REQUIRE(dtype == MK_DT_F16 || dtype == MK_DT_BF16);
  if (n == 0) return MK_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == MK_DT_F16)
    residual_add_kernel<f16><<<grid_for(n, 256), 256, 0, st>>>((const f16*)x, (const f16*)residual,
                                                               (f16*)out, n);
  else
    residual_add_kernel<bf16><<<grid_for(n, 256), 256, 0, st>>>(
        (const bf16*)x, (const bf16*)residual, (bf16*)out, n);
  MK_CHECK_LAUNCH();
  return MK_OK;
}

int mk_rms_norm(const void* x, const void* weight, void* y, int64_t rows, int64_t D, float eps,
                int x_dtype, int w_dtype, void* stream) {
  return norm_entry<false>(x, nullptr, weight, nullptr, y, rows, D, eps, x_dtype, w_dtype, stream);
}

int mk_residual_rms_norm(const void* x, const void* residual, const void* weight, void* z_out,
                         void* y_out, int64_t rows, int64_t D, float eps, int x_dtype,
                         int w_dtype, void* stream) {
  return norm_entry<true>(x, residual, weight, z_out, y_out, rows, D, eps, x_dtype, w_dtype,
                          stream);
}

}  // extern "C"
