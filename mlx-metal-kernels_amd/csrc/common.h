// Shared device helpers for the gfx950 quantized-decode kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, MFMA
// 16x16x32 f16/bf16 matrix cores, 160 KB of LDS per CU.  Activations are fp16
// or bf16, accumulation is fp32, quantized weights are uint8 codes (two 4-bit
// codes per byte, low nibble = even column).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mk_hip.h"

typedef _Float16 f16;
typedef __bf16 bf16;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define MK_WAVE 64

// Largest finite values of the activation types; outputs saturate to these
// like the reference's clip(result, finfo.min, finfo.max).
#define MK_F16_MAX 65504.0f
#define MK_BF16_MAX 3.3895313892515355e38f

// ---------------------------------------------------------------------------
// bit casts
// ---------------------------------------------------------------------------
template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From& v) {
  static_assert(sizeof(To) == sizeof(From), "bitcast size mismatch");
  return __builtin_bit_cast(To, v);
}

// ---------------------------------------------------------------------------
// activation-type traits
// ---------------------------------------------------------------------------
template <typename T>
struct ActTraits;

template <>
struct ActTraits<f16> {
  static constexpr float kMax = MK_F16_MAX;
  static __device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
  static __device__ __forceinline__ f16 from_f32(float v) { return (f16)v; }
};

template <>
struct ActTraits<bf16> {
  static constexpr float kMax = MK_BF16_MAX;
  static __device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
  static __device__ __forceinline__ bf16 from_f32(float v) { return (bf16)v; }
};

template <>
struct ActTraits<float> {
  static constexpr float kMax = 3.4028234663852886e38f;
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
};

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return ActTraits<T>::to_f32(v);
}
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return ActTraits<T>::from_f32(v);
}

// clip(v, -max, max) then round-to-nearest-even into T.  NaN propagates.
template <typename T>
__device__ __forceinline__ T saturate_cast(float v) {
  const float m = ActTraits<T>::kMax;
  v = v > m ? m : v;
  v = v < -m ? -m : v;
  return from_f32<T>(v);
}

// ---------------------------------------------------------------------------
// wave reductions (64 lanes)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, MK_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, MK_WAVE));
  return v;
}

// ---------------------------------------------------------------------------
// 128-bit global loads
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ldg128(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x2 ldg64(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}

// Streaming (read-once) 128-bit load: non-temporal hint keeps weights and KV
// pages from evicting the reused activation vector from L2.
__device__ __forceinline__ u32x4 ldg128_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// 8-byte read that is not expected to be reused (nontemporal)
__device__ __forceinline__ u32x2 ldg64_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

// Hide a constant from the optimizer so it lives in a VGPR: gfx9 VOP3
// instructions accept at most one scalar/literal operand, and
// v_and_or_b32(x, mask, magic) needs the magic in a vector register.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value
// {hi:src0, lo:src1} (selector values 0-3 pick src1, 4-7 pick src0).
__device__ __forceinline__ uint32_t perm_b32(uint32_t src0, uint32_t src1, uint32_t sel) {
  return __builtin_amdgcn_perm(src0, src1, sel);
}
// low halves: (lo16(a), lo16(b)) as (low, high) of the result
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return perm_b32(b, a, 0x05040100u);
}
// high halves: (hi16(a), hi16(b))
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return perm_b32(b, a, 0x07060302u);
}

// Workgroup barrier for LDS data only.  __syncthreads() is also a global
// memory fence, for which the compiler waits on every outstanding vector load
// (vmcnt(0)); here only the wave's LDS operations must be complete
// (lgkmcnt(0)), so weight loads issued earlier stay in flight across the
// barrier and are waited for where their registers are first used.  The
// memory clobber keeps the compiler from moving LDS (or any memory) accesses
// across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---------------------------------------------------------------------------
// host-side launch status
// ---------------------------------------------------------------------------
#define MK_CHECK_LAUNCH()                                 \
  do {                                                    \
    hipError_t _e = hipGetLastError();                    \
    if (_e != hipSuccess) return -(int)_e - 1000;         \
  } while (0)

#define MK_REQUIRE(cond)                 \
  do {                                   \
    if (!(cond)) return MK_ERR_INVALID;  \
  } while (0)

static inline bool mk_aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}
