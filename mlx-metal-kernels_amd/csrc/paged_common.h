// Device helpers shared by the paged cache writers (paged.hip) and the
// qkv projection whose epilogue writes the new token (gemv.hip).
#pragma once
#include "common.h"

namespace {

// page and in-page offset of sequence b's new token at position pos[b]
// (block table [B, max_blocks]); -1 for an out-of-range position or page id
__device__ __forceinline__ int slot_page(const int32_t* bt, const int32_t* pos, int b,
                                         int max_blocks, int P, int num_pages, int* off) {
  const int p = pos[b];
  if (p < 0 || p >= max_blocks * P) return -1;
  const int page = bt[(size_t)b * max_blocks + p / P];
  *off = p % P;
  if (page < 0 || page >= num_pages) return -1;
  return page;
}

// true when a later sequence writes the same slot (its write must win)
__device__ __forceinline__ bool superseded(const int32_t* bt, const int32_t* pos, int b, int B,
                                           int max_blocks, int P, int num_pages, int page,
                                           int off) {
  for (int b2 = b + 1; b2 < B; ++b2) {
    int o2;
    const int p2 = slot_page(bt, pos, b2, max_blocks, P, num_pages, &o2);
    if (p2 == page && o2 == off) return true;
  }
  return false;
}

// interleaved RoPE of one (even, odd) pair; products and sums rounded
// separately (no fma contraction), matching the reference's fp32 expression
__device__ __forceinline__ void rope_pair(float xe, float xo, float c, float s, float* ye,
                                          float* yo) {
#pragma clang fp contract(off)
  const float a = xe * c;
  const float b2 = xo * s;
  const float d = xe * s;
  const float e = xo * c;
  *ye = a - b2;
  *yo = d + e;
}

}  // namespace
