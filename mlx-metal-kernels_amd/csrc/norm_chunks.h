// The residual + RMSNorm prologue's share of the activation row for one
// thread of the gemv_dot_kernel workgroup (shared by the kernel and a host
// test, so every index the kernel can form is checked on the CPU).
//
// The row of K fp16 values is read in 16-byte chunks (K / 8 of them).  Thread
// t of nthr takes chunk t and, when nthr < K / 8, chunk t + nthr: at most two,
// so the dispatcher launches only when K / 8 <= 2 * nthr.  A thread whose
// chunk lies past the row still issues its load (every load counts in order)
// but reads a chunk inside the row instead -- chunk 0, or its first chunk --
// and leaves that value out of the norm (has0 / has1 false).
#pragma once

#if defined(__HIPCC__)
#define MK_HD __host__ __device__
#else
#define MK_HD
#endif

struct NormChunks {
  int c0, c1;    // chunk indices the loads read (always inside the row)
  bool has0, has1;  // whether each is this thread's own chunk of the norm
};

MK_HD inline NormChunks norm_prologue_chunks(int t, int nthr, int K) {
  const int nchunk = K / 8;
  const bool two = nthr < nchunk;
  const int a = t, b = two ? t + nthr : t;
  NormChunks r;
  r.has0 = a < nchunk;
  r.has1 = two && b < nchunk;
  r.c0 = r.has0 ? a : 0;
  r.c1 = b < nchunk ? b : r.c0;
  return r;
}
