"""CPU regression test for the norm prologue's activation indices.

gemv_dot_kernel's residual + RMSNorm prologue reads the row of K fp16 values
in 16-byte chunks, two per thread at most (csrc/norm_chunks.h).  A GPU memory
fault came from threads past K / 8 loading their chunk without a clamp, up
to 4 KB past x, the residual and the norm weight.  This test compiles the
kernel's own index function for the host (g++) and checks, for every row
length the dispatcher accepts (K % 32 == 0, K <= 8192) and every workgroup
size that satisfies its launch precondition (K / 8 <= 2 * threads), that

* every chunk a thread loads lies inside the row, and
* the chunks a thread counts in the norm cover the row exactly once.

The unclamped indexing the fault came from is checked the same way and must
fail, so the checker is shown to catch it."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "mlx-metal-kernels_amd", "csrc", "norm_chunks.h")

PROGRAM = r"""
#include <cstdio>
#include <vector>
#include "norm_chunks.h"

// the indexing before the fix: the second chunk was loaded unclamped
static NormChunks unclamped(int t, int nthr, int K) {
  NormChunks r = norm_prologue_chunks(t, nthr, K);
  r.c1 = nthr < K / 8 ? t + nthr : t;
  return r;
}

template <class F>
static int check(F chunks, bool report) {
  int bad = 0, cases = 0;
  for (int K = 32; K <= 8192; K += 32) {
    const int nchunk = K / 8;
    for (int nthr = 64; nthr <= 1024; nthr += 64) {
      if (nchunk > 2 * nthr) continue;  // the dispatcher's launch precondition
      ++cases;
      std::vector<int> cover(nchunk, 0);
      for (int t = 0; t < nthr; ++t) {
        const NormChunks c = chunks(t, nthr, K);
        // every 16-byte load reads elements [8c, 8c + 8) of the row
        if (c.c0 < 0 || c.c0 >= nchunk || c.c1 < 0 || c.c1 >= nchunk) {
          if (report && bad < 5) std::printf("out of row: K %d nthr %d t %d chunks %d %d\n", K, nthr, t, c.c0, c.c1);
          ++bad;
        }
        if (c.has0) cover[c.c0]++;
        if (c.has1) cover[c.c1]++;
      }
      for (int i = 0; i < nchunk; ++i)
        if (cover[i] != 1) {
          if (report && bad < 5) std::printf("chunk %d counted %d times: K %d nthr %d\n", i, cover[i], K, nthr);
          ++bad;
          break;
        }
    }
  }
  std::printf("cases %d bad %d\n", cases, bad);
  return bad;
}

int main() {
  const int fixed = check(norm_prologue_chunks, true);
  const int mutant = check(unclamped, false);
  std::printf("fixed %d mutant %d\n", fixed, mutant);
  return fixed == 0 && mutant > 0 ? 0 : 1;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs a host C++ compiler")
def test_norm_prologue_chunks_stay_in_the_row(tmp_path):
    src = tmp_path / "norm_chunks_check.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "norm_chunks_check"
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True)
    assert run.returncode == 0, run.stdout + run.stderr
    fixed, mutant = (int(v) for v in run.stdout.strip().splitlines()[-1].split()[1::2])
    assert fixed == 0 and mutant > 0
