"""libm_expf (qpack_amd/csrc/hip/libm_expf.hpp), the device restatement of the C library's expf used by the reference-order
mode, against the host C library's expf on every float input: compiled for the host with g++ and run exhaustively (the
reference's std::exp(float) calls, /root/reference/src/kernels_x86.cpp:420 and /root/reference/src/model_llama.cpp:163,
resolve to this expf)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROG = r'''
#include <math.h>
#include <stdio.h>
#include <string.h>
#include "libm_expf.hpp"
int main() {
  long long mism = 0, n = 0;
  #pragma omp parallel for reduction(+:mism, n) schedule(static, 1 << 20)
  for (long long u = 0; u < (1LL << 32); u++) {
    unsigned b = (unsigned)u; float x; memcpy(&x, &b, 4);
    if (x != x) continue;
    n++;
    const float a = expf(x), c = qph::libm_expf(x);
    unsigned ab, cb; memcpy(&ab, &a, 4); memcpy(&cb, &c, 4);
    if (ab != cb) mism++;
  }
  printf("%lld %lld\n", n, mism);
  return 0;
}
'''


def test_libm_expf_matches_libc_on_every_float(tmp_path):
    src = tmp_path / "expf_check.cpp"
    src.write_text(PROG)
    exe = tmp_path / "expf_check"
    subprocess.run(["g++", "-std=c++17", "-O2", "-fopenmp", "-ffp-contract=off", "-I",
                    os.path.join(ROOT, "qpack_amd/csrc/hip"), str(src), "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    n, mism = int(out[0]), int(out[1])
    assert n == (1 << 32) - 2 * ((1 << 23) - 1)
    assert mism == 0
