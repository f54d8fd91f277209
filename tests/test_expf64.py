"""The float64 exponential of the SiLU gate (tinyoai_amd/csrc/expf64.h),
compiled for the host with g++ and checked against the C library: its
float32 rounding (all the gate uses, stablelm.go:371-373) must equal the
C library's, and its float64 error stay within 2 ulp. The header holds only
IEEE operations with one rounding each (fma, rint, ldexp), so the device
computes the same bits."""
import os
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tinyoai_amd", "csrc")

DRIVER = r"""
#include "expf64.h"
#include <cstdio>
#include <random>
int main() {
  std::mt19937_64 rng(11);
  long n = 0, f32 = 0, over2 = 0, special = 0;
  auto check = [&](double x) {
    const double a = exp_f64(x), b = std::exp(x);
    n++;
    if (std::isnan(a) != std::isnan(b)) { f32++; return; }
    if (!std::isnan(a) && (float)a != (float)b) f32++;
    if (std::isfinite(b) && b > 2.3e-308) {
      const double ulp = std::nextafter(b, INFINITY) - b;
      if (std::fabs(a - b) > 2 * ulp) over2++;
    }
  };
  std::normal_distribution<double> N(0, 3);
  std::uniform_real_distribution<double> W(-745.2, 709.8);
  for (int i = 0; i < 3000000; i++) check(N(rng));
  for (int i = 0; i < 1000000; i++) check(W(rng));
  // a stride through the float32 gate values in [-20, 20] (exp(-g))
  for (float g = -20.f; g <= 20.f; g = std::nextafter(g, 30.f)) {
    check(-(double)g);
    for (int s = 0; s < 997 && g <= 20.f; s++) g = std::nextafter(g, 30.f);
  }
  const double sp[] = {0.0, -0.0, 709.78, 709.79, -745.13, -745.14, -708.5, -720.0, INFINITY, -INFINITY, NAN};
  for (double x : sp) {
    const double a = exp_f64(x), b = std::exp(x);
    if (!(a == b || (std::isnan(a) && std::isnan(b)))) special++;
  }
  std::printf("%ld %ld %ld %ld\n", n, f32, over2, special);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_exp_f64_matches_libm():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "t.cpp"), os.path.join(d, "t")
        with open(src, "w") as f:
            f.write(DRIVER)
        subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I", CSRC, src, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout.split()
    n, f32, over2, special = map(int, out)
    assert n > 4_000_000
    assert f32 == 0, f"{f32} float32 results differ from the C library"
    assert over2 == 0, f"{over2} results beyond 2 ulp"
    assert special == 0
