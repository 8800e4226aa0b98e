"""Exhaustive host check of the device quotient scheme in csrc/quant_math.h.

Every divisor a quantizer forms is max(amax * RN(1/L), 1e-12) for a bf16
amax (L = 127 or 448; amax_scale) and every dividend is a bf16 x with
|x| <= amax.  Over all
~1.07e9 such pairs per L, div_rn(x, s, RN(1/s)) (three fused ops) must equal
IEEE x / s bit for bit, except where |x / s| < 2^-70 (the residual underflows),
where both quotients produce the same code 0.  The header is compiled with
g++ exactly as the device includes it."""

from __future__ import annotations

import shutil
import subprocess

import pytest

from conftest import ROOT

SRC = r'''
#include "quant_math.h"
#include <cstdio>
#include <cstring>
static float bf(uint16_t h){ uint32_t b=(uint32_t)h<<16; float f; memcpy(&f,&b,4); return f; }
int main(){
  int rc = 0;
  for (int lim=0; lim<2; ++lim){
    const float L = lim ? h3q::kE4M3Max : h3q::kInt8Max;
    const float R = lim ? h3q::kE4M3Recip : h3q::kInt8Recip;
    long long bad_big = 0, bad_small = 0, total = 0;
    #pragma omp parallel for schedule(dynamic,64) reduction(+:bad_big,bad_small,total)
    for (uint32_t ah = 0; ah < 0x7F80; ++ah) {
      const float amax = bf((uint16_t)ah);
      const float s = h3q::amax_scale(amax, R);
      const float r = 1.0f / s;
      for (uint32_t xh = 0; xh <= ah; ++xh) {
        for (int sg = 0; sg < 2; ++sg) {
          const float x = bf((uint16_t)(xh | (sg << 15)));
          const float a = x / s;
          const float b = copysignf(h3q::div_rn(x, s, r), x);
          uint32_t ab, bb; memcpy(&ab, &a, 4); memcpy(&bb, &b, 4);
          ++total;
          if (ab != bb) { if (fabsf(a) >= 0x1p-70f || fabsf(b) >= 0x1p-70f) ++bad_big; else ++bad_small; }
        }
      }
    }
    printf("L=%g pairs=%lld mismatches_above_2^-70=%lld tiny=%lld\n", L, total, bad_big, bad_small);
    if (bad_big) rc = 1;
  }
  return rc;
}
'''


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_quotient_scheme_exhaustive(tmp_path):
    src = tmp_path / "divcheck.cpp"
    src.write_text(SRC)
    exe = tmp_path / "divcheck"
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
                    f"-I{ROOT / 'taomate-h3_amd' / 'csrc'}", str(src), "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert res.stdout.count("mismatches_above_2^-70=0") == 2
