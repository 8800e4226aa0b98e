"""Exhaustive host check of the device quotient scheme in csrc/quant_math.h.

Every divisor a quantizer forms is max(amax * RN(1/L), 1e-12) for a bf16
amax (L = 127 or 448; amax_scale) and every dividend is a bf16 x with
|x| <= amax.  Over all
~1.07e9 such pairs per L, div_rn(x, s, RN(1/s)) (three fused ops, its sign
restored by copysign) and div_rn_signed (the form the per-row quantizers use,
no copysign) must equal IEEE x / s bit for bit, except where
|x / s| < 2^-70 (the residual underflows), where both quotients have x's sign
and produce the same code +-0.  The header is compiled with
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
    long long bad_big = 0, bad_small = 0, bad_sign = 0, total = 0;
    #pragma omp parallel for schedule(dynamic,64) reduction(+:bad_big,bad_small,bad_sign,total)
    for (uint32_t ah = 0; ah < 0x7F80; ++ah) {
      const float amax = bf((uint16_t)ah);
      const float s = h3q::amax_scale(amax, R);
      const float r = 1.0f / s;
      for (uint32_t xh = 0; xh <= ah; ++xh) {
        for (int sg = 0; sg < 2; ++sg) {
          const float x = bf((uint16_t)(xh | (sg << 15)));
          const float a = x / s;
          const float b = copysignf(h3q::div_rn(x, s, r), x);
          const float c = h3q::div_rn_signed(x, s, r);
          uint32_t ab, bb, cb; memcpy(&ab, &a, 4); memcpy(&bb, &b, 4); memcpy(&cb, &c, 4);
          ++total;
          if (ab != bb) { if (fabsf(a) >= 0x1p-70f || fabsf(b) >= 0x1p-70f) ++bad_big; else ++bad_small; }
          if (ab != cb) { if (fabsf(a) >= 0x1p-70f || fabsf(c) >= 0x1p-70f) ++bad_big; else ++bad_small; }
          if ((ab ^ cb) & 0x80000000u) ++bad_sign;
        }
      }
    }
    printf("L=%g pairs=%lld mismatches_above_2^-70=%lld tiny=%lld sign=%lld\n", L, total, bad_big, bad_small,
           bad_sign);
    if (bad_big || bad_sign) rc = 1;
  }
  return rc;
}
'''


ANY_SRC = r'''
#include "quant_math.h"
#include <cstdio>
#include <cstring>
#include <cmath>
#include <vector>
static float bf(uint16_t h){ uint32_t b=(uint32_t)h<<16; float f; memcpy(&f,&b,4); return f; }
static uint32_t bits(float f){ uint32_t b; memcpy(&b,&f,4); return b; }
// bf16 round to nearest even of a binary32 value (NaN -> canonical NaN)
static uint16_t to_bf16(float f){ uint32_t b=bits(f); if ((b&0x7FFFFFFFu)>0x7F800000u) return 0x7FC0;
  return (uint16_t)((b+0x7FFFu+((b>>16)&1u))>>16); }
static long long check(const std::vector<float>& divisors, const char* what){
  long long bad=0, total=0;
  #pragma omp parallel for schedule(dynamic,16) reduction(+:bad,total)
  for (size_t d=0; d<divisors.size(); ++d){
    const float s=divisors[d], r=1.0f/s;
    for (uint32_t xh=0; xh<0x10000; ++xh){
      const float x=bf((uint16_t)xh);
      if (std::isnan(x)) continue;
      const float a=x/s, b=h3q::div_rn_any(x,s,r);
      const uint16_t ab=to_bf16(a), bb=to_bf16(b);
      ++total;
      // codes equal iff the bf16-rounded quotients are equal, or both are
      // below the smallest e4m3 magnitude (2^-10 rounds to 0) with one sign
      const bool tiny=std::fabs(bf(ab))<0x1p-11f && std::fabs(bf(bb))<0x1p-11f && ((ab^bb)&0x8000)==0;
      if (ab!=bb && !tiny) ++bad;
    }
  }
  printf("%s divisors=%zu pairs=%lld mismatches=%lld\n", what, divisors.size(), total, bad);
  return bad;
}
int main(){
  std::vector<float> bf16s;                          // every bf16 divisor but NaN, both signs
  for (uint32_t h=0; h<0x10000; ++h){ float v=bf((uint16_t)h); if (!std::isnan(v)) bf16s.push_back(v); }
  std::vector<float> sweep;                          // binary32 divisors: log-uniform, edge significands, specials
  uint64_t st=0x9E3779B97F4A7C15ull;
  for (int i=0;i<24000;++i){ st^=st<<13; st^=st>>7; st^=st<<17;
    const float e=(float)((int)(st%160)-80); uint32_t m=(uint32_t)(st>>40)&0x7FFFFFu;
    float v=std::ldexp(1.0f+(float)m/8388608.0f, (int)e); sweep.push_back(v); }
  for (int e=-140;e<=127;e+=3){ sweep.push_back(std::ldexp(1.0f,e)); sweep.push_back(std::ldexp(2.0f-0x1p-23f,e));
    sweep.push_back(std::ldexp(1.0f+0x1p-23f,e)); }
  sweep.push_back(0.0f); sweep.push_back(-0.0f); sweep.push_back(INFINITY); sweep.push_back(-INFINITY);
  sweep.push_back(0x1p-149f); sweep.push_back(0.0371f); sweep.push_back(1.0056f); sweep.push_back(-3.5f);
  long long bad=check(bf16s,"bf16") + check(sweep,"binary32");
  return bad?1:0;
}
'''


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_guarded_quotient_any_divisor(tmp_path):
    """div_rn_any (the per-tensor quantizer's quotient for static and
    bf16-rounded scales) against IEEE division, compared after the bf16
    rounding the quantizer applies: every bf16 numerator against every bf16
    divisor (zeros, infinities and subnormals included, both signs) and
    against ~25k binary32 divisors."""
    src = tmp_path / "anycheck.cpp"
    src.write_text(ANY_SRC)
    exe = tmp_path / "anycheck"
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
                    f"-I{ROOT / 'taomate-h3_amd' / 'csrc'}", str(src), "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=900)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert res.stdout.count("mismatches=0") == 2


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
