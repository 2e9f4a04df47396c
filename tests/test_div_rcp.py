"""The reciprocal division the kernels use in place of IEEE division gives the IEEE quotient:
y = RN(1/b), q0 = RN(a*y), r = fma(-q0, b, a), q1 = fma(r, y, q0).

Checked in C on this host (gcc's fmaf is a correctly rounded fused multiply-add, like gfx950's
v_fma_f32); quotients are compared bit for bit.  Three uses, three claims:

* quantisation by a block absmax b in [2^-40, 2^60] (came8_device.h: rcp_for_div): every
  significand of a in several binades with |a| in [2^-40, 2^100], skipping quotients above 2^100,
  which quantisation never produces (|a| <= b).  Smaller numerators give quotients below 2^-8,
  which round to code 0 whichever way they are divided.
* the clip divisor b in [1, 2^60]: every finite a with |a| >= 2^-40 (a normal quotient), over all
  binades up to the largest float (DivGuard's fast range).
* dequantisation scales absmax / 127 and absmax / 255: every 5th finite float a, subnormals
  included (scale_s8's fast form).
"""
import os
import shutil
import subprocess
import tempfile

import pytest

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static float div_fast(float a, float b, float y) { float q0 = a * y; float r = fmaf(-q0, b, a); return fmaf(r, y, q0); }
static unsigned long long tot = 0, bad = 0;
static void check(float a, float b, float y) {
  float q = a / b, q1 = div_fast(a, b, y);
  ++tot;
  if (memcmp(&q, &q1, 4) != 0) { if (bad < 5) printf("b=%a a=%a q=%a got=%a\n", b, a, q, q1); ++bad; }
}
static unsigned seed = 2024;
static float rand_sig(int e) { seed = seed * 1103515245u + 12345u; return ldexpf(fbits(0x3f800000u | ((seed >> 5) & 0x7fffff)), e); }
int main(int argc, char** argv) {
  const int mode = argv[1][0] - '0';
  if (mode == 0) {  /* quantisation divisors */
    const int eb[] = {-40, -20, -1, 0, 0, 1, 5, 12, 30, 59};
    const int ea[] = {-40, -7, 0, 3, 20, 99};
    for (int ib = 0; ib < 10; ++ib)
      for (int rep = 0; rep < 2; ++rep) {
        float b = rand_sig(eb[ib]);
        if (ib == 3 && rep == 0) b = 1.0f;
        if (ib == 4 && rep == 0) b = 127.0f;
        const float y = 1.0f / b;
        for (int ia = 0; ia < 6; ++ia)
          for (uint32_t m = 0; m < (1u << 23); m += 3) {
            const float a = ldexpf(fbits(0x3f800000u | m), ea[ia]);
            if (!(fabsf(a / b) <= 0x1p100f)) continue;
            check(a, b, y);
          }
      }
  } else if (mode == 1) {  /* clip divisors: b in [1, 2^60], every binade of a from 2^-40 up */
    const int eb[] = {0, 0, 1, 3, 7, 13, 20, 31, 44, 59, 60};
    for (int ib = 0; ib < 11; ++ib) {
      float b = ib == 0 ? 1.0f : (ib == 10 ? 0x1p60f : rand_sig(eb[ib]));
      const float y = 1.0f / b;
      for (int e = -40; e <= 127; ++e)
        for (uint32_t m = (uint32_t)e & 7u; m < (1u << 23); m += 61) {
          const float a = ldexpf(fbits(0x3f800000u | m), e);
          check(a, b, y);
          check(-a, b, y);
        }
    }
  } else {  /* 127 and 255 over every 5th finite float */
    const float bs[2] = {127.0f, 255.0f};
    for (int ib = 0; ib < 2; ++ib) {
      const float y = 1.0f / bs[ib];
      for (uint32_t u = 0; u < 0x7f800000u; u += 5) check(fbits(u), bs[ib], y);
    }
  }
  printf("%llu %llu\n", tot, bad);
  return 0;
}
"""


@pytest.fixture(scope="module")
def divcheck():
    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    d = tempfile.mkdtemp()
    src = os.path.join(d, "div.c")
    exe = os.path.join(d, "div")
    with open(src, "w") as f:
        f.write(SRC)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
    yield exe
    shutil.rmtree(d, ignore_errors=True)


@pytest.mark.parametrize("mode,min_total", [(0, 300_000_000), (1, 200_000_000), (2, 800_000_000)])
def test_reciprocal_division_is_exact(divcheck, mode, min_total):
    out = subprocess.run([divcheck, str(mode)], check=True, capture_output=True, text=True).stdout.strip().splitlines()
    tot, bad = (int(x) for x in out[-1].split())
    assert tot > min_total
    assert bad == 0, "\n".join(out)
