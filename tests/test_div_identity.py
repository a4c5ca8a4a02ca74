"""The pack kernels divide by a row scale s through its correctly rounded reciprocal
y = RN(1 / s): q = x y, r = fma(-q, s, x), q' = fma(r, y, q) (Markstein's correction,
htrc_amd/csrc/common.h div_by).  Checked here in IEEE fp32 (C, no contraction) against the
IEEE quotient: for |x| <= max|row| and s = max|row| / 127 the rounded codes (ties away from
zero, and ties to even) never differ, and the quotients differ only below 0.25."""
from __future__ import annotations

import shutil
import subprocess
import textwrap

import pytest

SRC = textwrap.dedent(r"""
    #include <math.h>
    #include <stdint.h>
    #include <stdio.h>
    #include <string.h>
    static float uf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
    static uint64_t st = 88172645463325252ull;
    static uint32_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return (uint32_t)(st >> 11); }
    static long n, bad_code, bad_big;
    static void check(float x, float amax) {
        float s = amax * (1.0f / 127.0f);
        if (s < 1e-20f) s = 1e-20f;
        const float y = 1.0f / s, want = x / s, q = x * y, got = fmaf(fmaf(-q, s, x), y, q);
        ++n;
        if (isnan(got) || roundf(got) != roundf(want) || rintf(got) != rintf(want)) ++bad_code;
        if (fabsf(want) >= 0.25f && memcmp(&got, &want, 4)) ++bad_big;
    }
    int main(void) {
        for (uint32_t a = 0; a < 65536; a += 16) {            /* 4096 bf16 row maxima */
            const float amax = fabsf(uf(a << 16));
            if (!isfinite(amax)) continue;
            for (uint32_t b = 0; b < 65536; ++b) {             /* every bf16 value */
                const float x = uf(b << 16);
                if (isfinite(x) && fabsf(x) <= amax) check(x, amax);
            }
        }
        for (long it = 0; it < 20000000L; ++it) {            /* random fp32 pairs */
            const uint32_t ua = rnd() & 0x7fffffffu;
            const float amax = uf(ua);
            const uint32_t ux = (rnd() & 3) ? ua - (rnd() & 0x00ffffffu) : (rnd() & 0x7fffffffu);
            float x = uf(ux);
            if (!isfinite(amax) || !isfinite(x) || fabsf(x) > amax) continue;
            check((rnd() & 1) ? -x : x, amax);
        }
        printf("%ld %ld %ld\n", n, bad_code, bad_big);
        return 0;
    }
""")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc is needed to build the fp32 check")
def test_reciprocal_division_gives_the_ieee_codes(tmp_path):
    src = tmp_path / "div.c"
    exe = tmp_path / "div"
    src.write_text(SRC)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=300).stdout.split()
    n, bad_code, bad_big = (int(x) for x in out)
    assert n > 100_000_000
    assert bad_code == 0 and bad_big == 0
