"""The libm boundary.  The reference's softmax and SiLU call glibc expf
(CpuRouterBackend.cpp:54, Activation.cpp:44); the kernels use the restated
algorithm in csrc/hm_expf.h.  That same header, compiled for the host with
g++, must equal the host expf on every float input it is checked on (and so
must its short path hm_expf_small_t on |x| < 88), and its 32-entry table must
equal bits(2^(i/32)) - (i << 47) computed in long double.

The default run strides through all 2^32 bit patterns (every 3rd); set
HM_EXPF_EXHAUSTIVE=1 to check every float (about a minute)."""
from __future__ import annotations

import os
import subprocess
import textwrap
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "hypermoe-engine_amd" / "csrc"

PROGRAM = textwrap.dedent(r"""
    #include <math.h>
    #include <stdio.h>
    #include <stdlib.h>
    #include <string.h>
    #include "hm_expf.h"
    int main(int argc, char** argv) {
        unsigned long long step = strtoull(argv[1], 0, 10);
        long long bad_tab = 0;
        for (int i = 0; i < 32; ++i) {
            long double v = exp2l((long double)i / 32.0L);
            double d = (double)v;
            unsigned long long u; memcpy(&u, &d, 8);
            if (u - ((unsigned long long)i << 47) != kHmExp2Table[i]) ++bad_tab;
        }
        long long n = 0, bad = 0;
        for (unsigned long long b = 0; b <= 0xffffffffull; b += step) {
            unsigned int bits = (unsigned int)b; float x; memcpy(&x, &bits, 4);
            if (x != x) continue;
            float a = expf(x), m = hm_expf(x);
            ++n;
            if (memcmp(&a, &m, 4)) { if (bad < 5) fprintf(stderr, "x=%a libm=%a mine=%a\n", x, a, m); ++bad; }
            if (fabsf(x) < 88.0f) {  /* the range where the kernels take the short path */
                float s = hm_expf_small_t(x, kHmExp2Table);
                if (memcmp(&a, &s, 4)) { if (bad < 5) fprintf(stderr, "small x=%a libm=%a mine=%a\n", x, a, s); ++bad; }
            }
        }
        printf("%lld %lld %lld\n", bad_tab, n, bad);
        return 0;
    }
""")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    d = tmp_path_factory.mktemp("expf")
    src = d / "check.cpp"
    src.write_text(PROGRAM)
    exe = d / "check"
    subprocess.run(["g++", "-std=c++20", "-O2", "-ffp-contract=off", f"-I{CSRC}", str(src),
                    "-o", str(exe), "-lm"], check=True)
    return exe


def test_expf_restatement_matches_host_libm(checker):
    step = 1 if os.environ.get("HM_EXPF_EXHAUSTIVE") == "1" else 3
    out = subprocess.run([str(checker), str(step)], capture_output=True, text=True, check=True)
    bad_tab, n, bad = map(int, out.stdout.split())
    assert bad_tab == 0, "exp2 table differs from long-double 2^(i/32)"
    assert n > ((1 << 32) - (1 << 25)) // step - 100  # all non-NaN patterns on the stride
    assert bad == 0, f"{bad} of {n} inputs differ from libm expf:\n{out.stderr}"
