"""The device exp (memvanta_amd/csrc/mvh_expf.h) equals the C library's expf,
which the reference's softmax and SwiGLU call, on every non-NaN binary32
input.  The header is compiled for the host and swept exhaustively."""
import os
import subprocess

import pytest

from conftest import ROOT

PROG = r"""
#include <math.h>
#include <stdio.h>
#include "mvh_expf.h"
int main(void) {
    long bad = 0, n = 0;
    #pragma omp parallel for reduction(+:bad, n) schedule(static)
    for (long long u = 0; u < (1LL << 32); ++u) {
        unsigned b = (unsigned)u; float x; memcpy(&x, &b, 4);
        if (isnan(x)) continue;
        float a = expf(x), c = mvh_expf(x); unsigned ua, uc;
        memcpy(&ua, &a, 4); memcpy(&uc, &c, 4); ++n; bad += ua != uc;
    }
    printf("%ld %ld\n", bad, n);
    return 0;
}
"""


@pytest.mark.slow
def test_expf_matches_libc_on_all_floats(tmp_path):
    src = tmp_path / "sweep.c"
    src.write_text(PROG)
    exe = tmp_path / "sweep"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-I", os.path.join(ROOT, "memvanta_amd", "csrc"),
                    "-o", str(exe), str(src), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    bad, n = int(out[0]), int(out[1])
    assert n == 4278190082
    assert bad == 0
