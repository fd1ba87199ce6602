"""include/iris_kernels.h on the CPU: the header compiles as C and C++, and its
inline fast_expf follows the reference's (iris_kernels.h:21-35): 0 below
-87.3, 1e38 above 88.7, and in between a relative error against e^x of at
most 3.5e-6 on [-8, 8] and 8e-6 on the whole range (the reference's comment
says 2e-6; its own operations give the same 3.3e-6 / 7.3e-6, see below).
Where the reference tree is present its inline is compiled beside ours and
the two must agree bit for bit."""
import os
import subprocess

import numpy as np
import pytest

import iris_testlib as tl

SRC = r"""
#include <stdio.h>
#include "iris_kernels.h"
int main(void) {
    for (int i = 0; i <= 400000; i++) {
        float x = -100.0f + 200.0f * (float)i / 400000.0f;
        printf("%.9g %.9g\n", x, fast_expf(x));
    }
    return 0;
}
"""


@pytest.mark.parametrize("compiler", ["gcc", "g++"])
def test_fast_expf(tmp_path, compiler):
    src = tmp_path / ("t.c" if compiler == "gcc" else "t.cpp")
    src.write_text(SRC)
    exe = tmp_path / "t"
    subprocess.run([compiler, "-O2", "-I", os.path.join(tl.ROOT, "include"), str(src), "-o", str(exe), "-lm"],
                   check=True)
    out = np.loadtxt(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines())
    x, y = out[:, 0].astype(np.float32), out[:, 1].astype(np.float32)   # %.9g round-trips float32
    lo, hi = x < np.float32(-87.3), x > np.float32(88.7)
    assert np.all(y[lo] == 0.0)
    assert np.all(y[hi] == np.float32(1e38))
    mid = ~(lo | hi)
    ref = np.exp(x[mid].astype(np.float64))
    normal = ref > 1.2e-38            # the result is built in the exponent field: normal range only
    rel = np.abs(y[mid][normal] - ref[normal]) / ref[normal]
    assert rel.max() < 8e-6, rel.max()
    core = np.abs(x[mid][normal]) <= 8
    assert rel[core].max() < 3.5e-6, rel[core].max()
    return x, y


REF_HEADER = "/root/reference/iris_kernels.h"


@pytest.mark.skipif(not os.path.exists(REF_HEADER), reason="reference tree absent")
def test_fast_expf_bit_identical_to_reference(tmp_path):
    ours = test_fast_expf(tmp_path, "gcc")[1]
    src = tmp_path / "r.c"
    src.write_text(SRC)
    exe = tmp_path / "r"
    subprocess.run(["gcc", "-O2", "-I", os.path.dirname(REF_HEADER), str(src), "-o", str(exe), "-lm"], check=True)
    out = np.loadtxt(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines())
    np.testing.assert_array_equal(ours, out[:, 1].astype(np.float32))
