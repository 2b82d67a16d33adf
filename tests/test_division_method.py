"""The append quantizers' IEEE division x / max(n, 1e-6) (div_by_norm in
kaplumba_amd/csrc/tq_append.h) is formed from the correctly rounded
reciprocal plus one fma refinement.  This CPU check runs the same
arithmetic for every f32 divisor significand against the hardware's IEEE
quotient (tests/csrc/division_method.c); the GPU tests then hold the kernels
bit-exact with the oracle's division, including the rows that take the
division itself (test_append_gpu.py::test_division_edge_vectors)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma_refined_reciprocal_equals_ieee_division(tmp_path):
    src = os.path.join(HERE, "csrc", "division_method.c")
    exe = str(tmp_path / "division_method")
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-pthread", src, "-o", exe, "-lm"],
                   check=True)
    out = subprocess.run([exe], check=True, capture_output=True, text=True, timeout=120).stdout.split()
    pairs, refined_bad, plain_bad = (int(v) for v in out)
    assert pairs == (1 << 23) * 64
    assert refined_bad == 0
    assert plain_bad > pairs // 10  # the plain product is often off: the check is not vacuous
