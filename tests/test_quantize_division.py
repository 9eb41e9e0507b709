"""The row quantisers' division-free quotient, checked exhaustively on the CPU.

The device quantisers (csrc/q38m_select.h, quant_scale and quantize8) form
rint(x/s) for bf16 x with |x| <= absmax, s = absmax/127, from r = RN(1/s)
and one Markstein correction step (two fmas) instead of an IEEE division
per value, for scales in [2^-120, FLT_MAX]; tiny and infinite scales keep
the division.  tests/quantize_division_check.c enumerates every such
(absmax, x) pair of bf16 values (5.3e8) and compares the rounded quotient
with rint of the correctly rounded division; the same float operations
(mul, fma, rint, IEEE division, subnormals kept) run on the device.  The
uncorrected product rint(RN(x r)) is counted as a control: it must differ
somewhere, or the check would not distinguish anything.  The GPU tests of
every quantiser (rows, tokens, decode mid rows) then compare the int8
outputs with the oracle's division.
"""
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("qdiv") / "check")
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", exe,
                    os.path.join(HERE, "quantize_division_check.c"), "-lm"], check=True)
    return exe


def test_markstein_quotient_rounds_like_the_division(checker):
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([checker], check=True, capture_output=True, text=True, env=env,
                         timeout=600).stdout
    m = re.search(r"pairs (\d+) mismatches (\d+) uncorrected_mismatches (\d+)", out)
    assert m, out
    pairs, mismatches, uncorrected = map(int, m.groups())
    assert pairs > 500_000_000
    assert mismatches == 0
    assert uncorrected > 0
