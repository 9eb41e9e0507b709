"""The chunk-path SwiGLU gate table (csrc/q38m_silu_gen.c ->
_build/q38m_silu_table.inc, read by the wide gate/up kernels).

silu(g) = g / (1 + exp(-g)) enters the contract with g already rounded to
bf16 (q38_moe_prefill.cu:449-461), so the table holds it for all 65,536 bf16
patterns.  Checked on the CPU:
- every entry against the oracle's evaluation (its exp, an IEEE float32
  division in numpy), bit for bit, NaN results as NaN;
- independently of the oracle, against float64 g / (1 + exp(-g)) within
  2 ulps over the normal range, and the exact special cases: silu(+-0) keeps
  the sign of zero, silu(g) = g once exp(-g) < 2^-25, silu(g) = g / 2 for
  subnormal g, silu(+inf) = +inf, silu(-inf) and silu(NaN) are NaN.
The GPU tests of the chunk path (tests/test_gpu_wide.py, tests/
test_gpu_formats.py) then compare the kernels that read it with the oracle.
"""
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import PACKAGE_DIR

TABLE = os.path.join(PACKAGE_DIR, "_build", "q38m_silu_table.inc")


@pytest.fixture(scope="module")
def table():
    subprocess.run(["make", "-C", PACKAGE_DIR, "-s", "_build/q38m_silu_table.inc"], check=True)
    with open(TABLE) as f:
        words = [int(w, 16) for w in re.findall(r"0x([0-9a-f]{8})u", f.read())]
    assert len(words) == 65536
    return np.array(words, dtype=np.uint32)


def gates():
    return (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)


def test_table_equals_oracle_silu(table, orc):
    g = gates()
    with np.errstate(all="ignore"):
        ref = g / (np.float32(1.0) + orc.expf(-g))
    got = table.view(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(table[~nan], ref.view(np.uint32)[~nan])


def test_table_against_float64_and_special_cases(table):
    g = gates()
    got = table.view(np.float32)
    finite = np.isfinite(g) & (np.abs(g) > np.float32(2.0 ** -126)) & (g > -87.0)
    g64 = g[finite].astype(np.float64)
    with np.errstate(over="ignore"):
        ref = g64 / (1.0 + np.exp(-g64))
    spacing = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    assert (np.abs(got[finite].astype(np.float64) - ref) / spacing).max() <= 2.0
    # +-0 and subnormal g: exp(-g) = 1, silu = g / 2 exactly
    sub = (np.abs(g) < np.float32(2.0 ** -126))
    assert np.array_equal(got[sub], g[sub] / np.float32(2.0))
    assert np.signbit(got[0x8000]) and got[0x8000] == 0.0 and not np.signbit(got[0])
    # large g: 1 + exp(-g) rounds to 1
    big = np.isfinite(g) & (g >= np.float32(18.0))
    assert np.array_equal(got[big], g[big])
    assert got[0x7F80] == np.inf
    assert np.isnan(got[0xFF80]) and np.isnan(got[0x7FC0]) and np.isnan(got[0xFFC0])
