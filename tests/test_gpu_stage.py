"""The C++ MoE stage (include/q38m_stage.hpp: run_moe, prepare/finish_hyper
and the slab x layer loop of run_prefill, cuda/cuda_backend.cu:1516-1605,
:1905-2022) compiled against libq38m.so and run on the GPU by its driver
program (host/run_moe_check.cpp, built by the package Makefile).

1,025 tokens through two config-2 layers: two 512-token slabs take
run_moe's grouped prefill branch and the one-token tail slab its decode
branch.  Every run_moe call's block output must equal the CPU oracle's MoE
step bit for bit, given the call's own inputs (the mixed rows the
hyper-connection prepare wrote, the router logits and the shared expert's
output and gate, which are floating-point GEMMs with their own tolerance
tests), and the stage's own loop must end in the same hyper state as the
loop written out call by call."""
import os
import subprocess

import numpy as np
import pytest

from conftest import PACKAGE_DIR
from helpers import Layer, W

pytestmark = pytest.mark.gpu

EXE = os.path.join(PACKAGE_DIR, "_build", "run_moe_check")


def load(path, dtype, shape):
    return np.fromfile(path, dtype=dtype).reshape(shape)


def test_cpp_stage_run_moe_and_slab_loop(q38m, orc, tmp_path):
    assert os.path.exists(EXE), "build the package (make -C qwen3.8-flash-next-dual-gpu_amd)"
    count, layers, seed = 1025, 2, W.CONFIGS[2]["seed"]
    print(f"run_moe_check: {count} tokens, {layers} layers, seed {seed}", flush=True)
    run = subprocess.run([EXE, str(tmp_path), str(count), str(layers), str(seed)],
                         capture_output=True, text=True, timeout=240)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "3 slabs, 2 layers done" in run.stdout
    final_explicit = np.fromfile(tmp_path / "final_explicit.bin", dtype=np.uint16)
    final_product = np.fromfile(tmp_path / "final_product.bin", dtype=np.uint16)
    assert final_explicit.size == count * 4 * W.HIDDEN
    assert np.array_equal(final_explicit, final_product)

    gfmt, dfmt = W.layer_policy(2, 0)
    slabs = [(0, 512), (1, 512), (2, 1)]
    for l in range(layers):
        layer = Layer(q38m, orc, seed, l, gfmt, dfmt)
        layer.drop_row_major()
        for s, tokens in slabs:
            stem = tmp_path / f"s{s}_l{l}_"
            mixed = load(str(stem) + "mixed.bin", np.uint16, (tokens, W.HIDDEN))
            logits = load(str(stem) + "logits.bin", np.float32, (tokens, W.EXPERTS))
            so = load(str(stem) + "shared_output.bin", np.uint16, (tokens, W.HIDDEN))
            sg = load(str(stem) + "shared_gate.bin", np.uint16, (tokens,))
            got = load(str(stem) + "block_output.bin", np.uint16, (tokens, W.HIDDEN))
            assert np.isfinite(orc.bf16_to_f32(mixed)).all()
            ref = orc.moe(mixed, layer.host_gu, layer.host_dn, logits=logits, shared_output=so,
                          shared_gate=sg)
            bad = int((got != ref["output"]).sum())
            assert bad == 0, f"layer {l} slab {s}: {bad} words differ"
        del layer
