"""Writes the committed fixtures under tests/golden/.

reference_topk_ties.json  -- the reference's top-k tie fixture
    (cuda/cuda_kernel_tests.cu:189-252): logits bf16(sin(e*0.037 + t*0.31))
    for 2 tokens x 512 experts with experts 3 and 7 forced to 2.0; ids by a
    Python sort on (value desc, id asc); weights exp(l_r - l_0) / sum in
    float64.
reference_grouped_kat.json -- the reference's one-hot grouped-MoE known
    answer (cuda/cuda_kernel_tests.cu:613-868) restated for the int8
    contract: 2 tokens, hidden one-hot 1.0 / 2.0 at column 0, all 10 routes
    on expert 0 with weight 0.1, gate row 0 / up row I / down row 0 one-hot
    at column 0 with unit scales.  Expected output word per token from the
    closed-form rounding sequence below (numpy float32 steps, float64 exp
    rounded to float32 -- independent of the oracle's exp).
config1_slice.npz -- the first 4 tokens of config 1 (seed 1): hidden,
    logits, and the oracle's ids / weights / output, a regression anchor
    for the oracle and a committed target for the GPU path.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests"))


def bf16_bits(x):
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return int((b + 0x7FFF + ((b >> 16) & 1)) >> 16)


def bf16r(x):
    return np.uint32(bf16_bits(x) << 16).view(np.float32)


def topk_ties():
    logits = np.empty((2, 512), np.float32)
    for t in range(2):
        for e in range(512):
            v = np.sin(np.float32(e) * np.float32(0.037) + np.float32(t) * np.float32(0.31),
                       dtype=np.float32)
            if e in (3, 7):
                v = np.float32(2.0)
            logits[t, e] = bf16r(v)
    ids, weights = [], []
    for t in range(2):
        order = sorted(range(512), key=lambda e: (-float(logits[t, e]), e))[:10]
        num = [math.exp(float(logits[t, e]) - float(logits[t, order[0]])) for e in order]
        ids.append(order)
        weights.append([n / sum(num) for n in num])
    return {"logits": logits.tolist(), "ids": ids, "weights": weights}


def kat_word(v):
    f32 = np.float32
    s_t = f32(v) / f32(127.0)
    q = np.rint(f32(v) / s_t)
    assert q == 127.0
    y = f32(127.0) * f32(1.0)
    y = y * s_t
    g = bf16r(y)
    u = bf16r(y)
    e = f32(math.exp(-float(g)))
    silu = g / (f32(1.0) + e)
    h = bf16r(silu * u)
    m = bf16r(h * f32(0.1))
    s_m = m / f32(127.0)
    assert np.rint(m / s_m) == 127.0
    o = (f32(127.0) * f32(1.0)) * s_m
    acc = f32(0.0)
    for _ in range(10):
        acc = f32(acc + o)
    return bf16_bits(acc)


def grouped_kat():
    return {"hidden_values": [1.0, 2.0], "route_weight": 0.1, "expert": 0,
            "expected_word_col0": [kat_word(1.0), kat_word(2.0)]}


def config1_slice():
    import oracle as O
    from conftest import load_product  # noqa: F401  (workloads lives in the package)
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "workloads", os.path.join(ROOT, "qwen3.8-flash-next-dual-gpu_amd", "workloads.py"))
    W = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(W)
    seed = W.CONFIGS[1]["seed"]
    gu_tag, dn_tag, h_tag, l_tag = W.layer_tags(0)
    T = 4
    gu = O.synth_weights(seed, gu_tag, 4, 32, 512, 2 * W.INTER, W.HIDDEN, 0.02)
    dn = O.synth_weights(seed, dn_tag, 4, 32, 512, W.HIDDEN, W.INTER, 0.02)
    hidden = O.synth_normal_bf16(seed, h_tag, T * W.HIDDEN).reshape(T, W.HIDDEN)
    logits = O.synth_logits(seed, l_tag, T)
    r = O.moe(hidden, gu, dn, logits=logits)
    return {"hidden": hidden, "logits": logits, "ids": r["ids"], "weights": r["weights"],
            "output": r["output"]}


def main():
    with open(os.path.join(HERE, "reference_topk_ties.json"), "w") as f:
        json.dump(topk_ties(), f)
    with open(os.path.join(HERE, "reference_grouped_kat.json"), "w") as f:
        json.dump(grouped_kat(), f, indent=1)
    np.savez(os.path.join(HERE, "config1_slice.npz"), **config1_slice())


if __name__ == "__main__":
    main()
