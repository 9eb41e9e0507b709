"""Pins the oracle's routing against closed forms.

- top-k: numpy lexsort (value desc, id asc) for the ids, the float64
  softmax-renormalised weights within 1e-6, the reference's tie fixture
  (cuda/cuda_kernel_tests.cu:189-252: sin(e*0.037 + t*0.31) with experts
  3 and 7 forced to 2.0, ids exact and weights within 1e-5), and heavy-tie
  logits.
- route plan: the reference's own checks (cuda/cuda_kernel_tests.cu:
  392-611) restated -- compile-time bounds 560/640/800 tasks and 52,552 B,
  the stable expert-major packing from a stable argsort, inverse, M=16
  tasks, fail-closed invalid id -- and the FNV-1a hashes from an
  independent Python FNV implementation.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN_DIR

FNV_OFFSET = 1469598103934665603
FNV_PRIME = 1099511628211
MASK64 = (1 << 64) - 1


def fnv_words(words, h=FNV_OFFSET):
    for w in words:
        h = ((h ^ int(w)) * FNV_PRIME) & MASK64
    return h


def expected_topk(logits, k=10):
    ids = np.empty((logits.shape[0], k), np.int64)
    w = np.empty((logits.shape[0], k), np.float64)
    for t, row in enumerate(logits):
        order = np.lexsort((np.arange(row.size), -row.astype(np.float64)))[:k]
        ids[t] = order
        num = np.exp(row[order].astype(np.float64) - float(row[order[0]]))
        w[t] = num / num.sum()
    return ids, w


def test_topk_random(orc):
    logits = orc.synth_logits(21, 2, 64)
    ids, w = orc.topk(logits)
    eids, ew = expected_topk(logits)
    assert np.array_equal(ids, eids)
    assert np.abs(w - ew).max() < 1e-6


def test_topk_heavy_ties(orc):
    rng = np.random.default_rng(3)
    logits = rng.integers(-3, 3, size=(32, 512)).astype(np.float32)
    ids, w = orc.topk(logits)
    eids, ew = expected_topk(logits)
    assert np.array_equal(ids, eids)
    assert np.abs(w - ew).max() < 1e-6


def test_topk_reference_tie_fixture(orc):
    with open(os.path.join(GOLDEN_DIR, "reference_topk_ties.json")) as f:
        fx = json.load(f)
    logits = np.array(fx["logits"], dtype=np.float32)
    ids, w = orc.topk(logits)
    assert ids.tolist() == fx["ids"]
    assert np.abs(w - np.array(fx["weights"])).max() <= 1e-5
    assert ids[0][0] == 3 and ids[0][1] == 7  # tie at 2.0 broken by id


def test_topk_unnormalised_denominator(orc):
    logits = orc.synth_logits(4, 2, 8)
    ids, w = orc.topk(logits, normalize=False)
    for t in range(8):
        full = np.exp(logits[t].astype(np.float64) - logits[t].max())
        want = full[ids[t]] / full.sum()
        assert np.abs(w[t] - want).max() < 1e-6


def test_plan_compile_time_bounds(orc):
    # cuda/cuda_kernel_tests.cu:529-533
    assert orc.max_tasks(128) == 560
    assert orc.max_tasks(256) == 640
    assert orc.max_tasks(512) == 800
    assert orc.plan_bytes(512) == 52552


def reference_pattern(tokens, repeated):
    a = np.arange(tokens * 10, dtype=np.int64)
    if repeated:
        return np.full(a.size, 7, np.int32)
    return ((a * 73 + (a // 10) * 17) % 512).astype(np.int32)


def check_plan(orc, ids, tokens):
    p = orc.parse_plan(orc.build_plan(ids, tokens, hashes=True), tokens)
    routes = tokens * 10
    counts = np.bincount(ids, minlength=512)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    ntasks = (counts + 15) // 16
    task_offsets = np.concatenate([[0], np.cumsum(ntasks)])
    assert p["magic"] == 0x52383351 and p["version"] == 1
    assert p["tokens"] == tokens and p["routes"] == routes and p["status"] == 0
    assert p["flags"] == 0 and p["reserved0"] == 0 and p["reserved1"] == 0
    assert p["active_experts"] == int((counts > 0).sum())
    assert p["task_count"] == int(task_offsets[-1]) <= orc.max_tasks(tokens)
    assert np.array_equal(p["counts"], counts)
    assert np.array_equal(p["offsets"], offsets)
    assert np.array_equal(p["task_offsets"], task_offsets)
    packed = np.argsort(ids, kind="stable")
    assert np.array_equal(p["packed"], packed)
    assert np.array_equal(p["inverse"][packed], np.arange(routes))
    tasks = p["tasks"]
    for e in np.nonzero(counts)[0]:
        for tile in range(ntasks[e]):
            t = tasks[task_offsets[e] + tile]
            assert t["packed_begin"] == offsets[e] + 16 * tile
            assert t["expert"] == e
            assert t["valid_rows"] == min(16, counts[e] - 16 * tile)
            assert t["flags"] == 0
    assert (tasks[task_offsets[-1]:].view(np.uint64) == 0).all()
    route_hash = fnv_words(ids)
    plan_hash = fnv_words(np.ravel(np.stack([offsets, task_offsets], 1)))
    plan_hash = fnv_words(packed, plan_hash)
    for t in tasks[:task_offsets[-1]]:
        plan_hash = fnv_words([int(t["packed_begin"]) | (int(t["expert"]) << 32),
                               int(t["valid_rows"]) | (int(t["flags"]) << 8)], plan_hash)
    assert p["route_hash"] == route_hash and p["plan_hash"] == plan_hash
    return p


@pytest.mark.parametrize("tokens,repeated", [(1, False), (128, False), (512, False),
                                             (512, True), (3, False)])
def test_plan_reference_cases(orc, tokens, repeated):
    check_plan(orc, reference_pattern(tokens, repeated), tokens)


def test_plan_routed_from_topk(orc):
    ids, _ = orc.topk(orc.synth_logits(8, 2, 512))
    check_plan(orc, ids.ravel(), 512)


def test_plan_without_hashes_zeroes_them(orc):
    ids = reference_pattern(16, False)
    with_h = orc.build_plan(ids, 16, hashes=True)
    without = orc.build_plan(ids, 16, hashes=False)
    p = orc.parse_plan(without, 16)
    assert p["route_hash"] == 0 and p["plan_hash"] == 0
    with_h[32:48] = 0
    assert np.array_equal(with_h, without)


def test_plan_invalid_expert_fails_closed(orc):
    # cuda/cuda_kernel_tests.cu:590-605: experts[4] = -1 -> kInvalidExpert
    tokens = 3
    ids = ((np.arange(30) * 19 + 5) % 512).astype(np.int32)
    ids[4] = -1
    ids[9] = 512
    p = orc.parse_plan(orc.build_plan(ids, tokens), tokens)
    assert p["status"] == 1
    valid = np.ones(30, bool)
    valid[[4, 9]] = False
    # identity initialisation of the reference for invalid assignments
    assert p["inverse"][4] == 4 and p["inverse"][9] == 9
    packed_valid = np.nonzero(valid)[0][np.argsort(ids[valid], kind="stable")]
    assert np.array_equal(p["packed"][:28], packed_valid)
    assert p["packed"][28] == 28 and p["packed"][29] == 29


def test_plan_rejects_bad_token_counts(orc):
    with pytest.raises(ValueError):
        orc.build_plan(np.zeros(5130, np.int32), 513)
