"""GPU parity of the hyper-connection prepare/finish (q38m_hyper_*,
cuda/q38_hyper.cu:52-114, cuda_backend.cu:1219-1252) with the oracle
restatement.  Bit-exact where the arithmetic is elementwise (repeat, SiLU
and sigmoid steps, stream mix, inject); within one bf16 ulp for the group
RMSNorm (its sum of squares is a reduction whose order the reference does
not fix); stage by stage for the whole prepare (each GEMM stage checked
within three bf16 ulps of the oracle fed the GPU's previous stage, the
mix bit-exact given the GPU's stages).  Then prepare -> MoE -> inject
chained on one layer: the MoE on the GPU's `mixed` equals the oracle bit
for bit, and so does the inject of its output."""
import ctypes

import numpy as np
import pytest

from helpers import Layer, W, device, host, prefill, stream, synth_logits, torch

pytestmark = pytest.mark.gpu


def bf(x):
    from conftest import load_oracle
    return load_oracle().f32_to_bf16(np.asarray(x, np.float32))


def ulp(r):
    r = np.abs(np.asarray(r, np.float64))
    _, e = np.frexp(np.where(r > 0, r, 2.0 ** -126))
    return np.ldexp(1.0, e - 8)


def close(orc, got, want, k):
    g = orc.bf16_to_f32(got).astype(np.float64)
    w = orc.bf16_to_f32(want).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= k * ulp(w) + 1e-30))


def activation_of_admissible_dot(orc, got, x, w, divisor, scale, silu):
    """The GEMM stages round an fp32 dot product to bf16 and then apply an
    activation that is bit-exact given that bf16 (tested above).  An fp32
    sum of n products differs from the exact dot by at most about
    n * 2^-24 * sum |x_i w_i| in the worst case and far less in practice;
    this allows delta = 64 * 2^-24 * sum |x_i w_i|.  Each GPU value must be
    the activation of a bf16 value within delta (plus one bf16 ulp) of the
    exact dot, or, where cancellation leaves the dot many bf16 steps inside
    that interval, within the activation's Lipschitz bound (SiLU slope at
    most 1.1, sigmoid at most 1/4) times scale / divisor of the exact
    activation, plus one output ulp.  Most values must be the activation
    of the exact dot's own bf16 rounding."""
    xf = orc.bf16_to_f32(x).astype(np.float64)
    wf = orc.bf16_to_f32(w).astype(np.float64)
    exact = xf @ wf.T
    delta = 64 * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T)
    centre = orc.f32_to_bf16(exact.astype(np.float32)).astype(np.int32)
    seeds = [centre] + [orc.f32_to_bf16((exact + sgn * delta).astype(np.float32)).astype(np.int32)
                        for sgn in (-1, 1)]
    ok = np.zeros(got.shape, bool)
    for seed in seeds:
        for d in (-2, -1, 0, 1, 2):
            cand = np.clip(seed + d, 0, 0xffff).astype(np.uint16)
            value = orc.bf16_to_f32(cand).astype(np.float64)
            near = np.abs(value - exact) <= delta + ulp(exact)
            ok |= near & (got == orc.hyper_activation(cand, divisor, scale, silu))
    v = exact / divisor
    want = scale * (v if silu else 1.0) / (1.0 + np.exp(-v))
    lipschitz = (1.1 if silu else 0.25) * scale / divisor
    g = orc.bf16_to_f32(got).astype(np.float64)
    ok |= np.abs(g - want) <= lipschitz * (delta + ulp(exact)) + ulp(want)
    exact_match = got == orc.hyper_activation(centre.astype(np.uint16), divisor, scale, silu)
    return bool(ok.all()) and exact_match.mean() > 0.95


def empty(n):
    t = torch()
    return t.empty(n, dtype=t.int16, device="cuda")


@pytest.mark.parametrize("hidden", [2048])
def test_repeat_norm_activation_mix_inject(q38m, orc, hidden):
    t = torch()
    rng = np.random.default_rng(hidden)
    tokens = 5
    emb = bf(rng.standard_normal((tokens, hidden)))
    hyp = empty(tokens * 4 * hidden)
    de = device(emb)
    q38m.call("q38m_hyper_repeat_embedding_bf16", de.data_ptr(), hyp.data_ptr(), tokens, hidden,
              stream(), 0)
    assert np.array_equal(host(hyp, np.uint16).reshape(tokens, 4, hidden),
                          orc.hyper_repeat_embedding(emb))

    x = bf(rng.standard_normal((tokens, 4, hidden)) * rng.uniform(0.05, 20, (tokens, 4, 1)))
    w = bf(rng.standard_normal((4, hidden)) * 0.1)
    dx, dw, out = device(x), device(w), empty(tokens * 4 * hidden)
    q38m.call("q38m_hyper_group_rmsnorm_bf16", dx.data_ptr(), dw.data_ptr(), out.data_ptr(),
              tokens, hidden, stream(), 0)
    got = host(out, np.uint16).reshape(tokens, 4, hidden)
    want = orc.hyper_group_rmsnorm(x, w)
    assert close(orc, got, want, 1)
    assert (got == want).mean() > 0.99

    a = bf(rng.standard_normal((tokens, 320)) * 8)
    da, ao = device(a), empty(tokens * 320)
    for divisor, scale, silu in ((4.0, 1.0, True), (1.0, 1.0, False), (4.0, 2.0, False)):
        name = "q38m_hyper_silu_scaled_bf16" if silu else "q38m_hyper_sigmoid_bf16"
        args = (divisor,) if silu else (divisor, scale)
        q38m.call(name, da.data_ptr(), ao.data_ptr(), tokens, 320, *args, stream(), 0)
        assert np.array_equal(host(ao, np.uint16).reshape(tokens, 320),
                              orc.hyper_activation(a, divisor, scale, silu))

    mixw = bf(rng.uniform(0, 1, (tokens, 4, hidden)))
    dm, mixed = device(mixw), empty(tokens * hidden)
    q38m.call("q38m_hyper_mix_bf16", dx.data_ptr(), dm.data_ptr(), mixed.data_ptr(), tokens,
              hidden, stream(), 0)
    assert np.array_equal(host(mixed, np.uint16).reshape(tokens, hidden), orc.hyper_mix(x, mixw))

    block = bf(rng.standard_normal((tokens, hidden)))
    inj = bf(rng.uniform(0, 2, (tokens, 4)))
    db, di, res = device(block), device(inj), empty(tokens * 4 * hidden)
    q38m.call("q38m_hyper_inject_bf16", dx.data_ptr(), db.data_ptr(), di.data_ptr(),
              res.data_ptr(), tokens, hidden, stream(), 0)
    assert np.array_equal(host(res, np.uint16).reshape(tokens, 4, hidden),
                          orc.hyper_inject(x, block, inj))


def run_prepare(q38m, hyper_d, norm_d, down_d, up_d, inj_d, tokens, hidden, low_rank):
    t = torch()
    scratch = t.empty(q38m.lib().q38m_hyper_prepare_scratch_bytes(tokens, hidden, low_rank) // 2,
                      dtype=t.int16, device="cuda")
    mixed = empty(tokens * hidden)
    injection = empty(tokens * 4)
    q38m.call("q38m_hyper_prepare_v1", hyper_d.data_ptr(), norm_d.data_ptr(), down_d.data_ptr(),
              up_d.data_ptr(), None if inj_d is None else inj_d.data_ptr(), tokens, hidden,
              low_rank, scratch.data_ptr(), mixed.data_ptr(), injection.data_ptr(), stream(), 0)
    t.cuda.synchronize()
    words = host(scratch, np.uint16)
    width = 4 * hidden
    stages = {"normalized": words[:tokens * width].reshape(tokens, 4, hidden),
              "mix": words[tokens * width:2 * tokens * width].reshape(tokens, width),
              "low": words[2 * tokens * width:2 * tokens * width + tokens * low_rank]
              .reshape(tokens, low_rank)}
    return host(mixed, np.uint16).reshape(tokens, hidden), host(injection, np.uint16).reshape(
        tokens, 4), stages


def hyper_weights(rng, hidden, low_rank):
    return (bf(rng.standard_normal((4, hidden)) * 0.1),
            bf(rng.standard_normal((low_rank, 4 * hidden)) * 0.03),
            bf(rng.standard_normal((4 * hidden, low_rank)) * 0.2),
            bf(rng.standard_normal((4, 4 * hidden)) * 0.03))


@pytest.mark.parametrize("tokens,hidden", [(1, 2048), (37, 2048), (512, 2048)])
def test_prepare_stage_by_stage(q38m, orc, tokens, hidden):
    rng = np.random.default_rng(tokens + hidden)
    low_rank = 320
    hyper = bf(rng.standard_normal((tokens, 4, hidden)))
    norm_w, down, up, inj = hyper_weights(rng, hidden, low_rank)
    mixed, injection, st = run_prepare(q38m, device(hyper), device(norm_w), device(down),
                                       device(up), device(inj), tokens, hidden, low_rank)
    want_norm = orc.hyper_group_rmsnorm(hyper, norm_w)
    assert close(orc, st["normalized"], want_norm, 1)
    flat = st["normalized"].reshape(tokens, -1)
    assert activation_of_admissible_dot(orc, st["low"], flat, down, 4.0, 1.0, True)
    assert activation_of_admissible_dot(orc, st["mix"], st["low"], up, 1.0, 1.0, False)
    assert np.array_equal(mixed, orc.hyper_mix(st["normalized"],
                                               st["mix"].reshape(tokens, 4, hidden)))
    assert activation_of_admissible_dot(orc, injection, flat, inj, 4.0, 2.0, False)
    # The whole chain against the oracle's own chain: mixed is a sum over
    # the four streams, so its error is bounded relative to the sum of the
    # terms' magnitudes (a few ulps of mix each), not to mixed itself.
    ref_mixed, _, ref = orc.hyper_prepare(hyper, norm_w, down, up, inj)
    terms = np.abs(orc.bf16_to_f32(ref["normalized"]).astype(np.float64) *
                   orc.bf16_to_f32(ref["mix"]).reshape(tokens, 4, hidden)).sum(axis=1) / 4
    g = orc.bf16_to_f32(mixed).astype(np.float64)
    w = orc.bf16_to_f32(ref_mixed).astype(np.float64)
    assert np.all(np.abs(g - w) <= 2.0 ** -5 * terms + ulp(w))
    assert (mixed == ref_mixed).mean() > 0.9


def test_prepare_moe_inject_chain(q38m, orc):
    """hyper -> prepare (H = 2048) -> MoE slab -> inject on one layer."""
    t = torch()
    tokens, hidden, low_rank = 64, W.HIDDEN, 320
    rng = np.random.default_rng(99)
    hyper = bf(rng.standard_normal((tokens, 4, hidden)))
    norm_w, down, up, inj = hyper_weights(rng, hidden, low_rank)
    hyper_d = device(hyper)
    mixed, injection, _ = run_prepare(q38m, hyper_d, device(norm_w), device(down), device(up),
                                      device(inj), tokens, hidden, low_rank)
    gfmt, dfmt = W.layer_policy(2, 0)
    layer = Layer(q38m, orc, W.CONFIGS[2]["seed"], 0, gfmt, dfmt)
    mixed_d = device(mixed).view(tokens, hidden)
    logits = synth_logits(q38m, 7, 3, tokens)
    ws = q38m.PrefillWorkspace_(tokens)
    block = prefill(q38m, layer, mixed_d, logits, ws)
    ref = orc.moe(mixed, layer.host_gu, layer.host_dn, logits=host(logits, np.float32))
    assert np.array_equal(host(block, np.uint16), ref["output"])
    out = empty(tokens * 4 * hidden)
    inj_d = device(injection)
    q38m.call("q38m_hyper_inject_bf16", hyper_d.data_ptr(), block.data_ptr(), inj_d.data_ptr(),
              out.data_ptr(), tokens, hidden, stream(), 0)
    t.cuda.synchronize()
    assert np.array_equal(host(out, np.uint16).reshape(tokens, 4, hidden),
                          orc.hyper_inject(hyper, ref["output"], injection))
