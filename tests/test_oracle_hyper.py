"""Oracle hyper-connection restatement (cuda/q38_hyper.cu:52-114, the
prepare_hyper/finish_hyper sequences of cuda/cuda_backend.cu:1219-1252)
pinned by closed forms and an independent float64 evaluation.  The
reference has no unit test for these kernels.

Pins:
- sigmoid(0) = 1/2 and silu(0) = 0 exactly; sigmoid and silu of random
  inputs within one bf16 ulp of a float64 evaluation; sigmoid(x) and
  sigmoid(-x) sum to 1 within two ulps;
- RMSNorm of a constant stream c with weight w is bf16((c / sqrt(c^2 +
  1e-6)) * (1 + w)); random streams within one ulp of a float64 evaluation;
  scaling a stream by 2^k (eps negligible) leaves the result unchanged;
- the stream mix of four equal streams with equal weights is bf16(n * m);
- inject with zero injection or a zero block returns the original, and with
  injection 1 equals the float32-rounded sum;
- the whole prepare within three ulps of an all-float64 evaluation that
  rounds to bf16 at the reference's kernel boundaries.
"""
import numpy as np

from conftest import load_oracle

orc = load_oracle()


def bf(x):
    return orc.f32_to_bf16(np.asarray(x, np.float32))


def f(h):
    return orc.bf16_to_f32(np.asarray(h, np.uint16)).astype(np.float64)


def ulp(r):
    r = np.abs(np.asarray(r, np.float64))
    _, e = np.frexp(np.where(r > 0, r, 2.0 ** -126))
    return np.ldexp(1.0, e - 8)


def within(got, want, k):
    g, w = f(got), f(want)
    return np.all(np.abs(g - w) <= k * ulp(w) + 1e-30)


def test_activation_closed_forms_and_float64():
    zero = bf(np.zeros(4))
    assert np.array_equal(orc.hyper_activation(zero, 4.0, 1.0, False), bf(np.full(4, 0.5)))
    assert np.array_equal(orc.hyper_activation(zero, 4.0, 1.0, True), bf(np.zeros(4)))
    rng = np.random.default_rng(0)
    x = bf(rng.standard_normal(4096) * 6)
    for divisor, scale, silu in ((4.0, 1.0, True), (1.0, 1.0, False), (4.0, 2.0, False)):
        v = f(x) / divisor
        s = 1.0 / (1.0 + np.exp(-v))
        want = bf(((v * s) if silu else s) * scale)
        assert within(orc.hyper_activation(x, divisor, scale, silu), want, 1)
    pos = f(orc.hyper_activation(x, 1.0, 1.0, False))
    neg = f(orc.hyper_activation(bf(-f(x)), 1.0, 1.0, False))
    assert np.all(np.abs(pos + neg - 1.0) <= 2 * ulp(np.maximum(pos, neg)))


def test_rmsnorm_closed_form_and_float64():
    h = 64
    c = np.array([0.5, -3.0, 1e-2, 7.0], np.float32)
    hyper = bf(np.broadcast_to(c[None, :, None], (1, 4, h)))
    w = bf(np.broadcast_to(np.array([0.0, 0.25, -0.5, 1.0], np.float32)[:, None], (4, h)))
    got = orc.hyper_group_rmsnorm(hyper, w)
    cf = f(bf(c))
    want = bf((cf / np.sqrt(cf * cf + 1e-6))[:, None] * (1.0 + f(w)))
    assert within(got[0], want, 1)
    rng = np.random.default_rng(1)
    x = bf(rng.standard_normal((3, 4, 256)) * rng.uniform(0.1, 10, (3, 4, 1)))
    wr = bf(rng.standard_normal((4, 256)) * 0.1)
    xf = f(x)
    inv = 1.0 / np.sqrt(np.mean(xf * xf, axis=-1, keepdims=True) + 1e-6)
    assert within(orc.hyper_group_rmsnorm(x, wr), bf(xf * inv * (1.0 + f(wr))), 1)
    big = bf(rng.standard_normal((2, 4, 256)) * 4)
    assert np.array_equal(orc.hyper_group_rmsnorm(big, wr),
                          orc.hyper_group_rmsnorm(bf(f(big) * 8.0), wr))


def test_mix_and_inject_closed_forms():
    rng = np.random.default_rng(2)
    n = bf(rng.standard_normal((2, 1, 128)))
    m = bf(rng.uniform(0, 1, (2, 1, 128)))
    n4, m4 = np.repeat(n, 4, axis=1), np.repeat(m, 4, axis=1)
    assert np.array_equal(orc.hyper_mix(n4, m4), bf(f(n[:, 0]) * f(m[:, 0])))
    orig = bf(rng.standard_normal((2, 4, 128)))
    block = bf(rng.standard_normal((2, 128)))
    assert np.array_equal(orc.hyper_inject(orig, block, bf(np.zeros((2, 4)))), orig)
    assert np.array_equal(orc.hyper_inject(orig, bf(np.zeros((2, 128))), bf(np.ones((2, 4)))),
                          orig)
    s32 = (f(orig).astype(np.float32) + f(block)[:, None, :].astype(np.float32))
    assert np.array_equal(orc.hyper_inject(orig, block, bf(np.ones((2, 4)))), bf(s32))


def test_prepare_against_float64_chain():
    rng = np.random.default_rng(3)
    t, h, r = 3, 128, 64
    hyper = bf(rng.standard_normal((t, 4, h)))
    norm_w = bf(rng.standard_normal((4, h)) * 0.1)
    down = bf(rng.standard_normal((r, 4 * h)) * 0.05)
    up = bf(rng.standard_normal((4 * h, r)) * 0.2)
    inj = bf(rng.standard_normal((4, 4 * h)) * 0.05)
    mixed, injection, mid = orc.hyper_prepare(hyper, norm_w, down, up, inj)
    # all-float64 chain, bf16 at the reference's kernel boundaries
    x = f(hyper)
    nrm = f(bf(x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6) * (1 + f(norm_w))))
    flat = nrm.reshape(t, -1)
    v = f(bf(flat @ f(down).T)) / 4
    low = f(bf(v / (1 + np.exp(-v))))
    mix = f(bf(1 / (1 + np.exp(-f(bf(low @ f(up).T))))))
    want_mixed = bf((nrm * mix.reshape(t, 4, h)).sum(axis=1) / 4)
    vi = f(bf(flat @ f(inj).T)) / 4
    want_inj = bf(2 / (1 + np.exp(-vi)))
    assert within(mixed, want_mixed, 3)
    assert within(injection, want_inj, 3)
    assert within(mid["normalized"], bf(nrm), 0)
