"""Pins the oracle's scalar arithmetic against independent references.

- exp: the contract's Cody-Waite + degree-7 Taylor exp against float64
  numpy.exp within 1 ulp over its whole normal range, exact at 0, and the
  documented overflow/flush edges.
- bf16 RNE: against torch's float32 -> bfloat16 cast (a library RNE), the
  reference's round-trip test values (tests/test_artifact_compiler.py:49-53)
  and hand-worked ties.
- fp16: against numpy's float16 cast, including subnormals and overflow.
- int4 packing: the reference's known answer [-7,-1,0,7] -> [0xF9, 0x70]
  (tests/test_artifact_compiler.py:66-71) through the oracle's unpacking.
- synthetic generators: distribution moments and ranges (not a retyping of
  the generator; a wrong sign/scale/range fails them).
"""
import numpy as np
import pytest
import torch


def ulp_error(got, ref64):
    spacing = np.spacing(np.abs(ref64).astype(np.float32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - ref64) / spacing


def test_expf_within_one_ulp(orc):
    x = np.linspace(-87.3, 88.7, 400001, dtype=np.float64).astype(np.float32)
    got = orc.expf(x)
    assert ulp_error(got, np.exp(x.astype(np.float64))).max() <= 1.0


def test_expf_special_values(orc):
    x = np.array([0.0, -0.0, 1.0, -1.0, 88.8, 100.0, -87.31, -200.0, np.inf, -np.inf],
                 dtype=np.float32)
    got = orc.expf(x)
    assert got[0] == 1.0 and got[1] == 1.0
    assert abs(got[2] - np.float32(np.e)) <= np.spacing(np.float32(np.e))
    assert np.isinf(got[4]) and np.isinf(got[5]) and np.isinf(got[8])
    assert got[6] == 0.0 and got[7] == 0.0 and got[9] == 0.0
    assert np.isnan(orc.expf(np.array([np.nan], dtype=np.float32)))[0]


def test_bf16_rne_matches_torch(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0),
        rng.standard_normal(1000).astype(np.float32) * np.float32(1e-30),
        np.array([3.3895314e38, -3.3895314e38, 1e-40, 0.0, -0.0], dtype=np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), ref)


def test_bf16_reference_roundtrip_and_ties(orc):
    # tests/test_artifact_compiler.py:49-53
    src = np.array([-448.0, -1.5, -0.0, 0.125, 1.0, 448.0], dtype=np.float32)
    back = orc.bf16_to_f32(orc.f32_to_bf16(src))
    np.testing.assert_allclose(back, src, rtol=0.008, atol=0.001)
    # ties to even: 1 + 2^-8 -> 1.0 ; 1 + 3*2^-8 -> 1 + 2^-6 ; just above a tie rounds up
    ties = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20],
                    dtype=np.float32)
    assert orc.f32_to_bf16(ties).tolist() == [0x3F80, 0x3F82, 0x3F81]


def test_f16_conversions_match_numpy(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        np.abs(rng.standard_normal(200000)).astype(np.float32) * np.float32(0.02),
        np.array([6.1035156e-05, 6.0e-05, 2.9802322e-08, 2.9802326e-08, 5.9604645e-08,
                  65504.0, 65519.99, 1e-12, -0.0, -3.0e-7], dtype=np.float32),
    ])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16(x), ref)
    assert orc.f32_to_f16(np.array([65520.0, 1e6], np.float32)).tolist() == [0x7C00, 0x7C00]
    h = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_int4_packing_known_answer(orc):
    # tests/test_artifact_compiler.py:66-71: [-7,-1,0,7] packs to [0xF9, 0x70]
    w = orc.HostWeights(np.array([0xF9, 0x70], np.uint8), np.zeros(1, np.uint16), 4, 0, 1, 1, 4)
    assert w.unpacked(0).tolist() == [[-7, -1, 0, 7]]
    # and -8 is representable (two's complement nibble 0x8)
    w = orc.HostWeights(np.array([0x78], np.uint8), np.zeros(1, np.uint16), 4, 0, 1, 1, 2)
    assert w.unpacked(0).tolist() == [[-8, 7]]


def test_synth_distributions(orc):
    n = 1 << 18
    z = orc.synth_normal_f32(11, 3, n)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert abs(float(((z - z.mean()) ** 3).mean())) < 0.03  # symmetric
    assert np.abs(z).max() < 7.0
    a = orc.f16_to_f32(orc.synth_abs_normal_f16(11, 4, n, 0.02))
    assert (a >= 0).all() and abs(a.mean() - 0.02 * np.sqrt(2 / np.pi)) < 3e-4
    w = orc.synth_uniform_w4(11, 5, n)
    vals = orc.HostWeights(w, np.zeros(1, np.uint16), 4, 0, 1, 1, n).unpacked(0).ravel()
    counts = np.bincount(vals.astype(np.int64) + 8, minlength=16)
    assert vals.min() == -8 and vals.max() == 7
    assert counts.min() > 0.9 * n / 16 and counts.max() < 1.1 * n / 16
    i8 = orc.synth_uniform_i8(11, 6, n)
    assert i8.min() == -127 and i8.max() == 127 and abs(i8.astype(np.float64).mean()) < 0.5
    # counter-based: a prefix of a longer draw is the shorter draw
    assert np.array_equal(orc.synth_normal_f32(11, 3, 1000), z[:1000])
    # different tags give different streams
    assert not np.array_equal(orc.synth_normal_f32(11, 4, 1000), z[:1000])


def test_logits_bias_is_added(orc):
    bias = np.linspace(-3, 3, 512).astype(np.float32)
    plain = orc.synth_logits(5, 2, 4)
    biased = orc.synth_logits(5, 2, 4, bias=bias)
    assert np.array_equal(biased, (plain + bias[None, :]).astype(np.float32))


def test_oracle_threads_bit_identical(orc):
    seed, T, H, I = 3, 6, 2048, 512
    gu = orc.synth_weights(seed, 10, 4, 32, 512, 2 * I, H, 0.02)
    dn = orc.synth_weights(seed, 20, 8, 0, 512, H, I, 0.002)
    hid = orc.synth_normal_bf16(seed, 1, T * H).reshape(T, H)
    lg = orc.synth_logits(seed, 2, T)
    threads = orc.num_threads()
    try:
        orc.set_threads(1)
        one = orc.moe(hid, gu, dn, logits=lg)["output"]
        orc.set_threads(max(2, threads))
        many = orc.moe(hid, gu, dn, logits=lg)["output"]
    finally:
        orc.set_threads(threads)
    assert np.array_equal(one, many)


@pytest.mark.parametrize("x", [1e-30, 0.37, 1.0, 2.5, 1e30])
def test_logf_close(orc, x):
    got = orc.lib().q38o_logf(x)
    assert abs(got - np.log(np.float64(np.float32(x)))) <= 2 * np.spacing(np.float32(abs(got) or 1))


def test_decode_combine_shared_is_one_fma(orc):
    """q38o_combine_shared: bf16(routed + shared * sigmoid(gate)) with the
    sum contracted into one fma (nvcc's default -fmad on the reference
    expression, cuda/q38_moe.cu:348-349).  Where the float64 sum of the
    exact product and routed is itself exact, rounding it once to float32
    is the fma; those elements must agree.  The rows also hold pairs found
    by search whose bf16 result differs between the fma and a separately
    rounded multiply-then-add, so an unfused restatement fails here."""
    rng = np.random.default_rng(348)
    tokens, hidden = 16, 256
    gate = orc.f32_to_bf16(rng.standard_normal(tokens) * 3)
    g = orc.bf16_to_f32(gate)
    sig = (np.float32(1.0) / (np.float32(1.0) + orc.expf(-g))).astype(np.float32)
    routed = orc.f32_to_bf16(rng.standard_normal((tokens, hidden)) * 4)
    shared = orc.f32_to_bf16(rng.standard_normal((tokens, hidden)) * 4)
    planted = 0
    for t in range(tokens):
        cr = orc.f32_to_bf16(rng.standard_normal(1 << 16) * 4)
        cs = orc.f32_to_bf16(rng.standard_normal(1 << 16) * 4)
        rf, sf = orc.bf16_to_f32(cr), orc.bf16_to_f32(cs)
        prod64 = sf.astype(np.float64) * np.float64(sig[t])
        sum64 = prod64 + rf.astype(np.float64)
        ok = ((sum64 - prod64) == rf) & ((sum64 - rf) == prod64)
        fused = orc.f32_to_bf16(sum64.astype(np.float32))
        unfused = orc.f32_to_bf16(rf + (sf * sig[t]).astype(np.float32))
        hits = np.flatnonzero(ok & (fused != unfused))[:4]
        routed[t, :hits.size], shared[t, :hits.size] = cr[hits], cs[hits]
        planted += hits.size
    assert planted >= 8
    got = orc.combine_shared(routed, shared, gate)
    r = orc.bf16_to_f32(routed).astype(np.float64)
    p = orc.bf16_to_f32(shared).astype(np.float64) * sig.astype(np.float64)[:, None]
    total = p + r
    exact = ((total - p) == r) & ((total - r) == p)
    assert exact.mean() > 0.9
    assert np.array_equal(got[exact], orc.f32_to_bf16(total.astype(np.float32))[exact])
    unfused = orc.f32_to_bf16(orc.bf16_to_f32(routed) +
                              (orc.bf16_to_f32(shared) * sig[:, None]).astype(np.float32))
    assert (got != unfused).sum() >= planted
