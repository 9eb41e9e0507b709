"""GPU parity of the building blocks against the CPU oracle, bit for bit:
the int8 MFMA lane layout, the contract's exp, the synthetic generators,
row quantisation, top-k, the route plan (all the reference's plan cases,
with and without hashes, double run over 0xa5-poisoned storage as in
cuda/cuda_kernel_tests.cu:412-468, fail-closed invalid ids), the bf16
gather (cuda_kernel_tests.cu:539-588), the MFMA16 weight layouts and the
residual add."""
import ctypes
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN_DIR
from helpers import W, device, host, stream, torch

pytestmark = pytest.mark.gpu


def sync():
    torch().cuda.synchronize()


def test_mfma_i8_lane_layout(q38m):
    rng = np.random.default_rng(0)
    a = rng.integers(-128, 128, (16, 32)).astype(np.int8)
    b = rng.integers(-128, 128, (32, 16)).astype(np.int8)
    t = torch()
    d = t.zeros(256, dtype=t.int32, device="cuda")
    da, db = device(a), device(b)  # keep both alive until the kernel has run
    q38m.call_selftest("q38m_debug_mfma_16x16x32_i8", da.data_ptr(), db.data_ptr(), d.data_ptr(),
              stream(), 0)
    got = host(d, np.int32).reshape(16, 16)
    assert np.array_equal(got, a.astype(np.int64) @ b.astype(np.int64))


def test_mfma_i8_32x32_lane_layout(q38m):
    rng = np.random.default_rng(3)
    a = rng.integers(-128, 128, (32, 32)).astype(np.int8)
    b = rng.integers(-128, 128, (32, 32)).astype(np.int8)
    t = torch()
    d = t.zeros(1024, dtype=t.int32, device="cuda")
    da, db = device(a), device(b)
    q38m.call_selftest("q38m_debug_mfma_32x32x32_i8", da.data_ptr(), db.data_ptr(), d.data_ptr(),
              stream(), 0)
    got = host(d, np.int32).reshape(32, 32)
    assert np.array_equal(got, a.astype(np.int64) @ b.astype(np.int64))


def test_expf_bitwise(q38m, orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        np.linspace(-90, 90, 300001, dtype=np.float32),
        rng.standard_normal(100000).astype(np.float32) * np.float32(30),
        np.array([0.0, -0.0, 88.72283, 88.72284, -87.3, -87.29999, np.inf, -np.inf],
                 dtype=np.float32)])
    t = torch()
    xd = device(x)
    out = t.empty_like(xd)
    q38m.call_selftest("q38m_debug_expf", xd.data_ptr(), x.size, out.data_ptr(), stream(), 0)
    got = host(out, np.float32)
    assert np.array_equal(got.view(np.uint32), orc.expf(x).view(np.uint32))


def test_bf16_hardware_conversion_sweep(q38m):
    """Every fp32 bit pattern: the hardware conversion (v_cvt_pk_bf16_f32)
    against the contract's integer round-to-nearest-even, on the device."""
    t = torch()
    result = device(np.array([0, 0xFFFFFFFF, 0, 0xFFFFFFFF], np.uint32).view(np.int32))
    q38m.call_selftest("q38m_debug_bf16_sweep", result.data_ptr(), stream(), 0)
    got = host(result, np.int32).view(np.uint32)
    print(f"bf16 sweep: mismatches {got[0]} (first {got[1]:#010x}), "
          f"non-NaN mismatches {got[2]} (first {got[3]:#010x})")
    assert got[2] == 0, f"non-NaN mismatch at {got[3]:#010x}"
    assert got[0] == 0, f"NaN mismatch at {got[1]:#010x}"


@pytest.mark.parametrize("kind", ["normal_f32", "bias_f32", "bf16", "abs_f16", "w4", "i8"])
def test_synth_matches_oracle(q38m, orc, kind):
    t = torch()
    n = 1 << 20
    seed, tag = 1234, 77
    if kind in ("normal_f32", "bias_f32"):
        bias = np.array(W.zipf_bias(9, 3, 1.1), np.float32) if kind == "bias_f32" else None
        out = t.empty(n, dtype=t.float32, device="cuda")
        q38m.synth_fill(q38m.SYNTH_NORMAL_F32, seed, tag, n, out, sigma=1.0,
                        bias=None if bias is None else device(bias))
        want = orc.synth_logits(seed, tag, n // 512, 512, bias=bias).ravel()
        got = host(out, np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    elif kind == "bf16":
        out = t.empty(n, dtype=t.int16, device="cuda")
        q38m.synth_fill(q38m.SYNTH_NORMAL_BF16, seed, tag, n, out, sigma=1.0)
        assert np.array_equal(host(out, np.uint16), orc.synth_normal_bf16(seed, tag, n))
    elif kind == "abs_f16":
        out = t.empty(n, dtype=t.int16, device="cuda")
        q38m.synth_fill(q38m.SYNTH_ABS_NORMAL_F16, seed, tag, n, out, sigma=0.02)
        assert np.array_equal(host(out, np.uint16), orc.synth_abs_normal_f16(seed, tag, n, 0.02))
    elif kind == "w4":
        out = t.empty(n // 2, dtype=t.uint8, device="cuda")
        q38m.synth_fill(q38m.SYNTH_UNIFORM_W4, seed, tag, n, out, lo=-8, hi=7)
        assert np.array_equal(host(out, np.uint8), orc.synth_uniform_w4(seed, tag, n))
    else:
        out = t.empty(n, dtype=t.int8, device="cuda")
        q38m.synth_fill(q38m.SYNTH_UNIFORM_I8, seed, tag, n, out, lo=-127, hi=127)
        assert np.array_equal(host(out, np.int8), orc.synth_uniform_i8(seed, tag, n))


@pytest.mark.parametrize("width", [512, 2048])
def test_quantize_rows_bitwise(q38m, orc, width):
    rng = np.random.default_rng(width)
    rows = 1000
    x = (rng.standard_normal((rows, width)) * rng.uniform(1e-3, 100, (rows, 1))).astype(np.float32)
    x[5] = 0.0
    x[9, 3] = 3e38
    # non-finite rows (an overflowed decode state): inf elements, a NaN
    x[11, 4], x[11, 8] = np.inf, -np.inf
    x[12, 6] = np.nan
    x[13] = np.inf
    h = orc.f32_to_bf16(x)
    t = torch()
    q = t.empty(rows * width, dtype=t.int8, device="cuda")
    s = t.empty(rows, dtype=t.float32, device="cuda")
    hd = device(h)
    q38m.call("q38m_quantize_rows_i8", hd.data_ptr(), rows, width, q.data_ptr(),
              s.data_ptr(), stream(), 0)
    wq, ws = orc.quantize_rows(h, width)
    assert np.array_equal(host(q, np.int8).reshape(rows, width), wq)
    assert np.array_equal(host(s, np.float32).view(np.uint32), ws.view(np.uint32))


def run_topk(q38m, logits, top_k=10, normalize=True):
    t = torch()
    tokens, experts = logits.shape
    ids = t.empty(tokens * top_k, dtype=t.int32, device="cuda")
    w = t.empty(tokens * top_k, dtype=t.float32, device="cuda")
    ld = device(logits)
    q38m.call("q38m_topk_router_f32", ld.data_ptr(), ids.data_ptr(), w.data_ptr(),
              tokens, experts, top_k, int(normalize), stream(), 0)
    return host(ids, np.int32).reshape(tokens, top_k), host(w, np.float32).reshape(tokens, top_k)


def run_topk_bf16(q38m, words, top_k=10, normalize=True):
    t = torch()
    tokens, experts = words.shape
    ids = t.empty(tokens * top_k, dtype=t.int32, device="cuda")
    w = t.empty(tokens * top_k, dtype=t.float32, device="cuda")
    ld = device(words.view(np.int16))
    q38m.call("q38m_topk_router_bf16", ld.data_ptr(), ids.data_ptr(), w.data_ptr(),
              tokens, experts, top_k, int(normalize), stream(), 0)
    return host(ids, np.int32).reshape(tokens, top_k), host(w, np.float32).reshape(tokens, top_k)


@pytest.mark.parametrize("case", ["synthetic", "ties", "reference_ties", "unnormalised",
                                  "signed_zeros", "top4", "experts256"])
def test_topk_bf16_bitwise(q38m, orc, case):
    """cuda_topk_router_bf16's surface: bf16 logits (the reference router's
    output type).  bf16 -> fp32 is exact, so the oracle runs on the widened
    values; rounding fp32 logits to bf16 also creates many exact ties."""
    rng = np.random.default_rng(31)
    top_k, normalize, experts = 10, case != "unnormalised", 512
    if case == "synthetic" or case == "unnormalised":
        logits = orc.synth_logits(11, 2, 256)
    elif case == "ties":
        logits = rng.integers(-3, 3, (200, 512)).astype(np.float32) * np.float32(0.125)
    elif case == "reference_ties":
        with open(os.path.join(GOLDEN_DIR, "reference_topk_ties.json")) as f:
            logits = np.array(json.load(f)["logits"], np.float32)
    elif case == "signed_zeros":
        logits = (-1.0 - np.abs(rng.standard_normal((64, 512)))).astype(np.float32)
        for row in logits:
            picks = rng.choice(512, 14, replace=False)
            row[picks] = np.where(rng.random(14) < 0.5, np.float32(0.0), np.float32(-0.0))
    elif case == "top4":
        logits, top_k = orc.synth_logits(12, 2, 100), 4
    else:
        logits, top_k, experts = orc.synth_logits(13, 2, 100)[:, :256].copy(), 8, 256
    words = orc.f32_to_bf16(logits).reshape(logits.shape[0], experts)
    widened = (words.astype(np.uint32) << 16).view(np.float32)
    ids, w = run_topk_bf16(q38m, words, top_k=top_k, normalize=normalize)
    wids, ww = orc.topk(widened, top_k=top_k, normalize=normalize)
    assert np.array_equal(ids, wids)
    assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))
    fids, fw = run_topk(q38m, widened, top_k=top_k, normalize=normalize)
    assert np.array_equal(ids, fids)
    assert np.array_equal(w.view(np.uint32), fw.view(np.uint32))


@pytest.mark.parametrize("case", ["synthetic", "zipf", "ties", "reference_ties", "unnormalised",
                                  "signed_zeros", "top4", "experts256"])
def test_topk_bitwise(q38m, orc, case):
    """512 experts with top_k <= 10 (normalised) run the ranked-key
    kernel; other shapes the wave-per-token kernel."""
    top_k, normalize = 10, case != "unnormalised"
    if case == "signed_zeros":
        rng = np.random.default_rng(12)
        logits = (-1.0 - np.abs(rng.standard_normal((64, 512)))).astype(np.float32)
        for row in logits:
            picks = rng.choice(512, 14, replace=False)
            row[picks] = np.where(rng.random(14) < 0.5, np.float32(0.0), np.float32(-0.0))
        ids, w = run_topk(q38m, logits)
        wids, ww = orc.topk(logits)
        assert np.array_equal(ids, wids)
        assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))
        return
    if case == "top4":
        logits = orc.synth_logits(7, 2, 200)
        ids, w = run_topk(q38m, logits, top_k=4)
        wids, ww = orc.topk(logits, top_k=4)
        assert np.array_equal(ids, wids)
        assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))
        return
    if case == "experts256":
        logits = orc.synth_logits(8, 2, 100)[:, :256].copy()
        ids, w = run_topk(q38m, logits, top_k=8)
        wids, ww = orc.topk(logits, top_k=8)
        assert np.array_equal(ids, wids)
        assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))
        return
    if case == "synthetic":
        logits = orc.synth_logits(5, 2, 512)
    elif case == "zipf":
        logits = orc.synth_logits(5, 2, 512, bias=np.array(W.zipf_bias(5, 9, 1.1), np.float32))
    elif case == "ties":
        logits = np.random.default_rng(2).integers(-2, 2, (300, 512)).astype(np.float32)
    elif case == "reference_ties":
        with open(os.path.join(GOLDEN_DIR, "reference_topk_ties.json")) as f:
            logits = np.array(json.load(f)["logits"], np.float32)
    else:
        logits = orc.synth_logits(6, 2, 64)
    normalize = case != "unnormalised"
    ids, w = run_topk(q38m, logits, normalize=normalize)
    wids, ww = orc.topk(logits, normalize=normalize)
    assert np.array_equal(ids, wids)
    assert np.array_equal(w.view(np.uint32), ww.view(np.uint32))


@pytest.mark.parametrize("tokens", [1, 64, 512])
def test_route_quantize_bitwise(q38m, orc, tokens):
    """q38m_moe_route_quantize_v1: top-10 ids and weights and the int8
    rows equal the oracle's top-k and row quantiser bit for bit."""
    t = torch()
    logits = orc.synth_logits(21, 2, tokens)
    logits[0, 17] = logits[0].max()  # a tie at the top
    rng = np.random.default_rng(tokens)
    x = (rng.standard_normal((tokens, 2048)) * rng.uniform(1e-3, 50, (tokens, 1))).astype(np.float32)
    if tokens > 3:
        x[3] = 0.0
    h = orc.f32_to_bf16(x)
    ld, hd = device(logits), device(h)
    ids = t.empty(tokens * 10, dtype=t.int32, device="cuda")
    w = t.empty(tokens * 10, dtype=t.float32, device="cuda")
    xq = t.empty(tokens * 2048, dtype=t.int8, device="cuda")
    xs = t.empty(tokens, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_route_quantize_v1", ld.data_ptr(), hd.data_ptr(), tokens, ids.data_ptr(),
              w.data_ptr(), xq.data_ptr(), xs.data_ptr(), stream(), 0)
    wids, ww = orc.topk(logits)
    wq, ws = orc.quantize_rows(h, 2048)
    assert np.array_equal(host(ids, np.int32).reshape(tokens, 10), wids)
    assert np.array_equal(host(w, np.float32).reshape(tokens, 10).view(np.uint32), ww.view(np.uint32))
    assert np.array_equal(host(xq, np.int8).reshape(tokens, 2048), wq)
    assert np.array_equal(host(xs, np.float32).view(np.uint32), ws.view(np.uint32))


def run_plan(q38m, ids, tokens, hashes, poison=None):
    t = torch()
    nbytes = q38m.route_plan_bytes(tokens)
    buf = t.empty(nbytes + 256, dtype=t.uint8, device="cuda")
    if poison is not None:
        buf.fill_(poison)
    base = (buf.data_ptr() + 255) // 256 * 256
    offset = base - buf.data_ptr()
    plan = q38m.bind_plan(base, nbytes, tokens)
    idd = device(ids)
    q38m.call("q38m_moe_build_route_plan_v1", idd.data_ptr(), tokens, ctypes.byref(plan),
              q38m.PLAN_FLAG_HASHES if hashes else 0, stream(), 0)
    return host(buf, np.uint8)[offset:offset + nbytes]


def reference_pattern(tokens, repeated):
    """Distinct ids within every token (what top-k gives), all one id
    ("all"), or distinct except one token that repeats an id ("one")."""
    a = np.arange(tokens * 10, dtype=np.int64)
    if repeated == "all":
        return np.full(a.size, 7, np.int32)
    ids = ((a * 73 + (a // 10) * 17) % 512).astype(np.int32)
    if repeated == "one":
        ids[10 * (tokens // 2) + 7] = ids[10 * (tokens // 2) + 3]
    return ids


@pytest.mark.parametrize("tokens,repeated", [(1, None), (2, None), (3, None), (128, None),
                                             (512, None), (512, "all"), (100, None),
                                             (300, "one"), (512, "one")])
@pytest.mark.parametrize("hashes", [False, True])
def test_plan_bitwise(q38m, orc, tokens, repeated, hashes):
    ids = reference_pattern(tokens, repeated)
    got = run_plan(q38m, ids, tokens, hashes)
    again = run_plan(q38m, ids, tokens, hashes, poison=0xA5)
    assert np.array_equal(got, again)
    assert np.array_equal(got, orc.build_plan(ids, tokens, hashes=hashes))


def test_plan_from_router_bitwise(q38m, orc):
    for seed, bias in ((3, None), (4, np.array(W.zipf_bias(4, 1, 1.1), np.float32))):
        ids, _ = orc.topk(orc.synth_logits(seed, 2, 512, bias=bias))
        got = run_plan(q38m, ids.ravel(), 512, True, poison=0x5A)
        assert np.array_equal(got, orc.build_plan(ids.ravel(), 512, hashes=True))


def test_plan_invalid_expert_fails_closed(q38m, orc):
    ids = ((np.arange(30) * 19 + 5) % 512).astype(np.int32)
    ids[4] = -1
    ids[17] = 600
    got = run_plan(q38m, ids, 3, True, poison=0xA5)
    p = orc.parse_plan(got, 3)
    assert p["status"] == 1
    assert np.array_equal(got, orc.build_plan(ids, 3, hashes=True))


def test_pack_hidden_gather(q38m, orc):
    tokens = 3
    ids = ((np.arange(30) * 19 + 5) % 512).astype(np.int32)
    hidden = np.zeros((tokens, 2048), np.uint16)
    for t_ in range(tokens):
        hidden[t_] = orc.f32_to_bf16((t_ * 4 + np.arange(2048) % 4).astype(np.float32))
    plan_img = orc.build_plan(ids, tokens)
    p = orc.parse_plan(plan_img, tokens)
    t = torch()
    out = t.empty(30 * 2048, dtype=t.int16, device="cuda")
    hd, pd = device(hidden), device(p["packed"].copy())
    q38m.call("q38m_moe_pack_hidden_v1", hd.data_ptr(), pd.data_ptr(), 30, 2048,
              out.data_ptr(), stream(), 0)
    got = host(out, np.uint16).reshape(30, 2048)
    assert np.array_equal(got, hidden[p["packed"] // 10])


def repack_w4_host(data, scales, experts, rows, cols, paired):
    """numpy restatement of the quad-major MFMA16 W4 layouts documented in
    q38m.h: [e][kq][slot][lane=(q,n)][j][byte i], byte i = nib(k0+i) |
    nib(k0+4+i) << 4; paired slots alternate tiles of the two row halves."""
    nib = np.empty(experts * rows * cols, np.uint8)
    nib[0::2] = data & 0xF
    nib[1::2] = data >> 4
    nib = nib.reshape(experts, rows // 16, 16, cols // 128, 4, 4, 8)  # e,rt,n,kq,j,q,k8
    sc = scales.reshape(experts, rows // 16, 16, cols // 128, 4)      # e,rt,n,kq,j
    tiles = rows // 16
    order = np.arange(tiles)
    if paired:
        order = np.stack([order[:tiles // 2], order[tiles // 2:]], 1).reshape(-1)
    nib = nib[:, order].transpose(0, 3, 1, 5, 2, 4, 6)  # e,kq,slot,q,n,j,k8
    out = nib[..., 0:4] | (nib[..., 4:8] << 4)
    sc = sc[:, order].transpose(0, 3, 1, 2, 4)          # e,kq,slot,n,j
    return out.reshape(-1), sc.reshape(-1)


def repack_w8_host(data, experts, rows, cols):
    d = data.reshape(experts, rows // 16, 16, cols // 64, 4, 16)  # e,rt,n,kb,q,16
    return d.transpose(0, 1, 3, 4, 2, 5).reshape(-1)


def test_repack_layouts(q38m, orc):
    E, R, C = 4, 64, 512
    w4 = q38m.synth_weights(3, 60, q38m.FORMAT_W4_SYM, 32, E, R, C, 0.02)
    for paired in (False, True):
        p4 = q38m.repack(w4, paired=paired)
        d, s = repack_w4_host(host(w4.data, np.uint8), host(w4.scales, np.uint16), E, R, C,
                              paired)
        assert np.array_equal(host(p4.data, np.uint8), d)
        assert np.array_equal(host(p4.scales, np.uint16), s)
    w8 = q38m.synth_weights(3, 62, q38m.FORMAT_W8_SYM, 0, E, R, C, 0.002)
    p8 = q38m.repack(w8)
    assert np.array_equal(host(p8.data, np.uint8), repack_w8_host(host(w8.data, np.uint8), E, R, C))
    assert np.array_equal(host(p8.scales, np.uint16), host(w8.scales, np.uint16))


def test_residual_add(q38m, orc):
    rng = np.random.default_rng(8)
    a = orc.f32_to_bf16(rng.standard_normal(4096).astype(np.float32) * 5)
    b = orc.f32_to_bf16(rng.standard_normal(4096).astype(np.float32) * 5)
    t = torch()
    out = t.empty(4096, dtype=t.int16, device="cuda")
    da, db = device(a), device(b)
    q38m.call("q38m_residual_add_bf16", da.data_ptr(), db.data_ptr(), out.data_ptr(), 4096,
              stream(), 0)
    want = orc.f32_to_bf16(orc.bf16_to_f32(a) + orc.bf16_to_f32(b))
    assert np.array_equal(host(out, np.uint16), want)
