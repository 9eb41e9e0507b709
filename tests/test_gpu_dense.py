"""The dense bf16 GEMMs on either side of the routed experts
(cuda/cuda_backend.cu:1518-1525, 1573-1601): the router logits and the
shared expert.  They are
floating-point results, checked against a float64 CPU evaluation within a
tolerance written here; the shared expert's SiLU multiply and everything
downstream of the logits / shared inputs are bit-exact.

Tolerances: an fp32 accumulation of K products is within
TOL_SUM * sum_k |a_k b_k| of the exact value (TOL_SUM = 2^-16, far above
the ~sqrt(K) * 2^-24 typical error, far below any layout mistake); bf16
outputs additionally within one bf16 step (2^-8 relative)."""
import ctypes

import numpy as np
import pytest

from helpers import (Layer, W, decode_fused, decode_scratch, device, host, prefill, stream,
                     synth_hidden, torch)

pytestmark = pytest.mark.gpu

TOL_SUM = 2.0 ** -16
BF16_STEP = 2.0 ** -8


def bf16_matrix(orc, rng, rows, cols, sigma):
    return orc.f32_to_bf16((rng.standard_normal((rows, cols)) * sigma).astype(np.float32))


def gemm(q38m, a_dev, b_dev, m, n, k, out_bf16):
    t = torch()
    if out_bf16:
        c = t.empty(m * n, dtype=t.int16, device="cuda")
        q38m.call("q38m_dense_gemm_bf16", a_dev.data_ptr(), b_dev.data_ptr(), m, n, k, None,
                  c.data_ptr(), stream(), 0)
    else:
        c = t.empty(m * n, dtype=t.float32, device="cuda")
        q38m.call("q38m_dense_gemm_bf16", a_dev.data_ptr(), b_dev.data_ptr(), m, n, k,
                  c.data_ptr(), None, stream(), 0)
    t.cuda.synchronize()
    return c


def check_close(orc, got, a, b, out_bf16):
    af = orc.bf16_to_f32(a).astype(np.float64)
    bf = orc.bf16_to_f32(b).astype(np.float64)
    exact = af @ bf.T
    bound = TOL_SUM * (np.abs(af) @ np.abs(bf).T)
    if out_bf16:
        got = orc.bf16_to_f32(got).astype(np.float64)
        bound = bound + BF16_STEP * np.abs(exact)
    assert np.all(np.abs(got - exact) <= bound)


# K-split 32 x 32 tiles (long K too: the hyper mix-down's 8192, and a
# ragged odd-step K), (K <= 1024 with at least 192 tiles of 64 x 64)
# workgroup-shared 64 x 64 tiles: ragged edges, a trailing half K chunk, a
# single half chunk, the largest K of that form; and one activation row
# (the GEMV form: the router and the shared down projection at one token,
# a row count that is not a multiple of the workgroup's four, a K whose
# last pass of chunks is partial, a single row)
@pytest.mark.parametrize("m,n,k", [(40, 512, 2048), (512, 2048, 512), (1, 512, 2048),
                                   (33, 1, 2048), (64, 96, 64), (130, 70, 96),
                                   (1000, 1000, 160), (640, 1600, 32), (1024, 768, 1024),
                                   (512, 2048, 320), (512, 320, 8192), (70, 100, 4128),
                                   (1, 2048, 512), (1, 1001, 4128), (1, 1, 32), (1, 320, 8192)])
@pytest.mark.parametrize("out_bf16", [False, True])
def test_dense_gemm(q38m, orc, m, n, k, out_bf16):
    rng = np.random.default_rng(m * 7 + n * 3 + k)
    a = bf16_matrix(orc, rng, m, k, 1.0)
    b = bf16_matrix(orc, rng, n, k, 0.05)
    c = gemm(q38m, device(a), device(b), m, n, k, out_bf16)
    got = host(c, np.uint16 if out_bf16 else np.float32).reshape(m, n)
    check_close(orc, got, a, b, out_bf16)


def test_router_logits_and_routes(q38m, orc):
    t = torch()
    rng = np.random.default_rng(5)
    tokens = 96
    hidden = bf16_matrix(orc, rng, tokens, W.HIDDEN, 1.0)
    router = bf16_matrix(orc, rng, W.EXPERTS, W.HIDDEN, 0.02)
    logits = t.empty(tokens * W.EXPERTS, dtype=t.float32, device="cuda")
    hd, rd = device(hidden), device(router)
    q38m.call("q38m_moe_router_v1", hd.data_ptr(), rd.data_ptr(), tokens, W.HIDDEN,
              logits.data_ptr(), stream(), 0)
    t.cuda.synchronize()
    got = host(logits, np.float32).reshape(tokens, W.EXPERTS)
    check_close(orc, got, hidden, router, False)
    # routes: the top-10 of the GPU logits equals the top-10 of the exact
    # logits wherever ranks 10 and 11 are further apart than the tolerance
    hf = orc.bf16_to_f32(hidden).astype(np.float64)
    rf = orc.bf16_to_f32(router).astype(np.float64)
    exact = hf @ rf.T
    bound = TOL_SUM * (np.abs(hf) @ np.abs(rf).T).max(axis=1)
    ids_gpu, _ = orc.topk(got)
    order = np.argsort(-exact, axis=1, kind="stable")
    decided = 0
    for tok in range(tokens):
        s = np.sort(exact[tok])[::-1]
        if s[9] - s[10] > 2 * bound[tok]:
            assert set(ids_gpu[tok]) == set(order[tok, :10])
            decided += 1
    assert decided >= tokens * 0.9


@pytest.mark.parametrize("tokens,top_k", [(1, 10), (37, 10), (512, 10), (96, 7)])
def test_router_topk_fused(q38m, orc, tokens, top_k):
    """q38m_moe_router_topk_v1 (logits kept on the CU, level-1 selection in
    the GEMM epilogue) equals q38m_moe_router_v1 -> q38m_topk_router_f32 and
    the oracle's top-k of those logits, bit for bit.  Experts 5 and 300 share
    a router row (exact ties, lower id first) and token 0 is all zeros (every
    logit 0: experts 0..9)."""
    t = torch()
    rng = np.random.default_rng(tokens * 31 + top_k)
    hidden = bf16_matrix(orc, rng, tokens, W.HIDDEN, 1.0)
    hidden[0] = 0
    router = bf16_matrix(orc, rng, W.EXPERTS, W.HIDDEN, 0.02)
    router[300] = router[5]
    hd, rd = device(hidden), device(router)
    logits = t.empty(tokens * W.EXPERTS, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_router_v1", hd.data_ptr(), rd.data_ptr(), tokens, W.HIDDEN,
              logits.data_ptr(), stream(), 0)
    ref_ids = t.empty(tokens * top_k, dtype=t.int32, device="cuda")
    ref_w = t.empty(tokens * top_k, dtype=t.float32, device="cuda")
    q38m.call("q38m_topk_router_f32", logits.data_ptr(), ref_ids.data_ptr(), ref_w.data_ptr(),
              tokens, W.EXPERTS, top_k, 1, stream(), 0)
    ws_bytes = q38m.lib().q38m_moe_router_topk_workspace_bytes(tokens)
    ws = t.empty(ws_bytes, dtype=t.uint8, device="cuda")
    ids = t.full((tokens * top_k,), -7, dtype=t.int32, device="cuda")
    w = t.full((tokens * top_k,), -1.0, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_router_topk_v1", hd.data_ptr(), rd.data_ptr(), tokens, W.HIDDEN, top_k,
              ws.data_ptr(), ws_bytes, ids.data_ptr(), w.data_ptr(), stream(), 0)
    t.cuda.synchronize()
    got_ids = host(ids, np.int32).reshape(tokens, top_k)
    got_w = host(w, np.float32).reshape(tokens, top_k)
    assert np.array_equal(got_ids, host(ref_ids, np.int32).reshape(tokens, top_k))
    assert np.array_equal(got_w.view(np.uint32),
                          host(ref_w, np.float32).reshape(tokens, top_k).view(np.uint32))
    orc_ids, orc_w = orc.topk(host(logits, np.float32).reshape(tokens, W.EXPERTS), top_k)
    assert np.array_equal(got_ids, orc_ids)
    assert np.array_equal(got_w.view(np.uint32), orc_w.view(np.uint32))
    assert list(got_ids[0]) == list(range(top_k))
    # the tie: wherever both tied experts are selected, 5 ranks directly above 300
    for row in got_ids:
        if 5 in row and 300 in row:
            assert list(row).index(300) == list(row).index(5) + 1


@pytest.mark.parametrize("tokens", [40, 1])
def test_shared_expert(q38m, orc, tokens):
    """Tiled at 40 tokens, the GEMV form at one token."""
    t = torch()
    rng = np.random.default_rng(9 + tokens)
    inter = W.INTER
    x = bf16_matrix(orc, rng, tokens, W.HIDDEN, 1.0)
    wg = bf16_matrix(orc, rng, inter, W.HIDDEN, 0.02)
    wu = bf16_matrix(orc, rng, inter, W.HIDDEN, 0.02)
    wd = bf16_matrix(orc, rng, W.HIDDEN, inter, 0.02)
    wo = bf16_matrix(orc, rng, 1, W.HIDDEN, 0.02)
    scratch = t.empty(q38m.lib().q38m_moe_shared_expert_scratch_bytes(tokens, inter) // 2,
                      dtype=t.int16, device="cuda")
    so = t.empty(tokens * W.HIDDEN, dtype=t.int16, device="cuda")
    sg = t.empty(tokens, dtype=t.int16, device="cuda")
    devs = [device(v) for v in (x, wg, wu, wd, wo)]
    q38m.call("q38m_moe_shared_expert_v1", *[d.data_ptr() for d in devs], tokens, W.HIDDEN, inter,
              scratch.data_ptr(), so.data_ptr(), sg.data_ptr(), stream(), 0)
    t.cuda.synchronize()
    words = host(scratch, np.uint16)
    g = words[:tokens * inter].reshape(tokens, inter)
    u = words[tokens * inter:2 * tokens * inter].reshape(tokens, inter)
    h = words[2 * tokens * inter:].reshape(tokens, inter)
    check_close(orc, g, x, wg, True)
    check_close(orc, u, x, wu, True)
    # the SiLU multiply is exact given g and u: bf16((g / (1 + exp(-g))) * u)
    gf = orc.bf16_to_f32(g)
    uf = orc.bf16_to_f32(u)
    denom = (np.float32(1.0) + orc.expf(-gf)).astype(np.float32)
    want_h = orc.f32_to_bf16(((gf / denom).astype(np.float32) * uf).astype(np.float32))
    assert np.array_equal(h, want_h)
    check_close(orc, host(so, np.uint16).reshape(tokens, W.HIDDEN), h, wd, True)
    check_close(orc, host(sg, np.uint16).reshape(tokens, 1), x, wo, True)


@pytest.mark.parametrize("tokens", [64, 1])
def test_moe_block_router_routed_shared(q38m, orc, tokens):
    """The whole MoE block on the device -- router logits, the routed
    experts, the shared expert and the gated combine -- equals the oracle's
    step on the same logits and shared inputs, bit for bit; at one token
    (the GEMV router and shared expert) through the decode entry point as
    well as the prefill one."""
    t = torch()
    gfmt, dfmt = W.layer_policy(2, 0)
    layer = Layer(q38m, orc, W.CONFIGS[2]["seed"], 0, gfmt, dfmt)
    rng = np.random.default_rng(17 + tokens)
    hidden = synth_hidden(q38m, 17, 1, tokens)
    router = device(bf16_matrix(orc, rng, W.EXPERTS, W.HIDDEN, 0.02))
    weights = [device(bf16_matrix(orc, rng, r, c, 0.02)) for r, c in
               ((W.INTER, W.HIDDEN), (W.INTER, W.HIDDEN), (W.HIDDEN, W.INTER), (1, W.HIDDEN))]
    logits = t.empty(tokens, W.EXPERTS, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_router_v1", hidden.data_ptr(), router.data_ptr(), tokens, W.HIDDEN,
              logits.data_ptr(), stream(), 0)
    scratch = t.empty(q38m.lib().q38m_moe_shared_expert_scratch_bytes(tokens, W.INTER) // 2,
                      dtype=t.int16, device="cuda")
    so = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    sg = t.empty(tokens, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_shared_expert_v1", hidden.data_ptr(), *[w.data_ptr() for w in weights],
              tokens, W.HIDDEN, W.INTER, scratch.data_ptr(), so.data_ptr(), sg.data_ptr(), stream(),
              0)
    ws = q38m.PrefillWorkspace_(tokens)
    out = prefill(q38m, layer, hidden, logits, ws, shared=(so, sg))
    ref = orc.moe(host(hidden, np.uint16), layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32), shared_output=host(so, np.uint16),
                  shared_gate=host(sg, np.uint16))
    assert np.array_equal(host(out, np.uint16), ref["output"])
    if tokens == 1:
        dec = decode_fused(q38m, layer, hidden, logits, decode_scratch(q38m), shared=(so, sg))
        assert np.array_equal(host(dec, np.uint16).ravel(), ref["output"].ravel())
        # the logits, shared output and gate themselves against float64
        check_close(orc, host(logits, np.float32).reshape(1, W.EXPERTS),
                    host(hidden, np.uint16).reshape(1, W.HIDDEN), host(router, np.uint16)
                    .reshape(W.EXPERTS, W.HIDDEN), False)
        check_close(orc, host(sg, np.uint16).reshape(1, 1),
                    host(hidden, np.uint16).reshape(1, W.HIDDEN),
                    host(weights[3], np.uint16).reshape(1, W.HIDDEN), True)


@pytest.mark.parametrize("policy,top_k,with_residual", [
    ("config", 10, False), ("config", 10, True), ("config", 7, True), ("interior", 10, True)])
def test_decode_block_equals_router_shared_decode(q38m, orc, policy, top_k, with_residual):
    """q38m_moe_decode_block_v1 (router GEMV; routed gate/up with the top-k
    and the shared gate/up; routed down with the shared down, the gated
    combine and the residual -- three launches) equals
    q38m_moe_router_v1 -> q38m_moe_shared_expert_v1 -> q38m_moe_decode_v1
    on the same token bit for bit, and the oracle fed the GPU's logits and
    shared inputs.  Formats: config 2's (W4 g32 gate/up, W8 down) and the
    reference artifact's interior layers (W4 g128, bf16 scales)."""
    t = torch()
    if policy == "config":
        gfmt, dfmt = W.layer_policy(2, 0)
        layer = Layer(q38m, orc, W.CONFIGS[2]["seed"], 0, gfmt, dfmt)
    else:
        fmt = ("w4", 4, 128, 0.02)
        layer = Layer(q38m, orc, W.CONFIGS[2]["seed"], 3, fmt, fmt, gate_up_bf16=True,
                      down_bf16=True)
    rng = np.random.default_rng(23 + top_k)
    hidden = synth_hidden(q38m, 23, 1, 1)
    router = device(bf16_matrix(orc, rng, W.EXPERTS, W.HIDDEN, 0.02))
    wg, wu, wd, wo = [device(bf16_matrix(orc, rng, r, c, 0.02)) for r, c in
                      ((W.INTER, W.HIDDEN), (W.INTER, W.HIDDEN), (W.HIDDEN, W.INTER),
                       (1, W.HIDDEN))]
    residual = synth_hidden(q38m, 23, 5, 1) if with_residual else None
    s = stream()

    logits = t.empty(1, W.EXPERTS, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_router_v1", hidden.data_ptr(), router.data_ptr(), 1, W.HIDDEN,
              logits.data_ptr(), s, 0)
    scratch = t.empty(q38m.lib().q38m_moe_shared_expert_scratch_bytes(1, W.INTER) // 2 + 8,
                      dtype=t.int16, device="cuda")
    so = t.empty(1, W.HIDDEN, dtype=t.int16, device="cuda")
    sg = t.empty(8, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_shared_expert_v1", hidden.data_ptr(), wg.data_ptr(), wu.data_ptr(),
              wd.data_ptr(), wo.data_ptr(), 1, W.HIDDEN, W.INTER, scratch.data_ptr(),
              so.data_ptr(), sg.data_ptr(), s, 0)
    want = decode_fused(q38m, layer, hidden, logits, decode_scratch(q38m), top_k=top_k,
                        shared=(so, sg), residual=residual)

    bscratch = t.full((q38m.lib().q38m_moe_decode_block_scratch_bytes() // 2,), -1,
                      dtype=t.int16, device="cuda")
    got = t.empty(1, W.HIDDEN, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_decode_block_v1", ctypes.byref(layer.gu.desc),
              ctypes.byref(layer.dn.desc), hidden.data_ptr(), router.data_ptr(), wg.data_ptr(),
              wu.data_ptr(), wd.data_ptr(), wo.data_ptr(), W.INTER, top_k,
              None if residual is None else residual.data_ptr(), bscratch.data_ptr(),
              got.data_ptr(), s, 0)
    t.cuda.synchronize()
    assert t.equal(got, want)
    ref = orc.moe(host(hidden, np.uint16).reshape(1, W.HIDDEN), layer.host_gu, layer.host_dn,
                  ids=None, logits=host(logits, np.float32).reshape(1, W.EXPERTS),
                  shared_output=host(so, np.uint16).reshape(1, W.HIDDEN),
                  shared_gate=host(sg, np.uint16)[:1]) if top_k == 10 else None
    if ref is not None:
        out = ref["output"]
        if residual is not None:
            out = orc.f32_to_bf16(orc.bf16_to_f32(host(residual, np.uint16).reshape(1, W.HIDDEN)) +
                                  orc.bf16_to_f32(out))
        assert np.array_equal(host(got, np.uint16).reshape(1, W.HIDDEN), out)
    ids = host(bscratch[:2 * top_k], np.int32)
    assert np.array_equal(ids, orc.topk(host(logits, np.float32).reshape(1, W.EXPERTS),
                                        top_k)[0].ravel())

