"""GPU parity of the chunk path (q38m_moe_prefill_wide_v1: one layer over up
to 32,768 tokens with 128-row tasks).

- the chunk plan against numpy's stable argsort of the expert ids (the
  expert-major stable order of cuda/q38_moe_prefill.cu:192-262), its counts,
  offsets, 128-row tasks and header; for T <= 512 its packed order, counts
  and offsets equal the oracle's V1 plan; invalid ids fail closed as V1;
- the whole step bit-exact against the slab path on the same inputs (every
  token of a 4096-token Zipf chunk) and against the oracle token by token
  on samples; at T = 512 every intermediate equals the slab path's;
- all-W4 layers (W4 down), the gated shared term and ragged sizes;
- the most skewed routing (every token to the same ten experts), plan and
  step.
"""
import ctypes

import numpy as np
import pytest

from helpers import (Layer, W, canonical_nan, device, host, oracle_chunk, pow2_normalize,
                     prefill, stream, synth_hidden, synth_logits, torch, ws_arrays)

pytestmark = pytest.mark.gpu

ROWS = 128


def wide_plan(q38m, ids_host, tokens):
    """Builds the chunk plan on the device; returns its arrays."""
    t = torch()
    nbytes = q38m.lib().q38m_moe_wide_plan_bytes(tokens)
    buf = t.full((nbytes + 256,), 0xA5, dtype=t.uint8, device="cuda")
    base = (buf.data_ptr() + 255) // 256 * 256
    plan = q38m.RoutePlan()
    q38m.call("q38m_moe_wide_plan_storage", base, nbytes, tokens, ctypes.byref(plan))
    scratch = t.empty(q38m.lib().q38m_moe_wide_plan_scratch_bytes(tokens) // 4,
                      dtype=t.int32, device="cuda")
    ids = t.from_numpy(np.ascontiguousarray(ids_host, dtype=np.int32).ravel()).cuda()
    q38m.call("q38m_moe_build_route_plan_wide", ids.data_ptr(), tokens, ctypes.byref(plan),
              scratch.data_ptr(), stream(), 0)
    t.cuda.synchronize()
    off = base - buf.data_ptr()
    raw = buf[off:off + nbytes].cpu().numpy()
    routes = tokens * 10
    max_tasks = q38m.lib().q38m_moe_wide_max_tasks(tokens)

    def take(ptr, count, dtype):
        start = ptr - base
        return raw[start:start + count * np.dtype(dtype).itemsize].view(dtype)

    header = take(plan.header, 16, np.uint32)
    return {
        "magic": header[0], "version": header[1], "tokens": header[2], "routes": header[3],
        "active": header[4], "task_count": header[5], "status": header[6],
        "counts": take(plan.expert_counts, 512, np.uint16),
        "offsets": take(plan.expert_offsets, 513, np.uint32),
        "task_offsets": take(plan.expert_task_offsets, 513, np.uint32),
        "packed": take(plan.packed_assignment, routes, np.uint32),
        "inverse": take(plan.assignment_to_packed, routes, np.uint32),
        "tasks": take(plan.tasks, 2 * max_tasks, np.uint32).reshape(max_tasks, 2),
        "max_tasks": max_tasks,
    }


def expected_plan(ids_host, tokens):
    """The chunk plan restated with numpy: stable argsort by expert id,
    128-row tiles of each expert's segment."""
    flat = np.ascontiguousarray(ids_host, dtype=np.int64).ravel()
    valid = (flat >= 0) & (flat < 512)
    order = np.argsort(np.where(valid, flat, 1 << 20), kind="stable")[:valid.sum()]
    counts = np.bincount(flat[valid], minlength=512)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    ntasks = (counts + ROWS - 1) // ROWS
    task_offsets = np.concatenate([[0], np.cumsum(ntasks)])
    tasks = []
    for e in range(512):
        for k in range(ntasks[e]):
            rows = min(ROWS, counts[e] - k * ROWS)
            tasks.append((offsets[e] + k * ROWS, e | (rows << 16)))
    return order, counts, offsets, task_offsets, np.array(tasks, dtype=np.uint32).reshape(-1, 2)


def zipf_ids(seed, tokens, s=1.1):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, 513) ** s
    p /= p.sum()
    perm = rng.permutation(512)
    out = np.empty((tokens, 10), np.int32)
    for t_ in range(tokens):
        out[t_] = perm[rng.choice(512, 10, replace=False, p=p)]
    return out


HOT_EXPERTS = np.array([3, 77, 150, 151, 260, 311, 400, 401, 402, 511], np.int32)


@pytest.mark.parametrize("tokens,kind", [(1, "uniform"), (3, "uniform"), (512, "uniform"),
                                         (2053, "zipf"), (4096, "zipf"), (32768, "uniform"),
                                         (32768, "hot")])
def test_wide_plan_matches_stable_sort(q38m, orc, tokens, kind):
    rng = np.random.default_rng(tokens)
    if kind == "zipf":
        ids = zipf_ids(tokens, tokens)
    elif kind == "hot":
        # every token routes to the same ten experts (in its own order):
        # ten 32,768-route segments of 256 full tasks each
        ids = np.stack([rng.permutation(HOT_EXPERTS) for _ in range(tokens)]).astype(np.int32)
    else:
        ids = np.stack([rng.choice(512, 10, replace=False) for _ in range(tokens)]).astype(np.int32)
    got = wide_plan(q38m, ids, tokens)
    order, counts, offsets, task_offsets, tasks = expected_plan(ids, tokens)
    routes = tokens * 10
    assert got["magic"] == 0x52383351 and got["version"] == 2 and got["status"] == 0
    assert got["tokens"] == tokens and got["routes"] == routes
    assert got["active"] == (counts > 0).sum()
    assert np.array_equal(got["packed"], order)
    assert np.array_equal(got["inverse"][order], np.arange(routes))
    assert np.array_equal(got["counts"], counts)
    assert np.array_equal(got["offsets"], offsets)
    assert np.array_equal(got["task_offsets"], task_offsets)
    assert got["task_count"] == len(tasks) <= got["max_tasks"]
    assert np.array_equal(got["tasks"][:len(tasks)], tasks)
    assert not got["tasks"][len(tasks):].any()
    if tokens <= 512:
        v1 = orc.parse_plan(orc.build_plan(ids.ravel(), tokens), tokens)
        assert np.array_equal(got["packed"], v1["packed"])
        assert np.array_equal(got["inverse"], v1["inverse"])


# 300 tokens: two 2048-route chunks; 32,768 tokens: 160 chunks, with
# invalid ids in chunks past 64 and 128 (the scan sums each chunk's
# invalid count in lane c % 64, pass c / 64)
@pytest.mark.parametrize("tokens,bad", [(300, {4: -1, 2500: 600}),
                                        (32768, {4: -1, 2500: 600, 131079: 512,
                                                 307203: -5})])
def test_wide_plan_invalid_ids_fail_closed(q38m, tokens, bad):
    ids = ((np.arange(tokens * 10) * 19 + 5) % 512).astype(np.int32)
    for at, v in bad.items():
        ids[at] = v
    got = wide_plan(q38m, ids, tokens)
    assert got["status"] == 1
    valid = (ids >= 0) & (ids < 512)
    order = np.argsort(np.where(valid, ids, 1 << 20), kind="stable")[:valid.sum()]
    nvalid = valid.sum()
    assert np.array_equal(got["packed"][:nvalid], order)
    assert np.array_equal(got["packed"][nvalid:], np.arange(nvalid, tokens * 10))
    for at in bad:
        assert got["inverse"][at] == at


def prefill_wide(q38m, layer, hidden, logits, ws, output=None, shared=None):
    t = torch()
    tokens = hidden.shape[0]
    if output is None:
        output = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    so, sg = (None, None) if shared is None else shared
    q38m.call("q38m_moe_prefill_wide_v1", ctypes.byref(layer.gu.desc),
              ctypes.byref(layer.dn.desc), hidden.data_ptr(),
              None if logits is None else logits.data_ptr(), tokens, ctypes.byref(ws.wide),
              None if so is None else so.data_ptr(), None if sg is None else sg.data_ptr(),
              output.data_ptr(), stream(), 0)
    return output


@pytest.fixture(scope="module")
def wide_layers(q38m, orc):
    cache = {}

    def get(config, layer=0):
        key = (config, layer)
        if key not in cache:
            gfmt, dfmt = W.layer_policy(config, layer)
            cache[key] = Layer(q38m, orc, W.CONFIGS[config]["seed"], layer, gfmt, dfmt)
        return cache[key]

    yield get
    cache.clear()


@pytest.mark.parametrize("values", ["finite", "non-finite"])
def test_wide_slab_equals_v1_with_intermediates(q38m, orc, wide_layers, values):
    """At T = 512 the chunk plan's packed order is the V1 order, so every
    intermediate of the chunk path equals the slab path's -- also word for
    word where tokens carry +inf, -inf or NaN (their gates go infinite or
    NaN: the chunk path's silu comes from a host-built table, the slab's
    from the device's exp and division, and both write NaN mid words as
    0x7fc0)."""
    layer = wide_layers(2)
    seed = W.CONFIGS[2]["seed"]
    hidden = synth_hidden(q38m, seed, 7, 512)
    logits = synth_logits(q38m, seed, 8, 512)
    if values == "non-finite":
        t = torch()
        bad = t.tensor([0x7f80, 0xff80, 0x7fc1, 0xffa0], dtype=t.int32).to(t.int16)
        for k, token in enumerate((3, 100, 101, 511)):
            hidden[token, 17 + 5 * k] = bad[k].item()
        hidden[200, :] = bad[2].item()  # a whole row of NaN
    ws1 = q38m.PrefillWorkspace_(512)
    out1 = prefill(q38m, layer, hidden, logits, ws1)
    wsw = q38m.WideWorkspace_(512)
    outw = prefill_wide(q38m, layer, hidden, logits, wsw)
    a, b = ws_arrays(ws1, 512), ws_arrays(wsw, 512)
    for name in ("ids", "xq", "weighted_mid", "mid_q"):
        assert np.array_equal(a[name], b[name]), name
    assert np.array_equal(a["route_output"].view(np.uint32), b["route_output"].view(np.uint32))
    assert np.array_equal(a["weights"].view(np.uint32), b["weights"].view(np.uint32))
    assert np.array_equal(host(out1, np.uint16), host(outw, np.uint16))
    if values == "non-finite":
        mid = a["weighted_mid"]
        nan = ((mid & 0x7f80) == 0x7f80) & ((mid & 0x7f) != 0)
        assert nan.any() and np.all(mid[nan] == 0x7fc0)
        # and the oracle writes the same mid words (NaN included) and output
        ref = orc.moe(host(hidden, np.uint16).reshape(512, W.HIDDEN), layer.host_gu,
                      layer.host_dn, logits=host(logits, np.float32).reshape(512, W.EXPERTS),
                      intermediates=True)
        assert np.array_equal(ref["weighted_mid"], mid)
        assert np.array_equal(canonical_nan(ref["output"]),
                              canonical_nan(host(out1, np.uint16).reshape(512, W.HIDDEN)))


def test_wide_config4_chunk(q38m, orc, wide_layers):
    """Config 4 (4096 tokens, Zipf s=1.1) in one chunk: every token equals
    the slab path's result and the oracle's (evaluated slab by slab), and a
    sample equals the oracle's token-by-token evaluation."""
    t = torch()
    layer = wide_layers(4)
    seed = W.CONFIGS[4]["seed"]
    bias = W.bias_for(4, 0)
    hidden = synth_hidden(q38m, seed, 1, 4096)
    logits = synth_logits(q38m, seed, 2, 4096, bias)
    wsw = q38m.WideWorkspace_(4096)
    outw = prefill_wide(q38m, layer, hidden, logits, wsw)
    ws1 = q38m.PrefillWorkspace_(512)
    out1 = t.empty(4096, W.HIDDEN, dtype=t.int16, device="cuda")
    for s in range(8):
        sl = slice(s * 512, (s + 1) * 512)
        prefill(q38m, layer, hidden[sl], logits[sl], ws1, output=out1[sl])
    got = host(outw, np.uint16)
    assert np.array_equal(got, host(out1, np.uint16))
    full = oracle_chunk(orc, host(hidden, np.uint16), host(logits, np.float32),
                        layer.host_gu, layer.host_dn)
    assert np.array_equal(got, full)
    rng = np.random.default_rng(44)
    sample = np.sort(rng.choice(4096, 64, replace=False))
    ref = orc.moe(host(hidden, np.uint16)[sample], layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32)[sample], grouped=False)
    assert np.array_equal(got[sample], ref["output"])
    # hot experts really span several 128-row tasks
    counts = wide_plan_counts(wsw)
    assert counts.max() > 2 * ROWS


def wide_plan_counts(wsw):
    torch().cuda.synchronize()
    base = wsw.buffer.data_ptr()
    start = wsw.ws.plan.expert_counts - base
    return wsw.buffer[start:start + 1024].cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("tokens", [1, 77, 1000])
def test_wide_all_w4_layer_and_shared(q38m, orc, wide_layers, tokens):
    """Config 5's all-W4 layer policy (W4 g32 down) with the gated shared
    term, at ragged chunk sizes, against the oracle token by token."""
    t = torch()
    layer = wide_layers(5, 0)
    seed = W.CONFIGS[5]["seed"]
    hidden = synth_hidden(q38m, seed, 11, tokens)
    logits = synth_logits(q38m, seed, 12, tokens, W.bias_for(5, 0))
    so = synth_hidden(q38m, seed, 13, tokens)
    sg = t.empty(tokens, dtype=t.int16, device="cuda")
    q38m.synth_fill(q38m.SYNTH_NORMAL_BF16, seed, 14, tokens, sg)
    wsw = q38m.WideWorkspace_(tokens)
    out = prefill_wide(q38m, layer, hidden, logits, wsw, shared=(so, sg))
    sample = np.arange(tokens) if tokens <= 100 else np.arange(0, tokens, 7)
    ref = orc.moe(host(hidden, np.uint16)[sample], layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32)[sample],
                  shared_output=host(so, np.uint16)[sample],
                  shared_gate=host(sg, np.uint16)[sample], grouped=False)
    assert np.array_equal(host(out, np.uint16)[sample], ref["output"])


def test_wide_hot_experts_chunk(q38m, orc, wide_layers):
    """The most skewed routing: a +40 logit bias on ten experts sends every
    token of a 2,048-token chunk to the same ten (each expert 2,048 rows,
    16 full 128-row tasks).  Every token equals the slab path's result and
    the oracle's."""
    t = torch()
    layer = wide_layers(4)
    seed = W.CONFIGS[4]["seed"]
    tokens = 2048
    bias = np.zeros(512, np.float32)
    bias[HOT_EXPERTS] = 40.0
    hidden = synth_hidden(q38m, seed, 51, tokens)
    logits = synth_logits(q38m, seed, 52, tokens, bias)
    wsw = q38m.WideWorkspace_(tokens)
    outw = prefill_wide(q38m, layer, hidden, logits, wsw)
    counts = wide_plan_counts(wsw)
    assert np.array_equal(np.flatnonzero(counts), np.sort(HOT_EXPERTS))
    assert (counts[HOT_EXPERTS] == tokens).all()
    ws1 = q38m.PrefillWorkspace_(512)
    out1 = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    for s in range(tokens // 512):
        sl = slice(s * 512, (s + 1) * 512)
        prefill(q38m, layer, hidden[sl], logits[sl], ws1, output=out1[sl])
    got = host(outw, np.uint16)
    assert np.array_equal(got, host(out1, np.uint16))
    full = oracle_chunk(orc, host(hidden, np.uint16), host(logits, np.float32),
                        layer.host_gu, layer.host_dn)
    assert np.array_equal(got, full)


def test_wide_config5_layer_full_chunk(q38m, orc, wide_layers):
    """One config-5 layer (W4/W8) over all 32,768 tokens of the stack in one
    chunk: every token against the oracle (evaluated slab by slab), and a
    64-token sample against its token-by-token evaluation."""
    layer = wide_layers(5, 1)
    seed = W.CONFIGS[5]["seed"]
    tokens = 32768
    _, _, h_tag, l_tag = W.layer_tags(1)
    hidden = synth_hidden(q38m, seed, h_tag, tokens)
    logits = synth_logits(q38m, seed, l_tag, tokens, W.bias_for(5, 1))
    wsw = q38m.WideWorkspace_(tokens)
    out = prefill_wide(q38m, layer, hidden, logits, wsw)
    got = host(out, np.uint16)
    full = oracle_chunk(orc, host(hidden, np.uint16), host(logits, np.float32),
                        layer.host_gu, layer.host_dn)
    mismatched = np.flatnonzero((got != full).any(axis=1))
    assert mismatched.size == 0, f"{mismatched.size} tokens differ, first {mismatched[:8]}"
    sample = np.arange(0, tokens, 512) + np.arange(64) % 7
    ref = orc.moe(host(hidden[sample.tolist()], np.uint16), layer.host_gu, layer.host_dn,
                  logits=host(logits[sample.tolist()], np.float32), grouped=False)
    assert np.array_equal(got[sample], ref["output"])


def _chunk_stack(q38m, orc, normalize=False, fresh_tokens=True, every_token=False):
    """Config 5's 48 layers (alternating all-W4 / W4-W8 policy, each with
    its own weights and Zipf s=0.8 router draw) on the chunk path over a
    2,048-token chunk with the residual add between layers.  At every
    layer the chained output equals the oracle on sampled tokens bit for
    bit (the device's input words for those tokens, NaNs canonicalised);
    optionally a fresh N(0,1) chunk through the layer does too.  With
    normalize, every token's state is rescaled by a power of two after the
    residual add (pow2_normalize).  The oracle evaluates a token on its ten
    routed experts only, gathered on the device, routes renumbered 0..9 in
    rank order.  With every_token, each layer's whole chained output is also
    compared with the oracle over all 2,048 tokens (the layer's full
    512-expert weights, slab by slab).  Returns the number of layers whose
    sampled outputs are finite."""
    t = torch()
    seed = W.CONFIGS[5]["seed"]
    tokens = 2048
    sample = np.array([0, 517, 1303, 2047])
    fmt = {4: q38m.FORMAT_W4_SYM, 8: q38m.FORMAT_W8_SYM}
    wsw = q38m.WideWorkspace_(tokens)
    state = synth_hidden(q38m, seed, 1, tokens)

    def subset(weights, ids, bits, group, rows, cols):
        per_data = weights.data.numel() // W.EXPERTS
        per_scale = weights.scales.numel() // W.EXPERTS
        index = t.as_tensor(ids, device="cuda", dtype=t.long)
        data = weights.data.view(W.EXPERTS, per_data).index_select(0, index)
        scales = weights.scales.view(W.EXPERTS, per_scale).index_select(0, index)
        return orc.HostWeights(host(data, np.uint8), host(scales, np.uint16), bits, group,
                               len(ids), rows, cols)

    class Repacked:
        pass

    routes = np.arange(10, dtype=np.int32)[None]
    finite_layers = 0
    for layer_index in range(48):
        gfmt, dfmt = W.layer_policy(5, layer_index)
        gu_tag, dn_tag, _, l_tag = W.layer_tags(layer_index)
        gu_rm = q38m.synth_weights(seed, gu_tag, fmt[gfmt[1]], gfmt[2], W.EXPERTS, 2 * W.INTER,
                                   W.HIDDEN, gfmt[3])
        dn_rm = q38m.synth_weights(seed, dn_tag, fmt[dfmt[1]], dfmt[2], W.EXPERTS, W.HIDDEN,
                                   W.INTER, dfmt[3])
        layer = Repacked()
        layer.gu, layer.dn = q38m.repack(gu_rm, paired=True), q38m.repack(dn_rm)
        logits = synth_logits(q38m, seed, l_tag, tokens, W.bias_for(5, layer_index))
        host_logits = host(logits, np.float32)[sample]
        if fresh_tokens:
            fresh = synth_hidden(q38m, seed, 2000 + layer_index, tokens)
            got_fresh = host(prefill_wide(q38m, layer, fresh, logits, wsw), np.uint16)
            host_fresh = host(fresh, np.uint16)[sample]
        host_in = host(state, np.uint16)[sample]
        out = prefill_wide(q38m, layer, state, logits, wsw)
        got_out = host(out, np.uint16)
        for k, token in enumerate(sample):
            ids, w = orc.topk(host_logits[k:k + 1])
            gu_sub = subset(gu_rm, ids[0], gfmt[1], gfmt[2], 2 * W.INTER, W.HIDDEN)
            dn_sub = subset(dn_rm, ids[0], dfmt[1], dfmt[2], W.HIDDEN, W.INTER)
            if fresh_tokens:
                ref = orc.moe(host_fresh[k:k + 1], gu_sub, dn_sub, ids=routes, weights=w,
                              grouped=False)
                assert np.array_equal(got_fresh[token:token + 1], ref["output"]), (
                    f"layer {layer_index}, fresh token {token}")
            ref = orc.moe(host_in[k:k + 1], gu_sub, dn_sub, ids=routes, weights=w,
                          grouped=False)
            assert np.array_equal(canonical_nan(got_out[token:token + 1]),
                                  canonical_nan(ref["output"])), (
                f"layer {layer_index}, chained token {token}")
        if every_token:
            full = oracle_chunk(
                orc, host(state, np.uint16), host(logits, np.float32),
                orc.HostWeights(host(gu_rm.data, np.uint8), host(gu_rm.scales, np.uint16),
                                gfmt[1], gfmt[2], W.EXPERTS, 2 * W.INTER, W.HIDDEN),
                orc.HostWeights(host(dn_rm.data, np.uint8), host(dn_rm.scales, np.uint16),
                                dfmt[1], dfmt[2], W.EXPERTS, W.HIDDEN, W.INTER))
            mismatched = np.flatnonzero((canonical_nan(got_out) != canonical_nan(full)).any(axis=1))
            assert mismatched.size == 0, (
                f"layer {layer_index}: {mismatched.size} tokens differ, first {mismatched[:8]}")
        finite_layers += int(np.isfinite(orc.bf16_to_f32(got_out[sample])).all())
        new_state = t.empty_like(state)
        q38m.call("q38m_residual_add_bf16", state.data_ptr(), out.data_ptr(),
                  new_state.data_ptr(), tokens * W.HIDDEN, stream(), 0)
        state = new_state
        if normalize:
            state = device(pow2_normalize(orc, host(state, np.uint16))).view(tokens, W.HIDDEN)
        del gu_rm, dn_rm, layer
    return finite_layers


def test_config5_stack_full_depth_chunk(q38m, orc):
    """Config 5 at full depth on the chunk path, on a fresh N(0,1) chunk
    and on the chained state.  The synthetic stack has no norm between
    layers and the MoE output grows about quadratically with its input, so
    the chained state overflows after a few layers; from there its words
    are compared with NaNs canonicalised."""
    assert _chunk_stack(q38m, orc) >= 3


def test_config5_stack_normalized_chunk_all_finite(q38m, orc):
    """The chained 48-layer chunk stack with config 5's weights and routes
    and a power-of-two rescale of every token's state between layers (rms
    back into [1, 2), exact in bf16; a stand-in for the norm of a real
    stack): at every layer all 2,048 tokens' outputs equal the oracle's
    word for word, and they stay finite."""
    assert _chunk_stack(q38m, orc, normalize=True, fresh_tokens=False, every_token=True) == 48
