"""GPU parity of the weight formats beyond the BASELINE pair (W4 g32 fp16
gate/up with W8 per-channel or W4 g32 fp16 down): W4 in groups of 64 and
128 columns, W8 in groups of 64 and 128 or per channel for either
projection, and bf16 scale words (the reference artifact's scale dtype,
tools/q38_artifact_compiler.py:232, with groups of 128).  The weight descriptor the reference's validate_expert_tensor
checks (cuda/q38_moe_prefill.cu:51-62) carries the format; every entry point
that takes expert weights runs each pair bit-exact against the oracle:

- the slab step (q38m_moe_prefill_v1) for 64 tokens with every intermediate;
- the fused decode (q38m_moe_decode_v1) for one token, which also equals the
  slab step at tokens == 1;
- the chunk step (q38m_moe_prefill_wide_v1) over 1024 Zipf-routed tokens
  (hot experts span several 128-row tasks, so every row-tile count of its
  kernels runs): every token equals the slab step over two 512-token slabs,
  and a sample equals the oracle token by token.

Scale magnitudes are |N(0, sigma)| as in the BASELINE synthesis.
"""
import numpy as np
import pytest

from helpers import (Layer, W, decode_fused, decode_scratch, host, prefill, staged_step,
                     synth_hidden, synth_logits, torch, ws_arrays)
from test_gpu_wide import prefill_wide

pytestmark = pytest.mark.gpu

# id -> (gate/up (bits, group, sigma), bf16?), (down (bits, group, sigma), bf16?)
FORMATS = {
    "w4g128bf16-w8g128bf16": (((4, 128, 0.02), True), ((8, 128, 0.002), True)),
    "w4g64-w4g64": (((4, 64, 0.02), False), ((4, 64, 0.02), False)),
    "w4g128-w4g128bf16": (((4, 128, 0.02), False), ((4, 128, 0.02), True)),
    "w4g32bf16-w8g64bf16": (((4, 32, 0.02), True), ((8, 64, 0.002), True)),
    "w4g64bf16-w8pcbf16": (((4, 64, 0.02), True), ((8, 0, 0.002), True)),
    "w4g128-w4g32": (((4, 128, 0.02), False), ((4, 32, 0.02), False)),
    # W8 gate/up: the reference's edge layers (0, 1, 46, 47) and MTP experts
    # are W8 g128 bf16 in both projections (tools/q38_quant_policy.py:164-190)
    "w8g128bf16-w8g128bf16": (((8, 128, 0.002), True), ((8, 128, 0.002), True)),
    "w8pc-w8pc": (((8, 0, 0.002), False), ((8, 0, 0.002), False)),
    "w8g64-w4g32": (((8, 64, 0.002), False), ((4, 32, 0.02), False)),
}
SEED = 9


@pytest.fixture(scope="module")
def format_layer(q38m, orc):
    """One layer per format pair; only the latest is kept (each holds about
    2.3 GB of device and 1.1 GB of host weights)."""
    held = {}

    def get(name):
        if name not in held:
            held.clear()
            torch().cuda.empty_cache()
            (gfmt, gbf16), (dfmt, dbf16) = FORMATS[name]
            held[name] = Layer(q38m, orc, SEED, 3, ("fmt",) + gfmt, ("fmt",) + dfmt,
                               gate_up_bf16=gbf16, down_bf16=dbf16)
        return held[name]

    yield get
    held.clear()


@pytest.mark.parametrize("name", list(FORMATS))
def test_format_slab_step_bitwise(q38m, orc, format_layer, name):
    layer = format_layer(name)
    tokens = 64
    hidden = synth_hidden(q38m, SEED, 21, tokens)
    logits = synth_logits(q38m, SEED, 22, tokens)
    ws = q38m.PrefillWorkspace_(tokens)
    out = prefill(q38m, layer, hidden, logits, ws)
    gpu = ws_arrays(ws, tokens)
    ref = orc.moe(host(hidden, np.uint16), layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32), intermediates=True)
    assert np.array_equal(gpu["ids"], ref["ids"])
    assert np.array_equal(gpu["weighted_mid"], ref["weighted_mid"])
    assert np.array_equal(gpu["mid_q"], ref["mid_q"])
    assert np.array_equal(gpu["route_output"].view(np.uint32),
                          ref["route_output"].view(np.uint32))
    got = host(out, np.uint16)
    assert np.array_equal(got, ref["output"])
    assert orc.bf16_to_f32(got).std() > 0.1


@pytest.mark.parametrize("name", list(FORMATS))
def test_format_decode_bitwise(q38m, orc, format_layer, name):
    layer = format_layer(name)
    hidden = synth_hidden(q38m, SEED, 31, 1)
    logits = synth_logits(q38m, SEED, 32, 1)
    out = decode_fused(q38m, layer, hidden, logits, decode_scratch(q38m))
    ref = orc.moe(host(hidden, np.uint16), layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32), grouped=False)
    got = host(out, np.uint16)
    assert np.array_equal(got, ref["output"])
    slab = prefill(q38m, layer, hidden, logits, q38m.PrefillWorkspace_(1))
    assert np.array_equal(got, host(slab, np.uint16))


@pytest.mark.parametrize("name", list(FORMATS))
def test_format_chunk_step_bitwise(q38m, orc, format_layer, name):
    t = torch()
    layer = format_layer(name)
    tokens = 1024
    hidden = synth_hidden(q38m, SEED, 41, tokens)
    logits = synth_logits(q38m, SEED, 42, tokens, W.bias_for(4, 0))
    wsw = q38m.WideWorkspace_(tokens)
    outw = prefill_wide(q38m, layer, hidden, logits, wsw)
    ws1 = q38m.PrefillWorkspace_(512)
    out1 = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    for s in range(tokens // 512):
        sl = slice(s * 512, (s + 1) * 512)
        prefill(q38m, layer, hidden[sl], logits[sl], ws1, output=out1[sl])
    got = host(outw, np.uint16)
    assert np.array_equal(got, host(out1, np.uint16))
    sample = np.arange(0, tokens, 37)
    ref = orc.moe(host(hidden, np.uint16)[sample], layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32)[sample], grouped=False)
    assert np.array_equal(got[sample], ref["output"])
    # hot experts span several 128-row tasks
    ids = ws_arrays(wsw, tokens)["ids"].ravel()
    assert np.bincount(ids, minlength=W.EXPERTS).max() > 2 * 128


@pytest.mark.parametrize("tokens", [1, 77, 600])
def test_edge_format_ragged_chunks(q38m, orc, format_layer, tokens):
    """The reference's edge-layer format (W8 g128 bf16 in both projections)
    through the chunk step at ragged sizes (one token, a partial first task,
    more than one slab), against the oracle token by token."""
    layer = format_layer("w8g128bf16-w8g128bf16")
    hidden = synth_hidden(q38m, SEED, 51, tokens)
    logits = synth_logits(q38m, SEED, 52, tokens, W.bias_for(4, 0))
    out = prefill_wide(q38m, layer, hidden, logits, q38m.WideWorkspace_(tokens))
    sample = np.arange(tokens) if tokens <= 100 else np.arange(0, tokens, 9)
    ref = orc.moe(host(hidden, np.uint16)[sample], layer.host_gu, layer.host_dn,
                  logits=host(logits, np.float32)[sample], grouped=False)
    assert np.array_equal(host(out, np.uint16)[sample], ref["output"])


@pytest.mark.parametrize("name", ["w8g128bf16-w8g128bf16", "w4g128-w4g128bf16"])
def test_format_staged_call_sequence(q38m, orc, format_layer, name):
    """The staged entry points (grouped gate/up, grouped down) take the
    descriptor's format too: the staged sequence equals the fused step."""
    layer = format_layer(name)
    hidden = synth_hidden(q38m, SEED, 61, 100)
    logits = synth_logits(q38m, SEED, 62, 100)
    fused = prefill(q38m, layer, hidden, logits, q38m.PrefillWorkspace_(100))
    staged = staged_step(q38m, layer, hidden, logits)
    assert np.array_equal(host(staged, np.uint16), host(fused, np.uint16))
