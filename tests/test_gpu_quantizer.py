"""GPU parity of the weight quantiser (q38m_quantize_expert_weights) with
the CPU oracle's restatement of quantize_groupwise
(tools/q38_artifact_compiler.py:193-253): packed bytes and fp16 or bf16
scale words bit for bit, for every supported format and group, then one layer
quantised on the device, repacked and run through the prefill step against
the oracle on the same quantised bytes."""
import ctypes

import numpy as np
import pytest

from helpers import W, device, host, prefill, stream, synth_hidden, synth_logits, torch

pytestmark = pytest.mark.gpu


def quantize_on_gpu(q38m, src_bf16_dev, fmt, group, experts, rows, cols, scale_bf16=False):
    t = torch()
    nbytes, sbytes = q38m.weights_bytes(fmt, group, experts, rows, cols)
    data = t.empty(nbytes, dtype=t.uint8, device="cuda")
    scales = t.empty(sbytes // 2, dtype=t.int16, device="cuda")
    dtype = q38m.SCALE_BF16 if scale_bf16 else q38m.SCALE_F16
    desc = q38m.ExpertWeights(data.data_ptr(), scales.data_ptr(), fmt, group, dtype,
                              q38m.LAYOUT_ROW_MAJOR, experts, rows, cols)
    q38m.call("q38m_quantize_expert_weights", src_bf16_dev.data_ptr(), ctypes.byref(desc),
              stream(), 0)
    t.cuda.synchronize()
    return data, scales


@pytest.mark.parametrize("scale_bf16", [False, True])
@pytest.mark.parametrize("bits,group", [(4, 32), (4, 64), (4, 128), (8, 0), (8, 32), (8, 128)])
def test_quantizer_bitwise(q38m, orc, bits, group, scale_bf16):
    rng = np.random.default_rng(100 + bits + group)
    experts, rows, cols = 3, 48, 1024
    w = (rng.standard_normal((experts * rows, cols)) *
         rng.choice([1e-7, 1e-5, 1e-3, 0.02, 1.0, 300.0], (experts * rows, 1))).astype(np.float32)
    w[7] = 0.0
    w[9, :64] = 0.0
    w[11, 5] = -65000.0
    h = orc.f32_to_bf16(w)
    fmt = q38m.FORMAT_W4_SYM if bits == 4 else q38m.FORMAT_W8_SYM
    data, scales = quantize_on_gpu(q38m, device(h), fmt, group, experts, rows, cols, scale_bf16)
    want_data, want_scales = orc.quantize_weights(h, bits, group, scale_bf16)
    assert np.array_equal(host(data, np.uint8).reshape(want_data.shape), want_data)
    assert np.array_equal(host(scales, np.uint16).reshape(want_scales.shape), want_scales)


# (gate/up group, gate/up bf16 scales, down bits, down group, down bf16 scales):
# the BASELINE formats, and the reference artifact's groups of 128 with bf16
# scales (tools/q38_artifact_compiler.py:193-253)
END_TO_END = {
    "baseline": (32, False, 8, 0, False),
    "artifact-g128-bf16": (128, True, 8, 128, True),
}


@pytest.mark.parametrize("case", sorted(END_TO_END))
def test_quantize_repack_prefill_end_to_end(q38m, orc, case):
    """A bf16 layer quantised on the device, repacked and run for 64 tokens
    equals the oracle on the same bytes."""
    ggroup, gbf16, dbits, dgroup, dbf16 = END_TO_END[case]
    t = torch()
    seed = 77
    gu_src = t.empty(W.EXPERTS * 2 * W.INTER * W.HIDDEN, dtype=t.int16, device="cuda")
    dn_src = t.empty(W.EXPERTS * W.HIDDEN * W.INTER, dtype=t.int16, device="cuda")
    q38m.synth_fill(q38m.SYNTH_NORMAL_BF16, seed, 11, gu_src.numel(), gu_src, sigma=0.05)
    q38m.synth_fill(q38m.SYNTH_NORMAL_BF16, seed, 12, dn_src.numel(), dn_src, sigma=0.05)
    dfmt = q38m.FORMAT_W4_SYM if dbits == 4 else q38m.FORMAT_W8_SYM
    gu_data, gu_scales = quantize_on_gpu(q38m, gu_src, q38m.FORMAT_W4_SYM, ggroup, W.EXPERTS,
                                         2 * W.INTER, W.HIDDEN, gbf16)
    dn_data, dn_scales = quantize_on_gpu(q38m, dn_src, dfmt, dgroup, W.EXPERTS, W.HIDDEN,
                                         W.INTER, dbf16)
    # the quantised bytes equal the oracle's on two experts of each tensor
    for src, data, scales, bits, group, bf16, rows, cols in (
            (gu_src, gu_data, gu_scales, 4, ggroup, gbf16, 2 * W.INTER, W.HIDDEN),
            (dn_src, dn_data, dn_scales, dbits, dgroup, dbf16, W.HIDDEN, W.INTER)):
        for e in (0, W.EXPERTS - 1):
            elems = rows * cols
            h = host(src[e * elems:(e + 1) * elems], np.uint16).reshape(rows, cols)
            wd, ws = orc.quantize_weights(h, bits, group, bf16)
            nb = elems * bits // 8
            ns = rows * (cols // (group or cols))
            assert np.array_equal(host(data[e * nb:(e + 1) * nb], np.uint8), wd.ravel())
            assert np.array_equal(host(scales[e * ns:(e + 1) * ns], np.uint16), ws.ravel())
    del gu_src, dn_src
    dtype = {False: q38m.SCALE_F16, True: q38m.SCALE_BF16}
    gu_rm = q38m.DeviceWeights(gu_data, gu_scales, q38m.FORMAT_W4_SYM, ggroup,
                               q38m.LAYOUT_ROW_MAJOR, W.EXPERTS, 2 * W.INTER, W.HIDDEN,
                               dtype[gbf16])
    dn_rm = q38m.DeviceWeights(dn_data, dn_scales, dfmt, dgroup, q38m.LAYOUT_ROW_MAJOR,
                               W.EXPERTS, W.HIDDEN, W.INTER, dtype[dbf16])

    class Quantised:
        pass

    layer = Quantised()
    layer.gu = q38m.repack(gu_rm, paired=True)
    layer.dn = q38m.repack(dn_rm)
    hidden = synth_hidden(q38m, seed, 1, 64)
    logits = synth_logits(q38m, seed, 2, 64)
    ws = q38m.PrefillWorkspace_(64)
    out = prefill(q38m, layer, hidden, logits, ws)
    host_gu = orc.HostWeights(host(gu_data, np.uint8), host(gu_scales, np.uint16), 4, ggroup,
                              W.EXPERTS, 2 * W.INTER, W.HIDDEN, gbf16)
    host_dn = orc.HostWeights(host(dn_data, np.uint8), host(dn_scales, np.uint16), dbits,
                              dgroup, W.EXPERTS, W.HIDDEN, W.INTER, dbf16)
    ref = orc.moe(host(hidden, np.uint16), host_gu, host_dn, logits=host(logits, np.float32))
    assert np.array_equal(host(out, np.uint16), ref["output"])
