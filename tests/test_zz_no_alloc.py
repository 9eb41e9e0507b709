"""The allocation-free slab step (q38m_moe_prefill_noalloc_v1; no
reference counterpart) against the slab step with a caller-owned workspace
(q38m_moe_prefill_v1), bit for bit, on two calls in a row with the second
smaller than the first: its device-resident workspace keeps the previous
call's contents, which must not leak into the next result.  Also its
limit: more than 64 tokens is an invalid argument."""
import ctypes

import numpy as np
import pytest

from helpers import Layer, W, host, prefill, stream, synth_hidden, synth_logits, torch

pytestmark = pytest.mark.gpu


def noalloc(q38m, layer, hidden, logits, tokens, shared=None):
    t = torch()
    out = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    so, sg = (None, None) if shared is None else (shared[0].data_ptr(), shared[1].data_ptr())
    q38m.call("q38m_moe_prefill_noalloc_v1", ctypes.byref(layer.gu.desc),
              ctypes.byref(layer.dn.desc), hidden.data_ptr(), logits.data_ptr(), tokens, so, sg,
              out.data_ptr(), stream(), 0)
    return out


@pytest.mark.parametrize("config", [1, 2])
def test_noalloc_equals_prefill_on_two_calls(q38m, orc, config):
    """config 1 (all-W4) runs gate/up and down as two launches, config 2
    (W4 + per-channel W8) as one, whose hand-off flags live in the
    device-resident workspace too."""
    t = torch()
    gfmt, dfmt = W.layer_policy(config, 0)
    layer = Layer(q38m, orc, W.CONFIGS[config]["seed"], 0, gfmt, dfmt, with_host=False)
    ws = q38m.PrefillWorkspace_(64)
    for tokens, tag in ((64, 11), (17, 12)):
        print(f"noalloc: config {config}, {tokens} tokens", flush=True)
        hidden = synth_hidden(q38m, 5, tag, tokens)
        logits = synth_logits(q38m, 5, tag + 100, tokens)
        so = synth_hidden(q38m, 5, tag + 200, tokens)
        sg = synth_hidden(q38m, 5, tag + 300, 1)[0, :tokens].contiguous()
        want = prefill(q38m, layer, hidden, logits, ws)
        got = noalloc(q38m, layer, hidden, logits, tokens)
        want_shared = prefill(q38m, layer, hidden, logits, ws, shared=(so, sg))
        got_shared = noalloc(q38m, layer, hidden, logits, tokens, shared=(so, sg))
        t.cuda.synchronize()
        assert np.array_equal(host(got, np.uint16), host(want, np.uint16)), tokens
        assert np.array_equal(host(got_shared, np.uint16), host(want_shared, np.uint16)), tokens


def test_noalloc_rejects_more_than_its_workspace_holds(q38m, orc):
    gfmt, dfmt = W.layer_policy(1, 0)
    layer = Layer(q38m, orc, W.CONFIGS[1]["seed"], 0, gfmt, dfmt, with_host=False)
    hidden = synth_hidden(q38m, 5, 21, 65)
    logits = synth_logits(q38m, 5, 22, 65)
    assert q38m.lib().q38m_moe_prefill_noalloc_scratch_bytes() == \
        q38m.lib().q38m_moe_prefill_workspace_bytes(64)
    with pytest.raises(q38m.InvalidArgument, match="64 tokens"):
        noalloc(q38m, layer, hidden, logits, 65)
    with pytest.raises(q38m.InvalidArgument):
        noalloc(q38m, layer, hidden, logits, 0)
