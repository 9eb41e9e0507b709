"""The checked build (libq38m_checked.so, include/q38m_checked.h): the
product library with the device index checks compiled in.  On valid inputs
its results equal the product library's bit for bit and its status word
stays clear; on a corrupted plan (an expert id past 512, a task row count
past 128, an inverse index past the routes -- values the plan builder never
writes) the check records a status bit and substitutes an in-range index,
so the kernel completes without reading or writing outside its buffers.
The product library never sees the corrupted plan."""
import ctypes

import numpy as np
import pytest

from helpers import (Layer, W, decode_fused, decode_scratch, host, prefill, stream,
                     synth_hidden, synth_logits, torch)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer(q38m, orc):
    gfmt, dfmt = W.layer_policy(2, 0)
    return Layer(q38m, orc, W.CONFIGS[2]["seed"], 0, gfmt, dfmt, with_host=False)


def wide(q38m, call, layer, hidden, logits, ws, out):
    call("q38m_moe_prefill_wide_v1", ctypes.byref(layer.gu.desc), ctypes.byref(layer.dn.desc),
         hidden.data_ptr(), logits.data_ptr(), hidden.shape[0], ctypes.byref(ws.wide), None,
         None, out.data_ptr(), stream(), 0)
    return out


def test_checked_build_equals_product_and_stays_clean(q38m, layer):
    """Slab (512 tokens), chunk (4,096 tokens) and decode (1 token) through
    both libraries: equal outputs, no status bit."""
    t = torch()
    q38m.checked_status(reset=True)
    hidden = synth_hidden(q38m, 71, 1, 512)
    logits = synth_logits(q38m, 71, 2, 512)
    ws = q38m.PrefillWorkspace_(512)
    want = prefill(q38m, layer, hidden, logits, ws).clone()
    got = prefill(q38m, layer, hidden, logits, ws, call=q38m.call_checked)
    t.cuda.synchronize()
    assert t.equal(got, want)

    big = 4096
    hidden = synth_hidden(q38m, 72, 1, big)
    logits = synth_logits(q38m, 72, 2, big, bias=W.bias_for(4, 0))
    wsw = q38m.WideWorkspace_(big)
    out = t.empty(big, W.HIDDEN, dtype=t.int16, device="cuda")
    want = wide(q38m, q38m.call, layer, hidden, logits, wsw, out).clone()
    got = wide(q38m, q38m.call_checked, layer, hidden, logits, wsw, out)
    t.cuda.synchronize()
    assert t.equal(got, want)

    one = synth_hidden(q38m, 73, 1, 1)
    one_logits = synth_logits(q38m, 73, 2, 1)
    want = decode_fused(q38m, layer, one, one_logits, decode_scratch(q38m)).clone()
    got = decode_fused(q38m, layer, one, one_logits, decode_scratch(q38m),
                       call=q38m.call_checked)
    t.cuda.synchronize()
    assert t.equal(got, want)
    assert q38m.checked_status() == 0


def test_checked_build_flags_a_corrupt_plan_and_completes(q38m, layer):
    """Staged gate/up and combine on a plan whose first task names expert
    600, whose second task claims 200 rows and whose first inverse index is
    past the routes: the checked kernels complete and report each."""
    t = torch()
    tokens = 64
    routes = tokens * W.TOPK
    s = stream()
    hidden = synth_hidden(q38m, 74, 1, tokens)
    logits = synth_logits(q38m, 74, 2, tokens)
    ids = t.empty(routes, dtype=t.int32, device="cuda")
    wts = t.empty(routes, dtype=t.float32, device="cuda")
    q38m.call("q38m_topk_router_f32", logits.data_ptr(), ids.data_ptr(), wts.data_ptr(), tokens,
              W.EXPERTS, W.TOPK, 1, s, 0)
    nbytes = q38m.route_plan_bytes(tokens)
    buf = t.zeros(nbytes + 256, dtype=t.uint8, device="cuda")
    base = (buf.data_ptr() + 255) // 256 * 256
    plan = q38m.bind_plan(base, nbytes, tokens)
    q38m.call("q38m_moe_build_route_plan_v1", ids.data_ptr(), tokens, ctypes.byref(plan), 0, s, 0)
    xq = t.empty(tokens, W.HIDDEN, dtype=t.int8, device="cuda")
    xs = t.empty(tokens, dtype=t.float32, device="cuda")
    q38m.call("q38m_quantize_rows_i8", hidden.data_ptr(), tokens, W.HIDDEN, xq.data_ptr(),
              xs.data_ptr(), s, 0)
    t.cuda.synchronize()

    def at(pointer):
        return pointer - buf.data_ptr()

    tasks_at = at(plan.tasks)
    task_words = buf[tasks_at:tasks_at + 16].view(t.int16)  # tasks 0 and 1
    assert int(task_words[2]) >= 0 and int(buf[tasks_at + 14]) <= 16
    task_words[2] = 600                 # task 0: expert (bytes 4-5)
    buf[tasks_at + 14] = 200            # task 1: valid_rows (byte 6 of record 1)
    inverse_at = at(plan.assignment_to_packed)
    buf[inverse_at:inverse_at + 4] = 255  # inverse[0] = 0xffffffff
    t.cuda.synchronize()

    q38m.checked_status(reset=True)
    mid = t.empty(routes, W.INTER, dtype=t.int16, device="cuda")
    q38m.call_checked("q38m_moe_grouped_gate_up_v1", ctypes.byref(layer.gu.desc),
                      xq.data_ptr(), xs.data_ptr(), plan.packed_assignment, wts.data_ptr(),
                      plan.tasks, q38m.max_tasks(tokens), mid.data_ptr(), q38m.MODE_GROUPED_MMQ,
                      s, 0)
    status = q38m.checked_status(reset=True)
    assert status & q38m.CHECK_EXPERT and status & q38m.CHECK_TASK_ROWS
    assert not status & (q38m.CHECK_ROUTE | q38m.CHECK_TOKEN)

    route_output = t.zeros(routes, W.HIDDEN, dtype=t.float32, device="cuda")
    out = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    q38m.call_checked("q38m_moe_reduce_top10_and_combine_shared_v1", route_output.data_ptr(),
                      plan.assignment_to_packed, None, None, tokens, out.data_ptr(), s, 0)
    assert q38m.checked_status(reset=True) == q38m.CHECK_ROUTE
    assert np.all(host(out, np.uint16) == 0)  # zero route outputs sum to +0
