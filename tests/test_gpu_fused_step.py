"""The one-launch gate/up + down (gate_up_down_kernel) against the staged
kernels it replaces.

q38m_moe_prefill_v1 runs gate/up, the mid quantisation and down as one
launch for W4 gate/up with per-channel W8 down (config 2's formats): down
workgroups wait on per-task flags that the gate/up workgroups set, and the
step's plan kernel clears the flags first.  Every intermediate must equal
what the staged entry points (q38m_moe_grouped_gate_up_v1,
q38m_quantize_rows_i8, q38m_moe_grouped_down_v1) compute from the same plan
and int8 rows, bit for bit, call after call on one workspace (a flag left
set by an earlier call would let a down workgroup read mid rows before they
are written), and the plan status must stay 0 (no wait ran out).
q38m_moe_grouped_gate_up_down_v1 is checked the same way over two calls
on one flag buffer (each call must leave its flags zero for the next), and
on a format pair it does not fuse.
"""
import ctypes

import numpy as np
import pytest

from helpers import (Layer, W, host, prefill, stream, synth_hidden, synth_logits, torch,
                     ws_arrays)

pytestmark = pytest.mark.gpu

STATUS_OFFSET = 24  # q38m_route_plan_header_v1.status


@pytest.fixture(scope="module")
def layer2(q38m, orc):
    gfmt, dfmt = W.layer_policy(2, 0)
    return Layer(q38m, orc, W.CONFIGS[2]["seed"], 0, gfmt, dfmt)


def staged_kernels(q38m, layer, ws, tokens):
    """gate/up, mid quantisation and down through the staged entry points on
    the workspace's plan and int8 rows."""
    t = torch()
    w = ws.ws
    routes = tokens * W.TOPK
    tasks = q38m.max_tasks(tokens)
    s = stream()
    mid = t.empty(routes, W.INTER, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_grouped_gate_up_v1", ctypes.byref(layer.gu.desc), w.xq, w.xs,
              w.plan.packed_assignment, w.expert_weights, w.plan.tasks, tasks, mid.data_ptr(),
              q38m.MODE_GROUPED_MMQ, s, 0)
    mq = t.empty(routes, W.INTER, dtype=t.int8, device="cuda")
    ms = t.empty(routes, dtype=t.float32, device="cuda")
    q38m.call("q38m_quantize_rows_i8", mid.data_ptr(), routes, W.INTER, mq.data_ptr(),
              ms.data_ptr(), s, 0)
    ro = t.empty(routes, W.HIDDEN, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_grouped_down_v1", ctypes.byref(layer.dn.desc), mq.data_ptr(),
              ms.data_ptr(), w.plan.tasks, tasks, ro.data_ptr(), q38m.MODE_GROUPED_MMQ, s, 0)
    t.cuda.synchronize()
    return {"weighted_mid": host(mid, np.uint16), "mid_q": host(mq, np.int8),
            "mid_s": host(ms, np.float32), "route_output": host(ro, np.float32)}


def assert_same(got, want):
    assert np.array_equal(got["weighted_mid"].reshape(-1), want["weighted_mid"].reshape(-1))
    assert np.array_equal(got["mid_q"].reshape(-1), want["mid_q"].reshape(-1))
    assert np.array_equal(got["mid_s"].view(np.uint32), want["mid_s"].view(np.uint32))
    assert np.array_equal(got["route_output"].reshape(-1).view(np.uint32),
                          want["route_output"].reshape(-1).view(np.uint32))


def plan_status(arrays):
    return int(arrays["plan"][STATUS_OFFSET:STATUS_OFFSET + 4].view(np.uint32)[0])


def test_step_calls_equal_staged_kernels(q38m, layer2):
    """Four calls of different sizes on one workspace (each plan kernel
    clears the previous call's flags): every intermediate equals the staged
    kernels', and no wait ran out."""
    ws = q38m.PrefillWorkspace_(512)
    for i, tokens in enumerate((512, 17, 300, 512)):
        hidden = synth_hidden(q38m, 31, 100 + i, tokens)
        logits = synth_logits(q38m, 31, 200 + i, tokens)
        prefill(q38m, layer2, hidden, logits, ws)
        got = ws_arrays(ws, tokens)
        assert plan_status(got) == 0
        assert_same(got, staged_kernels(q38m, layer2, ws, tokens))


@pytest.mark.parametrize("fusable", [True, False])
def test_gate_up_down_entry_point(q38m, orc, layer2, fusable):
    """q38m_moe_grouped_gate_up_down_v1 on flags cleared once
    (q38m_moe_clear_task_flags_v1 over garbage) equals the staged kernels on
    two calls in a row with different inputs, and leaves the flags and
    counters zero after each; on a pair it does not fuse (W4 down) it runs
    the three kernels."""
    t = torch()
    layer = layer2 if fusable else Layer(q38m, orc, W.CONFIGS[1]["seed"], 0,
                                         *W.layer_policy(1, 0))
    ws = q38m.PrefillWorkspace_(512)
    tasks = q38m.max_tasks(512)
    flags = t.full((9 * tasks,), 0x5A5A5A5A, dtype=t.int32, device="cuda")
    q38m.call("q38m_moe_clear_task_flags_v1", flags.data_ptr(), tasks, stream(), 0)
    status = t.zeros(1, dtype=t.int32, device="cuda")
    for call, tokens in enumerate((512, 300)):
        prefill(q38m, layer, synth_hidden(q38m, 32, 1 + call, tokens),
                synth_logits(q38m, 32, 11 + call, tokens), ws)
        want = staged_kernels(q38m, layer, ws, tokens)
        w = ws.ws
        routes = tokens * W.TOPK
        slots = q38m.max_tasks(tokens)
        mid = t.empty(routes, W.INTER, dtype=t.int16, device="cuda")
        mq = t.empty(routes, W.INTER, dtype=t.int8, device="cuda")
        ms = t.empty(routes, dtype=t.float32, device="cuda")
        ro = t.empty(routes, W.HIDDEN, dtype=t.float32, device="cuda")
        q38m.call("q38m_moe_grouped_gate_up_down_v1", ctypes.byref(layer.gu.desc),
                  ctypes.byref(layer.dn.desc), w.xq, w.xs, w.plan.packed_assignment,
                  w.expert_weights, w.plan.tasks, slots, mid.data_ptr(), mq.data_ptr(),
                  ms.data_ptr(), flags.data_ptr(), status.data_ptr(), ro.data_ptr(),
                  q38m.MODE_GROUPED_MMQ, stream(), 0)
        t.cuda.synchronize()
        assert int(status.item()) == 0
        got = {"weighted_mid": host(mid, np.uint16), "mid_q": host(mq, np.int8),
               "mid_s": host(ms, np.float32), "route_output": host(ro, np.float32)}
        assert_same(got, want)
        assert int(host(flags, np.int32).max()) == 0 and int(host(flags, np.int32).min()) == 0
