"""C ABI checks that need no GPU: libq38m.so loads, exports every function
include/q38m.h declares, keeps the reference's V1 plan byte layout
(include/q38/cuda_moe_prefill.h:24-48, 73-93; cuda_kernel_tests.cu:529-533),
and rejects every invalid argument the reference's host wrappers reject
(cuda/q38_moe_prefill.cu:44-68, :635-866; cuda/q38_moe.cu:352-385) before
touching a device."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import ROOT

HEADERS = [os.path.join(ROOT, "include", name)
           for name in ("q38m.h", "q38m_selftest.h", "q38m_phase.h", "q38m_checked.h")]


def declared_functions(headers=HEADERS[:1]):
    names = set()
    for header in headers:
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        names.update(re.findall(r"\b(q38m_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def exported_functions(path):
    """The q38m_ functions a shared library's dynamic symbol table defines."""
    out = subprocess.run(["nm", "-D", "--defined-only", path], check=True, capture_output=True,
                         text=True).stdout
    return sorted({line.split()[-1] for line in out.splitlines()
                   if line.split()[-1].startswith("q38m_") and line.split()[1] in "TW"})


def test_library_exports_every_declared_symbol(q38m):
    lib = q38m.lib()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(q38m.SIGNATURES), "binding and header disagree"
    assert lib.q38m_moe_compiled() == 1


def test_product_library_exports_exactly_its_header(q38m):
    """libq38m.so exports the operator surface of q38m.h and nothing else:
    the self checks and the phase log live in their own libraries."""
    assert exported_functions(q38m.LIB_PATH) == declared_functions()


def test_selftest_library_exports_its_header(q38m):
    names = declared_functions(HEADERS[1:2])
    assert names == ["q38m_debug_bf16_sweep", "q38m_debug_expf", "q38m_debug_mfma_16x16x32_i8",
                     "q38m_debug_mfma_32x32x32_i8"]
    assert exported_functions(q38m.SELFTEST_LIB_PATH) == names
    assert set(names) == set(q38m.SELFTEST_SIGNATURES)
    q38m.selftest_lib()
    with pytest.raises(q38m.InvalidArgument):
        q38m.call_selftest("q38m_debug_expf", None, 0, None, None, 0)


def test_timed_library_is_the_product_plus_the_phase_log(q38m):
    phase = declared_functions(HEADERS[2:3])
    assert phase == ["q38m_phase_calls_v1", "q38m_phase_log_v1"]
    assert exported_functions(q38m.TIMED_LIB_PATH) == sorted(declared_functions() + phase)
    assert ctypes.sizeof(q38m.PhaseRecord) == 272
    lib = q38m.timed_lib()
    # capacity must be a multiple of 512 records, and null with zero
    assert lib.q38m_phase_log_v1(None, 512, 0) == q38m.ERR_INVALID_ARGUMENT
    assert lib.q38m_phase_log_v1(None, 0, -1) == q38m.ERR_INVALID_ARGUMENT


def test_struct_layouts(q38m):
    assert ctypes.sizeof(q38m.Task) == 8
    assert ctypes.sizeof(q38m.PlanHeader) == 64
    assert q38m.PlanHeader.route_hash.offset == 32
    assert ctypes.sizeof(q38m.RoutePlan) == 56
    assert ctypes.sizeof(q38m.ExpertWeights) == 48


def test_plan_sizes_match_reference_bounds(q38m):
    lib = q38m.lib()
    assert lib.q38m_moe_prefill_routes_v1(512) == 5120
    assert lib.q38m_moe_prefill_max_tasks_v1(128) == 560
    assert lib.q38m_moe_prefill_max_tasks_v1(256) == 640
    assert lib.q38m_moe_prefill_max_tasks_v1(512) == 800
    assert lib.q38m_moe_prefill_max_tasks_v1(1) == 10
    assert lib.q38m_moe_route_plan_bytes_v1(512) == 52552


def test_plan_sizes_match_oracle(q38m, orc):
    for t in (1, 3, 64, 128, 500, 512):
        assert q38m.route_plan_bytes(t) == orc.plan_bytes(t)
        assert q38m.max_tasks(t) == orc.max_tasks(t)


def test_plan_storage_binding_offsets(q38m):
    base = 0x100000
    plan = q38m.bind_plan(base, q38m.route_plan_bytes(512), 512)
    routes = 5120
    assert plan.header == base
    assert plan.expert_counts == base + 64
    assert plan.expert_offsets == base + 64 + 1024
    assert plan.expert_task_offsets == base + 64 + 1024 + 2052
    assert plan.packed_assignment == base + 64 + 1024 + 2 * 2052
    assert plan.assignment_to_packed == plan.packed_assignment + 4 * routes
    assert plan.tasks == plan.assignment_to_packed + 4 * routes


def test_plan_storage_rejects_bad_allocations(q38m):
    with pytest.raises(q38m.InvalidArgument):
        q38m.bind_plan(0x100000, q38m.route_plan_bytes(512) - 1, 512)
    with pytest.raises(q38m.InvalidArgument):
        q38m.bind_plan(0x100008, q38m.route_plan_bytes(512), 512)
    for tokens in (0, 513):
        with pytest.raises(q38m.InvalidArgument):
            q38m.bind_plan(0x100000, 1 << 20, tokens)
    with pytest.raises(q38m.InvalidArgument):
        q38m.bind_plan(None, 1 << 20, 4)


def test_workspace_binding(q38m):
    lib = q38m.lib()
    sizes = [lib.q38m_moe_prefill_workspace_bytes(t) for t in (1, 64, 512)]
    assert sizes[0] < sizes[1] < sizes[2]
    assert lib.q38m_moe_prefill_workspace_bytes(0) == 0
    assert lib.q38m_moe_prefill_workspace_bytes(513) == 0
    ws = q38m.PrefillWorkspace()
    base = 0x1000000
    q38m.call("q38m_moe_prefill_workspace_bind", base, sizes[2], 512, ctypes.byref(ws))
    assert ws.max_tokens == 512 and ws.plan.header == base
    ptrs = [ws.expert_ids, ws.expert_weights, ws.xq, ws.xs, ws.weighted_mid, ws.mid_q,
            ws.mid_s, ws.route_output, ws.task_flags]
    assert ptrs == sorted(ptrs) and all(p % 256 == 0 for p in ptrs)
    assert ws.route_output + 5120 * 2048 * 4 <= ws.task_flags
    assert ws.task_flags + 9 * q38m.max_tasks(512) * 4 <= base + sizes[2]
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_prefill_workspace_bind", base + 16, sizes[2], 512, ctypes.byref(ws))


def fake_weights(q38m, fmt=2, group=32, layout=3, rows=1024, cols=2048, experts=512,
                 scale_dtype=1):
    return q38m.ExpertWeights(0x200000, 0x400000, fmt, group, scale_dtype, layout, experts, rows,
                              cols)


def test_gate_up_validation(q38m):
    good = fake_weights(q38m)
    args = [0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 800, 0x60000, 1, None, 0]

    def call(w, *override):
        a = list(args)
        for i, v in override:
            a[i] = v
        q38m.call("q38m_moe_grouped_gate_up_v1", ctypes.byref(w), *a)

    with pytest.raises(q38m.Unsupported):
        call(fake_weights(q38m, layout=0))
    # groups of 32, 64 and 128 with fp16 or bf16 scales are formats; these are not
    for bad in (fake_weights(q38m, fmt=3), fake_weights(q38m, group=16),
                fake_weights(q38m, group=96), fake_weights(q38m, group=256),
                fake_weights(q38m, group=0), fake_weights(q38m, scale_dtype=0),
                fake_weights(q38m, scale_dtype=3),
                fake_weights(q38m, rows=1280), fake_weights(q38m, cols=2560),
                fake_weights(q38m, experts=256),
                fake_weights(q38m, layout=2)):  # gate/up needs the paired layout
        with pytest.raises(q38m.InvalidArgument):
            call(bad)
    with pytest.raises(q38m.InvalidArgument):
        call(good, (5, 0))          # task_count == 0
    with pytest.raises(q38m.InvalidArgument):
        call(good, (5, 801))        # above the 512-token bound
    with pytest.raises(q38m.InvalidArgument):
        call(good, (0, None))       # null activations
    with pytest.raises(q38m.InvalidArgument):
        call(good, (0, 0x10001))    # misaligned activations
    # validate_grouped_mode (q38_moe_prefill.cu:64-68): grouped and grouped-safe only
    for mode in (0, q38m.MODE_LEGACY_ATOMIC_DIAGNOSTIC, 4):
        with pytest.raises(q38m.InvalidArgument, match="mode"):
            call(good, (7, mode))


def test_down_validation(q38m):
    w8 = fake_weights(q38m, fmt=3, group=0, layout=2, rows=2048, cols=512)
    args = [0x10000, 0x20000, 0x30000, 10, 0x40000, 2, None, 0]
    with pytest.raises(q38m.Unsupported):
        q38m.call("q38m_moe_grouped_down_v1",
                  ctypes.byref(fake_weights(q38m, fmt=3, group=0, layout=0, rows=2048, cols=512)),
                  *args)
    for group in (32, 96, 256):  # W8 down: per channel or groups of 64/128 only
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_grouped_down_v1",
                      ctypes.byref(fake_weights(q38m, fmt=3, group=group, layout=2, rows=2048,
                                                cols=512)), *args)
    for group in (0, 16, 256):  # W4 down: groups of 32/64/128 only
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_grouped_down_v1",
                      ctypes.byref(fake_weights(q38m, fmt=2, group=group, layout=2, rows=2048,
                                                cols=512)), *args)
    with pytest.raises(q38m.InvalidArgument):  # unknown scale dtype
        q38m.call("q38m_moe_grouped_down_v1",
                  ctypes.byref(fake_weights(q38m, fmt=3, group=0, layout=2, rows=2048, cols=512,
                                            scale_dtype=7)), *args)
    with pytest.raises(q38m.InvalidArgument):  # transposed shape
        q38m.call("q38m_moe_grouped_down_v1",
                  ctypes.byref(fake_weights(q38m, fmt=3, group=0, layout=2, rows=512, cols=2048)), *args)
    for mode in (0, 3):
        bad = list(args)
        bad[5] = mode
        with pytest.raises(q38m.InvalidArgument, match="mode"):
            q38m.call("q38m_moe_grouped_down_v1", ctypes.byref(w8), *bad)
    args[2] = None
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_grouped_down_v1", ctypes.byref(w8), *args)


def test_routing_and_quant_validation(q38m):
    plan = q38m.bind_plan(0x100000, q38m.route_plan_bytes(8), 8)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_build_route_plan_v1", 0x1000, 0, ctypes.byref(plan), 0, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_build_route_plan_v1", 0x1000, 513, ctypes.byref(plan), 0, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_build_route_plan_v1", 0x1000, 8, ctypes.byref(plan), 2, None, 0)
    broken = q38m.RoutePlan()
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_build_route_plan_v1", 0x1000, 8, ctypes.byref(broken), 0, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_topk_router_f32", 0x1000, 0x2000, 0x3000, 4, 512, 33, 1, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_topk_router_f32", 0x1000, 0x2000, 0x3000, 4, 500, 10, 1, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_topk_router_bf16", 0x1000, 0x2000, 0x3000, 4, 512, 33, 1, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_topk_router_bf16", 0x1000, 0x2000, 0x3000, 4, 500, 10, 1, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_topk_router_bf16", None, 0x2000, 0x3000, 4, 512, 10, 1, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_quantize_rows_i8", 0x1000, 4, 1536, 0x2000, 0x3000, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_reduce_top10_and_combine_shared_v1", 0x1000, 0x2000, 0x3000, None,
                  4, 0x4000, None, 0)  # shared output without its gate
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_pack_hidden_v1", 0x1000, 0x2000, 15, 2048, 0x3000, None, 0)


def test_weight_quantizer_validation(q38m):
    def desc(fmt=2, group=32, scale=1, layout=0, rows=1024, cols=2048, data=0x200000,
             scales=0x400000):
        return q38m.ExpertWeights(data, scales, fmt, group, scale, layout, 512, rows, cols)

    for d, err in [(desc(layout=2), q38m.InvalidArgument),        # not row-major
                   (desc(scale=0), q38m.InvalidArgument),         # scale dtype
                   (desc(scale=3), q38m.InvalidArgument),         # scale dtype
                   (desc(data=0x200008), q38m.InvalidArgument),   # misaligned data
                   (desc(group=16), q38m.Unsupported),            # W4 group 16
                   (desc(group=0), q38m.Unsupported),             # W4 per channel
                   (desc(fmt=3, group=0, cols=500), q38m.Unsupported),  # per channel, 500 cols
                   (desc(group=128, cols=2000), q38m.Unsupported)]:     # 2000 % 128
        with pytest.raises(err):
            q38m.call("q38m_quantize_expert_weights", 0x100000, ctypes.byref(d), None, 0)
    with pytest.raises(q38m.InvalidArgument):  # no source
        q38m.call("q38m_quantize_expert_weights", None, ctypes.byref(desc()), None, 0)


def test_route_quantize_validation(q38m):
    # logits, hidden, tokens, ids, weights, xq, xs
    good = [0x1000, 0x2000, 8, 0x3000, 0x4000, 0x5000, 0x6000]
    for i, bad in [(0, None), (1, None), (2, 0), (3, None), (4, None), (5, None), (6, None),
                   (0, 0x1004), (1, 0x2008), (5, 0x5004)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_route_quantize_v1", *args, None, 0)


def test_dense_validation(q38m):
    # a, b, m, n, k, c_f32, c_bf16
    good = [0x1000, 0x2000, 64, 512, 2048, 0x3000, None]
    for i, bad in [(0, None), (1, None), (2, 0), (3, 0), (4, 0), (4, 48), (5, None),
                   (2, 65535 * 32 + 1), (0, 0x1008), (1, 0x2002)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_dense_gemm_bf16", *args, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # both outputs
        q38m.call("q38m_dense_gemm_bf16", 0x1000, 0x2000, 64, 512, 2048, 0x3000, 0x4000, None, 0)
    # hidden, router, tokens, hidden_width, logits
    good = [0x1000, 0x2000, 8, 2048, 0x3000]
    for i, bad in [(0, None), (1, None), (2, 0), (3, 2560), (3, 1024), (4, None), (0, 0x1004)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_router_v1", *args, None, 0)
    # hidden, wg, wu, wd, wo, tokens, hidden_width, inter, scratch, shared_output, shared_gate
    good = [0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 8, 2048, 512, 0x6000, 0x7000, 0x8000]
    for i, bad in [(0, None), (4, None), (5, 0), (6, 2560), (7, 0), (7, 520), (8, None),
                   (9, None), (10, None), (3, 0x4008), (8, 0x6004)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_shared_expert_v1", *args, None, 0)
    assert q38m.lib().q38m_moe_shared_expert_scratch_bytes(8, 512) == 3 * 8 * 512 * 2
    # hidden, router, tokens, hidden_width, top_k, workspace, workspace_bytes, ids, weights
    ws = q38m.lib().q38m_moe_router_topk_workspace_bytes(8)
    assert ws == 8 * 8 * (10 * 8 + 4)
    good = [0x1000, 0x2000, 8, 2048, 10, 0x3000, ws, 0x4000, 0x5000]
    for i, bad in [(0, None), (1, None), (2, 0), (2, 65535 * 16 + 1), (3, 2560), (4, 0), (4, 11),
                   (5, None), (6, ws - 1), (7, None), (8, None), (0, 0x1004), (5, 0x3008)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_router_topk_v1", *args, None, 0)


def test_hyper_validation(q38m):
    # hyper, norm_weight, mix_down, mix_up, inject, tokens, hidden, low_rank, scratch, mixed, injection
    good = [0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 8, 2560, 320, 0x6000, 0x7000, 0x8000]
    for i, bad in [(0, None), (2, None), (5, 0), (6, 0), (6, 2564), (6, 8200), (7, 0), (7, 300),
                   (8, None), (9, None), (10, None), (0, 0x1008), (4, 0x5004)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_hyper_prepare_v1", *args, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # element count not a multiple of 8
        q38m.call("q38m_hyper_sigmoid_bf16", 0x1000, 0x2000, 3, 5, 1.0, 1.0, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # divisor must be positive
        q38m.call("q38m_hyper_silu_scaled_bf16", 0x1000, 0x2000, 8, 320, 0.0, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_hyper_inject_bf16", 0x1000, 0x2000, None, 0x3000, 8, 2560, None, 0)
    assert q38m.lib().q38m_hyper_prepare_scratch_bytes(8, 2560, 320) == 2 * 8 * 4 * 2560 * 2 + 8 * 320 * 2


def test_decode_and_step_validation(q38m):
    gu = fake_weights(q38m)
    dn = fake_weights(q38m, fmt=3, group=0, layout=2, rows=2048, cols=512)
    with pytest.raises(q38m.InvalidArgument):  # top_k above 10
        q38m.call("q38m_moe_routed_decode_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000,
                  0x2000, 0x3000, 11, 0x4000, 0x5000, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # no scratch
        q38m.call("q38m_moe_routed_decode_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000,
                  0x2000, 0x3000, 10, None, 0x5000, None, 0)
    # fused decode: gu, dn, hidden, logits, top_k, shared, gate, residual, scratch, out
    with pytest.raises(q38m.InvalidArgument):  # no logits
        q38m.call("q38m_moe_decode_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, None, 10,
                  None, None, None, 0x4000, 0x5000, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # top_k 0
        q38m.call("q38m_moe_decode_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2000, 0,
                  None, None, None, 0x4000, 0x5000, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # shared output without its gate
        q38m.call("q38m_moe_decode_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2000, 10,
                  0x6000, None, None, 0x4000, 0x5000, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # misaligned logits
        q38m.call("q38m_moe_decode_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2004, 10,
                  None, None, None, 0x4000, 0x5000, None, 0)
    with pytest.raises(q38m.Unsupported):  # row-major gate/up
        rm = fake_weights(q38m, layout=0)
        q38m.call("q38m_moe_decode_v1", ctypes.byref(rm), ctypes.byref(dn), 0x1000, 0x2000, 10,
                  None, None, None, 0x4000, 0x5000, None, 0)
    ws = q38m.PrefillWorkspace()
    q38m.call("q38m_moe_prefill_workspace_bind", 0x1000000,
              q38m.lib().q38m_moe_prefill_workspace_bytes(64), 64, ctypes.byref(ws))
    with pytest.raises(q38m.InvalidArgument):  # more tokens than the workspace holds
        q38m.call("q38m_moe_prefill_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2000, 65,
                  ctypes.byref(ws), None, None, 0x3000, None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_moe_prefill_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2000, 64,
                  ctypes.byref(ws), None, None, 0x3000, None, -1)  # negative device


def test_slab_step_on_a_chunk_workspace(q38m):
    """A chunk workspace holds more tokens than a slab: the slab entry point
    (whose plan kernel and task grid are sized for <= 512 tokens) must
    reject 513 tokens before any launch, and a chunk workspace bound for
    <= 512 tokens has task slots for a full V1 plan."""
    lib = q38m.lib()
    gu = fake_weights(q38m)
    dn = fake_weights(q38m, fmt=3, group=0, layout=2, rows=2048, cols=512)
    wide = q38m.WideWorkspace()
    base = 0x10000000
    q38m.call("q38m_moe_wide_workspace_bind", base, lib.q38m_moe_wide_workspace_bytes(4096), 4096,
              ctypes.byref(wide))
    assert wide.step.max_tokens == 4096
    for tokens in (513, 4096):
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_prefill_v1", ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2000,
                      tokens, ctypes.byref(wide.step), None, None, 0x3000, None, 0)
    for tokens in (1, 64, 300, 512, 600, 4096):
        slab = min(tokens, 512)
        task_bytes = lib.q38m_moe_wide_plan_bytes(tokens) - (
            64 + 1024 + 2 * 2052 + 2 * 4 * 10 * tokens)
        assert task_bytes >= 8 * lib.q38m_moe_prefill_max_tasks_v1(slab)
        assert task_bytes >= 8 * lib.q38m_moe_wide_max_tasks(tokens)
    # the slab step's hand-off flags: a V1 plan's task slots, inside the workspace
    for tokens in (64, 4096):
        q38m.call("q38m_moe_wide_workspace_bind", base, lib.q38m_moe_wide_workspace_bytes(tokens),
                  tokens, ctypes.byref(wide))
        step = wide.step
        assert step.route_output + 10 * tokens * 2048 * 4 <= step.task_flags
        assert (step.task_flags + 36 * lib.q38m_moe_prefill_max_tasks_v1(min(tokens, 512)) <=
                base + lib.q38m_moe_wide_workspace_bytes(tokens))


def test_gate_up_down_validation(q38m):
    """q38m_moe_grouped_gate_up_down_v1 rejects what either staged entry
    point rejects, and missing flags or status, before any launch."""
    gu = fake_weights(q38m)
    dn = fake_weights(q38m, fmt=3, group=0, layout=2, rows=2048, cols=512)
    # xq, xs, packed, weights, tasks, task_count, mid, mid_q, mid_s, flags, status, out, mode
    good = [0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 16, 0x6000, 0x7000, 0x8000, 0x9000,
            0xa000, 0xb000, q38m.MODE_GROUPED_MMQ]
    bad_values = [(0, None), (1, None), (2, None), (3, None), (4, None), (5, 0),
                  (5, q38m.max_tasks(512) + 1), (6, None), (7, None), (8, None), (9, None),
                  (10, None), (11, None), (12, 3), (9, 0x9002), (0, 0x1004)]
    for i, bad in bad_values:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_grouped_gate_up_down_v1", ctypes.byref(gu), ctypes.byref(dn),
                      *args, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # down given as gate/up
        q38m.call("q38m_moe_grouped_gate_up_down_v1", ctypes.byref(dn), ctypes.byref(dn), *good,
                  None, 0)
    for args in ([None, 16], [0x9000, 0], [0x9000, q38m.max_tasks(512) + 1], [0x9002, 16]):
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_clear_task_flags_v1", *args, None, 0)


def test_combine_shared_validation(q38m):
    # routed, shared, gate, output, tokens
    good = [0x1000, 0x2000, 0x3000, 0x4000, 4]
    for i, bad in [(0, None), (1, None), (2, None), (3, None), (4, 0)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_combine_shared_bf16", *args, None, 0)


def test_repack_and_synth_validation(q38m):
    src = fake_weights(q38m, layout=0)
    dst = fake_weights(q38m, layout=2)
    with pytest.raises(q38m.InvalidArgument):  # same layout on both sides
        q38m.call("q38m_repack_expert_weights", ctypes.byref(dst), ctypes.byref(dst), None, 0)
    with pytest.raises(q38m.InvalidArgument):  # shape mismatch
        q38m.call("q38m_repack_expert_weights", ctypes.byref(src),
                  ctypes.byref(fake_weights(q38m, layout=2, rows=2048)), None, 0)
    with pytest.raises(q38m.Unsupported):  # W4 per-channel has no MFMA16 layout
        q38m.call("q38m_repack_expert_weights", ctypes.byref(fake_weights(q38m, group=0, layout=0)),
                  ctypes.byref(fake_weights(q38m, group=0, layout=2)), None, 0)
    with pytest.raises(q38m.Unsupported):  # W4 groups of 32/64/128 only
        q38m.call("q38m_repack_expert_weights", ctypes.byref(fake_weights(q38m, group=256, layout=0)),
                  ctypes.byref(fake_weights(q38m, group=256, layout=3)), None, 0)
    with pytest.raises(q38m.Unsupported):  # W8 per channel or groups of 64/128 only
        q38m.call("q38m_repack_expert_weights",
                  ctypes.byref(fake_weights(q38m, fmt=3, group=32, layout=0, rows=2048, cols=512)),
                  ctypes.byref(fake_weights(q38m, fmt=3, group=32, layout=2, rows=2048, cols=512)),
                  None, 0)
    with pytest.raises(q38m.InvalidArgument):  # the scale dtype is kept
        q38m.call("q38m_repack_expert_weights", ctypes.byref(src),
                  ctypes.byref(fake_weights(q38m, layout=3, scale_dtype=2)), None, 0)
    w8_src = fake_weights(q38m, fmt=3, group=0, layout=0, rows=2064, cols=512)
    with pytest.raises(q38m.Unsupported):  # pairing needs an even number of row tiles
        q38m.call("q38m_repack_expert_weights", ctypes.byref(w8_src),
                  ctypes.byref(fake_weights(q38m, fmt=3, group=0, layout=3, rows=2064, cols=512)),
                  None, 0)
    with pytest.raises(q38m.InvalidArgument):
        q38m.call("q38m_synth_fill", 9, 1, 1, 16, 1.0, 0, 0, None, 0, 0x1000, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # odd W4 count
        q38m.call("q38m_synth_fill", 4, 1, 1, 15, 1.0, -8, 7, None, 0, 0x1000, None, 0)
    with pytest.raises(q38m.InvalidArgument):  # int4 range
        q38m.call("q38m_synth_fill", 4, 1, 1, 16, 1.0, -9, 7, None, 0, 0x1000, None, 0)


def test_weight_byte_counts(q38m):
    d, s = q38m.weights_bytes(2, 32, 512, 1024, 2048)
    assert (d, s) == (512 * 1024 * 1024, 512 * 1024 * 64 * 2)
    d, s = q38m.weights_bytes(3, 0, 512, 2048, 512)
    assert (d, s) == (512 * 2048 * 512, 512 * 2048 * 2)


def test_error_message_is_reported(q38m):
    try:
        q38m.bind_plan(0x100000, 10, 512)
    except q38m.InvalidArgument as exc:
        assert "too small" in str(exc)
    else:
        raise AssertionError("expected InvalidArgument")


CPP_PROGRAM = r"""
#include "q38m.hpp"
#include <cstdio>
int main() {
    static_assert(q38m::q38_moe_route_plan_bytes_v1(512) == 52552, "plan bytes");
    static_assert(q38m::q38_moe_prefill_max_tasks_v1(128) == 560, "max tasks");
    if (q38m_moe_route_plan_bytes_v1(512) != 52552) return 2;
    alignas(16) static unsigned char arena[1 << 16];
    auto plan = q38m::cuda_moe_route_plan_storage_v1(arena, sizeof(arena), 512);
    if (reinterpret_cast<unsigned char*>(plan.tasks) != arena + 52552 - 800 * 8) return 3;
    try {
        q38m::cuda_moe_route_plan_storage_v1(arena, 100, 512);
        return 4;
    } catch (const std::invalid_argument& e) {
        std::printf("invalid_argument: %s\n", e.what());
    }
    q38m_expert_weights_v1 rm{arena, arena, Q38M_FORMAT_W4_SYM, 32, Q38M_SCALE_F16,
                              Q38M_LAYOUT_ROW_MAJOR, 512, 1024, 2048};
    try {
        q38m::cuda_moe_grouped_gate_up_v1(rm, nullptr, nullptr, nullptr, nullptr, nullptr, 1,
                                          nullptr, q38m::Q38PrefillMoeModeV1::kGroupedMmq,
                                          nullptr, 0);
        return 5;
    } catch (const std::invalid_argument& e) {
        std::printf("unsupported layout: %s\n", e.what());
    }
    std::printf("ok\n");
    return 0;
}
"""


def test_cpp_wrapper_compiles_links_and_throws(tmp_path):
    import subprocess
    src = tmp_path / "wrapper.cpp"
    src.write_text(CPP_PROGRAM)
    exe = tmp_path / "wrapper"
    pkg = os.path.join(ROOT, "qwen3.8-flash-next-dual-gpu_amd")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    str(src), "-o", str(exe), "-L", pkg, "-lq38m", f"-Wl,-rpath,{pkg}",
                    "-Wl,-rpath,/opt/rocm/lib"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "too small" in out.stdout and "MFMA16" in out.stdout and out.stdout.endswith("ok\n")


def _function_with_comment(text, signature):
    """The comment block above `signature` through the function's closing brace."""
    start = text.index(signature)
    lines = text[:start].split("\n")[:-1]
    while lines and lines[-1].startswith("//"):
        lines.pop()
    begin = len("\n".join(lines)) + 1 if lines else 0
    return text[begin:text.index("\n}\n", start) + 3]


def test_integration_run_moe_is_the_compiled_stage_code():
    """INTEGRATION.md shows run_moe and the slab loop verbatim from
    include/q38m_stage.hpp, the header tests/test_gpu_stage.py compiles and
    runs against libq38m.so."""
    stage = open(os.path.join(ROOT, "include", "q38m_stage.hpp")).read()
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    for signature in ("inline void run_moe(", "inline std::uint16_t* run_prefill_moe("):
        body = _function_with_comment(stage, signature)
        assert body.count("\n") > 10
        assert "```cpp\n" + body + "```" in doc, signature
    assert "2560, 320" not in doc


def test_stage_header_compiles_and_validates_workspace(tmp_path):
    """The stage header builds with the host compiler and no vendor header;
    its workspace binder rejects a bad allocation before any device call."""
    import subprocess
    src = tmp_path / "stage.cpp"
    src.write_text(r'''
#include "q38m_stage.hpp"
#include <cstdio>
int main() {
    const std::size_t bytes = q38m::moe_stage_workspace_bytes(512);
    if (bytes == 0 || q38m::moe_stage_workspace_bytes(513) != 0) return 2;
    try {
        q38m::bind_moe_stage_workspace(reinterpret_cast<void*>(0x1000), bytes - 1, 512);
        return 3;
    } catch (const std::invalid_argument&) {}
    auto ws = q38m::bind_moe_stage_workspace(reinterpret_cast<void*>(0x100000), bytes, 512);
    if (ws.max_tokens != 512 || ws.moe.max_tokens != 512) return 4;
    const auto end = reinterpret_cast<std::uintptr_t>(ws.decode_scratch) +
                     q38m_moe_decode_scratch_bytes();
    if (end > 0x100000 + bytes) return 5;
    std::printf("ok\n");
    return 0;
}
''')
    exe = tmp_path / "stage"
    pkg = os.path.join(ROOT, "qwen3.8-flash-next-dual-gpu_amd")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-I",
                    os.path.join(ROOT, "include"), str(src), "-o", str(exe), "-L", pkg, "-lq38m",
                    f"-Wl,-rpath,{pkg}", "-Wl,-rpath,/opt/rocm/lib"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout == "ok\n", out.stdout + out.stderr


def test_checked_library_is_the_product_plus_the_status_word(q38m):
    checked = declared_functions(HEADERS[3:])
    assert checked == ["q38m_checked_status_v1"]
    assert exported_functions(q38m.CHECKED_LIB_PATH) == sorted(declared_functions() + checked)
    lib = q38m.checked_lib()
    assert lib.q38m_checked_status_v1(None, 0, 0) == q38m.ERR_INVALID_ARGUMENT
    # the checked build rejects the same arguments as the product library
    assert lib.q38m_moe_prefill_max_tasks_v1(512) == 800


def test_decode_block_validation(q38m):
    gu = fake_weights(q38m)
    dn = fake_weights(q38m, fmt=3, group=0, layout=2, rows=2048, cols=512)
    # gu, dn, hidden, router, w_gate, w_up, w_down, w_out_gate, shared_inter, top_k,
    # residual, scratch, output
    good = [ctypes.byref(gu), ctypes.byref(dn), 0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000,
            512, 10, None, 0x7000, 0x8000]
    for i, bad in [(2, None), (3, None), (4, None), (5, None), (6, None), (7, None),
                   (8, 256), (8, 1024), (9, 0), (9, 11), (11, None), (12, None),
                   (2, 0x1008), (3, 0x2002), (11, 0x7004), (10, 0x9001)]:
        args = list(good)
        args[i] = bad
        with pytest.raises(q38m.InvalidArgument):
            q38m.call("q38m_moe_decode_block_v1", *args, None, 0)
    with pytest.raises(q38m.Unsupported):  # row-major gate/up
        rm = fake_weights(q38m, layout=0)
        q38m.call("q38m_moe_decode_block_v1", ctypes.byref(rm), *good[1:], None, 0)
    assert q38m.lib().q38m_moe_decode_block_scratch_bytes() >= (
        q38m.lib().q38m_moe_decode_scratch_bytes() + 512 * 4 + 512 * 2 + 2)
