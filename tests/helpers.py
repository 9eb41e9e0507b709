"""GPU test plumbing: synthetic layers built on the device with the product's
generator, host copies for the oracle, and thin wrappers that run the
product's C ABI on torch-allocated buffers."""
import ctypes
import importlib.util
import os

import numpy as np

from conftest import PACKAGE_DIR, load_product

_spec = importlib.util.spec_from_file_location("q38m_workloads",
                                               os.path.join(PACKAGE_DIR, "workloads.py"))
W = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(W)


def torch():
    import torch as t
    return t


def host(tensor, dtype):
    """Device tensor -> numpy array reinterpreted as dtype."""
    return tensor.detach().cpu().numpy().view(dtype)


def device(array):
    t = torch()
    a = np.ascontiguousarray(array)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return t.from_numpy(a.copy()).cuda()


def stream():
    return torch().cuda.current_stream().cuda_stream


class Layer:
    """One MoE layer's weights: row-major on the device, repacked MFMA16 on
    the device, and the row-major bytes on the host for the oracle."""

    def __init__(self, q38m, orc, seed, layer, gate_up_fmt, down_fmt, with_host=True,
                 gate_up_bf16=False, down_bf16=False):
        gu_tag, dn_tag, _, _ = W.layer_tags(layer)
        _, gbits, ggroup, gsigma = gate_up_fmt
        _, dbits, dgroup, dsigma = down_fmt
        fmt = {4: q38m.FORMAT_W4_SYM, 8: q38m.FORMAT_W8_SYM}
        dtype = {False: q38m.SCALE_F16, True: q38m.SCALE_BF16}
        self.gu_rm = q38m.synth_weights(seed, gu_tag, fmt[gbits], ggroup, W.EXPERTS,
                                        2 * W.INTER, W.HIDDEN, gsigma,
                                        scale_dtype=dtype[gate_up_bf16])
        self.dn_rm = q38m.synth_weights(seed, dn_tag, fmt[dbits], dgroup, W.EXPERTS, W.HIDDEN,
                                        W.INTER, dsigma, scale_dtype=dtype[down_bf16])
        self.gu = q38m.repack(self.gu_rm, paired=True)
        self.dn = q38m.repack(self.dn_rm)
        self.host_gu = self.host_dn = None
        if with_host:
            self.host_gu = orc.HostWeights(host(self.gu_rm.data, np.uint8),
                                           host(self.gu_rm.scales, np.uint16), gbits, ggroup,
                                           W.EXPERTS, 2 * W.INTER, W.HIDDEN, gate_up_bf16)
            self.host_dn = orc.HostWeights(host(self.dn_rm.data, np.uint8),
                                           host(self.dn_rm.scales, np.uint16), dbits, dgroup,
                                           W.EXPERTS, W.HIDDEN, W.INTER, down_bf16)

    def drop_row_major(self):
        self.gu_rm = self.dn_rm = None


def synth_hidden(q38m, seed, tag, tokens):
    t = torch()
    out = t.empty(tokens * W.HIDDEN, dtype=t.int16, device="cuda")
    q38m.synth_fill(q38m.SYNTH_NORMAL_BF16, seed, tag, out.numel(), out)
    return out.view(tokens, W.HIDDEN)


def synth_logits(q38m, seed, tag, tokens, bias=None):
    t = torch()
    out = t.empty(tokens * W.EXPERTS, dtype=t.float32, device="cuda")
    b = None if bias is None else t.tensor(bias, dtype=t.float32, device="cuda")
    q38m.synth_fill(q38m.SYNTH_NORMAL_F32, seed, tag, out.numel(), out, bias=b)
    return out.view(tokens, W.EXPERTS)


def prefill(q38m, layer, hidden, logits, ws, output=None, shared=None, call=None):
    """Runs q38m_moe_prefill_v1 on device tensors (through `call`, by
    default the product library's); returns the bf16 output."""
    t = torch()
    tokens = hidden.shape[0]
    if output is None:
        output = t.empty(tokens, W.HIDDEN, dtype=t.int16, device="cuda")
    so, sg = (None, None) if shared is None else shared
    (call or q38m.call)("q38m_moe_prefill_v1", ctypes.byref(layer.gu.desc), ctypes.byref(layer.dn.desc),
              hidden.data_ptr(), None if logits is None else logits.data_ptr(), tokens,
              ctypes.byref(ws.ws), None if so is None else so.data_ptr(),
              None if sg is None else sg.data_ptr(), output.data_ptr(), stream(), 0)
    return output


def staged_step(q38m, layer, hidden, logits):
    """The reference's staged call sequence (run_moe, cuda_backend.cu:
    1516-1605) through the single-purpose entry points: top-k, route plan,
    token quantisation, grouped gate/up, mid quantisation, grouped down and
    the rank-order combine.  Returns the bf16 output."""
    t = torch()
    T = hidden.shape[0]
    R = T * W.TOPK
    s = stream()
    ids = t.empty(R, dtype=t.int32, device="cuda")
    wts = t.empty(R, dtype=t.float32, device="cuda")
    q38m.call("q38m_topk_router_f32", logits.data_ptr(), ids.data_ptr(), wts.data_ptr(), T,
              W.EXPERTS, W.TOPK, 1, s, 0)
    nbytes = q38m.route_plan_bytes(T)
    buf = t.empty(nbytes + 256, dtype=t.uint8, device="cuda")
    plan = q38m.bind_plan((buf.data_ptr() + 255) // 256 * 256, nbytes, T)
    q38m.call("q38m_moe_build_route_plan_v1", ids.data_ptr(), T, ctypes.byref(plan), 0, s, 0)
    xq = t.empty(T, W.HIDDEN, dtype=t.int8, device="cuda")
    xs = t.empty(T, dtype=t.float32, device="cuda")
    q38m.call("q38m_quantize_rows_i8", hidden.data_ptr(), T, W.HIDDEN, xq.data_ptr(),
              xs.data_ptr(), s, 0)
    tasks = q38m.max_tasks(T)
    mid = t.empty(R, W.INTER, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_grouped_gate_up_v1", ctypes.byref(layer.gu.desc), xq.data_ptr(),
              xs.data_ptr(), plan.packed_assignment, wts.data_ptr(), plan.tasks, tasks,
              mid.data_ptr(), q38m.MODE_GROUPED_MMQ, s, 0)
    mq = t.empty(R, W.INTER, dtype=t.int8, device="cuda")
    ms = t.empty(R, dtype=t.float32, device="cuda")
    q38m.call("q38m_quantize_rows_i8", mid.data_ptr(), R, W.INTER, mq.data_ptr(), ms.data_ptr(),
              s, 0)
    route_output = t.empty(R, W.HIDDEN, dtype=t.float32, device="cuda")
    q38m.call("q38m_moe_grouped_down_v1", ctypes.byref(layer.dn.desc), mq.data_ptr(),
              ms.data_ptr(), plan.tasks, tasks, route_output.data_ptr(), q38m.MODE_GROUPED_MMQ_SAFE,
              s, 0)
    out = t.empty(T, W.HIDDEN, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_reduce_top10_and_combine_shared_v1", route_output.data_ptr(),
              plan.assignment_to_packed, None, None, T, out.data_ptr(), s, 0)
    return out


def decode(q38m, layer, hidden, ids, weights, scratch, output=None, top_k=10):
    t = torch()
    if output is None:
        output = t.empty(1, W.HIDDEN, dtype=t.int16, device="cuda")
    q38m.call("q38m_moe_routed_decode_v1", ctypes.byref(layer.gu.desc),
              ctypes.byref(layer.dn.desc), hidden.data_ptr(), ids.data_ptr(), weights.data_ptr(),
              top_k, scratch.data_ptr(), output.data_ptr(), stream(), 0)
    return output


def decode_fused(q38m, layer, hidden, logits, scratch, output=None, top_k=10, shared=None,
                 residual=None, call=None):
    """Runs q38m_moe_decode_v1 (top-k from logits, routed experts, optional
    gated shared term and residual) on device tensors."""
    t = torch()
    if output is None:
        output = t.empty(1, W.HIDDEN, dtype=t.int16, device="cuda")
    so, sg = (None, None) if shared is None else shared
    (call or q38m.call)("q38m_moe_decode_v1", ctypes.byref(layer.gu.desc), ctypes.byref(layer.dn.desc),
              hidden.data_ptr(), logits.data_ptr(), top_k,
              None if so is None else so.data_ptr(), None if sg is None else sg.data_ptr(),
              None if residual is None else residual.data_ptr(), scratch.data_ptr(),
              output.data_ptr(), stream(), 0)
    return output


def decode_scratch(q38m):
    t = torch()
    return t.zeros(q38m.lib().q38m_moe_decode_scratch_bytes() // 2 + 64, dtype=t.int16,
                   device="cuda")


def scratch_ids(scratch, top_k=10):
    """The ids q38m_moe_decode_v1 leaves at the start of its scratch."""
    torch().cuda.synchronize()
    return host(scratch[:2 * top_k], np.int32).copy()


def ws_arrays(ws, tokens):
    """Workspace regions (views into the workspace's own device buffer)
    as numpy arrays."""
    t = torch()
    t.cuda.synchronize()
    r = tokens * 10
    base = ws.buffer.data_ptr()

    def grab(address, count, itemsize, np_dtype):
        offset = address - base
        raw = ws.buffer[offset:offset + count * itemsize]
        return raw.cpu().numpy().view(np_dtype)

    w = ws.ws
    return {
        "ids": grab(w.expert_ids, r, 4, np.int32).reshape(tokens, 10),
        "weights": grab(w.expert_weights, r, 4, np.float32).reshape(tokens, 10),
        "xq": grab(w.xq, tokens * W.HIDDEN, 1, np.int8).reshape(tokens, W.HIDDEN),
        "xs": grab(w.xs, tokens, 4, np.float32),
        "weighted_mid": grab(w.weighted_mid, r * W.INTER, 2, np.uint16).reshape(r, W.INTER),
        "mid_q": grab(w.mid_q, r * W.INTER, 1, np.int8).reshape(r, W.INTER),
        "mid_s": grab(w.mid_s, r, 4, np.float32),
        "route_output": grab(w.route_output, r * W.HIDDEN, 4, np.float32).reshape(r, W.HIDDEN),
        "plan": grab(w.plan.header, load_product().route_plan_bytes(ws.max_tokens), 1, np.uint8),
    }


def canonical_nan(words):
    """bf16 words with every NaN as 0x7fc0: a NaN's sign and payload depend
    on the instruction set that produced it (x86 and the GPU differ), not on
    the arithmetic, and nothing downstream reads them."""
    w = np.array(words, dtype=np.uint16, copy=True)
    w[((w & 0x7f80) == 0x7f80) & ((w & 0x007f) != 0)] = 0x7fc0
    return w


def pow2_normalize(orc, words):
    """Scales each row of bf16 words by 2^-k, k = floor(log2(row rms)),
    which brings every row's rms into [1, 2).  Only exponents change, so the
    scaling is exact; it is the chained tests' deterministic stand-in for
    the norm a model applies between its MoE layers (the product has none:
    the reference's layer ends at the residual add)."""
    w = np.ascontiguousarray(words, dtype=np.uint16)
    f = orc.bf16_to_f32(w)
    rms = np.sqrt(np.mean(f.astype(np.float64) ** 2, axis=-1, keepdims=True))
    assert np.isfinite(rms).all() and (rms > 0).all()
    scaled = f * np.exp2(-np.floor(np.log2(rms))).astype(np.float32)
    out = orc.f32_to_bf16(scaled).reshape(w.shape)
    assert np.array_equal(orc.bf16_to_f32(out), scaled)  # exact
    return out


def oracle_chunk(orc, hidden, logits, gate_up, down, slab=512):
    """The oracle over a chunk of any size, evaluated as consecutive slabs
    through its grouped path (T <= 512 per call): a token's output depends
    only on its own row, logits and routes (per-token and per-route
    quantisation, rank-order combine), so the slabs' outputs are the
    chunk's.  hidden: bf16 words [T][H]; logits: fp32 [T][E]."""
    tokens = hidden.shape[0]
    out = np.empty(hidden.shape, dtype=np.uint16)
    for s0 in range(0, tokens, slab):
        sl = slice(s0, min(tokens, s0 + slab))
        out[sl] = orc.moe(np.ascontiguousarray(hidden[sl]), gate_up, down,
                          logits=np.ascontiguousarray(logits[sl]), grouped=True)["output"]
    return out
