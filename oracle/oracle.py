"""ctypes + numpy binding of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
this module (see q38m_oracle.h for the reference lines each function
follows and how each is pinned).
"""
import ctypes
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
# Q38M_ORACLE_LIB selects another build of the same source (the sanitizer
# build of `make -C oracle check-sanitize`).
LIB_PATH = os.environ.get("Q38M_ORACLE_LIB") or os.path.join(ORACLE_DIR, "_build",
                                                             "libq38m_oracle.so")

EXPERTS = 512
TOPK = 10
MMQ_M = 16


class Weights(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("bits", ctypes.c_uint32), ("group", ctypes.c_uint32),
                ("experts", ctypes.c_uint32), ("rows", ctypes.c_uint32),
                ("cols", ctypes.c_uint32), ("scale_bf16", ctypes.c_uint32)]


class MoeIO(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
                ("inter", ctypes.c_uint32),
                ("hidden_states", ctypes.c_void_p), ("logits", ctypes.c_void_p),
                ("ids", ctypes.c_void_p), ("weights", ctypes.c_void_p),
                ("gate_up", ctypes.POINTER(Weights)), ("down", ctypes.POINTER(Weights)),
                ("shared_output", ctypes.c_void_p), ("shared_gate", ctypes.c_void_p),
                ("output", ctypes.c_void_p), ("plan", ctypes.c_void_p),
                ("xq", ctypes.c_void_p), ("xs", ctypes.c_void_p),
                ("weighted_mid", ctypes.c_void_p), ("mid_q", ctypes.c_void_p),
                ("mid_s", ctypes.c_void_p), ("route_output", ctypes.c_void_p)]


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_INT = ctypes.c_int

_SIGS = {
    "q38o_f32_to_bf16": (ctypes.c_uint16, [_F]),
    "q38o_bf16_to_f32": (_F, [ctypes.c_uint16]),
    "q38o_f32_to_f16": (ctypes.c_uint16, [_F]),
    "q38o_f16_to_f32": (_F, [ctypes.c_uint16]),
    "q38o_expf": (_F, [_F]),
    "q38o_logf": (_F, [_F]),
    "q38o_expf_array": (None, [_P, _SZ, _P]),
    "q38o_f32_to_bf16_array": (None, [_P, _SZ, _P]),
    "q38o_f32_to_f16_array": (None, [_P, _SZ, _P]),
    "q38o_f16_to_f32_array": (None, [_P, _SZ, _P]),
    "q38o_rand64": (_U64, [_U64, _U64, _U64]),
    "q38o_synth_normal_f32": (None, [_U64, _U64, _F, _INT, _SZ, _P]),
    "q38o_synth_normal_bf16": (None, [_U64, _U64, _F, _SZ, _P]),
    "q38o_synth_abs_normal_f16": (None, [_U64, _U64, _F, _SZ, _P]),
    "q38o_synth_logits": (None, [_U64, _U64, _F, _P, _U32, _U32, _P]),
    "q38o_synth_uniform_w4": (None, [_U64, _U64, _INT, _INT, _SZ, _P]),
    "q38o_synth_uniform_i8": (None, [_U64, _U64, _INT, _INT, _SZ, _P]),
    "q38o_topk": (_INT, [_P, _U32, _U32, _U32, _INT, _P, _P]),
    "q38o_routes": (_U32, [_U32]),
    "q38o_max_tasks": (_U32, [_U32]),
    "q38o_plan_bytes": (_SZ, [_U32]),
    "q38o_build_plan": (_INT, [_P, _U32, _INT, _P]),
    "q38o_quantize_rows": (None, [_P, _U32, _U32, _P, _P]),
    "q38o_quantize_weights": (ctypes.c_int, [_P, ctypes.c_uint64, _U32, ctypes.c_int, _U32, _P, _P,
                                             ctypes.c_int]),
    "q38o_row_value": (_F, [ctypes.POINTER(Weights), _U32, _U32, _P]),
    "q38o_row_accumulators": (None, [ctypes.POINTER(Weights), _U32, _U32, _P, _P]),
    "q38o_gate_up": (None, [ctypes.POINTER(Weights), _U32, _U32, _P, _P, _P, _P, _P]),
    "q38o_down": (None, [ctypes.POINTER(Weights), _U32, _U32, _P, _P, _P, _P]),
    "q38o_combine": (None, [_P, _P, _P, _P, _U32, _U32, _P]),
    "q38o_combine_shared": (None, [_P, _P, _P, _U32, _U32, _P]),
    "q38o_moe_prefill": (_INT, [ctypes.POINTER(MoeIO)]),
    "q38o_moe_per_token": (_INT, [ctypes.POINTER(MoeIO)]),
    "q38o_num_threads": (_INT, []),
    "q38o_set_num_threads": (None, [_INT]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C oracle`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


# ---- scalar conversions ---------------------------------------------------

def expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().q38o_expf_array(_p(x), x.size, _p(out))
    return out


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().q38o_f32_to_bf16_array(_p(x), x.size, _p(out))
    return out


def bf16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().q38o_f32_to_f16_array(_p(x), x.size, _p(out))
    return out


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().q38o_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


# ---- synthetic data ------------------------------------------------------

def synth_normal_f32(seed, tag, n, sigma=1.0, absolute=False):
    out = np.empty(n, dtype=np.float32)
    lib().q38o_synth_normal_f32(seed, tag, sigma, int(absolute), n, _p(out))
    return out


def synth_normal_bf16(seed, tag, n, sigma=1.0):
    out = np.empty(n, dtype=np.uint16)
    lib().q38o_synth_normal_bf16(seed, tag, sigma, n, _p(out))
    return out


def synth_abs_normal_f16(seed, tag, n, sigma):
    out = np.empty(n, dtype=np.uint16)
    lib().q38o_synth_abs_normal_f16(seed, tag, sigma, n, _p(out))
    return out


def synth_logits(seed, tag, tokens, experts=EXPERTS, sigma=1.0, bias=None):
    out = np.empty((tokens, experts), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().q38o_synth_logits(seed, tag, sigma, _p(b), tokens, experts, _p(out))
    return out


def synth_uniform_w4(seed, tag, n, lo=-8, hi=7):
    out = np.empty(n // 2, dtype=np.uint8)
    lib().q38o_synth_uniform_w4(seed, tag, lo, hi, n, _p(out))
    return out


def synth_uniform_i8(seed, tag, n, lo=-127, hi=127):
    out = np.empty(n, dtype=np.int8)
    lib().q38o_synth_uniform_i8(seed, tag, lo, hi, n, _p(out))
    return out


# ---- weights ---------------------------------------------------------------

class HostWeights:
    """Canonical row-major weights in host memory."""

    def __init__(self, data, scales, bits, group, experts, rows, cols, scale_bf16=False):
        self.data = np.ascontiguousarray(data, dtype=np.uint8)
        self.scales = np.ascontiguousarray(scales, dtype=np.uint16)
        self.bits, self.group = bits, group
        self.experts, self.rows, self.cols = experts, rows, cols
        self.scale_bf16 = bool(scale_bf16)
        self.desc = Weights(_p(self.data), _p(self.scales), bits, group, experts, rows, cols,
                            int(self.scale_bf16))

    def unpacked(self, expert):
        """int8 [rows][cols] of one expert."""
        if self.bits == 8:
            per = self.rows * self.cols
            return self.data[expert * per:(expert + 1) * per].view(np.int8).reshape(
                self.rows, self.cols)
        per = self.rows * self.cols // 2
        b = self.data[expert * per:(expert + 1) * per]
        low = (b & 0x0F).astype(np.int16)
        high = (b >> 4).astype(np.int16)
        low = np.where(low >= 8, low - 16, low)
        high = np.where(high >= 8, high - 16, high)
        out = np.empty(self.rows * self.cols, dtype=np.int8)
        out[0::2] = low
        out[1::2] = high
        return out.reshape(self.rows, self.cols)

    def scale_matrix(self, expert):
        """fp32 scales [rows][groups] (groups = 1 for per-channel)."""
        g = self.cols // self.group if self.group else 1
        per = self.rows * g
        words = self.scales[expert * per:(expert + 1) * per]
        f = bf16_to_f32(words) if self.scale_bf16 else f16_to_f32(words)
        return f.reshape(self.rows, g)


def synth_weights(seed, tag, bits, group, experts, rows, cols, scale_sigma, scale_bf16=False):
    """Host twin of the product's synth_weights (same counter streams)."""
    n = experts * rows * cols
    data = synth_uniform_w4(seed, tag, n) if bits == 4 else \
        synth_uniform_i8(seed, tag, n).view(np.uint8)
    nscales = n // group if group else experts * rows
    if scale_bf16:
        scales = synth_normal_bf16(seed, tag + 1, nscales, scale_sigma) & np.uint16(0x7FFF)
    else:
        scales = synth_abs_normal_f16(seed, tag + 1, nscales, scale_sigma)
    return HostWeights(data, scales, bits, group, experts, rows, cols, scale_bf16)


# ---- routing ---------------------------------------------------------------

def topk(logits, top_k=TOPK, normalize=True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    tokens, experts = logits.shape
    ids = np.empty((tokens, top_k), dtype=np.int32)
    w = np.empty((tokens, top_k), dtype=np.float32)
    rc = lib().q38o_topk(_p(logits), tokens, experts, top_k, int(normalize), _p(ids), _p(w))
    if rc:
        raise ValueError("invalid top-k input")
    return ids, w


def plan_bytes(tokens):
    return lib().q38o_plan_bytes(tokens)


def max_tasks(tokens):
    return lib().q38o_max_tasks(tokens)


def build_plan(ids, tokens, hashes=False):
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    buf = np.zeros(plan_bytes(tokens), dtype=np.uint8)
    rc = lib().q38o_build_plan(_p(ids), tokens, int(hashes), _p(buf))
    if rc:
        raise ValueError("invalid plan input")
    return buf


def parse_plan(buf, tokens):
    """Splits a V1 plan image into named numpy views."""
    routes = tokens * TOPK
    mt = max_tasks(tokens)
    hdr = buf[:64]
    u32 = hdr[:32].view(np.uint32)
    u64 = hdr[32:64].view(np.uint64)
    off = 64
    counts = buf[off:off + 1024].view(np.uint16); off += 1024
    offsets = buf[off:off + 2052].view(np.uint32); off += 2052
    task_offsets = buf[off:off + 2052].view(np.uint32); off += 2052
    packed = buf[off:off + 4 * routes].view(np.uint32); off += 4 * routes
    inverse = buf[off:off + 4 * routes].view(np.uint32); off += 4 * routes
    tasks_raw = buf[off:off + 8 * mt]
    tasks = np.zeros(mt, dtype=[("packed_begin", "<u4"), ("expert", "<u2"),
                                ("valid_rows", "u1"), ("flags", "u1")])
    tasks_view = tasks_raw.view(tasks.dtype)
    return {
        "magic": int(u32[0]), "version": int(u32[1]), "tokens": int(u32[2]),
        "routes": int(u32[3]), "active_experts": int(u32[4]), "task_count": int(u32[5]),
        "status": int(u32[6]), "flags": int(u32[7]), "route_hash": int(u64[0]),
        "plan_hash": int(u64[1]), "reserved0": int(u64[2]), "reserved1": int(u64[3]),
        "counts": counts, "offsets": offsets, "task_offsets": task_offsets,
        "packed": packed, "inverse": inverse, "tasks": tasks_view,
    }


def quantize_rows(x_bf16, width):
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16).reshape(-1, width)
    rows = x.shape[0]
    q = np.empty((rows, width), dtype=np.int8)
    s = np.empty(rows, dtype=np.float32)
    lib().q38o_quantize_rows(_p(x), rows, width, _p(q), _p(s))
    return q, s


def quantize_weights(w_bf16, bits, group, scale_bf16=False):
    """Weight quantiser (quantize_groupwise restated): bf16 words [rows][cols]
    -> (data bytes [rows][cols*bits/8], fp16 (or bf16) scale words
    [rows][cols/group])."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    rows, cols = w.reshape(-1, w.shape[-1]).shape
    g = group or cols
    data = np.zeros((rows, cols * bits // 8), dtype=np.uint8)
    scales = np.empty((rows, cols // g), dtype=np.uint16)
    rc = lib().q38o_quantize_weights(_p(w), rows, cols, bits, group, _p(data), _p(scales),
                                     int(scale_bf16))
    if rc:
        raise ValueError(f"invalid quantiser shape rows={rows} cols={cols} bits={bits} group={group}")
    return data, scales


def row_accumulators(w, expert, row, x_i8):
    x = np.ascontiguousarray(x_i8, dtype=np.int8)
    groups = w.cols // w.group if w.group else 1
    out = np.empty(groups, dtype=np.int32)
    lib().q38o_row_accumulators(ctypes.byref(w.desc), expert, row, _p(x), _p(out))
    return out


def row_value(w, expert, row, x_i8):
    x = np.ascontiguousarray(x_i8, dtype=np.int8)
    return lib().q38o_row_value(ctypes.byref(w.desc), expert, row, _p(x))


# ---- whole step ------------------------------------------------------------

def moe(hidden_bf16, gate_up, down, logits=None, ids=None, weights=None, shared_output=None,
        shared_gate=None, grouped=True, intermediates=False):
    """Runs one MoE layer.  grouped=True goes through the V1 plan (T <= 512);
    grouped=False evaluates token by token (any T)."""
    hidden = np.ascontiguousarray(hidden_bf16, dtype=np.uint16)
    tokens, H = hidden.shape
    I = down.cols
    R = tokens * TOPK
    out = np.empty((tokens, H), dtype=np.uint16)
    if logits is not None:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        ids = np.empty((tokens, TOPK), dtype=np.int32)
        weights = np.empty((tokens, TOPK), dtype=np.float32)
    else:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        weights = np.ascontiguousarray(weights, dtype=np.float32)
    so = None if shared_output is None else np.ascontiguousarray(shared_output, dtype=np.uint16)
    sg = None if shared_gate is None else np.ascontiguousarray(shared_gate, dtype=np.uint16)
    io = MoeIO()
    io.tokens, io.hidden, io.inter = tokens, H, I
    io.hidden_states = _p(hidden)
    io.logits = _p(logits)
    io.ids, io.weights = _p(ids), _p(weights)
    io.gate_up = ctypes.pointer(gate_up.desc)
    io.down = ctypes.pointer(down.desc)
    io.shared_output, io.shared_gate = _p(so), _p(sg)
    io.output = _p(out)
    res = {"output": out, "ids": ids, "weights": weights}
    if intermediates and grouped:
        res["plan"] = np.zeros(plan_bytes(tokens), dtype=np.uint8)
        res["xq"] = np.empty((tokens, H), dtype=np.int8)
        res["xs"] = np.empty(tokens, dtype=np.float32)
        res["weighted_mid"] = np.empty((R, I), dtype=np.uint16)
        res["mid_q"] = np.empty((R, I), dtype=np.int8)
        res["mid_s"] = np.empty(R, dtype=np.float32)
        res["route_output"] = np.empty((R, H), dtype=np.float32)
        for name in ("plan", "xq", "xs", "weighted_mid", "mid_q", "mid_s", "route_output"):
            setattr(io, name, _p(res[name]))
    fn = lib().q38o_moe_prefill if grouped else lib().q38o_moe_per_token
    rc = fn(ctypes.byref(io))
    if rc:
        raise ValueError(f"oracle MoE step failed with status {rc}")
    return res


def combine_shared(routed_bf16, shared_bf16, gate_bf16):
    """Decode combine of bf16 rows (cuda/q38_moe.cu:337-350): [T][H] words,
    gate [T] words -> bf16(fma(shared, sigmoid(gate), routed))."""
    routed = np.ascontiguousarray(routed_bf16, dtype=np.uint16)
    shared = np.ascontiguousarray(shared_bf16, dtype=np.uint16)
    gate = np.ascontiguousarray(gate_bf16, dtype=np.uint16)
    tokens, hidden = routed.shape
    assert shared.shape == routed.shape and gate.shape == (tokens,)
    out = np.empty_like(routed)
    lib().q38o_combine_shared(_p(routed), _p(shared), _p(gate), tokens, hidden, _p(out))
    return out


def set_threads(n):
    lib().q38o_set_num_threads(n)


def num_threads():
    return lib().q38o_num_threads()


# ---- hyper-connection prepare/finish (floating point) ---------------------
# Restatement of cuda/q38_hyper.cu:52-114 and the prepare_hyper /
# finish_hyper sequences of cuda/cuda_backend.cu:1219-1252, in float32 with
# bf16 rounding between steps as the reference stores bf16 after every
# kernel.  exp is this library's expf (the reference calls CUDA's expf);
# a * b + c written in the reference is evaluated as one rounding (fma),
# emulated exactly in float64 since every product here is of bf16 values.
# Pins: tests/test_oracle_hyper.py (closed forms and a float64 evaluation).
HYPER_STREAMS = 4


def _bf(x):
    return bf16_to_f32(f32_to_bf16(np.asarray(x, dtype=np.float32)))


def _fma(a, b, c):
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) +
            np.asarray(c, np.float64)).astype(np.float32)


def hyper_repeat_embedding(embedding_bf16):
    """[T][H] -> [T][4][H] (q38_hyper.cu:52-61)."""
    e = np.asarray(embedding_bf16, np.uint16)
    return np.repeat(e[:, None, :], HYPER_STREAMS, axis=1)


def hyper_group_rmsnorm(hyper_bf16, weight_bf16):
    """[T][4][H], weight [4][H] -> bf16 [T][4][H] (q38_hyper.cu:63-85):
    x * rsqrt(mean(x^2) + 1e-6) * (1 + w) per (token, stream).  The sum of
    squares is evaluated in float64 (the reference's tree order is not part
    of its contract; parity is a tolerance)."""
    x = bf16_to_f32(np.asarray(hyper_bf16, np.uint16))
    w = bf16_to_f32(np.asarray(weight_bf16, np.uint16))
    hidden = x.shape[-1]
    mean = (np.square(x.astype(np.float64)).sum(axis=-1) / hidden).astype(np.float32)
    inverse = (np.float32(1.0) / np.sqrt(mean + np.float32(1e-6))).astype(np.float32)
    y = (x * inverse[..., None]).astype(np.float32) * (np.float32(1.0) + w)
    return f32_to_bf16(y.astype(np.float32))


def hyper_activation(x_bf16, divisor, scale, silu):
    """bf16(f(x / divisor) * scale), f = silu or sigmoid (q38_hyper.cu:87-97)."""
    v = (bf16_to_f32(np.asarray(x_bf16, np.uint16)) / np.float32(divisor)).astype(np.float32)
    sigmoid = (np.float32(1.0) / (np.float32(1.0) + expf(-v))).astype(np.float32)
    out = (v * sigmoid if silu else sigmoid).astype(np.float32) * np.float32(scale)
    return f32_to_bf16(out.astype(np.float32))


def hyper_mix(normalized_bf16, mix_bf16):
    """[T][4][H] x [T][4][H] -> bf16 [T][H]: the stream sum in stream order,
    then / 4 (q38_hyper.cu:99-114)."""
    n = bf16_to_f32(np.asarray(normalized_bf16, np.uint16))
    m = bf16_to_f32(np.asarray(mix_bf16, np.uint16))
    acc = np.zeros(n.shape[:1] + n.shape[2:], np.float32)
    for s in range(HYPER_STREAMS):
        acc = _fma(n[:, s], m[:, s], acc)
    return f32_to_bf16((acc / np.float32(HYPER_STREAMS)).astype(np.float32))


def hyper_inject(original_bf16, block_bf16, injection_bf16):
    """bf16(original[s][i] + block[i] * injection[s]) (q38_hyper.cu:116-135)."""
    o = bf16_to_f32(np.asarray(original_bf16, np.uint16))
    b = bf16_to_f32(np.asarray(block_bf16, np.uint16))
    g = bf16_to_f32(np.asarray(injection_bf16, np.uint16))
    return f32_to_bf16(_fma(b[:, None, :], g[:, :, None], o))


def hyper_gemv(x_bf16, w_bf16):
    """cuda_gemv_bf16 over a preserved bf16 matrix [N][K]: bf16 of the dot
    product (evaluated in float64; the reference's order is cuBLAS's)."""
    x = bf16_to_f32(np.asarray(x_bf16, np.uint16)).astype(np.float64)
    w = bf16_to_f32(np.asarray(w_bf16, np.uint16)).astype(np.float64)
    return f32_to_bf16((x @ w.T).astype(np.float32))


def hyper_prepare(hyper_bf16, norm_bf16, mix_down_bf16, mix_up_bf16, inject_bf16=None):
    """prepare_hyper (cuda_backend.cu:1219-1243): returns (mixed [T][H],
    injection [T][4] or None, and the intermediates for tests)."""
    t = hyper_bf16.shape[0]
    normalized = hyper_group_rmsnorm(hyper_bf16, norm_bf16)
    flat = normalized.reshape(t, -1)
    low = hyper_activation(hyper_gemv(flat, mix_down_bf16), HYPER_STREAMS, 1.0, True)
    mix = hyper_activation(hyper_gemv(low, mix_up_bf16), 1.0, 1.0, False)
    mixed = hyper_mix(normalized, mix.reshape(normalized.shape))
    injection = None
    if inject_bf16 is not None:
        injection = hyper_activation(hyper_gemv(flat, inject_bf16), HYPER_STREAMS, 2.0, False)
    return mixed, injection, {"normalized": normalized, "low": low, "mix": mix}
