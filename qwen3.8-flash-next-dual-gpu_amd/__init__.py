"""ctypes binding of libq38m.so, the MI355X MoE data plane (C ABI in
include/q38m.h).

The product is the C ABI; this module is the plumbing the tests and
bench.py use to call it with torch-allocated device memory.  Function
names and argument order follow the C ABI, which mirrors the reference's
operator surface (include/q38/cuda_moe_prefill.h:98-133,
include/q38/cuda_moe.h:17-39, include/q38/cuda_kernels.h:83-91).  Errors
raise InvalidArgument (the reference's std::invalid_argument) or
DeviceError (std::runtime_error), like the reference's host wrappers.

Loading never falls back to anything: if libq38m.so is missing this
module raises at the first call.
"""
import ctypes
import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
# Q38M_LIB_PATH names another build of the same library (the host-sanitized
# one of the ABI tests); there is no fallback either way.
LIB_PATH = os.environ.get("Q38M_LIB_PATH") or os.path.join(PACKAGE_DIR, "libq38m.so")

OK = 0
ERR_INVALID_ARGUMENT = 1
ERR_DEVICE = 2
ERR_UNSUPPORTED = 3

ROUTE_EXPERTS = 512
ROUTE_TOPK = 10
MMQ_M = 16
MODE_GROUPED_MMQ = 1
MODE_GROUPED_MMQ_SAFE = 2
MODE_LEGACY_ATOMIC_DIAGNOSTIC = 3
SLAB_MAX_TOKENS = 512
NOALLOC_MAX_TOKENS = 64
HIDDEN = 2048
INTERMEDIATE = 512
PLAN_MAGIC_V1 = 0x52383351
PLAN_FLAG_HASHES = 1

FORMAT_W4_SYM = 2
FORMAT_W8_SYM = 3
SCALE_F16 = 1
SCALE_BF16 = 2
LAYOUT_ROW_MAJOR = 0
LAYOUT_MFMA16 = 2
LAYOUT_MFMA16_PAIRED = 3

SYNTH_NORMAL_F32 = 1
SYNTH_NORMAL_BF16 = 2
SYNTH_ABS_NORMAL_F16 = 3
SYNTH_UNIFORM_W4 = 4
SYNTH_UNIFORM_I8 = 5


class Q38MError(RuntimeError):
    pass


class InvalidArgument(Q38MError, ValueError):
    pass


class DeviceError(Q38MError):
    pass


class Unsupported(Q38MError):
    pass


class Task(ctypes.Structure):
    _fields_ = [("packed_begin", ctypes.c_uint32), ("expert", ctypes.c_uint16),
                ("valid_rows", ctypes.c_uint8), ("flags", ctypes.c_uint8)]


class PlanHeader(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_uint32), ("version", ctypes.c_uint32),
                ("tokens", ctypes.c_uint32), ("routes", ctypes.c_uint32),
                ("active_experts", ctypes.c_uint32), ("task_count", ctypes.c_uint32),
                ("status", ctypes.c_uint32), ("flags", ctypes.c_uint32),
                ("route_hash", ctypes.c_uint64), ("plan_hash", ctypes.c_uint64),
                ("reserved0", ctypes.c_uint64), ("reserved1", ctypes.c_uint64)]


class RoutePlan(ctypes.Structure):
    _fields_ = [("header", ctypes.c_void_p), ("expert_counts", ctypes.c_void_p),
                ("expert_offsets", ctypes.c_void_p), ("expert_task_offsets", ctypes.c_void_p),
                ("packed_assignment", ctypes.c_void_p), ("assignment_to_packed", ctypes.c_void_p),
                ("tasks", ctypes.c_void_p)]


class ExpertWeights(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("format", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
                ("scale_dtype", ctypes.c_uint32), ("layout", ctypes.c_uint32),
                ("experts", ctypes.c_uint32), ("rows", ctypes.c_uint32),
                ("columns", ctypes.c_uint32)]


class PrefillWorkspace(ctypes.Structure):
    _fields_ = [("max_tokens", ctypes.c_uint32), ("plan", RoutePlan),
                ("expert_ids", ctypes.c_void_p), ("expert_weights", ctypes.c_void_p),
                ("xq", ctypes.c_void_p), ("xs", ctypes.c_void_p),
                ("weighted_mid", ctypes.c_void_p), ("mid_q", ctypes.c_void_p),
                ("mid_s", ctypes.c_void_p), ("route_output", ctypes.c_void_p),
                ("task_flags", ctypes.c_void_p)]


class WideWorkspace(ctypes.Structure):
    _fields_ = [("step", PrefillWorkspace), ("plan_scratch", ctypes.c_void_p)]


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I32 = ctypes.c_int32
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); every entry point of include/q38m.h
SIGNATURES = {
    "q38m_moe_prefill_routes_v1": (_U32, [_U32]),
    "q38m_moe_prefill_max_tasks_v1": (_U32, [_U32]),
    "q38m_moe_route_plan_bytes_v1": (_SZ, [_U32]),
    "q38m_moe_route_plan_storage_v1": (_INT, [_P, _SZ, _U32, ctypes.POINTER(RoutePlan)]),
    "q38m_topk_router_f32": (_INT, [_P, _P, _P, _U32, _U32, _U32, _INT, _P, _INT]),
    "q38m_topk_router_bf16": (_INT, [_P, _P, _P, _U32, _U32, _U32, _INT, _P, _INT]),
    "q38m_moe_route_quantize_v1": (_INT, [_P, _P, _U32, _P, _P, _P, _P, _P, _INT]),
    "q38m_moe_build_route_plan_v1": (_INT, [_P, _U32, ctypes.POINTER(RoutePlan), _U32, _P, _INT]),
    "q38m_moe_pack_hidden_v1": (_INT, [_P, _P, _U32, _U32, _P, _P, _INT]),
    "q38m_quantize_rows_i8": (_INT, [_P, _U32, _U32, _P, _P, _P, _INT]),
    "q38m_residual_add_bf16": (_INT, [_P, _P, _P, _U64, _P, _INT]),
    "q38m_moe_grouped_gate_up_v1": (_INT, [ctypes.POINTER(ExpertWeights), _P, _P, _P, _P, _P,
                                           _U32, _P, _U32, _P, _INT]),
    "q38m_moe_grouped_down_v1": (_INT, [ctypes.POINTER(ExpertWeights), _P, _P, _P, _U32, _P,
                                        _U32, _P, _INT]),
    "q38m_moe_grouped_gate_up_down_v1": (_INT, [ctypes.POINTER(ExpertWeights),
                                                ctypes.POINTER(ExpertWeights), _P, _P, _P, _P, _P,
                                                _U32, _P, _P, _P, _P, _P, _P, _U32, _P, _INT]),
    "q38m_moe_clear_task_flags_v1": (_INT, [_P, _U32, _P, _INT]),
    "q38m_moe_reduce_top10_and_combine_shared_v1": (_INT, [_P, _P, _P, _P, _U32, _P, _P, _INT]),
    "q38m_moe_combine_shared_bf16": (_INT, [_P, _P, _P, _P, _U32, _P, _INT]),
    "q38m_moe_prefill_workspace_bytes": (_SZ, [_U32]),
    "q38m_moe_prefill_workspace_bind": (_INT, [_P, _SZ, _U32, ctypes.POINTER(PrefillWorkspace)]),
    "q38m_moe_prefill_v1": (_INT, [ctypes.POINTER(ExpertWeights), ctypes.POINTER(ExpertWeights),
                                   _P, _P, _U32, ctypes.POINTER(PrefillWorkspace), _P, _P, _P,
                                   _P, _INT]),
    "q38m_moe_prefill_noalloc_scratch_bytes": (_SZ, []),
    "q38m_moe_prefill_noalloc_v1": (_INT, [ctypes.POINTER(ExpertWeights),
                                           ctypes.POINTER(ExpertWeights), _P, _P, _U32, _P, _P,
                                           _P, _P, _INT]),
    "q38m_moe_wide_max_tasks": (_U32, [_U32]),
    "q38m_moe_wide_plan_bytes": (_SZ, [_U32]),
    "q38m_moe_wide_plan_scratch_bytes": (_SZ, [_U32]),
    "q38m_moe_wide_plan_storage": (_INT, [_P, _SZ, _U32, ctypes.POINTER(RoutePlan)]),
    "q38m_moe_build_route_plan_wide": (_INT, [_P, _U32, ctypes.POINTER(RoutePlan), _P, _P, _INT]),
    "q38m_moe_wide_workspace_bytes": (_SZ, [_U32]),
    "q38m_moe_wide_workspace_bind": (_INT, [_P, _SZ, _U32, ctypes.POINTER(WideWorkspace)]),
    "q38m_moe_prefill_wide_v1": (_INT, [ctypes.POINTER(ExpertWeights),
                                        ctypes.POINTER(ExpertWeights), _P, _P, _U32,
                                        ctypes.POINTER(WideWorkspace), _P, _P, _P, _P, _INT]),
    "q38m_moe_decode_scratch_bytes": (_SZ, []),
    "q38m_moe_routed_decode_v1": (_INT, [ctypes.POINTER(ExpertWeights),
                                         ctypes.POINTER(ExpertWeights), _P, _P, _P, _U32, _P, _P,
                                         _P, _INT]),
    "q38m_moe_decode_v1": (_INT, [ctypes.POINTER(ExpertWeights), ctypes.POINTER(ExpertWeights),
                                  _P, _P, _U32, _P, _P, _P, _P, _P, _P, _INT]),
    "q38m_moe_decode_block_scratch_bytes": (_SZ, []),
    "q38m_moe_decode_block_v1": (_INT, [ctypes.POINTER(ExpertWeights),
                                        ctypes.POINTER(ExpertWeights), _P, _P, _P, _P, _P, _P,
                                        _U32, _U32, _P, _P, _P, _P, _INT]),
    "q38m_expert_weights_bytes": (_SZ, [ctypes.POINTER(ExpertWeights), ctypes.POINTER(_SZ)]),
    "q38m_repack_expert_weights": (_INT, [ctypes.POINTER(ExpertWeights),
                                          ctypes.POINTER(ExpertWeights), _P, _INT]),
    "q38m_quantize_expert_weights": (_INT, [_P, ctypes.POINTER(ExpertWeights), _P, _INT]),
    "q38m_dense_gemm_bf16": (_INT, [_P, _P, _U32, _U32, _U32, _P, _P, _P, _INT]),
    "q38m_moe_router_v1": (_INT, [_P, _P, _U32, _U32, _P, _P, _INT]),
    "q38m_moe_router_topk_workspace_bytes": (_SZ, [_U32]),
    "q38m_moe_router_topk_v1": (_INT, [_P, _P, _U32, _U32, _U32, _P, _SZ, _P, _P, _P, _INT]),
    "q38m_moe_shared_expert_scratch_bytes": (_SZ, [_U32, _U32]),
    "q38m_moe_shared_expert_v1": (_INT, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, _P, _P, _P,
                                         _INT]),
    "q38m_hyper_repeat_embedding_bf16": (_INT, [_P, _P, _U32, _U32, _P, _INT]),
    "q38m_hyper_group_rmsnorm_bf16": (_INT, [_P, _P, _P, _U32, _U32, _P, _INT]),
    "q38m_hyper_silu_scaled_bf16": (_INT, [_P, _P, _U32, _U32, _F, _P, _INT]),
    "q38m_hyper_sigmoid_bf16": (_INT, [_P, _P, _U32, _U32, _F, _F, _P, _INT]),
    "q38m_hyper_mix_bf16": (_INT, [_P, _P, _P, _U32, _U32, _P, _INT]),
    "q38m_hyper_inject_bf16": (_INT, [_P, _P, _P, _P, _U32, _U32, _P, _INT]),
    "q38m_hyper_prepare_scratch_bytes": (_SZ, [_U32, _U32, _U32]),
    "q38m_hyper_prepare_v1": (_INT, [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, _P, _P, _P, _INT]),
    "q38m_synth_fill": (_INT, [_U32, _U64, _U64, _U64, _F, _I32, _I32, _P, _U32, _P, _P, _INT]),
    "q38m_moe_compiled": (_INT, []),
    "q38m_last_error": (ctypes.c_char_p, []),
}

# The test suite's self checks (include/q38m_selftest.h), in their own
# library: libq38m.so exports none of them.
SELFTEST_LIB_PATH = os.path.join(PACKAGE_DIR, "libq38m_selftest.so")
SELFTEST_SIGNATURES = {
    "q38m_debug_expf": (_INT, [_P, _U32, _P, _P, _INT]),
    "q38m_debug_bf16_sweep": (_INT, [_P, _P, _INT]),
    "q38m_debug_mfma_16x16x32_i8": (_INT, [_P, _P, _P, _P, _INT]),
    "q38m_debug_mfma_32x32x32_i8": (_INT, [_P, _P, _P, _P, _INT]),
}

# The timing build (include/q38m_phase.h): the product entry points plus
# the phase log.
TIMED_LIB_PATH = os.path.join(PACKAGE_DIR, "libq38m_timed.so")
PHASE_SIGNATURES = {
    "q38m_phase_log_v1": (_INT, [_P, _U32, _INT]),
    "q38m_phase_calls_v1": (_U32, []),
}


# The checked build (include/q38m_checked.h): the product entry points with
# the device index checks compiled in, plus their status word.
CHECKED_LIB_PATH = os.path.join(PACKAGE_DIR, "libq38m_checked.so")
CHECKED_SIGNATURES = {"q38m_checked_status_v1": (_INT, [_P, _INT, _INT])}
CHECK_EXPERT = 1
CHECK_TASK_ROWS = 2
CHECK_ROUTE = 4
CHECK_TOKEN = 8


class PhaseRecord(ctypes.Structure):
    _fields_ = [("stamp", ctypes.c_uint64 * 16), ("wave_stamp", ctypes.c_uint64 * 16),
                ("kernel", ctypes.c_uint32),
                ("block", ctypes.c_uint32), ("call", ctypes.c_uint32), ("valid", ctypes.c_uint32)]


_lib = None
_selftest_lib = None
_timed_lib = None
_checked_lib = None


def _open(path, signatures):
    if not os.path.exists(path):
        raise Q38MError(f"{path} is not built; run __graft_entry__.build()")
    handle = ctypes.CDLL(path)
    for name, (restype, argtypes) in signatures.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def lib():
    """Loads libq38m.so (raises OSError/Q38MError when it is not built)."""
    global _lib
    if _lib is None:
        _lib = _open(LIB_PATH, SIGNATURES)
    return _lib


def selftest_lib():
    """Loads libq38m_selftest.so, the test suite's self-check kernels."""
    global _selftest_lib
    if _selftest_lib is None:
        _selftest_lib = _open(SELFTEST_LIB_PATH, SELFTEST_SIGNATURES)
    return _selftest_lib


def timed_lib():
    """Loads libq38m_timed.so, the timing build (its own copy of every entry
    point, with phase timestamps in the decode kernels)."""
    global _timed_lib
    if _timed_lib is None:
        _timed_lib = _open(TIMED_LIB_PATH, {**SIGNATURES, **PHASE_SIGNATURES})
    return _timed_lib


def _check(rc):
    if rc == OK:
        return
    message = lib().q38m_last_error().decode(errors="replace")
    if rc == ERR_INVALID_ARGUMENT:
        raise InvalidArgument(message)
    if rc == ERR_UNSUPPORTED:
        raise Unsupported(message)
    raise DeviceError(message)


def checked_lib():
    """Loads libq38m_checked.so, the checked build (its own copy of every
    entry point, with the device index checks compiled in)."""
    global _checked_lib
    if _checked_lib is None:
        _checked_lib = _open(CHECKED_LIB_PATH, {**SIGNATURES, **CHECKED_SIGNATURES})
    return _checked_lib


def call(name, *args):
    """Calls an int-returning entry point and raises on a non-OK status."""
    _check(getattr(lib(), name)(*args))


def call_checked(name, *args):
    """Calls an entry point of the checked build and raises on a non-OK status."""
    handle = checked_lib()
    rc = getattr(handle, name)(*args)
    if rc != OK:
        message = handle.q38m_last_error().decode(errors="replace")
        raise (InvalidArgument if rc == ERR_INVALID_ARGUMENT else DeviceError)(message)


def checked_status(reset=True, device=0):
    """The checked build's status bits (CHECK_*) since the last reset."""
    word = ctypes.c_uint32(0)
    call_checked("q38m_checked_status_v1", ctypes.byref(word), 1 if reset else 0, device)
    return word.value


def call_selftest(name, *args):
    """Calls a self-check entry point of libq38m_selftest.so."""
    rc = getattr(selftest_lib(), name)(*args)
    if rc == ERR_INVALID_ARGUMENT:
        raise InvalidArgument(f"{name}: invalid argument")
    if rc != OK:
        raise DeviceError(f"{name}: status {rc}")


def call_timed(name, *args):
    """Calls an entry point of the timing build and raises on a non-OK status."""
    handle = timed_lib()
    rc = getattr(handle, name)(*args)
    if rc != OK:
        message = handle.q38m_last_error().decode(errors="replace")
        raise (InvalidArgument if rc == ERR_INVALID_ARGUMENT else DeviceError)(message)


# ---------------------------------------------------------------------------
# torch conveniences (device memory and streams are plumbing only)
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def ptr(tensor):
    return None if tensor is None else tensor.data_ptr()


def stream_handle(stream=None):
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def device_index(tensor):
    return tensor.device.index if tensor.device.index is not None else 0


class DeviceWeights:
    """Expert weights resident in device memory plus their descriptor."""

    def __init__(self, data, scales, fmt, group, layout, experts, rows, columns,
                 scale_dtype=SCALE_F16):
        self.data = data
        self.scales = scales
        self.desc = ExpertWeights(ptr(data), ptr(scales), fmt, group, scale_dtype, layout,
                                  experts, rows, columns)

    @property
    def nbytes(self):
        return self.data.numel() * self.data.element_size() + \
            self.scales.numel() * self.scales.element_size()


def weights_bytes(fmt, group, experts, rows, columns):
    desc = ExpertWeights(None, None, fmt, group, SCALE_F16, LAYOUT_ROW_MAJOR, experts, rows,
                         columns)
    scale_bytes = _SZ(0)
    data_bytes = lib().q38m_expert_weights_bytes(ctypes.byref(desc), ctypes.byref(scale_bytes))
    return data_bytes, scale_bytes.value


def synth_fill(kind, seed, tag, count, out, sigma=1.0, lo=0, hi=0, bias=None, stream=None):
    call("q38m_synth_fill", kind, seed, tag, count, sigma, lo, hi, ptr(bias),
         0 if bias is None else bias.numel(), ptr(out), stream_handle(stream), device_index(out))


def synth_weights(seed, tag, fmt, group, experts, rows, columns, scale_sigma, device="cuda",
                  stream=None, scale_dtype=SCALE_F16):
    """Row-major synthetic weights: int4 U[-8,7] / int8 U[-127,127] and
    |N(0, scale_sigma)| scales (counter streams tag and tag+1): fp16, or
    bf16 (the bf16 normal stream with its sign bit cleared)."""
    torch = _torch()
    data_bytes, scale_bytes = weights_bytes(fmt, group, experts, rows, columns)
    data = torch.empty(data_bytes, dtype=torch.uint8, device=device)
    scales = torch.empty(scale_bytes // 2, dtype=torch.int16, device=device)
    elements = experts * rows * columns
    if fmt == FORMAT_W4_SYM:
        synth_fill(SYNTH_UNIFORM_W4, seed, tag, elements, data, lo=-8, hi=7, stream=stream)
    else:
        synth_fill(SYNTH_UNIFORM_I8, seed, tag, elements, data, lo=-127, hi=127, stream=stream)
    if scale_dtype == SCALE_BF16:
        synth_fill(SYNTH_NORMAL_BF16, seed, tag + 1, scales.numel(), scales, sigma=scale_sigma,
                   stream=stream)
        scales.bitwise_and_(0x7FFF)
    else:
        synth_fill(SYNTH_ABS_NORMAL_F16, seed, tag + 1, scales.numel(), scales,
                   sigma=scale_sigma, stream=stream)
    return DeviceWeights(data, scales, fmt, group, LAYOUT_ROW_MAJOR, experts, rows, columns,
                         scale_dtype)


def repack(weights, paired=False, stream=None):
    """Row-major -> MFMA16 device layout (a new allocation).  paired=True
    gives the gate/up layout (tile t next to tile t + rows/32)."""
    torch = _torch()
    data = torch.empty_like(weights.data)
    scales = torch.empty_like(weights.scales)
    d = weights.desc
    layout = LAYOUT_MFMA16_PAIRED if paired else LAYOUT_MFMA16
    out = DeviceWeights(data, scales, d.format, d.group_size, layout, d.experts, d.rows,
                        d.columns, d.scale_dtype)
    call("q38m_repack_expert_weights", ctypes.byref(weights.desc), ctypes.byref(out.desc),
         stream_handle(stream), device_index(data))
    return out


class PrefillWorkspace_:
    """One device allocation bound as the whole-step workspace."""

    def __init__(self, max_tokens, device="cuda"):
        torch = _torch()
        nbytes = lib().q38m_moe_prefill_workspace_bytes(max_tokens)
        if nbytes == 0:
            raise InvalidArgument(f"invalid workspace token count {max_tokens}")
        self.buffer = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
        base = self.buffer.data_ptr()
        aligned = (base + 255) // 256 * 256
        self.ws = PrefillWorkspace()
        call("q38m_moe_prefill_workspace_bind", aligned, nbytes, max_tokens,
             ctypes.byref(self.ws))
        self.max_tokens = max_tokens


class WideWorkspace_:
    """One device allocation bound as the chunk (up to 32,768 tokens) workspace."""

    def __init__(self, max_tokens, device="cuda"):
        torch = _torch()
        nbytes = lib().q38m_moe_wide_workspace_bytes(max_tokens)
        if nbytes == 0:
            raise InvalidArgument(f"invalid chunk workspace token count {max_tokens}")
        self.buffer = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
        base = self.buffer.data_ptr()
        aligned = (base + 255) // 256 * 256
        self.wide = WideWorkspace()
        call("q38m_moe_wide_workspace_bind", aligned, nbytes, max_tokens,
             ctypes.byref(self.wide))
        self.ws = self.wide.step
        self.max_tokens = max_tokens


def route_plan_bytes(tokens):
    return lib().q38m_moe_route_plan_bytes_v1(tokens)


def max_tasks(tokens):
    return lib().q38m_moe_prefill_max_tasks_v1(tokens)


def bind_plan(allocation_ptr, nbytes, tokens):
    plan = RoutePlan()
    call("q38m_moe_route_plan_storage_v1", allocation_ptr, nbytes, tokens, ctypes.byref(plan))
    return plan
