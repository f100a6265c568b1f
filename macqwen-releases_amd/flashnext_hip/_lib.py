"""ctypes binding of ``libmqmoe.so`` (the gfx950 C ABI in ``include/mqmoe.h``).

The library is loaded from ``macqwen-releases_amd/lib/libmqmoe.so`` (built in
tree by ``macqwen-releases_amd/csrc/Makefile``).  There is no fallback: a
missing or unloadable library raises :class:`NativeUnavailable`.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("MQMOE_LIB", PACKAGE_ROOT / "lib" / "libmqmoe.so"))

MQ_OK = 0
MQ_ERR_INVALID = -1
MQ_ERR_DEVICE = -2
MQ_ERR_LAUNCH = -3
MQ_ERR_UNSUPPORTED = -4
MQ_F32 = 0
MQ_BF16 = 1
MQ_SLOT_BIT = 0x80000000
MQ_DECODE_RETURN_ALL = 1
MQ_DECODE_UNFUSED_UP = 2
MQ_DECODE_GENERIC_COMBINE = 4
MQ_SWIGLU_SCALAR = 1
MQ_SWIGLU_TABLE = 2
MQ_DEVFLAG_BAD_ROUTE = 1
MQ_DEVFLAG_BAD_ROW = 2

# Every symbol the header declares (checked by the CPU test suite).
EXPORTS = (
    "mq_available", "mq_init", "mq_last_error", "mq_check_device_errors", "mq_version",
    "mq_abi_struct_size", "mq_record_layout",
    "mq_q4_unpack", "mq_q4_dequant", "mq_q4_qmv", "mq_gather_qmv",
    "mq_swiglu", "mq_sigmoid", "mq_bf16_round_check", "mq_stream_probe", "mq_hop_probe", "mq_mfma_probe",
    "mq_route_topk", "mq_moe_decode", "mq_moe_layer", "mq_grouped_workspace_size",
    "mq_moe_grouped", "mq_moe_grouped_static", "mq_gather_qmm_workspace_size", "mq_gather_qmm",
    "mq_pool_refill_async", "mq_pool_refill_gather_async",
)


class NativeUnavailable(RuntimeError):
    """The HIP library is missing, failed to load, or no gfx950 device is usable."""


class NativeError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"mqmoe error {code}: {message}")
        self.code = code


class MqProjection(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("biases", ctypes.c_void_p),
        ("pool", ctypes.c_void_p),
        ("pool_header", ctypes.c_uint64),
        ("pool_stride", ctypes.c_uint64),
        ("off_weight", ctypes.c_uint64),
        ("off_scales", ctypes.c_uint64),
        ("off_biases", ctypes.c_uint64),
        ("stream_pack", ctypes.c_void_p),
        ("pool_slots", ctypes.c_uint32),
        ("stream_records", ctypes.c_uint32),
    ]


class MqMoeArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int),
        ("gate", MqProjection),
        ("up", MqProjection),
        ("down", MqProjection),
        ("routes", ctypes.c_void_p),
        ("scores", ctypes.c_void_p),
        ("score_dtype", ctypes.c_int),
        ("keeps", ctypes.c_void_p),
        ("shared_y", ctypes.c_void_p),
        ("shared", ctypes.c_void_p),
        ("shared_gate", ctypes.c_void_p),
        ("shared_expert", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("gate_out", ctypes.c_void_p),
        ("up_out", ctypes.c_void_p),
        ("act_out", ctypes.c_void_p),
        ("down_out", ctypes.c_void_p),
        ("tokens", ctypes.c_uint32),
        ("slots", ctypes.c_uint32),
        ("hidden", ctypes.c_uint32),
        ("inter", ctypes.c_uint32),
        ("expert_count", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
    ]


class MqRouteArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("gate_w", ctypes.c_void_p),
        ("logits_in", ctypes.c_void_p),
        ("shared_gate_w", ctypes.c_void_p),
        ("slot_table", ctypes.c_void_p),
        ("logits_out", ctypes.c_void_p),
        ("inds", ctypes.c_void_p),
        ("scores", ctypes.c_void_p),
        ("score_dtype", ctypes.c_int),
        ("scores_raw", ctypes.c_void_p),
        ("routes", ctypes.c_void_p),
        ("keeps", ctypes.c_void_p),
        ("shared_gate", ctypes.c_void_p),
        ("tokens", ctypes.c_uint32),
        ("hidden", ctypes.c_uint32),
        ("experts", ctypes.c_uint32),
        ("top_k", ctypes.c_uint32),
        ("threshold", ctypes.c_float),
        ("min_keep", ctypes.c_uint32),
        ("blend", ctypes.c_float),
    ]


class MqGroupedArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("gate", MqProjection),
        ("up", MqProjection),
        ("down", MqProjection),
        ("routes", ctypes.c_void_p),
        ("scores", ctypes.c_void_p),
        ("shared", ctypes.c_void_p),
        ("shared_expert", ctypes.c_void_p),  # host array of 3 MqProjection
        ("shared_gate", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("tokens", ctypes.c_uint32),
        ("slots", ctypes.c_uint32),
        ("hidden", ctypes.c_uint32),
        ("inter", ctypes.c_uint32),
        ("expert_count", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
    ]


class MqGatherArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_rows", ctypes.c_void_p),
        ("routes", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("w", MqProjection),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("x_count", ctypes.c_uint32),
        ("rows", ctypes.c_uint32),
        ("in_width", ctypes.c_uint32),
        ("out_width", ctypes.c_uint32),
        ("expert_count", ctypes.c_uint32),
        ("group_size", ctypes.c_uint32),
    ]


_LIB = None
_LOAD_ERROR: str | None = None


def _declare(lib) -> None:
    c = ctypes
    vp, u32, u64, i32 = c.c_void_p, c.c_uint32, c.c_uint64, c.c_int
    sig = {
        "mq_available": ([], i32),
        "mq_init": ([], i32),
        "mq_last_error": ([c.c_char_p, u32], i32),
        "mq_check_device_errors": ([vp, c.POINTER(c.c_uint32)], i32),
        "mq_version": ([], i32),
        "mq_abi_struct_size": ([i32], u64),
        "mq_record_layout": ([u32, u32, u32, c.POINTER(c.c_uint64), c.POINTER(c.c_uint64)], i32),
        "mq_q4_unpack": ([vp, vp, u64, vp], i32),
        "mq_q4_dequant": ([vp, vp, vp, vp, u32, u32, u32, vp], i32),
        "mq_q4_qmv": ([vp, i32, vp, vp, vp, vp, u32, u32, u32, u32, vp], i32),
        "mq_gather_qmv": ([vp, i32, i32, c.POINTER(MqProjection), vp, vp, u32, u32, u32, u32, u32, u32, vp], i32),
        "mq_swiglu": ([vp, vp, vp, u64, i32, u32, vp], i32),
        "mq_sigmoid": ([vp, vp, u64, i32, vp], i32),
        "mq_bf16_round_check": ([u64, u64, vp, vp], i32),
        "mq_route_topk": ([c.POINTER(MqRouteArgs), vp], i32),
        "mq_moe_decode": ([c.POINTER(MqMoeArgs), vp], i32),
        "mq_moe_layer": ([c.POINTER(MqRouteArgs), c.POINTER(MqMoeArgs), vp], i32),
        "mq_grouped_workspace_size": ([u32, u32, u32, u32, u32, i32], u64),
        "mq_moe_grouped": ([c.POINTER(MqGroupedArgs), vp], i32),
        "mq_moe_grouped_static": ([c.POINTER(MqGroupedArgs), vp], i32),
        "mq_gather_qmm_workspace_size": ([u32, u32], u64),
        "mq_gather_qmm": ([c.POINTER(MqGatherArgs), vp], i32),
        "mq_pool_refill_async": ([vp, u64, u64, u32, vp, vp, u32, u64, vp, vp], i32),
        "mq_pool_refill_gather_async": ([vp, u64, u64, u32, vp, vp, u32, u64, vp, vp], i32),
        "mq_stream_probe": ([vp, u32, u64, u32, vp, vp], i32),
        "mq_hop_probe": ([vp, u32, vp, u32, vp], i32),
        "mq_mfma_probe": ([u32, u32, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res


def load(path: str | os.PathLike | None = None):
    """Load (once) and return the ctypes library; raise NativeUnavailable on failure."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None and path is None:
        return _LIB
    target = Path(path) if path is not None else LIB_PATH
    if not target.exists():
        _LOAD_ERROR = f"{target} not found (build it with macqwen-releases_amd/csrc/Makefile)"
        raise NativeUnavailable(_LOAD_ERROR)
    try:
        lib = ctypes.CDLL(str(target), mode=ctypes.RTLD_GLOBAL)
    except OSError as exc:
        _LOAD_ERROR = f"cannot load {target}: {exc}"
        raise NativeUnavailable(_LOAD_ERROR) from exc
    _declare(lib)
    for which, struct in enumerate((MqProjection, MqMoeArgs, MqRouteArgs, MqGroupedArgs, MqGatherArgs)):
        native = int(lib.mq_abi_struct_size(which))
        if native != ctypes.sizeof(struct):
            _LOAD_ERROR = (f"{target} is out of date: sizeof({struct.__name__}) is {native} in the "
                           f"library but {ctypes.sizeof(struct)} in the binding; rebuild it")
            raise NativeUnavailable(_LOAD_ERROR)
    if path is None:
        _LIB = lib
        init_device()
    return lib


def init_device() -> None:
    """Resolve the library's per-device state (its device error flags) on the
    current device; a no-op when no gfx950 device is visible."""
    lib = _LIB
    if lib is not None and lib.mq_available() == 1:
        check(lib.mq_init(), lib)


def last_error(lib=None) -> str:
    lib = lib or load()
    buf = ctypes.create_string_buffer(1024)
    lib.mq_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int, lib=None) -> None:
    """Raise the Python exception matching a negative status code."""
    if rc >= 0:
        return
    message = last_error(lib)
    if rc == MQ_ERR_INVALID:
        raise ValueError(message)
    if rc == MQ_ERR_DEVICE:
        raise NativeUnavailable(message)
    raise NativeError(rc, message)


def check_device_errors(stream=None) -> int:
    """Synchronise ``stream`` and raise if a kernel flagged a bad route word."""
    lib = load()
    flags = ctypes.c_uint32(0)
    check(lib.mq_check_device_errors(stream, ctypes.byref(flags)), lib)
    return int(flags.value)


def record_layout(hidden: int, inter: int, group_size: int = 32):
    """Offsets of the nine record parts and the record stride, from the library."""
    lib = load()
    offs = (ctypes.c_uint64 * 9)()
    stride = ctypes.c_uint64()
    check(lib.mq_record_layout(hidden, inter, group_size, offs, ctypes.byref(stride)), lib)
    return list(offs), int(stride.value)
