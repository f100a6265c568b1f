"""ctypes binding of the oracle's C restatement (``oracle/c/mq_oracle.c``).

Test infrastructure: used to cross-check the numpy oracle and as the timed
CPU baseline.  Build with ``make -C oracle``.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libmq_oracle.so"
_LIB = None


def load():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, u32, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
        lib.mqo_decode_layer.argtypes = [vp, u32, u32, u32, u32, u32, u32, vp, vp] + [vp] * 18 + [vp, vp, i32]
        lib.mqo_decode_layer.restype = i32
        lib.mqo_qmv.argtypes = [vp, vp, vp, vp, vp, u32, u32, u32, u32, i32]
        lib.mqo_qmv.restype = i32
        lib.mqo_max_threads.restype = i32
        _LIB = lib
    return _LIB


def _p(a):
    return None if a is None else np.ascontiguousarray(a).ctypes.data


def decode_layer(x_bits, router_w, records, k, *, shared=None, shared_gate_w=None, threads=0):
    """Router + routed experts + optional shared expert; returns (out bf16 bits, inds)."""
    lib = load()
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    tokens, hidden = x_bits.shape
    inter = records.gate.out_width
    experts = records.gate.packed.shape[0]
    out = np.empty((tokens, hidden), dtype=np.uint16)
    inds = np.empty((tokens, k), dtype=np.uint32)
    keep = [x_bits, router_w, shared_gate_w]
    banks = []
    for bank in (records.gate, records.up, records.down):
        banks += [bank.packed, bank.scales, bank.biases]
    if shared is not None:
        for bank in shared:
            banks += [bank.packed, bank.scales, bank.biases]
    else:
        banks += [None] * 9
    banks = [None if b is None else np.ascontiguousarray(b) for b in banks]
    keep += banks
    rc = lib.mqo_decode_layer(_p(x_bits), tokens, hidden, inter, experts, k, records.gate.group_size,
                              _p(router_w), _p(shared_gate_w), *[_p(b) for b in banks],
                              _p(out), _p(inds), int(threads))
    if rc != 0:
        raise RuntimeError(f"mqo_decode_layer failed: {rc}")
    return out, inds


def qmv(x_bits, packed, scales, biases, group=32, threads=0):
    lib = load()
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, k = x_bits.shape
    n = packed.shape[0]
    y = np.empty((rows, n), dtype=np.float32)
    packed, scales, biases = (np.ascontiguousarray(a) for a in (packed, scales, biases))
    rc = lib.mqo_qmv(_p(x_bits), _p(packed), _p(scales), _p(biases), _p(y), rows, n, k, group, int(threads))
    if rc != 0:
        raise RuntimeError(f"mqo_qmv failed: {rc}")
    return y


def max_threads() -> int:
    return int(load().mqo_max_threads())
