"""ctypes wrapper of the C restatement (oracle/moe_ref.c) — test infrastructure.

Used by the CPU tests (as a second oracle) and by the ``cpu_baseline`` leg of
bench.py.  Activation tensors travel as uint16 bit patterns.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

from . import moe_oracle as O

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libmoe_ref.so"
DT = {"float16": 0, "bfloat16": 1}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        lib.moe_ref_threads.argtypes = [I]
        lib.moe_ref_threads.restype = I
        lib.moe_ref_route.argtypes = [P, I64, I64, P, P, P, I64, I, I, I, I, P, P, P]
        lib.moe_ref_route.restype = I
        lib.moe_ref_dispatch.argtypes = [P, I64, I64, P, P]
        lib.moe_ref_dispatch.restype = I
        lib.moe_ref_forward.argtypes = [P, I64, I64, I64, I64, I, I, I, I] + [P] * 12 + [P, P, P]
        lib.moe_ref_forward.restype = I
        _lib = lib
    return _lib


def threads(n: int = 0) -> int:
    """Set (n > 0) and return the OpenMP thread count."""
    return load().moe_ref_threads(n)


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def bits(a, act: str) -> np.ndarray:
    return np.ascontiguousarray(O.to_bits(a, act))


def route(x_bits, wr, sr_bits, br_bits, gs, k, norm, act):
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    T, H = x_bits.shape
    E = wr.shape[0]
    probs = np.zeros((T, E), np.uint16)
    ids = np.zeros((T, k), np.int32)
    scores = np.zeros((T, k), np.uint16)
    wr = np.ascontiguousarray(wr, np.uint32)
    sr_bits = np.ascontiguousarray(sr_bits, np.uint16)
    br_bits = np.ascontiguousarray(br_bits, np.uint16)
    rc = load().moe_ref_route(_p(x_bits), T, H, _p(wr), _p(sr_bits), _p(br_bits), E, gs, k,
                              int(norm), DT[act], _p(probs), _p(ids), _p(scores))
    assert rc == 0, rc
    return probs, ids, scores


def dispatch(ids, E):
    ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
    off = np.zeros(E + 1, np.int32)
    srt = np.zeros(max(ids.size, 1), np.int32)
    rc = load().moe_ref_dispatch(_p(ids), ids.size, E, _p(off), _p(srt))
    assert rc == 0, rc
    return off, srt[: ids.size]


class Layer:
    """One MoE layer's operands as contiguous arrays for the C restatement."""

    def __init__(self, weights: dict, act: str):
        self.act = act
        self.ops = []
        for name in ("router", "gate", "up", "down"):
            wq, s, b = weights[name]
            self.ops += [np.ascontiguousarray(wq, np.uint32), bits(s, act), bits(b, act)]
        self.E = weights["router"][0].shape[0]
        self.I = weights["gate"][0].shape[1]
        self.H = weights["down"][0].shape[1]

    @classmethod
    def from_arrays(cls, arrays: list, act: str):
        """Operands already in C layout: 12 arrays (u32 words, u16 scale/bias bits)."""
        self = cls.__new__(cls)
        self.act = act
        self.ops = [np.ascontiguousarray(a) for a in arrays]
        self.E = arrays[0].shape[0]
        self.I = arrays[3].shape[1]
        self.H = arrays[9].shape[1]
        return self


def forward(x_bits, layer: Layer, k: int, norm: bool, gs: int):
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    T, H = x_bits.shape
    y = np.zeros((T, H), np.uint16)
    ids = np.zeros((T, k), np.int32)
    scores = np.zeros((T, k), np.uint16)
    rc = load().moe_ref_forward(_p(x_bits), T, H, layer.I, layer.E, k, int(norm), gs,
                                DT[layer.act], *[_p(a) for a in layer.ops], _p(y), _p(ids),
                                _p(scores))
    assert rc == 0, rc
    return y, ids, scores
