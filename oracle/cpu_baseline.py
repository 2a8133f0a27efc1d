"""ctypes binding of the CPU baseline (cpu_baseline.c) -- measurement
infrastructure for bench.py's cpu_baseline leg, never the product path.

``load(build_dir)`` compiles cpu_baseline.c for the CPU it runs on
(-O3 -march=native, OpenMP) into ``build_dir`` and loads it.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


class Baseline:
    def __init__(self, path: str):
        L = C.CDLL(path)
        L.cpb_set_threads.argtypes = [C.c_int]
        L.cpb_max_threads.restype = C.c_int
        vp, i64 = C.c_void_p, C.c_int64
        L.cpb_u4_matvec.argtypes = [vp, vp, vp, i64, i64, i64, vp, vp]
        L.cpb_moe_layer_token.argtypes = [vp, i64, vp, C.c_float, vp, vp]
        self.lib = L
        self.path = path

    def set_threads(self, n: int) -> None:
        if self.lib.cpb_set_threads(int(n)) != 0:
            raise ValueError("bad thread count")

    def matvec(self, q: np.ndarray, s: np.ndarray, z: np.ndarray, n: int, k: int, group: int,
               x: np.ndarray, y: np.ndarray) -> None:
        rc = self.lib.cpb_u4_matvec(q.ctypes.data, s.ctypes.data, z.ctypes.data, n, k, group,
                                    x.ctypes.data, y.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"cpb_u4_matvec failed ({rc})")

    def layer(self, experts, shared, gate_vec, norm, hidden, inter, group):
        """A layer record for k selected experts: experts = [(gu, dn)] where
        gu/dn are (q, s, z) numpy triples; shared = (gu, dn)."""
        return _Layer(experts, shared, gate_vec, norm, hidden, inter, group)

    def moe_token(self, layer: "_Layer", w: np.ndarray, eps: float, r: np.ndarray,
                  out: np.ndarray) -> None:
        rc = self.lib.cpb_moe_layer_token(C.addressof(layer.c), len(layer.experts),
                                          w.ctypes.data, eps, r.ctypes.data, out.ctypes.data)
        if rc != 0:
            raise RuntimeError(f"cpb_moe_layer_token failed ({rc})")


class _LayerC(C.Structure):
    _fields_ = [("gu_q", C.c_void_p), ("gu_s", C.c_void_p), ("gu_z", C.c_void_p),
                ("dn_q", C.c_void_p), ("dn_s", C.c_void_p), ("dn_z", C.c_void_p),
                ("shared_gate_vec", C.c_void_p), ("norm_weight", C.c_void_p),
                ("hidden", C.c_int64), ("inter", C.c_int64), ("group", C.c_int64)]


class _Layer:
    def __init__(self, experts, shared, gate_vec, norm, hidden, inter, group):
        self.experts = experts
        slots = list(experts) + [shared]
        self._keep = [slots, gate_vec, norm]

        def arr(i, j):
            return (C.c_void_p * len(slots))(*[sl[i][j].ctypes.data for sl in slots])

        self._ptrs = [arr(i, j) for i in range(2) for j in range(3)]
        self.c = _LayerC(*[C.cast(p, C.c_void_p) for p in self._ptrs],
                         gate_vec.ctypes.data, norm.ctypes.data, hidden, inter, group)


def build(build_dir: str) -> str:
    """Compile the baseline for this CPU into build_dir; returns the path."""
    out = os.path.join(build_dir, "libcpu_baseline.so")
    subprocess.run(["make", "-s", "-C", HERE, "baseline", f"BASELINE_OUT={out}"], check=True,
                   stdout=subprocess.DEVNULL)
    return out


def load(build_dir: str) -> Baseline:
    return Baseline(build(build_dir))
