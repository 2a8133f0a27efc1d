"""Test helpers: move device weights to the CPU oracle, compare results."""

from __future__ import annotations

import json
import os

import numpy as np

import oracle


def f16_bits(t) -> np.ndarray:
    """float16 torch tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().cpu().contiguous().numpy().view(np.uint16)


def f16_to_f32(t) -> np.ndarray:
    return oracle.f16_values(f16_bits(t))


def u4_to_oracle(w) -> oracle.U4Tensor:
    e = w.experts
    q = w.qweight.detach().cpu().contiguous().numpy().reshape(e, w.rows, w.k // 2)
    s = f16_bits(w.scale).reshape(e, w.rows, w.k // w.group)
    z = w.zp.detach().cpu().contiguous().numpy().reshape(e, -1)
    return oracle.U4Tensor(np.ascontiguousarray(q), np.ascontiguousarray(s),
                           np.ascontiguousarray(z), w.rows, w.k, w.group)


def moe_to_oracle(layer) -> oracle.MoeWeights:
    return oracle.MoeWeights(u4_to_oracle(layer.gate_up), u4_to_oracle(layer.down),
                             u4_to_oracle(layer.shared_gate_up), u4_to_oracle(layer.shared_down),
                             f16_bits(layer.shared_gate_vec))


def max_rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (the parity metric; 2e-3 bar)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / (den if den > 0 else 1.0))


def compare(got, ref) -> dict:
    """The reference's component acceptance statistics
    (benchmarks/intel-qwen36-35b-a3b-gguf-q4km/acceptance-matrix.json:367-374:
    cosine >= 0.999, rel-L2 <= 0.002) plus max relative error."""
    g = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    rl2 = float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-300))
    cos = float(np.dot(g, r) / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-300))
    return {"max_rel": max_rel_err(g, r), "rel_l2": rl2, "cosine": cos,
            "max_abs": float(np.max(np.abs(g - r))) if g.size else 0.0}


def assert_parity(got, ref, tol=2e-3, what=""):
    c = compare(got, ref)
    log = os.environ.get("AIMA_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"what": what, "tol": tol, **c}) + "\n")
    assert np.all(np.isfinite(np.asarray(got, np.float64))), f"{what}: non-finite output"
    assert c["max_rel"] <= tol, f"{what}: {c}"
    assert c["rel_l2"] <= tol, f"{what}: {c}"
    assert c["cosine"] >= 0.999, f"{what}: {c}"
    return c
