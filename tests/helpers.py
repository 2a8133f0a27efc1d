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


# ---------------------------------------------------------------------------
# End-to-end parity of a layer stack: the measured floor
# ---------------------------------------------------------------------------
# Free-running through 40 layers, any two correct implementations drift
# apart: the f16 residual r_{L+1} = f16(r_L + ffn_L) turns every last-bit
# difference of ffn_L (a different f32 summation order is enough) into an
# f16 rounding flip, and the next layers carry and mix it.  How far they
# drift is measured on the CPU, on the test's own inputs, with the oracle
# chain run three ways: in the reference's order and precision (ref), in
# f64 (exact up to the stack's f16 h and r roundings), and under the
# device's precision model (oracle.MODEL_DECODE_PLAN / MODEL_PREFILL: its
# f16 SwiGLU, f16 weight operand, f16 contributions and summation orders).
# The floor towards the reference is max(d(ref, exact), d(model, ref)), and
# towards the exact chain max(d(ref, exact), d(model, exact)): the
# reference's own distance from exact arithmetic, and what the device's
# rounding points alone cost.  The device must land within FLOOR_MARGIN
# times each floor (or within 2e-3).  The margin covers the spread between
# single realizations of the drift: on the CPU, equally valid orders of the
# same arithmetic land 0.6x - 1.8x apart from each other.  Per layer,
# teacher-forced, the 2e-3 bar applies unchanged.
FLOOR_MARGIN = 2.0


def stack_chains(mws, norms, x_bits, ids, w, eps, model_flags, threads):
    """ref / exact / model chains of the oracle (f16 bits of the last r) and
    their distances: mws[L] oracle weights, ids/w [L][T][k] into mws[L]."""
    ch = {name: oracle.moe_stack_chain_model(mws, norms, x_bits, ids, w, eps=eps, flags=fl,
                                             threads=threads)
          for name, fl in (("ref", 0), ("exact", oracle.MODEL_F64), ("model", model_flags))}
    vals = {n: oracle.f16_values(v) for n, v in ch.items()}
    ch["ref_vs_exact"] = compare(vals["ref"], vals["exact"])
    ch["model_vs_ref"] = compare(vals["model"], vals["ref"])
    ch["model_vs_exact"] = compare(vals["model"], vals["exact"])
    return ch


def assert_end_to_end(got, chains, what, margin=FLOOR_MARGIN):
    """got: device result (f32 values of the f16 output) of the same chain."""
    ref = oracle.f16_values(chains["ref"])
    exact = oracle.f16_values(chains["exact"])
    vs_ref, vs_exact = compare(got, ref), compare(got, exact)
    out = {"vs_ref": vs_ref, "vs_exact": vs_exact}
    for key in ("ref_vs_exact", "model_vs_ref", "model_vs_exact"):
        out[key] = chains[key]
    log = os.environ.get("AIMA_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"what": what, "end_to_end": out, "margin": margin}) + "\n")
    assert np.all(np.isfinite(np.asarray(got, np.float64))), f"{what}: non-finite output"
    for m in ("max_rel", "rel_l2"):
        floor_ref = max(chains["ref_vs_exact"][m], chains["model_vs_ref"][m])
        floor_exact = max(chains["ref_vs_exact"][m], chains["model_vs_exact"][m])
        assert vs_ref[m] <= max(2e-3, margin * floor_ref), f"{what}: {m} vs ref {out}"
        assert vs_exact[m] <= max(2e-3, margin * floor_exact), f"{what}: {m} vs exact {out}"
    assert vs_ref["cosine"] >= 0.9999, f"{what}: {out}"
    return out
