#!/usr/bin/env python3
"""Writes tests/golden/golden.npz: expected outputs produced by the
reference's own CPU code (engine/src/gguf_loader.cpp, built into oracle/_ref
in this container) for seeded inputs.

Inputs are regenerated from their seeds by ``inputs(case)`` (numpy PCG64) and
pinned by a SHA-256 of their bytes, so only outputs are stored.  The GPU box
has no reference tree: its tests regenerate the inputs, check the hashes and
compare the HIP results with these reference outputs.

Cases
* matvec_k2048_n512: matvec_tensor on the exactly dequantized U4 matrix.
* router_*: select_router_topk on seeded logits (one case with ties).
* moe_layer_h{H}: run_qwen36_moe_ffn_layer on exactly dequantized U4 experts
  (F32 GGUF written by the shim): RMSNorm, router matvec + top-8, routed
  experts, shared expert, residual.  Stored: ffn_norm, router ids/weights,
  moe_out, shared_down, ffn_out, residual (all f32).
* schedule_t64: the oracle's BuildGroupedSchedule restatement (the reference's
  grouped runtime needs OpenCL and is not built here; this case is a
  regression vector, pinned independently by test_schedule_oracle.py).

Run:  python tests/golden/make_golden.py   (needs oracle/_ref)
"""

from __future__ import annotations

import hashlib
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

OUT = os.path.join(HERE, "golden.npz")
GROUP = 128


def rand_u4(rng, e, rows, k, group=GROUP):
    q = rng.integers(0, 256, (e, rows, k // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (e, rows, k // group))) + 1e-3).astype(np.float16)
    z = rng.integers(0, 256, (e, rows * (k // group) // 2), dtype=np.uint8)
    return oracle.U4Tensor(q, s.view(np.uint16), z, rows, k, group)


def dequant(t: oracle.U4Tensor):
    return np.stack([oracle.u4_dequant(t.qweight[e], t.scale[e], t.zp[e], t.rows, t.k, t.group)
                     for e in range(t.experts)])


MOE_CASES = {"moe_layer_h2048": (2048, 512, 16, 301), "moe_layer_h512": (512, 128, 16, 302)}


def inputs(case: str) -> dict:
    """Seeded inputs of a case (numpy arrays; f16 values as uint16 bits)."""
    if case == "matvec_k2048_n512":
        rng = np.random.default_rng(201)
        t = rand_u4(rng, 1, 512, 2048)
        x = rng.standard_normal(2048).astype(np.float16)
        return {"w": t, "x": x.view(np.uint16)}
    if case.startswith("router_"):
        rng = np.random.default_rng(202 if case == "router_plain" else 203)
        logits = rng.standard_normal((16, 256)).astype(np.float32)
        if case == "router_ties":
            logits[:, 100:140] = logits[:, 7:8]
            logits[3] = 0.0
        return {"logits": logits}
    if case in MOE_CASES:
        H, I, E, seed = MOE_CASES[case]
        rng = np.random.default_rng(seed)
        d = {"gate_up": rand_u4(rng, E, 2 * I, H), "down": rand_u4(rng, E, H, I),
             "shared_gate_up": rand_u4(rng, 1, 2 * I, H), "shared_down": rand_u4(rng, 1, H, I),
             "gate_vec": (rng.standard_normal(H) / np.sqrt(H)).astype(np.float16).view(np.uint16),
             "router": (rng.standard_normal((E, H)) * 0.05).astype(np.float32),
             "norm_w": (1 + 0.01 * rng.standard_normal(H)).astype(np.float32),
             "residual": rng.standard_normal(H).astype(np.float16).view(np.uint16)}
        return d
    if case == "schedule_t64":
        rng = np.random.default_rng(204)
        ids = np.stack([rng.permutation(16)[:8] for _ in range(64)]).astype(np.int32)
        w = rng.random((64, 8)).astype(np.float32)
        return {"ids": ids, "w": w}
    raise KeyError(case)


CASES = ["matvec_k2048_n512", "router_plain", "router_ties", "moe_layer_h2048",
         "moe_layer_h512", "schedule_t64"]


def digest(d: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(d):
        v = d[k]
        if isinstance(v, oracle.U4Tensor):
            for a in (v.qweight, v.scale, v.zp):
                h.update(np.ascontiguousarray(a).tobytes())
        else:
            h.update(np.ascontiguousarray(v).tobytes())
    return h.hexdigest()


def moe_weights(d) -> oracle.MoeWeights:
    return oracle.MoeWeights(d["gate_up"], d["down"], d["shared_gate_up"], d["shared_down"],
                             d["gate_vec"])


def main():
    ref = oracle.Ref()
    out = {}
    tmp = tempfile.mkdtemp()
    for case in CASES:
        d = inputs(case)
        out[f"{case}/sha256"] = np.frombuffer(digest(d).encode(), np.uint8)
        if case == "matvec_k2048_n512":
            x = oracle.f16_values(d["x"])
            out[f"{case}/y"] = ref.matvec_f32(dequant(d["w"])[0], x, tmp)
        elif case.startswith("router_"):
            ids, nws = [], []
            for row in d["logits"]:
                i, _, nw = ref.select_router_topk(row, 8)
                ids.append(i)
                nws.append(nw)
            out[f"{case}/ids"] = np.stack(ids)
            out[f"{case}/weights"] = np.stack(nws)
        elif case in MOE_CASES:
            r = ref.moe_ffn_layer_f32(tmp, dequant(d["gate_up"]), dequant(d["down"]),
                                      dequant(d["shared_gate_up"])[0],
                                      dequant(d["shared_down"])[0], d["router"],
                                      oracle.f16_values(d["gate_vec"]), d["norm_w"],
                                      oracle.f16_values(d["residual"]), 1e-6)
            for name in ("ffn_norm", "ids", "normalized_weights", "moe_out", "shared_down",
                         "ffn_out", "residual"):
                out[f"{case}/{name}"] = r[name]
        elif case == "schedule_t64":
            s = oracle.build_grouped_schedule(d["ids"], 16, d["w"])
            for name in ("offsets", "token_map", "inverse_map", "compact_weights"):
                out[f"{case}/{name}"] = s[name]
        print(f"{case}: done", flush=True)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
