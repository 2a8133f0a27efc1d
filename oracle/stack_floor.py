"""CPU measurement of the end-to-end parity floor of a 40-layer MoE FFN stack
(test infrastructure: runs the oracle only, never the product library).

Runs the oracle chain h = f16(rmsnorm(r)), r = f16(r + ffn(h)) through
``--layers`` layers under several precision models (see
``orc_moe_ffn_tokens_model`` in u4moe_oracle.c) and prints how far each lands
from the reference's own f32 order and from f64 arithmetic.  Layers are
synthesized with the benchmark distributions (hidden 2048, inter 512, the 8
routed experts a token selects + the shared expert, top-8 weights from
N(0, 1) logits over 256 experts).

    python oracle/stack_floor.py --layers 40 --tokens 8 --seed 1
"""

from __future__ import annotations

import argparse
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402

MODELS = [("reference order", 0), ("f64 (exact)", oracle.MODEL_F64),
          ("chunked dot products", oracle.MODEL_CHUNKED),
          ("SwiGLU rounded to f16", oracle.MODEL_ACT_F16),
          ("decode plan", oracle.MODEL_DECODE_PLAN), ("grouped prefill", oracle.MODEL_PREFILL)]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--threads", type=int, default=min(16, os.cpu_count() or 1))
    args = ap.parse_args()
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    from tests.helpers import compare, moe_to_oracle

    T, k = args.tokens, 8
    mws, norms, ids, ws = [], [], [], []
    for l in range(args.layers):
        lw = pkg.synth.moe_layer(hidden=2048, inter=512, experts=k,
                                 seed=args.seed * 1000 + l, device="cpu")
        mws.append(moe_to_oracle(lw))
        norms.append(lw.norm_weight.numpy())
        g = torch.Generator().manual_seed(args.seed * 1000 + 500 + l)
        _, w8 = oracle.router_topk_tokens(torch.randn((T, 256), generator=g).numpy(), k)
        ids.append(np.tile(np.arange(k, dtype=np.int32), (T, 1)))  # the 8 synthesized experts
        ws.append(w8.astype(np.float32))
    x = torch.randn((T, 2048), generator=torch.Generator().manual_seed(args.seed + 77))
    xb = x.to(torch.float16).numpy().view(np.uint16)
    out = {}
    for name, flags in MODELS:
        t0 = time.time()
        out[name] = oracle.f16_values(oracle.moe_stack_chain_model(
            mws, norms, xb, ids, ws, flags=flags, threads=args.threads))
        print(f"# {name}: {time.time() - t0:.1f} s", flush=True)
    print("chain | vs reference order (max_rel, rel-L2) | vs f64 (max_rel, rel-L2)")
    for name, _ in MODELS:
        a = compare(out[name], out["reference order"])
        b = compare(out[name], out["f64 (exact)"])
        print(f"{name} | {a['max_rel']:.3e}, {a['rel_l2']:.3e} | {b['max_rel']:.3e}, "
              f"{b['rel_l2']:.3e}")


if __name__ == "__main__":
    main()
