"""Per-phase timing of the persistent decode kernel (diagnostics).

Runs the 40-layer config-4a decode (256 experts, top-8, hidden 2048, inter
512, group 128; synthetic seeded weights) through ``DecodePlan`` on the
trace build of the library (``make -C csrc trace``), whose kernel writes a
100 MHz real-time stamp per block at each phase boundary, and prints the
median / p90 / max of every phase over layers 2..37 and all 256 blocks.

    python decode_trace.py [--routed] [--lib PATH]

``--routed`` traces the true-decode instance (every layer routed from its
own normalized input); the default traces the logits-fed plan.  Stamps are
taken by one thread of each block (the wave named per phase below), so a
phase is the time between two stamps of the same block.
"""

import argparse
import ctypes as C
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import __graft_entry__  # noqa: E402

# slot -> boundary (see AIMA_TRACE in csrc/moe_decode_persistent.hip)
FED_PHASES = [(0, 1, "r_L read -> barrier #1 (sums of squares)"),
              (1, 2, "#1 -> #2 (RMSNorm, operands)"),
              (2, 3, "#2 -> gate/up dots done (wave 4)"),
              (3, 4, "dots -> #3"),
              (4, 5, "#3 -> activations published"),
              (5, 6, "act published -> XCD act read (hop)"),
              (6, 7, "act read -> #4 (staging)"),
              (7, 8, "#4 -> P published (down dots)"),
              (8, 9, "P published -> P read (cross-XCD hop)"),
              (9, 10, "P read -> r_{L+1} rows stored (relay)")]
ROUTED_PHASES = [(0, 1, "r_L read -> barrier #1"),
                 (1, 2, "#1 -> #2 (RMSNorm, operands)"),
                 (2, 11, "#2 -> XCD logits read (router dot + hop)"),
                 (11, 12, "logits read -> #2b (ranking)"),
                 (11, 16, "  logits read -> ranked (wave 0)"),
                 (11, 17, "  logits read -> probabilities (wave 1)"),
                 (12, 14, "#2b -> routed rows issued (wave 2)"),
                 (12, 18, "#2b -> routed rows issued (wave 1)"),
                 (12, 15, "#2b -> route confirmed (wave 1)"),
                 (12, 19, "#2b -> gate/up rows in registers (wave 4)"),
                 (12, 3, "#2b -> gate/up dots done (wave 4)"),
                 (3, 4, "dots -> #3"),
                 (4, 5, "#3 -> activations published"),
                 (5, 6, "act published -> XCD act read (hop)"),
                 (6, 7, "act read -> #4 (staging)"),
                 (7, 20, "  #4 -> down rows in registers (wave 0)"),
                 (7, 8, "#4 -> P published (down dots)"),
                 (8, 9, "P published -> P read (cross-XCD hop)"),
                 (9, 10, "P read -> r_{L+1} rows stored (relay)")]
# the streaming wave of the weight-ring instance (logits-fed plan) against
# the compute waves' barriers
RING_PHASES = [(2, 28, "#2 -> gate/up dots done (wave 0)"),
               (2, 29, "#2 -> gate/up dots done (wave 1)"),
               (2, 30, "#2 -> gate/up dots done (wave 5)"),
               (2, 3, "#2 -> gate/up dots done (wave 4)"),
               (14, 1, "wave 0 at #1 -> #1 passed"),
               (1, 11, "#1 -> wave 0 at #2"),
               (1, 12, "#1 -> wave 4 at #2"),
               (1, 13, "#1 -> stream: batch 3 written"),
               (1, 26, "#1 -> stream: batch 3 written, 0 issued"),
               (11, 2, "wave 0 at #2 -> #2 passed"),
               (2, 17, "#2 -> stream: batch 0 written"),
               (2, 27, "#2 -> stream: batch 0 written, 1 issued"),
               (21, 22, "stream: #3 -> batch 1 written"),
               (22, 23, "stream: batch 1 written -> at #4"),
               (25, 7, "wave 0 at #4 -> #4 passed"),
               (23, 7, "stream at #4 -> #4 passed"),
               (7, 24, "#4 -> stream: batch 2 written, 3 issued")]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--routed", action="store_true")
    ap.add_argument("--lib", default=os.path.join(HERE, "csrc", "_trace",
                                                  "libaima_u4moe_trace.so"))
    args = ap.parse_args()
    pkg = __graft_entry__.load_package()
    pkg._lib.LIB_PATH = os.path.abspath(args.lib)
    lib = pkg._lib.lib()
    if not hasattr(lib, "aima_debug_set_decode_trace"):
        raise SystemExit(f"{args.lib} is not a trace build (make -C csrc trace)")
    ops, synth = pkg.ops, pkg.synth
    dev = torch.device("cuda:0")
    n, H, I, E, K = 40, 2048, 512, 256, 8
    layers = [synth.moe_layer(H, I, E, 128, seed=4000 + l, device=dev) for l in range(n)]
    x = synth.activations(1, H, 41, dev)[0].contiguous()
    out = torch.empty(H, dtype=torch.float16, device=dev)
    if args.routed:
        routers = [synth.u4_weight(1, E, H, 128, synth.generator(2041 + l, dev), dev)
                   for l in range(n)]
        plan = ops.DecodePlan(layers, K, routers=routers)
        run = lambda: plan.run(x, routers=routers, out=out)  # noqa: E731
        phases = ROUTED_PHASES
    else:
        logits = torch.stack([synth.router_logits(1, E, 1041 + l, dev)[0] for l in range(n)])
        plan = ops.DecodePlan(layers, K)
        run = lambda: plan.run(x, router_logits=logits, out=out)  # noqa: E731
        phases = FED_PHASES
    for _ in range(10):
        run()
    torch.cuda.synchronize()
    plan.check()
    lib.aima_debug_set_decode_trace.argtypes = [C.c_void_p]
    tr = torch.zeros(41 * 256 * 32, dtype=torch.int64, device=dev)
    pkg._lib.check(lib.aima_debug_set_decode_trace(tr.data_ptr()), "set decode trace")
    for _ in range(3):
        run()
    torch.cuda.synchronize()
    plan.check()
    raw = tr.cpu().numpy().reshape(41, 256, 32)
    xcd = raw[40, :, 31].copy()  # the hardware XCD id of every block
    A = raw.astype(np.float64) * 10.0  # ns

    def st(v):
        v = np.asarray(v)
        return "%7.0f %7.0f %7.0f" % (np.median(v), np.percentile(v, 90), np.max(v))

    print(f"{'routed' if args.routed else 'logits-fed'} plan, trace build, 40 layers x 256 blocks")
    print("launch (entry -> last relay store): %.1f us; prologue (entry -> layer 0) median %.0f ns"
          % ((A[39, :, 10].max() - A[40, :, 0].min()) / 1000,
             np.median(A[40, :, 1] - A[40, :, 0])))
    print("%-44s %7s %7s %7s  (ns, layers 2..37, all blocks)" % ("phase", "median", "p90", "max"))
    for a0, a1, name in phases:
        print("%-44s %s" % (name, st(np.concatenate([A[l][:, a1] - A[l][:, a0]
                                                     for l in range(2, 38)]))))
    if not args.routed:
        simd = raw[40, :, 16:25]
        maps, counts = np.unique(simd, axis=0, return_counts=True)
        for m, c in sorted(zip(maps.tolist(), counts.tolist()), key=lambda t: -t[1])[:3]:
            print("SIMD of waves 0..8 (last: the streaming wave): %s in %d blocks" % (m, c))
        for a0, a1, name in RING_PHASES:
            print("%-44s %s" % (name, st(np.concatenate([A[l][:, a1] - A[l][:, a0]
                                                         for l in range(2, 38)]))))
        print("%-44s %s" % ("stream at #1 -> #1 passed", st(np.concatenate(
            [A[l][:, 1] - A[l - 1][:, 24] for l in range(2, 38)]))))
    hop = [A[l, :, 0] - A[l - 1, :, 10].max() for l in range(2, 38)]
    print("%-44s %s" % ("last r_L store -> r_L read (residual hop)", st(np.concatenate(hop))))
    # The hops measured from the last stamp a reader depends on (block b is
    # rank b / 8 of the XCD it recorded): the act hop waits for the 32 blocks
    # of its XCD, the relay of rank j for rank j of every XCD, the layer
    # start for the 32 relays of its XCD.
    j_of = np.arange(256) // 8

    def by_xcd(v):
        return np.array([v[xcd == xcd[b]].max() for b in range(256)])

    def by_rank(v):
        return np.array([v[j_of == j_of[b]].max() for b in range(256)])

    act_src = [by_xcd(A[l, :, 5]) for l in range(2, 38)]
    p_src = [by_rank(A[l, :, 8]) for l in range(2, 38)]
    r_src = [by_xcd(A[l - 1, :, 10]) for l in range(2, 38)]
    for name, s, dst in [("last XCD act published -> act read", act_src, 6),
                         ("last P of the rank published -> P read", p_src, 9)]:
        print("%-44s %s" % (name, st(np.concatenate([A[l, :, dst] - s[i]
                                                       for i, l in enumerate(range(2, 38))]))))
    print("%-44s %s" % ("last XCD relay store -> r_L read",
                        st(np.concatenate([A[l, :, 0] - r_src[i]
                                           for i, l in enumerate(range(2, 38))]))))
    lay = [A[l + 1, :, 0] - A[l, :, 0] for l in range(2, 38)]
    print("%-44s %s" % ("layer (r_L read -> r_{L+1} read)", st(np.concatenate(lay))))


if __name__ == "__main__":
    main()
