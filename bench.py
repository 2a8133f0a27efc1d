#!/usr/bin/env python3
"""Benchmark of the U4 MoE hot path on one MI355X.

Headline workload (BASELINE.json metric "MoE-FFN decode us/token + HBM GB/s
%peak; grouped prefill tok/s at T=2048"): the 40-layer MoE FFN stack of
config 4 (40 x 256 routed experts + 40 shared experts resident, hidden 2048,
expert intermediate 512, group-128 U4, ~17 GB), one batch-1 decode step per
"step": router top-8 from seeded logits for all 40 layers, then RMSNorm ->
MoE FFN -> residual through every layer; consecutive steps take four seeded
routings in turn.  ``value`` is us per decode token.

The same line carries
* ``roofline``: the dominant kernel, the persistent decode kernel (one launch
  runs all 40 layers): algorithmic bytes per launch (the 8 routed + 1 shared
  experts' U4 weights, scales and zero points of every layer, plus the
  activations) / its event-timed average launch time on the launch stream;
  ``traffic`` is the HBM bytes per launch measured with rocprofv3 PMC
  counters (FETCH_SIZE + WRITE_SIZE, calibrated against a plain copy of
  known size), read from the committed profile summary;
* ``prefill``: grouped prefill of one layer at T=2048 (config 2, Zipf(1.1)
  skewed routing) in tok/s and MFMA fraction, and the 40-layer T=16384 chunk
  (config 4b);
* ``configs``: config 0 (U4 matvec), 1 (one decode layer), 3 (LM-head matvec);
* ``cpu_baseline``: the CPU oracle (restatement of the reference CPU path) on
  this host's cores for a bounded sample of the same decode workload.
Inputs are synthetic (seeded), weights random-init, all resident in HBM
before timing.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
H, I, E, K_TOP, GROUP, LAYERS = 2048, 512, 256, 8, 128, 40
EPS = 1e-6
ROUTE_SETS = 4  # routings the decode steps take in turn


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def u4_bytes(rows, k, group=GROUP):
    return rows * k // 2 + rows * (k // group) * 2 + rows * (k // group) // 2


GATEUP_EXPERT_B = u4_bytes(2 * I, H)   # 1,089,536
DOWN_EXPERT_B = u4_bytes(H, I)         # 544,768
EXPERT_B = GATEUP_EXPERT_B + DOWN_EXPERT_B  # 1,634,304


def timed(torch, fn, iters, warmup=2):
    for _ in range(warmup):
        fn()
    stream = torch.cuda.current_stream()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(iters):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) * 1e3 / iters  # us per call


def graphed(torch, fn):
    """Capture fn into a HIP graph (after a warm run); returns replay callable."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g.replay


def _host_u4(t, idx=None):
    """Device U4 weight (optionally experts idx only) -> numpy (q, s, z) per expert."""
    import numpy as np
    import torch

    q, sc, z = t.qweight, t.scale, t.zp
    if idx is not None:
        ii = torch.as_tensor([int(i) for i in idx], dtype=torch.int64, device=q.device)
        q, sc, z = q.index_select(0, ii), sc.index_select(0, ii), z.index_select(0, ii)
    q = q.cpu().numpy()
    sc = sc.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    z = z.cpu().numpy()
    if idx is None:
        return [(q.reshape(t.rows, -1), sc.reshape(t.rows, -1), z.reshape(-1))]
    return [(q[i], sc[i], z[i]) for i in range(len(idx))]


def _stats(samples):
    srt = sorted(samples)
    return {"min": round(srt[0], 3), "median": round(srt[len(srt) // 2], 3),
            "mean": round(sum(srt) / len(srt), 3), "repeats": len(srt)}


def _time_cpu(fn, min_s=0.6, min_reps=3):
    fn()  # warm
    samples = []
    t_end = time.perf_counter() + min_s
    while time.perf_counter() < t_end or len(samples) < min_reps:
        t0 = time.perf_counter()
        fn()
        samples.append((time.perf_counter() - t0) * 1e6)
    return samples


def cpu_baseline(torch, pkg, layers, x, ids, w, dev):
    """The reference CPU path (oracle/cpu_baseline.c: the row-parallel U4
    matvec and MoE layer of gguf_loader.cpp, scale / zero point hoisted per
    group, OpenMP) compiled here with -O3 -march=native, at 1 thread and at
    this process's CPU share, for configs 0, 1, 2, 3, 4a and 4b.  Only the
    experts a sample touches are copied to the host."""
    import tempfile

    import numpy as np

    from oracle import cpu_baseline as cpb

    base = cpb.load(tempfile.mkdtemp(prefix="aima_cpb_"))
    share = len(os.sched_getaffinity(0))
    nthreads = max(1, min(16, share))  # the box grants one GPU 16 host cores
    gen = pkg.synth.generator(0, dev)
    m0 = pkg.synth.u4_weight(1, 4096, 2048, GROUP, gen, dev)
    m3 = pkg.synth.u4_weight(1, 248320, 2048, GROUP, pkg.synth.generator(3, dev), dev)
    mats = {"config0": (_host_u4(m0)[0], 4096), "config3": (_host_u4(m3)[0], 248320)}
    del m3
    xv = np.random.default_rng(0).normal(size=2048).astype(np.float32)
    x_np = x.float().cpu().numpy()
    ids_np, w_np = ids.cpu().numpy(), w.cpu().numpy()

    def layer_rec(L, sel):
        lay = layers[L]
        ex = list(zip(_host_u4(lay.gate_up, sel), _host_u4(lay.down, sel)))
        sh = (_host_u4(lay.shared_gate_up)[0], _host_u4(lay.shared_down)[0])
        return base.layer(ex, sh, lay.shared_gate_vec.float().cpu().numpy(),
                          lay.norm_weight.cpu().numpy(), H, I, GROUP)

    decode_layers = [(layer_rec(L, ids_np[L]), w_np[L]) for L in range(LAYERS)]
    # prefill samples: config 2 (one layer, Zipf routing) token by token, and
    # config 4b (40 layers, uniform routing) for two tokens
    T2 = 16
    xs2 = pkg.synth.activations(2048, H, 2, dev)[:T2].float().cpu().numpy()
    i2, w2 = pkg.select_router_topk(pkg.synth.router_logits(2048, E, 3, dev, zipf_s=1.1), K_TOP)
    i2, w2 = i2[:T2].cpu().numpy(), w2[:T2].cpu().numpy()
    p2 = [(layer_rec(0, i2[t]), w2[t]) for t in range(T2)]
    T4 = 2
    xs4 = pkg.synth.activations(16384, H, 43, dev)[:T4].float().cpu().numpy()
    lg4 = torch.stack([pkg.synth.router_logits(16384, E, 2044 + l, dev)[:T4] for l in range(LAYERS)])
    i4, w4 = pkg.select_router_topk(lg4, K_TOP)
    i4, w4 = i4.cpu().numpy(), w4.cpu().numpy()
    p4 = [[(layer_rec(L, i4[L, t]), w4[L, t]) for L in range(LAYERS)] for t in range(T4)]

    out = np.empty(H, np.float32)

    def stack(r0, recs):
        r, nxt = r0.copy(), np.empty_like(r0)
        for lay, wl in recs:
            base.moe_token(lay, wl, EPS, r, nxt)
            r, nxt = nxt, r
        return r

    def mv(name):
        (q, sc, z), n = mats[name]
        y = np.empty(n, np.float32)
        return lambda: base.matvec(q, sc, z, n, 2048, GROUP, xv, y)

    work = {
        "config0_matvec_K2048_N4096": ("us/matvec", mv("config0"), 1),
        "config1_decode_layer": ("us/token", lambda: base.moe_token(decode_layers[0][0],
                                                                     decode_layers[0][1], EPS,
                                                                     x_np, out), 1),
        "config2_prefill_T2048": ("tok/s", lambda: [base.moe_token(l_, w_, EPS, xs2[t], out)
                                                     for t, (l_, w_) in enumerate(p2)], T2),
        "config3_lm_head_N248320": ("us/matvec", mv("config3"), 1),
        "config4a_decode_40L": ("us/token", lambda: stack(x_np, decode_layers), 1),
        "config4b_prefill_40L_T16384": ("tok/s", lambda: [stack(xs4[t], p4[t])
                                                          for t in range(T4)], T4),
    }
    recs = {}
    for name, (unit, fn, ntok) in work.items():
        rec = {"unit": unit}
        for th in sorted({1, nthreads}):
            base.set_threads(th)
            st = _stats(_time_cpu(fn))
            if unit == "tok/s":
                st = {"tok_s": round(ntok / (st["median"] * 1e-6), 2), "us_per_call": st,
                      "tokens_per_call": ntok}
            rec[f"threads_{th}"] = st
        recs[name] = rec
        log(f"cpu baseline {name}: {rec}")
    head = recs["config4a_decode_40L"][f"threads_{nthreads}"]
    return {"value": head["median"], "unit": "us/token", "cores": nthreads, "kind": "port",
            "sample": f"config 4a: one decode token through all 40 layers (8 routed + shared "
                      f"expert per layer), median of {head['repeats']}; every config at 1 and "
                      f"{nthreads} threads in 'configs' (prefill configs token by token, the "
                      f"reference CPU layer function: {T2} tokens of config 2, {T4} of 4b)",
            "build": "gcc -O3 -march=native -fopenmp (built on this host)",
            "host_cpu": _cpu_model(), "host_cpus_visible": share, "configs": recs}


def profiled_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (profiles/*_pmc.md lines "traffic_bytes_per_launch <kernel> <bytes>"), or
    None when no summary records it."""
    d = os.path.join(ROOT, "profiles")
    if not os.path.isdir(d):
        return None
    for name in sorted(os.listdir(d)):
        if not name.endswith("_pmc.md"):
            continue
        for line in open(os.path.join(d, name)):
            parts = line.strip().strip("`").split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == kernel:
                return int(parts[2])
    return None


def _cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name (virtualized hosts
    may report only the family name), x86 family / model / stepping, the
    widest vector extension and the logical CPU count."""
    fields = {}
    n = 0
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                continue
            key, val = (t.strip() for t in line.split(":", 1))
            if key == "processor":
                n += 1
            if key in ("model name", "cpu family", "model", "stepping", "flags") and \
                    key not in fields:
                fields[key] = val
    except OSError:
        return "unknown"
    flags = fields.get("flags", "").split()
    vec = next((f for f in ("avx512f", "avx2", "avx") if f in flags), "none")
    return (f"{fields.get('model name', 'unknown')} (family {fields.get('cpu family', '?')} "
            f"model {fields.get('model', '?')} stepping {fields.get('stepping', '?')}, "
            f"{vec}, {n} logical CPUs)")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="only the headline decode step (for profiling runs)")
    ap.add_argument("--prefill-tokens", type=int, default=2048,
                    help="with --prefill-only: tokens of the one timed layer (2048 = config 2 "
                         "with Zipf routing; other values use uniform routing, as config 4b)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config 2 grouped prefill (one layer, T=2048), timed with "
                         "--steps launches; prints its JSON entry (for profiling runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy 5 times (PMC counter "
                         "calibration) and exit")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py measures one GPU: the batch-1 decode and grouped prefill path here "
              "is single-device (multi-GPU sharding is a design note, not a build target); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        n = 1 << 30
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "copies": 5}), flush=True)
        return

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    from aima_u4moe import ops, synth  # noqa: E402

    dev = torch.device("cuda:0")
    if args.prefill_only:
        layer = synth.moe_layer(hidden=H, inter=I, experts=E, group=GROUP, seed=4000, device=dev)
        layers_c = ops._layers_c([layer])
        res = prefill_config2(torch, pkg, ops, synth, layer, layers_c, dev, args.steps,
                              args.warmup, T=args.prefill_tokens)
        key = ("prefill_config2_T2048" if args.prefill_tokens == 2048
               else f"prefill_layer_T{args.prefill_tokens}_uniform")
        print(json.dumps({key: res}), flush=True)
        return
    log(f"device {torch.cuda.get_device_name(0)}; building 40-layer stack")
    t0 = time.perf_counter()
    layers = [synth.moe_layer(hidden=H, inter=I, experts=E, group=GROUP, seed=4000 + l,
                              device=dev) for l in range(LAYERS)]
    layers_c = ops._layers_c(layers)
    torch.cuda.synchronize()
    log(f"stack resident in {time.perf_counter() - t0:.1f}s, "
        f"{sum(l.gate_up.nbytes + l.down.nbytes + l.shared_bytes() for l in layers) / 1e9:.2f} GB")

    # ------------------------------------------------------------------ decode
    x = synth.activations(1, H, 41, dev)[0].contiguous()
    # ROUTE_SETS routings (per-layer logits), taken in turn by consecutive
    # steps of the persistent plan, so that no step re-reads the experts the
    # step before it read (the union over the sets, ~2 GB, is far past the
    # 256 MB last-level cache)
    logit_sets = [torch.stack([synth.router_logits(1, E, 1041 + 97 * s + l, dev)[0]
                               for l in range(LAYERS)]) for s in range(ROUTE_SETS)]
    logits = logit_sets[0]
    ws = ops.Workspace(dev)
    out = torch.empty(H, dtype=torch.float16, device=dev)
    ids_buf = torch.empty((LAYERS, K_TOP), dtype=torch.int32, device=dev)
    w_buf = torch.empty((LAYERS, K_TOP), dtype=torch.float32, device=dev)
    lib = pkg._lib

    def decode_step_multikernel():
        lib.call("aima_router_topk", logits.data_ptr(), LAYERS, E, K_TOP,
                 ops.MIN_WEIGHT_SUM, ids_buf.data_ptr(), w_buf.data_ptr(), ops._stream())
        ops.moe_stack_decode(layers, x, ids_buf, w_buf, EPS, ws=ws, out=out, layers_c=layers_c)

    multi_us = timed(torch, decode_step_multikernel, max(10, args.steps // 10), warmup=3)
    log(f"decode multi-kernel: {multi_us:.1f} us/token")
    ws.check()
    # true decode: each layer routes from its own hidden state (router U4 FC
    # [256][2048] + top-8 per layer, then the layer), multi-kernel
    routers = [synth.u4_weight(1, E, H, GROUP, synth.generator(2041 + l, dev), dev)
               for l in range(LAYERS)]
    routed_us = timed(torch, lambda: ops.moe_stack_decode_routed(layers, routers, x, K_TOP,
                                                                 epsilon=EPS, ws=ws),
                      max(10, args.steps // 10), warmup=3)
    log(f"decode multi-kernel, routed from h: {routed_us:.1f} us/token")
    ws.check()
    # true decode inside the resident plan: every layer routes from its own
    # normalized input in the same persistent launch
    rplan = ops.DecodePlan(layers, k=K_TOP, routers=routers)
    routed_plan_us = timed(torch, lambda: rplan.run(x, routers=routers, epsilon=EPS, out=out),
                           args.steps, warmup=args.warmup)
    rplan.check()
    log(f"decode persistent, routed from h: {routed_plan_us:.1f} us/token")
    rplan.close()
    del rplan, routers
    plan = ops.DecodePlan(layers, k=K_TOP)
    step_no = [0]

    def decode_step_set(sidx):
        plan.run(x, router_logits=logit_sets[sidx], epsilon=EPS, out=out)

    def decode_step():
        decode_step_set(step_no[0] % ROUTE_SETS)
        step_no[0] += 1

    eager_us = timed(torch, decode_step, args.steps, warmup=args.warmup)
    log(f"decode persistent eager: {eager_us:.1f} us/token")
    replays = [graphed(torch, lambda s=s: decode_step_set(s)) for s in range(ROUTE_SETS)]

    def replay():
        replays[step_no[0] % ROUTE_SETS]()
        step_no[0] += 1

    graph_us = timed(torch, replay, args.steps, warmup=args.warmup)
    log(f"decode persistent graph: {graph_us:.1f} us/token")
    plan.check()
    step_us = min(eager_us, graph_us)
    decode_mode = "hip-graph" if graph_us <= eager_us else "eager"
    torch.cuda.synchronize()
    ids_np = ids_buf.cpu().numpy()
    n_unique = sum(len(set(r)) for r in ids_np)
    weight_bytes = LAYERS * (K_TOP * EXPERT_B + EXPERT_B)  # 8 routed + shared per layer
    act_bytes = LAYERS * (H * 2 * 3 + H * 4 + (K_TOP + 1) * I * 2 * 2 + H * 2)
    decode_gbs = (weight_bytes + act_bytes) / step_us / 1e3

    # dominant kernel: the persistent decode kernel, one launch per token; its
    # algorithmic bytes are the 8 routed + 1 shared experts of all 40 layers
    # plus the activations, timed back to back on the launch stream
    per_launch_us = timed(torch, decode_step, args.steps, warmup=3)
    plan.check()  # every timed launch finished without a device error
    achieved = (weight_bytes + act_bytes) / per_launch_us / 1e3
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": profiled_traffic("decode_persistent_kernel"),
                "kernel": "decode_persistent_kernel", "bytes_per_launch": weight_bytes + act_bytes,
                "avg_launch_us": round(per_launch_us, 3)}
    log(f"persistent decode kernel: {per_launch_us:.2f} us/launch, {achieved:.0f} GB/s")

    result = {
        "metric": "MoE-FFN decode us/token + HBM GB/s %peak; grouped prefill tok/s at T=2048",
        "value": round(step_us, 2), "unit": "us/token", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_us / 1e3, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u4xf16",
        "data": "synthetic (seeded U4 weights, f16 activations, f32 router logits)",
        "config": {"workload": "config4a: 40-layer MoE FFN decode step, batch 1, top-8/256 + "
                               "shared expert, hidden 2048, inter 512, U4 group 128",
                   "routings": ROUTE_SETS,
                   "layers": LAYERS, "experts": E, "top_k": K_TOP, "hidden": H, "inter": I,
                   "group": GROUP, "parallelism": "single-gpu"},
        "decode": {"us_per_token": round(step_us, 2), "eager_us": round(eager_us, 2),
                   "graph_us": round(graph_us, 2), "mode": decode_mode,
                   "multikernel_us": round(multi_us, 2),
                   "routed_multikernel_us": round(routed_us, 2),
                   "routed_plan_us": round(routed_plan_us, 2),
                   "algorithmic_bytes": weight_bytes + act_bytes,
                   "hbm_gbs": round(decode_gbs, 1),
                   "hbm_frac": round(decode_gbs / HBM_PEAK_GBS, 4),
                   "unique_experts_per_step": int(n_unique)},
        "roofline": roofline,
    }

    if not args.no_extras:
        pf = prefill_bench(torch, pkg, ops, synth, layers, layers_c, dev)
        result["prefill"] = pf
        # the prefill half of the metric as flat scalars
        c2, c4 = pf["config2_T2048"], pf["config4b_T16384_40L"]
        result.update({"prefill_T2048_us": c2["us"], "prefill_T2048_tok_s": c2["tok_s"],
                       "prefill_T2048_mfma_frac": c2["mfma_frac"],
                       "prefill_4b_ms": round(c4["us"] / 1e3, 3),
                       "prefill_4b_tok_s": c4["tok_s"], "prefill_4b_mfma_frac": c4["mfma_frac"]})
        result["configs"] = matvec_bench(torch, ops, synth, layers, layers_c, dev, ids_buf,
                                         w_buf)

    if not args.no_cpu_baseline:
        log("cpu baseline (reference CPU path, all configs, 1 and N threads)")
        cb = cpu_baseline(torch, pkg, layers, x, ids_buf, w_buf, dev)
        result["cpu_baseline"] = cb
        # each CPU record beside the GPU's number for the same config
        gpu = {"config4a_decode_40L": (step_us, roofline["frac"])}
        if not args.no_extras:
            cf = result["configs"]
            gpu.update({
                "config0_matvec_K2048_N4096": (cf["config0_matvec_K2048_N4096"]["us"],
                                               cf["config0_matvec_K2048_N4096"]["hbm_frac"]),
                "config1_decode_layer": (cf["config1_decode_layer"]["us"],
                                         cf["config1_decode_layer"]["hbm_frac"]),
                "config3_lm_head_N248320": (cf["config3_lm_head_N248320"]["us"],
                                            cf["config3_lm_head_N248320"]["hbm_frac"]),
                "config2_prefill_T2048": (c2["tok_s"], c2["mfma_frac"]),
                "config4b_prefill_40L_T16384": (c4["tok_s"], c4["mfma_frac"])})
        for name, (v, frac) in gpu.items():
            cb["configs"][name]["gpu"] = {"value": v, "roofline_frac": frac}
    print(json.dumps(result), flush=True)


def prefill_config2(torch, pkg, ops, synth, layer, layers_c, dev, iters=50, warmup=5,
                    T=2048):
    """Config 2: one layer, T=2048, Zipf(1.1)-skewed routing (another T: one
    layer of that many tokens with uniform routing, as in config 4b)."""
    x = synth.activations(T, H, 2, dev)
    ids, w = ops.select_router_topk(synth.router_logits(T, E, 3, dev,
                                                        zipf_s=1.1 if T == 2048 else None), K_TOP)
    ws = ops.Workspace(dev)
    o = torch.empty_like(x)

    def run():
        lc = layers_c[0]
        import ctypes as C
        buf = ws.get(pkg._lib.size_query("aima_moe_prefill_workspace_size", C.byref(lc), T,
                                         K_TOP))
        pkg._lib.call("aima_moe_grouped_prefill", C.byref(lc), x.data_ptr(), None, T,
                      ids.data_ptr(), w.data_ptr(), K_TOP, o.data_ptr(), buf.data_ptr(),
                      buf.numel(), ops._stream())

    us = timed(torch, run, iters, warmup=warmup)
    ws.check()
    flops = (T * K_TOP + T) * 2 * (H * 2 * I + I * H)
    counts = torch.bincount(ids.reshape(-1).long(), minlength=E)
    active = int((counts > 0).sum())
    wbytes = active * EXPERT_B + EXPERT_B
    tf = flops / us / 1e6
    res = {"us": round(us, 2), "tok_s": round(T / us * 1e6, 1),
           "tflops": round(tf, 2), "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
           "hbm_weight_gbs": round(wbytes / us / 1e3, 1),
           "active_experts": active, "max_group": int(counts.max()),
           "flops": flops}
    log(f"prefill T={T}: {us:.1f} us, {T / us * 1e6:.0f} tok/s, {tf:.1f} TFLOP/s")
    return res


def prefill_bench(torch, pkg, ops, synth, layers, layers_c, dev):
    out = {"config2_T2048": prefill_config2(torch, pkg, ops, synth, layers[0], layers_c, dev)}
    # config 4b: 40 layers, T=16384
    T = 16384
    x = synth.activations(T, H, 43, dev)
    logits = torch.stack([synth.router_logits(T, E, 2044 + l, dev) for l in range(LAYERS)])
    ids, w = ops.select_router_topk(logits, K_TOP)
    del logits
    ws2 = ops.Workspace(dev)
    o = torch.empty_like(x)

    def run4b():
        ops.moe_stack_prefill(layers, x, ids, w, EPS, ws=ws2, out=o, layers_c=layers_c)

    us = timed(torch, run4b, 3, warmup=1)
    ws2.check()
    flops = LAYERS * (T * K_TOP + T) * 2 * (H * 2 * I + I * H)
    tf = flops / us / 1e6
    out["config4b_T16384_40L"] = {"us": round(us, 1), "tok_s": round(T / us * 1e6, 1),
                                  "tflops": round(tf, 2),
                                  "mfma_frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                                  "flops": flops}
    log(f"prefill 40L T=16384: {us / 1e3:.2f} ms, {tf:.1f} TFLOP/s")
    return out


def matvec_bench(torch, ops, synth, layers, layers_c, dev, ids_buf, w_buf):
    out = {}
    # config 0: K=2048, N=4096 over 64 rotating weight copies (~280 MB, past the caches)
    gen = synth.generator(0, dev)
    copies = [synth.u4_weight(1, 4096, 2048, GROUP, gen, dev) for _ in range(64)]
    x = synth.activations(1, 2048, 0, dev)[0].contiguous()
    y = torch.empty(4096, dtype=torch.float16, device=dev)
    import ctypes as C
    lib = ops._lib

    def mv_all():
        for wgt in copies:
            lib.call("aima_u4_matvec", x.data_ptr(), wgt.qweight.data_ptr(),
                     wgt.scale.data_ptr(), wgt.zp.data_ptr(), 4096, 2048, GROUP, y.data_ptr(),
                     0, ops._stream())

    rep = graphed(torch, mv_all)
    us = timed(torch, rep, 20, warmup=2) / len(copies)
    b0 = u4_bytes(4096, 2048) + 2048 * 2 + 4096 * 2
    out["config0_matvec_K2048_N4096"] = {"us": round(us, 3), "gbs": round(b0 / us / 1e3, 1),
                                         "hbm_frac": round(b0 / us / 1e3 / HBM_PEAK_GBS, 4),
                                         "bytes": b0}
    del copies
    # config 1: one decode layer, cycling over the 40 resident layers (cache-cold)
    ws = ops.Workspace(dev)
    o = torch.empty(H, dtype=torch.float16, device=dev)
    res = synth.activations(1, H, 5, dev)[0].contiguous()
    rows = [(ids_buf[l].contiguous(), w_buf[l].contiguous()) for l in range(LAYERS)]
    buf = ws.get(ops.size_query("aima_moe_decode_workspace_size", C.byref(layers_c[0]), K_TOP))

    def layer_all():
        for l in range(LAYERS):
            lib.call("aima_moe_ffn_decode", C.byref(layers_c[l]), x.data_ptr(), res.data_ptr(),
                     rows[l][0].data_ptr(), rows[l][1].data_ptr(), K_TOP, o.data_ptr(),
                     buf.data_ptr(), buf.numel(), ops._stream())

    rep = graphed(torch, layer_all)
    us = timed(torch, rep, 20, warmup=2) / LAYERS
    b1 = (K_TOP + 1) * EXPERT_B
    out["config1_decode_layer"] = {"us": round(us, 3), "gbs": round(b1 / us / 1e3, 1),
                                   "hbm_frac": round(b1 / us / 1e3 / HBM_PEAK_GBS, 4),
                                   "weight_bytes": b1}
    # config 3: LM-head-sized matvec, K=2048, N=248320, f32 logits
    wl = synth.u4_weight(1, 248320, 2048, GROUP, synth.generator(3, dev), dev)
    xl = synth.activations(1, 2048, 3, dev)[0].contiguous()
    us = timed(torch, lambda: ops.matvec_u4(xl, wl, out_dtype=torch.float32), 50, warmup=5)
    b3 = u4_bytes(248320, 2048) + 2048 * 2 + 248320 * 4
    out["config3_lm_head_N248320"] = {"us": round(us, 2), "gbs": round(b3 / us / 1e3, 1),
                                      "hbm_frac": round(b3 / us / 1e3 / HBM_PEAK_GBS, 4),
                                      "bytes": b3}
    # the same LM head with its top-8 (logits kept; one launch at K = 2048):
    # back-to-back calls through the C ABI with preallocated outputs (the
    # Python wrapper's allocations and size query would outlast the GPU
    # work, and a graph replay adds its own launch overhead on this system)
    lws = ops.Workspace(dev)
    nl = 248320
    lbuf = lws.get(ops.size_query("aima_topk_workspace_size", nl, 8))
    lg = torch.empty(nl, dtype=torch.float32, device=dev)
    tid = torch.empty(8, dtype=torch.int32, device=dev)
    tval = torch.empty(8, dtype=torch.float32, device=dev)

    def lm_head_call():
        ops.call("aima_u4_lm_head_topk", xl.data_ptr(), wl.qweight.data_ptr(),
                 wl.scale.data_ptr(), wl.zp.data_ptr(), nl, 2048, GROUP, 8, lg.data_ptr(),
                 tid.data_ptr(), tval.data_ptr(), lbuf.data_ptr(), lbuf.numel(), ops._stream())

    us = timed(torch, lm_head_call, 50, warmup=5)
    lws.check()
    out["lm_head_topk8_N248320"] = {"us": round(us, 2), "gbs": round(b3 / us / 1e3, 1),
                                    "hbm_frac": round(b3 / us / 1e3 / HBM_PEAK_GBS, 4),
                                    "bytes": b3}
    del wl
    # the K=2048 fanout (multi-output fixed FC, N = [1, 512, 512, 256]) and the
    # device router (U4 FC 2048 -> 256, then top-8), each over ~270 MB of
    # rotating weight copies (past the caches)
    fan_rows = (1, 512, 512, 256)
    fan_dts = [torch.float16, torch.float16, torch.float16, torch.float32]
    fans = [[synth.u4_weight(1, n, 2048, GROUP, gen, dev) for n in fan_rows] for _ in range(200)]
    xf = synth.activations(1, 2048, 9, dev)[0].contiguous()

    def fan_all():
        for f in fans:
            ops.matvec_u4_multi(xf, f, fan_dts)

    rep = graphed(torch, fan_all)
    us = timed(torch, rep, 5, warmup=1) / len(fans)
    bf = sum(u4_bytes(n, 2048) for n in fan_rows) + 2048 * 2 + (1 + 512 + 512) * 2 + 256 * 4
    out["fanout_K2048_N1_512_512_256"] = {"us": round(us, 3), "gbs": round(bf / us / 1e3, 1),
                                          "hbm_frac": round(bf / us / 1e3 / HBM_PEAK_GBS, 4),
                                          "bytes": bf}
    del fans
    routers = [synth.u4_weight(1, 256, 2048, GROUP, gen, dev) for _ in range(1000)]

    def router_all():
        for r in routers:
            ops.router_fc_topk(xf, r, K_TOP)

    rep = graphed(torch, router_all)
    us = timed(torch, rep, 5, warmup=1) / len(routers)
    br = u4_bytes(256, 2048) + 2048 * 2 + 256 * 4
    out["router_fc_topk_E256"] = {"us": round(us, 3), "gbs": round(br / us / 1e3, 1),
                                  "hbm_frac": round(br / us / 1e3 / HBM_PEAK_GBS, 4), "bytes": br}
    del routers
    log(f"config0 {out['config0_matvec_K2048_N4096']['us']} us, config1 "
        f"{out['config1_decode_layer']['us']} us, config3 {out['config3_lm_head_N248320']['us']} us, "
        f"fanout {out['fanout_K2048_N1_512_512_256']['us']} us, router "
        f"{out['router_fc_topk_E256']['us']} us")
    return out


if __name__ == "__main__":
    main()
