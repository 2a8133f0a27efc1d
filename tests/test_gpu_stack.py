"""GPU parity for the layer stacks (config 4): RMSNorm between layers, f16
activations carried layer to layer.  Small stacks are checked on every token;
the full 40-layer x 256-expert stack (~17 GB resident) is checked on the
decode token and on sampled prefill tokens (tokens are independent through
an MoE FFN stack, so a token subset is an exact check of those rows)."""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import (assert_end_to_end, assert_parity, f16_bits, f16_to_f32, moe_to_oracle,
                           stack_chains, u4_to_oracle)

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)
EPS = 1e-6


def oracle_stack(layers_np, norms, x_bits, ids, w):
    """ids/w: [L][T][k] (already remapped to each layer's oracle experts)."""
    r = x_bits
    for L, mw in enumerate(layers_np):
        rf = oracle.f16_values(r)
        h = oracle.f16_values(oracle.float_to_half(oracle.rms_norm_rows(rf, norms[L], EPS))
                              .reshape(rf.shape))
        o = oracle.moe_ffn_tokens(mw, h, ids[L], w[L], residual=rf, threads=THREADS)
        r = oracle.float_to_half(o).reshape(o.shape)
    return r


def compact_oracle_layer(layer, used):
    """Oracle weights holding only the experts in `used` (in that order)."""
    idx = torch.as_tensor(np.asarray(used, np.int64), device=layer.gate_up.qweight.device)

    def pick(w):
        sub = type(w)(w.qweight.index_select(0, idx).contiguous(),
                      w.scale.index_select(0, idx).contiguous(),
                      w.zp.index_select(0, idx).contiguous(), w.rows, w.k, w.group)
        return u4_to_oracle(sub)

    return oracle.MoeWeights(pick(layer.gate_up), pick(layer.down),
                             u4_to_oracle(layer.shared_gate_up), u4_to_oracle(layer.shared_down),
                             f16_bits(layer.shared_gate_vec))


def remap(ids_np):
    used, inv = np.unique(ids_np, return_inverse=True)
    return used, inv.reshape(ids_np.shape).astype(np.int32)


def make_stack(pkg, dev, n_layers, H, I, E, seed):
    return [pkg.synth.moe_layer(hidden=H, inter=I, experts=E, seed=seed + l, device=dev)
            for l in range(n_layers)]


def routing(pkg, dev, n_layers, T, E, seed, k=8):
    logits = torch.stack([pkg.synth.router_logits(T, E, seed + 1000 + l, dev)
                          for l in range(n_layers)])
    return pkg.select_router_topk(logits, k)


def test_small_stack_decode_and_prefill(pkg, dev):
    layers = make_stack(pkg, dev, 3, 512, 128, 16, seed=500)
    lnp = [moe_to_oracle(l) for l in layers]
    norms = [l.norm_weight.cpu().numpy() for l in layers]
    # decode
    x = pkg.synth.activations(1, 512, 1, dev)
    ids, w = routing(pkg, dev, 3, 1, 16, 2)
    out = pkg.moe_stack_decode(layers, x[0], ids[:, 0].contiguous(), w[:, 0].contiguous(),
                               epsilon=EPS)
    torch.cuda.synchronize()
    ref = oracle_stack(lnp, norms, f16_bits(x), ids.cpu().numpy(), w.cpu().numpy())
    assert_parity(f16_to_f32(out), oracle.f16_values(ref[0]), what="small stack decode")
    # prefill
    T = 97
    x = pkg.synth.activations(T, 512, 3, dev)
    ids, w = routing(pkg, dev, 3, T, 16, 4)
    out = pkg.moe_stack_prefill(layers, x, ids, w, epsilon=EPS)
    torch.cuda.synchronize()
    ids_np, w_np = ids.cpu().numpy(), w.cpu().numpy()
    # teacher-forced: every GPU layer starts from the oracle's input (2e-3 bar)
    r = f16_bits(x)
    for L in range(len(layers)):
        nxt = oracle_stack([lnp[L]], [norms[L]], r, ids_np[L:L + 1], w_np[L:L + 1])
        got = pkg.moe_stack_prefill([layers[L]], torch.from_numpy(r.view(np.float16)).to(dev),
                                    ids[L:L + 1].contiguous(), w[L:L + 1].contiguous(),
                                    epsilon=EPS)
        torch.cuda.synchronize()
        assert_parity(f16_to_f32(got), oracle.f16_values(nxt),
                      what=f"small stack prefill layer {L}")
        r = nxt
    # free-running: against the measured floor of the same chain
    chains = stack_chains(lnp, norms, f16_bits(x), ids_np, w_np, EPS, oracle.MODEL_PREFILL,
                          THREADS)
    assert np.array_equal(chains["ref"], r)
    assert_end_to_end(f16_to_f32(out), chains, "small stack prefill end-to-end")


def test_stack_single_layer_equals_layer_ops(pkg, dev):
    """One stack layer == RMSNorm, then the decode layer with the residual."""
    layers = make_stack(pkg, dev, 1, 2048, 512, 32, seed=700)
    x = pkg.synth.activations(1, 2048, 7, dev)[0]
    ids, w = routing(pkg, dev, 1, 1, 32, 8)
    a = pkg.moe_stack_decode(layers, x, ids[:, 0].contiguous(), w[:, 0].contiguous(), EPS)
    h = pkg.apply_rms_norm(x[None], layers[0].norm_weight, EPS)[0]
    b = pkg.run_moe_ffn_layer(layers[0], h, ids[0, 0].contiguous(), w[0, 0].contiguous(),
                              residual=x)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.fixture(scope="module")
def stack40(pkg, dev):
    layers = make_stack(pkg, dev, 40, 2048, 512, 256, seed=4000)
    yield layers
    del layers
    torch.cuda.empty_cache()


def compact_chain(stack, ids_np):
    """Per layer, oracle weights holding only the experts the tokens select,
    and the tokens' ids into them (ids_np [L][T][k])."""
    mws, rids = [], []
    for L, layer in enumerate(stack):
        used, rid = remap(ids_np[L])
        mws.append(compact_oracle_layer(layer, used))
        rids.append(rid)
    return mws, np.stack(rids)


def _oracle_layer(layer, r_bits, ids_np, w_np, mw=None):
    """One stack layer on the oracle for a few tokens, using only the experts
    they select: r_{L+1} = f16(r + ffn(f16(rmsnorm(r)))).  With mw (from
    compact_chain) ids_np are already ids into mw."""
    if mw is None:
        used, rid = remap(ids_np)
        mw = compact_oracle_layer(layer, used)
    else:
        rid = ids_np
    rf = oracle.f16_values(r_bits)
    h = oracle.f16_values(oracle.float_to_half(
        oracle.rms_norm_rows(rf, layer.norm_weight.cpu().numpy(), EPS)).reshape(rf.shape))
    o = oracle.moe_ffn_tokens(mw, h, rid, w_np, residual=rf, threads=THREADS)
    return oracle.float_to_half(o).reshape(o.shape)


def test_config4a_decode_40_layers(pkg, dev, stack40):
    """Config 4a through the multi-kernel stack: every layer teacher-forced
    at the 2e-3 bar; the 40-layer call equals 40 chained 1-layer calls bit
    for bit; the free-running result within the measured floor."""
    x = pkg.synth.activations(1, 2048, 41, dev)
    ids, w = routing(pkg, dev, 40, 1, 256, 42)
    out = pkg.moe_stack_decode(stack40, x[0], ids[:, 0].contiguous(), w[:, 0].contiguous(), EPS)
    torch.cuda.synchronize()
    ids_np, w_np = ids.cpu().numpy(), w.cpu().numpy()
    mws, rids = compact_chain(stack40, ids_np)
    norms = [l.norm_weight.cpu().numpy() for l in stack40]
    r = f16_bits(x)
    chained = x[0]
    for L, layer in enumerate(stack40):
        nxt = _oracle_layer(layer, r, rids[L], w_np[L], mw=mws[L])
        got = pkg.moe_stack_decode([layer], torch.from_numpy(r[0].view(np.float16)).to(dev),
                                   ids[L].contiguous(), w[L].contiguous(), EPS)
        chained = pkg.moe_stack_decode([layer], chained, ids[L].contiguous(),
                                       w[L].contiguous(), EPS)
        torch.cuda.synchronize()
        assert_parity(f16_to_f32(got), oracle.f16_values(nxt[0]), what=f"config4a layer {L}")
        r = nxt
    assert torch.equal(chained, out), "40-layer stack differs from 40 chained 1-layer calls"
    chains = stack_chains(mws, norms, f16_bits(x), rids, w_np, EPS, oracle.MODEL_ACT_F16 |
                          oracle.MODEL_CHUNKED, THREADS)
    assert np.array_equal(chains["ref"], r)
    assert_end_to_end(f16_to_f32(out), chains, "config4a multi-kernel end-to-end")


def test_config4b_prefill_40_layers_full_tiles(pkg, dev, stack40):
    """Config 4b, T = 16384 (full 256-row tiles, every expert ~512 rows).
    Layer by layer at the full T: each GPU layer runs on the GPU's own input
    for all tokens, and the oracle runs the same layer on the same input rows
    for sampled tokens (teacher-forced per layer at the 2e-3 bar).  The
    40-layer stack (fused combine: next layer's RMSNorm and shared gate in
    the combine kernel) equals the layer-by-layer runs bit for bit, and the
    sampled tokens' end-to-end result lies within the measured floor of
    their oracle chains."""
    T = 16384
    x = pkg.synth.activations(T, 2048, 43, dev)
    ids, w = routing(pkg, dev, 40, T, 256, 44)
    out = pkg.moe_stack_prefill(stack40, x, ids, w, EPS)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    sel = np.array([0, 1, 777, 5000, 8191, 12345, 16000, 16383])
    ids_np = ids.cpu().numpy()[:, sel]
    w_np = w.cpu().numpy()[:, sel]
    r = x
    for L, layer in enumerate(stack40):
        nxt = pkg.moe_stack_prefill([layer], r, ids[L:L + 1].contiguous(),
                                    w[L:L + 1].contiguous(), EPS)
        torch.cuda.synchronize()
        ref = _oracle_layer(layer, f16_bits(r)[sel], ids_np[L], w_np[L])
        assert_parity(f16_to_f32(nxt)[sel], oracle.f16_values(ref),
                      what=f"config4b layer {L} (T=16384)")
        r = nxt
    assert torch.equal(r, out), "fused 40-layer stack differs from the layer-by-layer runs"
    mws, rids = compact_chain(stack40, ids_np)
    norms = [l.norm_weight.cpu().numpy() for l in stack40]
    chains = stack_chains(mws, norms, f16_bits(x)[sel], rids, w_np, EPS, oracle.MODEL_PREFILL,
                          THREADS)
    assert_end_to_end(f16_to_f32(out)[sel], chains, "config4b end-to-end (8 sampled tokens)")


def test_stack_prefill_fused_combine_three_layers(pkg, dev):
    """H = 2048 stacks fuse the next layer's RMSNorm and shared gate into the
    combine kernel: a 3-layer stack equals three 1-layer stacks bit for bit,
    and layers 1 and 2 match the oracle teacher-forced on every token."""
    layers = make_stack(pkg, dev, 3, 2048, 512, 32, seed=1500)
    T = 200
    x = pkg.synth.activations(T, 2048, 1501, dev)
    ids, w = routing(pkg, dev, 3, T, 32, 1502)
    out = pkg.moe_stack_prefill(layers, x, ids, w, EPS)
    r = x
    for L in range(3):
        nxt = pkg.moe_stack_prefill([layers[L]], r, ids[L:L + 1].contiguous(),
                                    w[L:L + 1].contiguous(), EPS)
        torch.cuda.synchronize()
        if L > 0:
            ref = _oracle_layer(layers[L], f16_bits(r), ids.cpu().numpy()[L], w.cpu().numpy()[L])
            assert_parity(f16_to_f32(nxt), oracle.f16_values(ref), what=f"fused stack layer {L}")
        r = nxt
    assert torch.equal(out, r)


# ---------------------------------------------------------------------------
# resident persistent decode (one launch for all layers)
# ---------------------------------------------------------------------------

def test_decode_plan_ring_matches_register_prefetch(pkg, dev, monkeypatch):
    """The weight-ring instance (the default for 128-wide groups: a streaming
    wave fills an LDS ring one layer ahead) and the register-prefetch
    instance (AIMA_DECODE_RING=0) run the same arithmetic on the same rows:
    bit-identical outputs, repeated runs, k = 8 and k = 3."""
    layers = make_stack(pkg, dev, 3, 2048, 512, 16, seed=990)
    monkeypatch.setenv("AIMA_DECODE_RING", "0")
    plain = {k: pkg.DecodePlan(layers, k=k) for k in (8, 3)}
    monkeypatch.delenv("AIMA_DECODE_RING")
    ring = {k: pkg.DecodePlan(layers, k=k) for k in (8, 3)}
    for rep in range(3):
        x = pkg.synth.activations(1, 2048, 991 + rep, dev)[0].contiguous()
        logits = torch.stack([pkg.synth.router_logits(1, 16, 995 + 10 * rep + l, dev)[0]
                              for l in range(3)])
        for k in (8, 3):
            a = plain[k].run(x, router_logits=logits)
            b = ring[k].run(x, router_logits=logits)
            torch.cuda.synchronize()
            assert plain[k].error_bits() == 0 and ring[k].error_bits() == 0
            assert torch.equal(a, b), (rep, k)


def test_decode_plan_small_stack(pkg, dev):
    """3 layers of the real width (16 experts): persistent kernel vs oracle,
    routing from logits and from explicit ids/weights; repeated runs (the
    per-launch epochs must never match stale words of an earlier launch)."""
    layers = make_stack(pkg, dev, 3, 2048, 512, 16, seed=900)
    lnp = [moe_to_oracle(l) for l in layers]
    norms = [l.norm_weight.cpu().numpy() for l in layers]
    plan = pkg.DecodePlan(layers, k=8)
    for rep in range(4):
        x = pkg.synth.activations(1, 2048, 60 + rep, dev)
        logits = torch.stack([pkg.synth.router_logits(1, 16, 70 + rep * 10 + l, dev)[0]
                              for l in range(3)])
        ids, w = pkg.select_router_topk(logits, 8)
        a = plan.run(x[0], router_logits=logits)
        b = plan.run(x[0], ids=ids, weights=w)
        torch.cuda.synchronize()
        assert plan.error_bits() == 0
        assert torch.equal(a, b)
        ref = oracle_stack(lnp, norms, f16_bits(x), ids.cpu().numpy()[:, None],
                           w.cpu().numpy()[:, None])
        assert_parity(f16_to_f32(a), oracle.f16_values(ref[0]), what=f"plan small rep={rep}")


@pytest.mark.parametrize("k", [8, 3])
def test_decode_plan_routes_match_select_router_topk(pkg, dev, k):
    """At 256 experts the plan ranks each layer's logits in its prologue and
    confirms the ranking on the probabilities; the result must be the
    routes of select_router_topk bit for bit: the plan run from logits
    equals the plan run on select_router_topk's ids and weights, also with
    tied logits (4 distinct values repeated) and with a run of equal top
    logits, where the probability ranking decides."""
    layers = make_stack(pkg, dev, 3, 2048, 512, 256, seed=1300 + k)
    plan = pkg.DecodePlan(layers, k=k)
    x = pkg.synth.activations(1, 2048, 1310 + k, dev)[0]
    base = torch.stack([pkg.synth.router_logits(1, 256, 1320 + k + l, dev)[0] for l in range(3)])
    tied = base.clone()
    tied[1] = base[1, torch.arange(256, device=dev) % 4]
    tied[2, 17:27] = tied[2].max() + 0.5
    for logits in (base, tied):
        ids, w = pkg.select_router_topk(logits, k)
        a = plan.run(x, router_logits=logits)
        b = plan.run(x, ids=ids, weights=w)
        torch.cuda.synchronize()
        assert plan.error_bits() == 0
        assert torch.equal(a, b)


@pytest.mark.parametrize("k", [1, 4])
def test_decode_plan_small_k(pkg, dev, k):
    """Fewer than 8 routed experts: the XCDs of the missing ranks compute only
    their shared-expert slice (2 layers of the real width vs the oracle)."""
    layers = make_stack(pkg, dev, 2, 2048, 512, 16, seed=1200 + k)
    lnp = [moe_to_oracle(l) for l in layers]
    norms = [l.norm_weight.cpu().numpy() for l in layers]
    plan = pkg.DecodePlan(layers, k=k)
    x = pkg.synth.activations(1, 2048, 95 + k, dev)
    logits = torch.stack([pkg.synth.router_logits(1, 16, 96 + k + l, dev)[0] for l in range(2)])
    ids, w = pkg.select_router_topk(logits, k)
    out = plan.run(x[0], router_logits=logits)
    torch.cuda.synchronize()
    assert plan.error_bits() == 0
    ref = oracle_stack(lnp, norms, f16_bits(x), ids.cpu().numpy()[:, None],
                       w.cpu().numpy()[:, None])
    assert_parity(f16_to_f32(out), oracle.f16_values(ref[0]), what=f"plan k={k}")


@pytest.mark.parametrize("group", [64, 256])
def test_decode_plan_other_groups(pkg, dev, group):
    """Group sizes other than 128 run the general kernel instance (per-row
    scale and zero-point loads): 2 layers of the real width vs the oracle."""
    layers = [pkg.synth.moe_layer(hidden=2048, inter=512, experts=16, group=group,
                                  seed=980 + l, device=dev) for l in range(2)]
    lnp = [moe_to_oracle(l) for l in layers]
    norms = [l.norm_weight.cpu().numpy() for l in layers]
    plan = pkg.DecodePlan(layers, k=8)
    x = pkg.synth.activations(1, 2048, 90, dev)
    logits = torch.stack([pkg.synth.router_logits(1, 16, 91 + l, dev)[0] for l in range(2)])
    ids, w = pkg.select_router_topk(logits, 8)
    out = plan.run(x[0], router_logits=logits)
    torch.cuda.synchronize()
    assert plan.error_bits() == 0
    ref = oracle_stack(lnp, norms, f16_bits(x), ids.cpu().numpy()[:, None],
                       w.cpu().numpy()[:, None])
    assert_parity(f16_to_f32(out), oracle.f16_values(ref[0]), what=f"plan group {group}")


def test_decode_plan_flags_bad_ids(pkg, dev):
    layers = make_stack(pkg, dev, 2, 2048, 512, 16, seed=950)
    plan = pkg.DecodePlan(layers, k=8)
    x = pkg.synth.activations(1, 2048, 1, dev)[0]
    ids = torch.arange(8, dtype=torch.int32, device=dev).repeat(2, 1).contiguous()
    ids[1, 3] = 40  # out of range for 16 experts
    w = torch.full((2, 8), 0.125, device=dev)
    out = plan.run(x, ids=ids, weights=w)
    torch.cuda.synchronize()
    bits = plan.error_bits()
    assert bits & pkg._lib.AIMA_DEVERR_EXPERT_RANGE and not bits & pkg._lib.AIMA_DEVERR_TIMEOUT
    assert torch.isfinite(out.float()).all()


def test_decode_plan_graph_replays(pkg, dev):
    """Captured once, replayed several times with eager work in between; every
    replay equals the eager result."""
    layers = make_stack(pkg, dev, 2, 2048, 512, 16, seed=960)
    plan = pkg.DecodePlan(layers, k=8)
    x = pkg.synth.activations(1, 2048, 5, dev)[0].contiguous()
    logits = torch.stack([pkg.synth.router_logits(1, 16, 80 + l, dev)[0] for l in range(2)])
    out = torch.empty(2048, dtype=torch.float16, device=dev)
    eager = plan.run(x, router_logits=logits).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run(x, router_logits=logits, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run(x, router_logits=logits, out=out)
    for _ in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        plan.run(x, router_logits=logits)  # eager work between replays
        torch.cuda.synchronize()
    assert plan.error_bits() == 0


def test_config4a_decode_plan_40_layers(pkg, dev, stack40):
    """The 40-layer persistent decode (one launch): every layer teacher-forced
    (1-layer plans on the oracle's inputs) at the 2e-3 bar; the 40-layer
    launch equals 40 chained 1-layer launches fed their own outputs, bit for
    bit (so the per-layer evidence holds for the fused launch's layers); the
    free-running result within the measured floor."""
    x = pkg.synth.activations(1, 2048, 141, dev)
    logits = torch.stack([pkg.synth.router_logits(1, 256, 2141 + l, dev)[0] for l in range(40)])
    ids, w = pkg.select_router_topk(logits, 8)
    plan = pkg.DecodePlan(stack40, k=8)
    out = plan.run(x[0], router_logits=logits)
    torch.cuda.synchronize()
    assert plan.error_bits() == 0
    ids_np, w_np = ids.cpu().numpy()[:, None], w.cpu().numpy()[:, None]
    mws, rids = compact_chain(stack40, ids_np)
    norms = [l.norm_weight.cpu().numpy() for l in stack40]
    r = f16_bits(x)
    chained = x[0].contiguous()
    for L, layer in enumerate(stack40):
        nxt = _oracle_layer(layer, r, rids[L], w_np[L], mw=mws[L])
        one = pkg.DecodePlan([layer], k=8)
        got = one.run(torch.from_numpy(r[0].view(np.float16)).to(dev), ids=ids[L:L + 1],
                      weights=w[L:L + 1])
        chained = one.run(chained, ids=ids[L:L + 1], weights=w[L:L + 1])
        torch.cuda.synchronize()
        assert one.error_bits() == 0
        assert_parity(f16_to_f32(got), oracle.f16_values(nxt[0]), what=f"plan layer {L}")
        one.close()
        r = nxt
    assert torch.equal(chained, out), "40-layer plan differs from 40 chained 1-layer plans"
    # the register-prefetch instance gives the same 40-layer result
    os.environ["AIMA_DECODE_RING"] = "0"
    try:
        plain = pkg.DecodePlan(stack40, k=8)
    finally:
        del os.environ["AIMA_DECODE_RING"]
    again = plain.run(x[0], router_logits=logits)
    torch.cuda.synchronize()
    assert plain.error_bits() == 0 and torch.equal(again, out)
    plain.close()
    chains = stack_chains(mws, norms, f16_bits(x), rids, w_np, EPS, oracle.MODEL_DECODE_PLAN,
                          THREADS)
    assert np.array_equal(chains["ref"], r)
    assert_end_to_end(f16_to_f32(out), chains, "plan 40-layer end-to-end")


def test_stack_decode_routed_true_decode(pkg, dev):
    """Routing from each layer's own normalized input (router U4 FC + top-k),
    teacher-forced per layer: a 1-layer routed call on the oracle's residual
    picks the oracle's routes (ids exact where the k-th / (k+1)-th logit gap
    exceeds the f32 rounding of the logits, weights at the 2e-3 bar) and its
    output matches the oracle layer on those routes at the 2e-3 bar; the
    3-layer call equals 3 chained 1-layer calls bit for bit."""
    nl, H, I, E, k = 3, 512, 128, 16, 8
    layers = make_stack(pkg, dev, nl, H, I, E, seed=1300)
    routers = [pkg.synth.u4_weight(1, E, H, 128, pkg.synth.generator(1400 + l, dev), dev)
               for l in range(nl)]
    x = pkg.synth.activations(1, H, 9, dev)[0]
    out, ids, w = pkg.moe_stack_decode_routed(layers, routers, x, k, epsilon=EPS)
    chained = x
    for l in range(nl):
        chained, il, wl = pkg.moe_stack_decode_routed([layers[l]], [routers[l]], chained, k,
                                                      epsilon=EPS)
        torch.cuda.synchronize()
        assert torch.equal(il[0], ids[l]) and torch.equal(wl[0], w[l])
    assert torch.equal(chained, out), "3-layer routed stack differs from chained 1-layer calls"
    lnp = [moe_to_oracle(l) for l in layers]
    norms = [l.norm_weight.cpu().numpy() for l in layers]
    r = f16_bits(x)[None]
    checked = 0
    for l in range(nl):
        rf = oracle.f16_values(r)
        h = oracle.f16_values(oracle.float_to_half(oracle.rms_norm_rows(rf, norms[l], EPS))
                              .reshape(rf.shape))
        o = u4_to_oracle(routers[l])
        logits = oracle.u4_matvec(o.qweight[0], o.scale[0], o.zp[0], E, H, h[0], group=128,
                                  threads=THREADS)
        rid, rw = oracle.router_topk_tokens(logits[None].astype(np.float32), k)
        got, gi, gw = pkg.moe_stack_decode_routed(
            [layers[l]], [routers[l]], torch.from_numpy(r[0].view(np.float16)).to(dev), k,
            epsilon=EPS)
        torch.cuda.synchronize()
        gi, gw = gi.cpu().numpy(), gw.cpu().numpy()
        srt = np.sort(logits)[::-1]
        if srt[k - 1] - srt[k] > 1e-4 * max(1.0, abs(srt[k - 1])):
            assert np.array_equal(gi[0], rid[0]), l
            assert_parity(gw[0], rw[0], what=f"routed stack weights layer {l}")
            checked += 1
        dev_ref = oracle.moe_ffn_tokens(lnp[l], h, gi, gw, residual=rf, threads=THREADS)
        assert_parity(f16_to_f32(got), oracle.f16_values(oracle.float_to_half(dev_ref)),
                      what=f"routed stack layer {l}")
        o2 = oracle.moe_ffn_tokens(lnp[l], h, rid, rw, residual=rf, threads=THREADS)
        r = oracle.float_to_half(o2).reshape(o2.shape)
    assert checked >= 2
