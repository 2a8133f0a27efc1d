"""GPU parity for true decode inside the resident plan (DecodePlan with
routers): every layer routes from its own normalized input in the same
persistent launch, as run_qwen36_moe_ffn_layer does per layer
(gguf_loader.cpp:5704-5711: ffn_norm -> router FC -> select_router_topk ->
experts).

Evidence, per run:
  * the selection is bit-exact: the oracle's select_router_topk on the
    plan's own logits gives the plan's ids (and weights within 1e-6, the
    f64 exp of the device library against the host's);
  * the logits are within 2e-3 of the oracle's U4 FC on the oracle's
    normalized input (layer 0 starts from the same residual; later layers
    from the oracle stack fed the plan's routes);
  * the output equals, bit for bit, the logits-fed plan run on the plan's
    own routes (same kernel arithmetic, the route source aside), and the
    oracle stack on those routes at the 2e-3 bar."""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_bits, f16_to_f32, moe_to_oracle, u4_to_oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)
EPS = 1e-6


def _stack(pkg, dev, n, E, seed, group=128):
    return [pkg.synth.moe_layer(hidden=2048, inter=512, experts=E, group=group, seed=seed + l,
                                device=dev) for l in range(n)]


def _routers(pkg, dev, n, E, seed, group=128):
    return [pkg.synth.u4_weight(1, E, 2048, group, pkg.synth.generator(seed + l, dev), dev)
            for l in range(n)]


def _check_routes(pkg, layers, routers, x, routes, k, group, n_check=None):
    """Selection exact on the plan's logits; logits against the oracle's FC
    on the oracle's h (stack fed the plan's routes).  Returns the oracle's
    final residual bits when every layer was stepped."""
    ids = routes.expert_ids.cpu().numpy()
    w = routes.weights.cpu().numpy()
    lg = routes.logits.cpu().numpy()
    L, E = lg.shape
    ref_ids, ref_w = oracle.router_topk_tokens(lg, k)
    assert np.array_equal(ids, ref_ids), (ids, ref_ids)
    assert_parity(w, ref_w, tol=1e-6, what="plan router weights")
    r = f16_bits(x)[None]
    n_check = L if n_check is None else n_check
    for l in range(n_check):
        lay = layers[l]
        rf = oracle.f16_values(r)
        h = oracle.f16_values(oracle.float_to_half(
            oracle.rms_norm_rows(rf, lay.norm_weight.cpu().numpy(), EPS)).reshape(rf.shape))
        ro = u4_to_oracle(routers[l])
        want = oracle.u4_matvec(ro.qweight[0], ro.scale[0], ro.zp[0], E, 2048, h[0],
                                group=group, threads=THREADS)
        assert_parity(lg[l], want, what=f"plan router logits layer {l}")
        if l + 1 < n_check or n_check == L:
            used, inv = np.unique(ids[l], return_inverse=True)
            mw = _compact(lay, used)
            o = oracle.moe_ffn_tokens(mw, h, inv.reshape(1, k).astype(np.int32), w[l:l + 1],
                                      residual=rf, threads=THREADS)
            r = oracle.float_to_half(o).reshape(o.shape)
    return r


def _compact(layer, used):
    idx = torch.as_tensor(np.asarray(used, np.int64), device=layer.gate_up.qweight.device)

    def pick(t):
        sub = type(t)(t.qweight.index_select(0, idx).contiguous(),
                      t.scale.index_select(0, idx).contiguous(),
                      t.zp.index_select(0, idx).contiguous(), t.rows, t.k, t.group)
        return u4_to_oracle(sub)

    return oracle.MoeWeights(pick(layer.gate_up), pick(layer.down),
                             u4_to_oracle(layer.shared_gate_up), u4_to_oracle(layer.shared_down),
                             f16_bits(layer.shared_gate_vec))


@pytest.mark.parametrize("k,group", [(8, 128), (4, 64)])
def test_routed_plan_small_stack(pkg, dev, k, group):
    """3 layers of the real width, 16 experts, repeated runs interleaved with
    logits-fed runs (per-launch epochs never match an earlier launch)."""
    n, E = 3, 16
    layers = _stack(pkg, dev, n, E, 1500 + k, group)
    routers = _routers(pkg, dev, n, E, 1600 + k, group)
    plan = pkg.DecodePlan(layers, k=k, routers=routers)
    for rep in range(3):
        x = pkg.synth.activations(1, 2048, 1700 + rep, dev)[0].contiguous()
        routes = plan.route_buffers()
        out = plan.run(x, routers=routers, route_out=routes)
        fed = plan.run(x, ids=routes.expert_ids, weights=routes.weights)
        torch.cuda.synchronize()
        assert plan.error_bits() == 0
        assert torch.equal(out, fed)
        ref = _check_routes(pkg, layers, routers, x, routes, k, group)
        assert_parity(f16_to_f32(out), oracle.f16_values(ref[0]),
                      what=f"routed plan k={k} g={group} rep={rep}")
    # without route_out the result is the same
    again = plan.run(x, routers=routers)
    torch.cuda.synchronize()
    assert torch.equal(again, out)


def test_routed_plan_ties(pkg, dev):
    """Routers whose 16 rows are 4 distinct rows repeated: every logit ties
    with three others, and the selection must take equal probabilities in
    id order (the oracle on the plan's logits, exact)."""
    n, E, k = 2, 16, 8
    layers = _stack(pkg, dev, n, E, 1750)
    routers = []
    for l, r in enumerate(_routers(pkg, dev, n, E, 1760)):
        idx = torch.arange(E, device=dev) % 4
        G = r.scale.shape[-1]
        zp = r.zp.view(E, G // 2)[idx].reshape(-1).contiguous()
        routers.append(type(r)(r.qweight[idx].contiguous(), r.scale[idx].contiguous(), zp,
                               r.rows, r.k, r.group))
    plan = pkg.DecodePlan(layers, k=k, routers=routers)
    x = pkg.synth.activations(1, 2048, 1770, dev)[0].contiguous()
    routes = plan.route_buffers()
    out = plan.run(x, routers=routers, route_out=routes)
    torch.cuda.synchronize()
    assert plan.error_bits() == 0
    lg = routes.logits.cpu().numpy()
    assert all(len(np.unique(row)) <= 4 for row in lg)
    ref = _check_routes(pkg, layers, routers, x, routes, k, 128)
    assert_parity(f16_to_f32(out), oracle.f16_values(ref[0]), what="routed plan ties")


def test_routed_plan_graph_replays(pkg, dev):
    """Captured once, replayed with eager work in between: every replay equals
    the eager routed run, routes included."""
    n, E = 2, 16
    layers = _stack(pkg, dev, n, E, 1800)
    routers = _routers(pkg, dev, n, E, 1810)
    plan = pkg.DecodePlan(layers, k=8, routers=routers)
    x = pkg.synth.activations(1, 2048, 1820, dev)[0].contiguous()
    eager_routes = plan.route_buffers()
    eager = plan.run(x, routers=routers, route_out=eager_routes).clone()
    routes = plan.route_buffers()
    out = torch.empty(2048, dtype=torch.float16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run(x, routers=routers, route_out=routes, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        plan.run(x, routers=routers, route_out=routes, out=out)
    for _ in range(3):
        out.zero_()
        routes.expert_ids.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(routes.expert_ids, eager_routes.expert_ids)
        assert torch.equal(routes.logits, eager_routes.logits)
        plan.run(x, ids=eager_routes.expert_ids, weights=eager_routes.weights)
        torch.cuda.synchronize()
    assert plan.error_bits() == 0


def test_routed_plan_rejects_misuse(pkg, dev):
    layers = _stack(pkg, dev, 2, 16, 1900)
    plan = pkg.DecodePlan(layers, k=8)
    x = pkg.synth.activations(1, 2048, 1, dev)[0].contiguous()
    with pytest.raises(ValueError):
        plan.run(x, route_out=plan.route_buffers())  # no routers registered
    bad = _routers(pkg, dev, 2, 8, 1910)  # 8 experts for a 16-expert layer
    with pytest.raises(ValueError):
        plan.run(x, routers=bad)
    routers = _routers(pkg, dev, 2, 16, 1920)
    with pytest.raises(ValueError):
        plan.run(x, routers=routers, router_logits=torch.zeros((2, 16), device=dev))


@pytest.fixture(scope="module")
def stack40r(pkg, dev):
    layers = _stack(pkg, dev, 40, 256, 4000)
    routers = _routers(pkg, dev, 40, 256, 5000)
    yield layers, routers
    del layers, routers
    torch.cuda.empty_cache()


def test_config4a_routed_plan_40_layers(pkg, dev, stack40r):
    """The headline shape with true decode: 40 layers x 256 experts, k = 8.
    Every layer's selection exact on its logits and equal to the logits-fed
    plan on the same routes; logits of the first 3 layers against the
    oracle's FC; the fused launch equal to 40 chained 1-layer launches."""
    layers, routers = stack40r
    plan = pkg.DecodePlan(layers, k=8, routers=routers)
    x = pkg.synth.activations(1, 2048, 4141, dev)[0].contiguous()
    routes = plan.route_buffers()
    out = plan.run(x, routers=routers, route_out=routes)
    fed = plan.run(x, ids=routes.expert_ids, weights=routes.weights)
    torch.cuda.synchronize()
    assert plan.error_bits() == 0
    assert torch.equal(out, fed)
    _check_routes(pkg, layers, routers, x, routes, 8, 128, n_check=3)
    # distinct experts per layer, all in range
    ids = routes.expert_ids.cpu().numpy()
    assert ((ids >= 0) & (ids < 256)).all()
    assert all(len(set(row)) == 8 for row in ids)
    # the 40-layer launch equals 40 chained 1-layer routed launches fed their
    # own outputs, routes and logits included, bit for bit
    chained = x
    for l in range(40):
        one = pkg.DecodePlan([layers[l]], k=8, routers=[routers[l]])
        rl = one.route_buffers()
        chained = one.run(chained, routers=[routers[l]], route_out=rl)
        torch.cuda.synchronize()
        assert one.error_bits() == 0
        assert torch.equal(rl.expert_ids[0], routes.expert_ids[l]), l
        assert torch.equal(rl.weights[0], routes.weights[l]), l
        assert torch.equal(rl.logits[0], routes.logits[l]), l
        one.close()
    assert torch.equal(chained, out), "40-layer routed plan differs from chained 1-layer plans"
