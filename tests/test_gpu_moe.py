"""GPU parity for the MoE FFN: batch-1 decode (config 1), the device grouped
schedule (bit-exact), the grouped prefill (config 2) and small edge cases."""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_to_f32, moe_to_oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)


@pytest.fixture(scope="module")
def layer_full(pkg, dev):
    """Config 1/2 layer: H=2048, 256 routed experts, I=512, shared I=512, group 128."""
    layer = pkg.synth.moe_layer(hidden=2048, inter=512, experts=256, seed=1, device=dev)
    return layer, moe_to_oracle(layer)


@pytest.fixture(scope="module")
def layer_small(pkg, dev):
    layer = pkg.synth.moe_layer(hidden=512, inter=128, experts=16, seed=21, device=dev)
    return layer, moe_to_oracle(layer)


def _decode(pkg, dev, layer, mw, seed, residual=True, k=8):
    H, E = layer.hidden, layer.experts
    x = pkg.synth.activations(1, H, seed, dev)[0]
    logits = pkg.synth.router_logits(1, E, seed + 1, dev)
    ids, w = pkg.select_router_topk(logits, k)
    res = pkg.synth.activations(1, H, seed + 2, dev)[0] if residual else None
    out = pkg.run_moe_ffn_layer(layer, x, ids[0].contiguous(), w[0].contiguous(), residual=res)
    torch.cuda.synchronize()
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x)[None], ids.cpu().numpy(), w.cpu().numpy(),
                                residual=None if res is None else f16_to_f32(res)[None],
                                threads=1)
    return f16_to_f32(out), ref[0]


def test_config1_decode(pkg, dev, layer_full):
    layer, mw = layer_full
    for seed in (0, 10, 20):
        got, ref = _decode(pkg, dev, layer, mw, seed)
        assert_parity(got, ref, what=f"config1 seed={seed}")


def test_decode_without_residual(pkg, dev, layer_full):
    layer, mw = layer_full
    got, ref = _decode(pkg, dev, layer, mw, 5, residual=False)
    assert_parity(got, ref, what="no residual")


@pytest.mark.parametrize("k", [1, 4, 8, 16])
def test_decode_small_topk(pkg, dev, layer_small, k):
    layer, mw = layer_small
    got, ref = _decode(pkg, dev, layer, mw, 30 + k, k=k)
    assert_parity(got, ref, what=f"small k={k}")


@pytest.mark.parametrize("k", [23, 24, 40])
def test_decode_wide_topk(pkg, dev, k):
    """k + 1 > 24 slots: the down phase takes its slots in several batches."""
    layer = pkg.synth.moe_layer(hidden=512, inter=128, experts=40, seed=23, device=dev)
    g = np.random.default_rng(50 + k)
    ids = g.permutation(40)[:k].astype(np.int32)[None]  # router top-k stops at 16
    w = g.random(k).astype(np.float32)
    w = (w / w.sum())[None]
    x = pkg.synth.activations(1, 512, 51 + k, dev)[0]
    res = pkg.synth.activations(1, 512, 52 + k, dev)[0]
    out = pkg.run_moe_ffn_layer(layer, x, torch.from_numpy(ids[0]).to(dev),
                                torch.from_numpy(w[0]).to(dev), residual=res)
    torch.cuda.synchronize()
    ref = oracle.moe_ffn_tokens(moe_to_oracle(layer), f16_to_f32(x)[None], ids, w,
                                residual=f16_to_f32(res)[None], threads=1)
    assert_parity(f16_to_f32(out), ref[0], what=f"wide k={k}")


def test_decode_flags_bad_expert_id(pkg, dev, layer_small):
    layer, _ = layer_small
    ws = pkg.Workspace(dev)
    x = pkg.synth.activations(1, layer.hidden, 1, dev)[0]
    ids = torch.tensor([0, 1, 2, 3, 4, 5, 6, 99], dtype=torch.int32, device=dev)
    w = torch.full((8,), 0.125, device=dev)
    out = pkg.run_moe_ffn_layer(layer, x, ids, w, ws=ws)
    torch.cuda.synchronize()
    assert ws.error_bits() & pkg._lib.AIMA_DEVERR_EXPERT_RANGE
    assert torch.isfinite(out.float()).all()
    assert ws.error_bits() == 0  # reading clears the word


# ---------------------------------------------------------------------------
# grouped schedule
# ---------------------------------------------------------------------------

# (1024, 1024, 16): the largest expert count and k, 16 chunks of 1024
# assignments; (2049, 256, 8): a partial last chunk of 8 assignments.
@pytest.mark.parametrize("T,E,k,zipf", [(2048, 256, 8, 1.1), (1, 256, 8, None),
                                        (37, 16, 8, None), (1000, 64, 6, None),
                                        (16384, 256, 8, None), (2049, 256, 8, 1.1),
                                        (1024, 1024, 16, 1.1), (1025, 1024, 16, None),
                                        (3, 1024, 16, None)])
def test_schedule_bit_exact(pkg, dev, T, E, k, zipf):
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, E, seed=T, device=dev,
                                                            zipf_s=zipf), k)
    s = pkg.build_grouped_schedule(ids, w, E)
    torch.cuda.synchronize()
    r = oracle.build_grouped_schedule(ids.cpu().numpy(), E, w.cpu().numpy())
    for name in ("offsets", "token_map", "inverse_map", "compact_weights"):
        assert np.array_equal(s[name].cpu().numpy(), r[name]), name


def test_schedule_flags_errors(pkg, dev):
    ws = pkg.Workspace(dev)
    ids = torch.tensor([[0, 1, 2, 3], [4, 5, 6, 4]], dtype=torch.int32, device=dev)
    w = torch.ones((2, 4), device=dev)
    pkg.build_grouped_schedule(ids, w, 8, ws=ws)
    assert ws.error_bits() == pkg._lib.AIMA_DEVERR_EXPERT_DUPLICATE
    ids = torch.tensor([[0, 1, 2, 8]], dtype=torch.int32, device=dev)
    pkg.build_grouped_schedule(ids, torch.ones((1, 4), device=dev), 8, ws=ws)
    assert ws.error_bits() & pkg._lib.AIMA_DEVERR_EXPERT_RANGE


@pytest.mark.parametrize("T", [200, 3000])
def test_schedule_flags_duplicate_across_chunks(pkg, dev, T):
    """At k = 6, token 170 holds assignments 1020..1025, across the boundary of
    the 1024-assignment blocks of the schedule.  A duplicate between its rank
    0 and rank 5 (in different blocks) is flagged, with 2 blocks (T = 200) and
    18 (T = 3000); a clean routing flags nothing and ranks as the oracle."""
    ws = pkg.Workspace(dev)
    g = torch.Generator(device="cpu")
    g.manual_seed(T)
    ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(T)]).to(torch.int32)
    ids = ids.to(dev)
    w = torch.ones((T, 6), device=dev)
    s = pkg.build_grouped_schedule(ids, w, 64, ws=ws)
    torch.cuda.synchronize()
    assert ws.error_bits() == 0
    r = oracle.build_grouped_schedule(ids.cpu().numpy(), 64, w.cpu().numpy())
    assert np.array_equal(s["token_map"].cpu().numpy(), r["token_map"])
    bad = ids.clone()
    bad[170, 5] = bad[170, 0]
    pkg.build_grouped_schedule(bad, w, 64, ws=ws)
    assert ws.error_bits() == pkg._lib.AIMA_DEVERR_EXPERT_DUPLICATE


# ---------------------------------------------------------------------------
# grouped prefill
# ---------------------------------------------------------------------------

def _prefill(pkg, dev, layer, mw, T, seed, zipf=None, residual=False, k=8, tokens=None):
    H, E = layer.hidden, layer.experts
    x = pkg.synth.activations(T, H, seed, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, E, seed + 1, dev, zipf_s=zipf), k)
    res = pkg.synth.activations(T, H, seed + 2, dev) if residual else None
    out = pkg.grouped_moe_prefill(layer, x, ids, w, residual=res)
    torch.cuda.synchronize()
    sel = np.arange(T) if tokens is None else np.asarray(tokens)
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x)[sel], ids.cpu().numpy()[sel],
                                w.cpu().numpy()[sel],
                                residual=None if res is None else f16_to_f32(res)[sel],
                                threads=THREADS)
    return f16_to_f32(out)[sel], ref


def test_config2_prefill(pkg, dev, layer_full):
    """T=2048, Zipf(1.1)-skewed routing, every token against the oracle."""
    layer, mw = layer_full
    got, ref = _prefill(pkg, dev, layer, mw, 2048, seed=2, zipf=1.1)
    assert_parity(got, ref, what="config2")


def test_prefill_uniform_routing_residual(pkg, dev, layer_full):
    layer, mw = layer_full
    got, ref = _prefill(pkg, dev, layer, mw, 512, seed=40, residual=True)
    assert_parity(got, ref, what="uniform+residual")


@pytest.mark.parametrize("T", [1, 2, 37, 129, 300])
def test_prefill_ragged(pkg, dev, layer_small, T):
    layer, mw = layer_small
    got, ref = _prefill(pkg, dev, layer, mw, T, seed=T, residual=(T % 2 == 1))
    assert_parity(got, ref, what=f"ragged T={T}")


def test_prefill_all_tokens_same_experts(pkg, dev, layer_small):
    """Every token routes to experts 0..7: a few maximal groups, most empty."""
    layer, mw = layer_small
    T = 333
    x = pkg.synth.activations(T, layer.hidden, 9, dev)
    ids = torch.arange(8, dtype=torch.int32, device=dev).repeat(T, 1).contiguous()
    w = torch.full((T, 8), 0.125, device=dev)
    out = pkg.grouped_moe_prefill(layer, x, ids, w)
    torch.cuda.synchronize()
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x), ids.cpu().numpy(), w.cpu().numpy(),
                                threads=THREADS)
    assert_parity(f16_to_f32(out), ref, what="same experts")


def test_prefill_matches_decode(pkg, dev, layer_small):
    """One token through the grouped path equals the decode path's result."""
    layer, _ = layer_small
    x = pkg.synth.activations(1, layer.hidden, 77, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(1, 16, 78, dev), 8)
    a = pkg.grouped_moe_prefill(layer, x, ids, w)[0]
    b = pkg.run_moe_ffn_layer(layer, x[0], ids[0].contiguous(), w[0].contiguous())
    torch.cuda.synchronize()
    assert_parity(f16_to_f32(a), f16_to_f32(b), tol=2e-3, what="prefill vs decode")


def test_prefill_runtime_contract(pkg, dev, layer_small):
    layer, mw = layer_small
    rt = pkg.GroupedU4PrefillRuntime(dev)
    h = rt.LoadLayer(layer)
    T = 200
    x = pkg.synth.activations(T, layer.hidden, 5, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, 16, 6, dev), 8)
    run = rt.RunLayer(h, pkg.GroupedU4PrefillInput(x, ids, w, warmup=1, repeat=3,
                                                   capture_intermediates=True,
                                                   include_shared=True))
    assert len(run.timing.samples_us) == 3 and run.timing.minimum_us > 0
    assert run.active_experts > 0 and run.max_group_size > 0
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x), ids.cpu().numpy(), w.cpu().numpy(),
                                threads=THREADS)
    assert_parity(f16_to_f32(run.output), ref, what="runtime")
    st = rt.stats()
    assert st["run_count"] == 1 and st["layer_count"] == 1
    with pytest.raises(KeyError):
        rt.RunLayer(99, pkg.GroupedU4PrefillInput(x, ids, w, include_shared=True))


def test_decode_phases_compose(pkg, dev, layer_full):
    """gate_up then down == the one-call decode (same kernels, same order)."""
    layer, _ = layer_full
    x = pkg.synth.activations(1, 2048, 91, dev)[0]
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(1, 256, 92, dev), 8)
    ids, w = ids[0].contiguous(), w[0].contiguous()
    res = pkg.synth.activations(1, 2048, 93, dev)[0]
    act, sigma = pkg.moe_decode_gate_up(layer, x, ids)
    a = pkg.moe_decode_down(layer, act, sigma, ids, w, residual=res)
    b = pkg.run_moe_ffn_layer(layer, x, ids, w, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # the activations themselves against the oracle's SwiGLU (f32 -> f16 rounding)
    mw = moe_to_oracle(layer)
    d = oracle.moe_ffn_token_detail(mw, f16_to_f32(x), None, ids.cpu().numpy(),
                                    w.cpu().numpy())
    ref_act = np.concatenate([d["selected_swiglu"], d["shared_swiglu"]]).reshape(9, 512)
    assert_parity(f16_to_f32(act), ref_act, what="decode SwiGLU activations")
    assert abs(float(sigma.item()) - float(d["shared_gate"][1])) < 1e-5


def test_prefill_largest_batch(pkg, dev, layer_full):
    """T = 233016, the largest batch whose row offsets stay below 2^31 bytes
    (tokens * (k + 1) * inter < 2^30 f16 elements at k = 8, inter = 512):
    every token finite, sampled tokens against the oracle."""
    layer, mw = layer_full
    T = 233016
    x = pkg.synth.activations(T, 2048, 77, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, 256, 78, dev), 8)
    out = pkg.grouped_moe_prefill(layer, x, ids, w)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    sel = torch.tensor([0, 1, 116508, T - 2, T - 1], device=dev)
    got = f16_to_f32(out[sel])
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x[sel]), ids[sel].cpu().numpy(),
                                w[sel].cpu().numpy(), threads=THREADS)
    assert_parity(got, ref, what="largest batch")
    del out, x
