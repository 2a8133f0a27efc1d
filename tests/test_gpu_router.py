"""GPU parity for the batched router (the grouped prefill's native router,
grouped_s8_u4_prefill_runtime.cpp:1085-1101): f32 logits of every token
against a float64 product (the GEMM pinned by the mathematics: a different
f32 summation order moves a logit by ~1e-7 relative), the selection bit-exact
against the oracle's select_router_topk on the GPU's own logits, and the
runtime's native_router run equal to a run fed those routes."""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity

pytestmark = pytest.mark.gpu


def _router(E, H, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return (torch.randn((E, H), generator=g, device=dev) * 0.05).contiguous()


@pytest.mark.parametrize("T,E,k,H", [(300, 256, 8, 2048), (1, 256, 8, 2048),
                                     (2048, 256, 8, 2048), (77, 16, 4, 2048),
                                     (33, 100, 8, 528)])
def test_router_gemm_topk(pkg, dev, T, E, k, H):
    """Tiles of 64 tokens x 64 experts: partial tiles in both dimensions
    (T = 1, 33, 77, 300; E = 16, 100) and a hidden size whose K halves are
    not a multiple of the 64-wide steps (528)."""
    x = pkg.synth.activations(T, H, T + E, dev).float()
    W = _router(E, H, T + 1, dev)
    ids, w, logits = pkg.router_gemm_topk(x, W, k)
    torch.cuda.synchronize()
    ref = (x.double().cpu().numpy() @ W.double().cpu().numpy().T)
    got = logits.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    ref_ids, ref_w = oracle.router_topk_tokens(got, k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert_parity(w.cpu().numpy(), ref_w, tol=1e-6, what="router weights")


def test_router_gemm_f16_input(pkg, dev):
    """An f16 input is widened exactly: the same logits as its f32 copy."""
    T, H, E = 129, 2048, 256
    x16 = pkg.synth.activations(T, H, 5, dev)
    W = _router(E, H, 6, dev)
    a = pkg.router_gemm_topk(x16, W, 8)
    b = pkg.router_gemm_topk(x16.float(), W, 8)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_run_layer_native_router(pkg, dev):
    """RunLayer(native_router) == RunLayer fed the batched router's routes,
    bit for bit; sampled tokens match the oracle's routed sum."""
    layer = pkg.synth.moe_layer(hidden=2048, inter=512, experts=256, seed=8, device=dev)
    T, k = 512, 8
    x = pkg.synth.activations(T, 2048, 9, dev).float()
    W = _router(256, 2048, 10, dev)
    rt = pkg.GroupedU4PrefillRuntime(dev)
    h = rt.LoadLayer(layer, router_weight=W)
    native = rt.RunLayer(h, pkg.GroupedU4PrefillInput(x, None, None, native_router=True,
                                                      warmup=1, repeat=3))
    ids, w, _ = pkg.router_gemm_topk(x, W, k)
    fed = rt.RunLayer(h, pkg.GroupedU4PrefillInput(x, ids, w.reshape(-1)))
    torch.cuda.synchronize()
    assert native.native_router and not fed.native_router
    assert torch.equal(native.output, fed.output)
    assert len(native.timing.stage_us) == 5 and all(s > 0 for s in native.timing.stage_us)
    assert rt.stats()["native_router_run_count"] == 1
    sel = np.array([0, 1, 255, 511])
    from tests.helpers import moe_to_oracle
    ref = oracle.moe_routed_tokens(moe_to_oracle(layer), x.cpu().numpy()[sel],
                                   ids.cpu().numpy()[sel], w.cpu().numpy()[sel], threads=4)
    assert_parity(native.output.cpu().numpy()[sel], ref, what="native router RunLayer")
    with pytest.raises(ValueError):
        rt2 = pkg.GroupedU4PrefillRuntime(dev)
        rt2.RunLayer(rt2.LoadLayer(layer), pkg.GroupedU4PrefillInput(x, None, None,
                                                                    native_router=True))
