"""GPU parity for the decode-layer trace (ffn_layer_trace): every field of
the Qwen36MoeFfnLayerResult / RouterTopKSelection counterpart
(gguf_loader.hpp:138-161) against the oracle's restatement of
run_qwen36_moe_ffn_layer (gguf_loader.cpp:5654-5782).

Each stage is checked teacher-forced: the oracle stage runs on the GPU's own
input to that stage, so a mismatch names the stage.  Float stages are held
to the 2e-3 bar; the selection ids and the elementwise sums (weighting,
rank-order aggregate, gating, ffn_out) are exact."""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_to_f32, moe_to_oracle, u4_to_oracle

pytestmark = pytest.mark.gpu
EPS = 1e-6


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("shape", [(2048, 512, 256, 8), (512, 128, 16, 4)])
def test_ffn_layer_trace_matches_oracle_stages(pkg, dev, shape):
    H, I, E, k = shape
    layer = pkg.synth.moe_layer(hidden=H, inter=I, experts=E, seed=H + E, device=dev)
    mw = moe_to_oracle(layer)
    router = pkg.synth.u4_weight(1, E, H, 128, pkg.synth.generator(H + 7, dev), dev)
    ro = u4_to_oracle(router)
    residual = pkg.synth.activations(1, H, H + 3, dev)[0]
    r = pkg.ffn_layer_trace(layer, router, residual, EPS, k)
    torch.cuda.synchronize()
    res32 = f16_to_f32(residual)

    # ffn_norm: the GPU rounds the normalized input to f16 (the decode input)
    norm_ref = oracle.rms_norm(res32, _np(layer.norm_weight), EPS)
    x = f16_to_f32(r.ffn_norm)
    assert_parity(x, norm_ref, what="ffn_norm")

    # router logits on the GPU's ffn_norm, then the selection on its logits
    logits = _np(r.router_logits)
    assert_parity(logits, oracle.u4_matvec(ro.qweight[0], ro.scale[0], ro.zp[0], E, H, x),
                  what="router_logits")
    ids_ref, w_ref, nw_ref = oracle.select_router_topk(logits, k)
    ids = _np(r.router.expert_ids)
    assert np.array_equal(ids, ids_ref), (ids, ids_ref)
    assert_parity(_np(r.router.weights), w_ref, tol=1e-6, what="router weights")
    assert_parity(_np(r.router.normalized_weights), nw_ref, tol=1e-6, what="normalized weights")

    # the expert stages on the GPU's input and route
    nw = _np(r.router.normalized_weights)
    d = oracle.moe_ffn_token_detail(mw, x, res32, ids, nw)
    assert_parity(_np(r.selected_gate_up), d["selected_gate_up"], what="selected_gate_up")
    assert_parity(f16_to_f32(r.selected_swiglu), d["selected_swiglu"], what="selected_swiglu")
    assert_parity(_np(r.shared_gate_up), d["shared_gate_up"], what="shared_gate_up")
    assert_parity(f16_to_f32(r.shared_swiglu), d["shared_swiglu"], what="shared_swiglu")
    assert_parity(_np(r.shared_gate), d["shared_gate"][:1], what="shared_gate")
    assert_parity(_np(r.shared_gate_sigmoid), d["shared_gate"][1:], what="shared_gate_sigmoid")
    # down: the oracle takes the GPU's f16 activations as its input
    sel_down = np.concatenate([
        oracle.u4_matvec(mw.down.qweight[e], mw.down.scale[e], mw.down.zp[e], H, I,
                         f16_to_f32(r.selected_swiglu)[j * I:(j + 1) * I])
        for j, e in enumerate(ids)])
    assert_parity(_np(r.selected_down), sel_down, what="selected_down")
    sh_down = oracle.u4_matvec(mw.shared_down.qweight[0], mw.shared_down.scale[0],
                               mw.shared_down.zp[0], H, I, f16_to_f32(r.shared_swiglu))
    assert_parity(_np(r.shared_down), sh_down, what="shared_down")

    # elementwise sums: exact against the oracle's restatement on the GPU's rows
    weighted = oracle.apply_expert_weights(_np(r.selected_down), nw, H)
    assert np.array_equal(_np(r.weighted_selected_down), weighted)
    moe = oracle.aggregate_experts(weighted, k, H)
    assert np.array_equal(_np(r.moe_out), moe)
    gated = (_np(r.shared_down) * _np(r.shared_gate_sigmoid)[0]).astype(np.float32)
    assert np.array_equal(_np(r.shared_gated), gated)
    assert np.array_equal(_np(r.ffn_out), (moe + gated).astype(np.float32))
    # the complete layer: against the oracle's chain, and bit for bit the
    # product decode on the same input and route
    assert_parity(_np(r.ffn_out), d["ffn_out"], what="ffn_out")
    assert_parity(f16_to_f32(r.residual), d["residual"], what="residual")
    out = pkg.run_moe_ffn_layer(layer, r.ffn_norm, r.router.expert_ids,
                                r.router.normalized_weights, residual=residual)
    torch.cuda.synchronize()
    assert torch.equal(out, r.residual)


def test_ffn_layer_trace_rejects_bad_router(pkg, dev):
    layer = pkg.synth.moe_layer(hidden=512, inter=128, experts=16, seed=3, device=dev)
    bad = pkg.synth.u4_weight(1, 8, 512, 128, pkg.synth.generator(1, dev), dev)
    residual = pkg.synth.activations(1, 512, 1, dev)[0]
    with pytest.raises(ValueError):
        pkg.ffn_layer_trace(layer, bad, residual)
