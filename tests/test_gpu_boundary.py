"""GPU parity of the drop-in boundary forms.

* the f16 MFMA weight operand of the grouped GEMM (aima_u4_dequant_f16, the
  same dequant8 routine): bit-exact f16(f32(q - z) * f32(s)) for EVERY finite
  f16 scale, q and z;
* small group scales (down into the f16 subnormals) through the grouped
  prefill at the config-2 shape and through the decode layer;
* RunLayer's contract (aima_moe_grouped_prefill_ex): f32 routed-only output,
  int32 top-k at a byte stride, f32 hidden states;
* the split gate / up tensors of MOE3GemmFusedCompressed in every MoE entry
  point: bit-identical to the concatenated form, and against the oracle.
"""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_bits, f16_to_f32, moe_to_oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)


def test_dequant_f16_exhaustive(pkg, dev):
    """Row r has scale bits finite[r] in all 16 groups; group g has zero
    point g and element kk of a group the code kk % 16, so every (q, z, s)
    with s any finite f16 appears 8 times."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = bits[np.isfinite(bits.view(np.float16))]
    n, K, G = finite.size, 2048, 16
    assert n == 63488
    codes = np.arange(K) % 16
    row_q = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)          # [K/2]
    qweight = torch.from_numpy(np.tile(row_q, (n, 1))).to(dev)
    scale = torch.from_numpy(np.repeat(finite[:, None], G, axis=1).view(np.int16)).to(dev)
    zrow = np.arange(G)
    zrow = (zrow[0::2] | (zrow[1::2] << 4)).astype(np.uint8)              # [G/2]
    zp = torch.from_numpy(np.tile(zrow, n)).to(dev)
    w = pkg.U4Weight(qweight, scale.view(torch.float16), zp, n, K, 128)
    got = f16_bits(pkg.u4_dequant_f16(w))                                # [n][K]
    torch.cuda.synchronize()
    # the mathematics: (q - z) * s is exact in f32; numpy rounds to nearest even
    q = (np.arange(K) % 128) % 16
    z = np.arange(K) // 128
    s = finite.view(np.float16).astype(np.float32)
    exp = ((q - z).astype(np.float32)[None, :] * s[:, None]).astype(np.float16).view(np.uint16)
    bad = np.argwhere(got != exp)
    assert bad.size == 0, f"{len(bad)} mismatches, first (row, k) {bad[:4].tolist()}"
    # and the oracle's f32 dequantization rounded to f16, on every 8th row
    sub = slice(0, n, 8)
    ref = oracle.u4_dequant(qweight[sub].cpu().numpy(), scale[sub].cpu().numpy().view(np.uint16),
                            zp.reshape(n, G // 2)[sub].cpu().numpy(), (n + 7) // 8, K, 128)
    assert np.array_equal(oracle.float_to_half(ref.reshape(-1)), got[sub].reshape(-1))


@pytest.fixture(scope="module")
def layer_tiny_scales(pkg, dev):
    """Config-2 layer with scales log-uniform over [2^-20, 2^-10] (about
    40 % of them f16 subnormals)."""
    layer = pkg.synth.moe_layer(hidden=2048, inter=512, experts=256, seed=77, device=dev,
                                scale_log2=(-20, -10))
    s = layer.gate_up.scale.float()
    assert (s < 2 ** -14).float().mean() > 0.3 and (s <= 2 ** -10).all()
    return layer, moe_to_oracle(layer)


def test_prefill_small_scales_config2(pkg, dev, layer_tiny_scales):
    layer, mw = layer_tiny_scales
    T = 2048
    x = pkg.synth.activations(T, 2048, 78, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, 256, 79, dev, zipf_s=1.1), 8)
    out = pkg.grouped_moe_prefill(layer, x, ids, w)
    routed = pkg.grouped_moe_prefill_routed(layer, x, ids, w.reshape(-1))
    torch.cuda.synchronize()
    xf, ids_np, w_np = f16_to_f32(x), ids.cpu().numpy(), w.cpu().numpy()
    ref = oracle.moe_ffn_tokens(mw, xf, ids_np, w_np, threads=THREADS)
    assert_parity(f16_to_f32(out), ref, what="config2 small scales, full")
    ref_r = oracle.moe_routed_tokens(mw, xf, ids_np, w_np, threads=THREADS)
    assert_parity(routed.cpu().numpy(), ref_r, what="config2 small scales, routed f32")


def test_decode_small_scales(pkg, dev, layer_tiny_scales):
    layer, mw = layer_tiny_scales
    x = pkg.synth.activations(1, 2048, 80, dev)[0]
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(1, 256, 81, dev), 8)
    out = pkg.run_moe_ffn_layer(layer, x, ids[0].contiguous(), w[0].contiguous())
    torch.cuda.synchronize()
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x)[None], ids.cpu().numpy(), w.cpu().numpy(),
                                threads=1)
    assert_parity(f16_to_f32(out), ref[0], what="decode small scales")


@pytest.fixture(scope="module")
def layer_c2(pkg, dev):
    layer = pkg.synth.moe_layer(hidden=2048, inter=512, experts=256, seed=90, device=dev)
    return layer, moe_to_oracle(layer)


def test_run_layer_contract(pkg, dev, layer_c2):
    """Strided int32 top-k (12 ids per row, the last 4 garbage), weights
    [T * 8], f32 hidden states -> f32 routed sum, against the oracle."""
    layer, mw = layer_c2
    T, k = 512, 8
    x16 = pkg.synth.activations(T, 2048, 91, dev)
    x32 = x16.float() + 1e-3 * torch.randn(T, 2048, device=dev)  # not f16-representable
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, 256, 92, dev), k)
    wide = torch.full((T, 12), 9999, dtype=torch.int32, device=dev)
    wide[:, :k] = ids
    out = pkg.grouped_moe_prefill_routed(layer, x32, wide, w.reshape(-1), topk_stride=48)
    # the same through a byte buffer
    raw = wide.view(torch.uint8).reshape(-1)
    out_b = pkg.grouped_moe_prefill_routed(layer, x32, raw, w.reshape(-1), topk_stride=48)
    # f32 input == its f16 rounding given as f16
    out_h = pkg.grouped_moe_prefill_routed(layer, x32.half(), ids, w)
    torch.cuda.synchronize()
    assert torch.equal(out, out_b) and torch.equal(out, out_h)
    ref = oracle.moe_routed_tokens(mw, x32.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(),
                                   threads=THREADS)
    assert_parity(out.cpu().numpy(), ref, what="RunLayer routed f32, f32 input")


def test_run_layer_intermediates_and_stages(pkg, dev, layer_c2):
    """Runtime RunLayer: stage timings and the intermediates of the timed run."""
    layer, mw = layer_c2
    T, k = 300, 8
    x = pkg.synth.activations(T, 2048, 93, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, 256, 94, dev), k)
    rt = pkg.GroupedU4PrefillRuntime(dev)
    h = rt.LoadLayer(layer)
    run = rt.RunLayer(h, pkg.GroupedU4PrefillInput(x, ids, w.reshape(-1), warmup=1, repeat=3,
                                                   capture_intermediates=True))
    assert run.output.dtype == torch.float32 and run.output.shape == (T, 2048)
    # router (no native router here: ~0), schedule, gate/up, down, combine
    assert len(run.timing.stage_us) == 5 and all(s > 0 for s in run.timing.stage_us[1:])
    assert not run.native_router
    assert sum(run.timing.stage_us) <= max(run.timing.samples_us) * 1.1 + 5
    sched = oracle.build_grouped_schedule(ids.cpu().numpy(), 256, w.cpu().numpy())
    assert np.array_equal(run.inverse_map.cpu().numpy(), sched["inverse_map"])
    assert np.array_equal(run.token_map.cpu().numpy(), sched["token_map"])
    # the output is the rank-ordered f32 sum of the captured contributions
    contrib = run.grouped_contributions_f16.float()
    inv = run.inverse_map.long().reshape(T, k)
    acc = torch.zeros(T, 2048, device=dev)
    for r in range(k):
        acc = acc + contrib[inv[:, r]]
    assert torch.equal(acc, run.output)
    # the run record's intermediates, as the reference's
    # (grouped_s8_u4_prefill_runtime.hpp:101-107): SwiGLU rows unweighted in
    # f16 and f32, contributions w_r * down in f16 and f32; each f16 row is
    # the f32 one rounded to nearest even, bit for bit
    A = T * k
    sw16, sw32 = run.grouped_swiglu_f16, run.grouped_swiglu_f32
    c16, c32 = run.grouped_contributions_f16[:A], run.grouped_contributions_f32
    assert sw32.shape == (A, 512) and c32.shape == (A, 2048)
    assert torch.equal(sw16[:A], sw32.half())
    assert torch.equal(c16, c32.half())
    for t in (0, T // 2, T - 1):
        d = oracle.moe_ffn_token_detail(mw, f16_to_f32(x[t]), None, ids[t].cpu().numpy(),
                                        w[t].cpu().numpy())
        wt = w[t].cpu().numpy()[:, None]
        assert_parity(sw32[inv[t]].cpu().numpy(), d["selected_swiglu"].reshape(k, 512),
                      what=f"swiglu f32 token {t}")
        assert_parity(c32[inv[t]].cpu().numpy(), d["selected_down"].reshape(k, 2048) * wt,
                      what=f"contributions f32 token {t}")
    # capturing changes no arithmetic: a plain run gives the same output
    again = rt.RunLayer(h, pkg.GroupedU4PrefillInput(x, ids, w.reshape(-1), repeat=1))
    assert torch.equal(again.output, run.output)
    # the reference's timing record (grouped_s8_u4_prefill_runtime.hpp:86-98):
    # device inputs need no upload or host preparation; the device schedule
    # is the schedule stage; setup and complete minimum follow from them
    tm = run.timing
    assert tm.input_upload_us == 0.0 and tm.schedule_prepare_us == 0.0
    assert tm.device_schedule_us == tm.stage_us[1] > 0
    assert tm.schedule_upload_us == tm.device_schedule_us
    assert tm.schedule_setup_us == tm.schedule_prepare_us + tm.schedule_upload_us
    assert tm.complete_minimum_us == tm.minimum_us + tm.schedule_prepare_us
    # host inputs are uploaded first (hidden states: input_upload_us; top-k
    # rows and router weights: schedule_prepare_us), with the same output
    host = rt.RunLayer(h, pkg.GroupedU4PrefillInput(x.cpu(), ids.cpu(), w.reshape(-1).cpu(),
                                                    repeat=2))
    assert torch.equal(host.output, run.output)
    th = host.timing
    assert th.input_upload_us > 0 and th.schedule_prepare_us > 0
    assert th.schedule_setup_us == th.schedule_prepare_us + th.schedule_upload_us
    assert th.complete_minimum_us == th.minimum_us + th.schedule_prepare_us
    ref = oracle.moe_routed_tokens(mw, f16_to_f32(x), ids.cpu().numpy(), w.cpu().numpy(),
                                   threads=THREADS)
    assert_parity(run.output.cpu().numpy(), ref, what="runtime routed")


@pytest.fixture(scope="module")
def split_pair(pkg, dev, layer_c2):
    layer, mw = layer_c2
    return layer, layer.to_split(), mw


def test_split_decode_matches(pkg, dev, split_pair):
    layer, split, mw = split_pair
    x = pkg.synth.activations(1, 2048, 95, dev)[0]
    res = pkg.synth.activations(1, 2048, 96, dev)[0]
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(1, 256, 97, dev), 8)
    ids, w = ids[0].contiguous(), w[0].contiguous()
    a = pkg.run_moe_ffn_layer(layer, x, ids, w, residual=res)
    b = pkg.run_moe_ffn_layer(split, x, ids, w, residual=res)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ref = oracle.moe_ffn_tokens(mw, f16_to_f32(x)[None], ids.cpu().numpy()[None],
                                w.cpu().numpy()[None], residual=f16_to_f32(res)[None], threads=1)
    assert_parity(f16_to_f32(b), ref[0], what="split decode")


def test_split_prefill_matches(pkg, dev, split_pair):
    layer, split, mw = split_pair
    T = 256
    x = pkg.synth.activations(T, 2048, 98, dev)
    ids, w = pkg.select_router_topk(pkg.synth.router_logits(T, 256, 99, dev), 8)
    a = pkg.grouped_moe_prefill(layer, x, ids, w)
    b = pkg.grouped_moe_prefill(split, x, ids, w)
    ra = pkg.grouped_moe_prefill_routed(layer, x, ids, w)
    rb = pkg.grouped_moe_prefill_routed(split, x, ids, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(ra, rb)
    ref = oracle.moe_routed_tokens(mw, f16_to_f32(x), ids.cpu().numpy(), w.cpu().numpy(),
                                   threads=THREADS)
    assert_parity(rb.cpu().numpy(), ref, what="split prefill routed")


def test_split_decode_plan_matches(pkg, dev):
    """The persistent plan reads both forms through its resolved table."""
    layers = [pkg.synth.moe_layer(2048, 512, 256, 128, seed=100 + l, device=dev)
              for l in range(3)]
    splits = [l.to_split() for l in layers]
    x = pkg.synth.activations(1, 2048, 103, dev)[0].contiguous()
    logits = torch.stack([pkg.synth.router_logits(1, 256, 104 + l, dev)[0] for l in range(3)])
    pa, pb = pkg.DecodePlan(layers, 8), pkg.DecodePlan(splits, 8)
    a = pa.run(x, router_logits=logits)
    b = pb.run(x, router_logits=logits)
    torch.cuda.synchronize()
    pa.check()
    pb.check()
    assert torch.equal(a, b)
    pa.close()
    pb.close()


@pytest.mark.parametrize("include_shared", [False, True])
def test_moe_3gemm_fused_compressed_logits(pkg, dev, layer_c2, include_shared):
    """MOE3GemmFusedCompressed's contract (aima_moe_grouped_prefill_logits):
    router logits in, with the Zipf skew of config 2 and a run of tied
    logits.  The device's routes are the oracle's select_router_topk on
    those logits (ids exact, weights at 1e-6), the output equals the
    ids-fed entry point on the same routes bit for bit, and sampled tokens
    match the oracle at the 2e-3 bar.  Split gate / up tensors, as the op
    takes them."""
    layer, mw = layer_c2
    split = layer.to_split()
    T, E, k = 2048, 256, 8
    x = pkg.synth.activations(T, 2048, 130, dev)
    logits = pkg.synth.router_logits(T, E, 131, dev, zipf_s=1.1)
    logits[5, 40:52] = logits[5].max() + 1.0  # 12 equal top logits: ids decide
    res = pkg.synth.activations(T, 2048, 132, dev) if include_shared else None
    out, ids, w = pkg.moe_3gemm_fused_compressed(x, logits, split, k,
                                                 include_shared=include_shared, residual=res)
    torch.cuda.synchronize()
    ref_ids, ref_w = oracle.router_topk_tokens(logits.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ref_ids)
    assert ids[5].cpu().tolist() == list(range(40, 48))
    assert_parity(w.cpu().numpy(), ref_w, tol=1e-6, what="fused-op router weights")
    if include_shared:
        fed = pkg.grouped_moe_prefill(layer, x, ids, w, residual=res)
    else:
        fed = pkg.grouped_moe_prefill_routed(layer, x, ids, w.reshape(-1))
    torch.cuda.synchronize()
    assert torch.equal(out, fed)
    sel = np.array([0, 5, 1000, T - 1])
    xs = f16_to_f32(x)[sel]
    if include_shared:
        ref = oracle.moe_ffn_tokens(mw, xs, ref_ids[sel], ref_w[sel],
                                    residual=f16_to_f32(res)[sel], threads=THREADS)
        assert_parity(f16_to_f32(out)[sel], ref, what="fused-op full output")
    else:
        ref = oracle.moe_routed_tokens(mw, xs, ref_ids[sel], ref_w[sel], threads=THREADS)
        assert_parity(out.cpu().numpy()[sel], ref, what="fused-op routed output")
