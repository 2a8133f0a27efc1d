"""GPU parity: U4 dequant (bit-exact) and the batch-1 U4 matvec (configs 0
and 3 of the benchmark, plus every supported K and group) against the oracle."""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_bits, f16_to_f32, u4_to_oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)


def _weight(pkg, dev, rows, k, group, seed):
    gen = pkg.synth.generator(seed, dev)
    return pkg.synth.u4_weight(1, rows, k, group, gen, dev)


@pytest.mark.parametrize("rows,k,group", [(4096, 2048, 128), (96, 512, 64), (40, 256, 32),
                                          (17, 1024, 256)])
def test_dequant_bit_exact(pkg, dev, rows, k, group):
    w = _weight(pkg, dev, rows, k, group, seed=rows)
    got = pkg.u4_dequant(w).cpu().numpy()
    o = u4_to_oracle(w)
    exp = oracle.u4_dequant(o.qweight[0], o.scale[0], o.zp[0], rows, k, group)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def _matvec_case(pkg, dev, rows, k, group, seed, out_dtype=torch.float16):
    w = _weight(pkg, dev, rows, k, group, seed)
    x = pkg.synth.activations(1, k, seed + 1, dev)[0]
    y = pkg.matvec_u4(x, w, out_dtype=out_dtype)
    torch.cuda.synchronize()
    o = u4_to_oracle(w)
    ref = oracle.u4_matvec(o.qweight[0], o.scale[0], o.zp[0], rows, k, f16_to_f32(x),
                           group=group, threads=THREADS)
    got = y.float().cpu().numpy()
    return got, ref


def test_config0_matvec(pkg, dev):
    """K=2048, N=4096, group 128, seed 0, f16 out."""
    got, ref = _matvec_case(pkg, dev, 4096, 2048, 128, seed=0)
    c = assert_parity(got, ref, what="config0")
    # the f16 output is the round-to-nearest of an f32 sum within ~1e-5 of the oracle's
    assert c["max_rel"] < 5e-4, c


@pytest.mark.parametrize("k", [128, 256, 512, 1024, 4096, 8192])
@pytest.mark.parametrize("rows", [37, 256])
def test_matvec_shapes(pkg, dev, k, rows):
    got, ref = _matvec_case(pkg, dev, rows, k, 128, seed=k + rows, out_dtype=torch.float32)
    c = assert_parity(got, ref, what=f"k={k} rows={rows}")
    assert c["max_rel"] < 1e-4, c


@pytest.mark.parametrize("group", [32, 64, 256])
def test_matvec_groups(pkg, dev, group):
    got, ref = _matvec_case(pkg, dev, 300, 2048, group, seed=group, out_dtype=torch.float32)
    c = assert_parity(got, ref, what=f"group={group}")
    assert c["max_rel"] < 1e-4, c


@pytest.mark.parametrize("k,rows,group", [(2048, 20001, 64), (512, 70001, 32),
                                           (4096, 17001, 256), (128, 300001, 128)])
def test_matvec_many_rows(pkg, dev, k, rows, group):
    """Row counts that take the 8-pass kernel instance, with a partial last
    block (scales and zero points staged per block)."""
    got, ref = _matvec_case(pkg, dev, rows, k, group, seed=rows, out_dtype=torch.float32)
    c = assert_parity(got, ref, what=f"k={k} rows={rows} group={group}")
    assert c["max_rel"] < 1e-4, c


def test_config3_lm_head(pkg, dev):
    """K=2048, N=248320 (vocab rows), f32 logits."""
    got, ref = _matvec_case(pkg, dev, 248320, 2048, 128, seed=3, out_dtype=torch.float32)
    c = assert_parity(got, ref, what="config3")
    assert c["max_rel"] < 1e-4, c
    assert np.argmax(got) == np.argmax(ref)


def test_router_topk_matches_oracle(pkg, dev):
    for T, E, k, zipf in ((2048, 256, 8, 1.1), (333, 256, 8, None), (64, 16, 8, None),
                          (16, 1000, 16, None)):
        logits = pkg.synth.router_logits(T, E, seed=T + E, device=dev, zipf_s=zipf)
        ids, w = pkg.select_router_topk(logits, k)
        torch.cuda.synchronize()
        rid, rw = oracle.router_topk_tokens(logits.cpu().numpy(), k)
        assert np.array_equal(ids.cpu().numpy(), rid), (T, E, k)
        np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-7)


def test_router_ties_pick_lower_id(pkg, dev):
    logits = torch.zeros((4, 64), device=dev)
    logits[1, 10:20] = 1.0
    logits[2, ::3] = 2.0
    ids, w = pkg.select_router_topk(logits, 8)
    torch.cuda.synchronize()
    rid, rw = oracle.router_topk_tokens(logits.cpu().numpy(), 8)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert list(ids[0].cpu().numpy()) == list(range(8))


def test_rmsnorm_matches_oracle(pkg, dev):
    x = pkg.synth.activations(8, 2048, seed=5, device=dev)
    wt = 1.0 + 0.01 * torch.randn(2048, device=dev)
    out = pkg.apply_rms_norm(x, wt, 1e-6)
    torch.cuda.synchronize()
    ref = oracle.rms_norm_rows(f16_to_f32(x), wt.cpu().numpy(), 1e-6)
    refh = oracle.f16_values(oracle.float_to_half(ref)).reshape(ref.shape)
    got = f16_to_f32(out)
    # f16 outputs agree except where the f32 results straddle a rounding point
    assert np.mean(f16_bits(out).reshape(-1) == oracle.float_to_half(ref)) > 0.99
    assert_parity(got, refh, tol=1e-3, what="rmsnorm")
