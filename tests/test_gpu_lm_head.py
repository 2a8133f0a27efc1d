"""GPU parity for the device top-k and the U4 LM head with top-k
(q4x8_matvec.cl:973-1021): value descending, lower index first among equal
values, bit-exact against the oracle's restatement."""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_to_f32, u4_to_oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)


@pytest.mark.parametrize("n", [1, 100, 1024, 1025, 70001, 248320, 1048576])
@pytest.mark.parametrize("k", [1, 8, 16])
def test_topk_matches_oracle_with_ties(pkg, dev, n, k):
    if k > n:
        pytest.skip("k > n")
    g = torch.Generator(device=dev)
    g.manual_seed(n * 31 + k)
    # integer-valued: every value repeats many times, so ties decide the order
    v = torch.randint(-50, 50, (n,), generator=g, device=dev).float()
    ids, vals = pkg.topk_f32(v, k)
    torch.cuda.synchronize()
    ref_i, ref_v = oracle.lm_head_topk(v.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ref_i)
    assert np.array_equal(vals.cpu().numpy(), ref_v)


@pytest.mark.parametrize("n,k", [(4096, 8), (300000, 16), (70, 16), (130, 8)])
def test_topk_constant_and_sparse(pkg, dev, n, k):
    """All-equal values leave thousands of pairs at the block threshold (the
    per-wave fallback); small n leaves most waves empty (no threshold)."""
    for v in (torch.full((n,), 3.0, device=dev), torch.arange(n, device=dev).float() % 7):
        ids, vals = pkg.topk_f32(v, k)
        torch.cuda.synchronize()
        ref_i, ref_v = oracle.lm_head_topk(v.cpu().numpy(), k)
        assert np.array_equal(ids.cpu().numpy(), ref_i)
        assert np.array_equal(vals.cpu().numpy(), ref_v)


def test_topk_distinct_and_infinite(pkg, dev):
    v = torch.randn(300000, device=dev)
    v[::7] = -float("inf")
    v[12345] = float("inf")
    ids, vals = pkg.topk_f32(v, 16)
    torch.cuda.synchronize()
    ref_i, ref_v = oracle.lm_head_topk(v.cpu().numpy(), 16)
    assert ids[0].item() == 12345
    assert np.array_equal(ids.cpu().numpy(), ref_i) and np.array_equal(vals.cpu().numpy(), ref_v)


@pytest.mark.parametrize("k", [1, 8])
def test_lm_head_topk_config3(pkg, dev, k):
    """K=2048, N=248320: logits are the matvec's bit for bit, the selection is
    the oracle's on them, and the logits match the oracle's matvec."""
    w = pkg.synth.u4_weight(1, 248320, 2048, 128, pkg.synth.generator(3, dev), dev)
    x = pkg.synth.activations(1, 2048, 3, dev)[0]
    ids, vals, logits = pkg.lm_head_topk(x, w, k)
    single = pkg.matvec_u4(x, w, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(logits, single)
    lg = logits.cpu().numpy()
    ref_i, ref_v = oracle.lm_head_topk(lg, k)
    assert np.array_equal(ids.cpu().numpy(), ref_i) and np.array_equal(vals.cpu().numpy(), ref_v)
    o = u4_to_oracle(w)
    ref_logits = oracle.u4_matvec(o.qweight[0], o.scale[0], o.zp[0], 248320, 2048, f16_to_f32(x),
                                  group=128, threads=THREADS)
    assert_parity(lg, ref_logits, what="lm head logits")
    assert ids[0].item() == int(np.argmax(ref_logits))


def test_topk_rejects_bad_sizes(pkg, dev):
    v = torch.zeros(16, device=dev)
    with pytest.raises(pkg.AimaError):
        pkg.topk_f32(v, 17)
    with pytest.raises(pkg.AimaError):
        pkg.topk_f32(torch.zeros(1048577, device=dev), 8)
