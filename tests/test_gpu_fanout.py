"""GPU parity for the multi-output fixed FC (one input, 1 to 4 U4 matrices in
one launch, iq36_fixed_fc_multi_output.cl) and the device router (U4 FC to
the expert logits, then top-k; gguf_loader.cpp:5708-5711)."""

import os

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_to_f32, u4_to_oracle

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)


def _weight(pkg, dev, rows, k, group, seed):
    return pkg.synth.u4_weight(1, rows, k, group, pkg.synth.generator(seed, dev), dev)


def _oracle_matvec(w, x):
    o = u4_to_oracle(w)
    return oracle.u4_matvec(o.qweight[0], o.scale[0], o.zp[0], w.rows, w.k, f16_to_f32(x),
                            group=w.group, threads=THREADS)


@pytest.mark.parametrize("rows,k,group", [
    ((1, 512, 512, 256), 2048, 128),        # the K = 2048 fanout of the reference
    ((1024, 1024, 64), 1024, 64),           # arity 3
    ((300,), 2048, 32),                     # arity 1
    ((1, 8192, 8192, 256), 2048, 128),      # enough rows for the 8-pass blocks
])
def test_multi_output_matches_single(pkg, dev, rows, k, group):
    ws = [_weight(pkg, dev, n, k, group, seed=10 * i + n) for i, n in enumerate(rows)]
    x = pkg.synth.activations(1, k, seed=sum(rows), device=dev)[0]
    dts = [torch.float32 if i == len(rows) - 1 else torch.float16 for i in range(len(rows))]
    ys = pkg.matvec_u4_multi(x, ws, dts)
    singles = [pkg.matvec_u4(x, w, out_dtype=d) for w, d in zip(ws, dts)]
    torch.cuda.synchronize()
    for i, (y, s, w) in enumerate(zip(ys, singles, ws)):
        assert y.dtype == dts[i] and y.numel() == w.rows
        assert torch.equal(y, s), f"output {i} differs from the single matvec"
        assert_parity(y.float().cpu().numpy(), _oracle_matvec(w, x), what=f"output {i}")


def test_multi_output_rejects_bad_calls(pkg, dev):
    x = pkg.synth.activations(1, 2048, seed=1, device=dev)[0]
    w = _weight(pkg, dev, 64, 2048, 128, seed=1)
    with pytest.raises(ValueError):
        pkg.matvec_u4_multi(x, [w] * 5)
    with pytest.raises(ValueError):
        pkg.matvec_u4_multi(x, [w, _weight(pkg, dev, 64, 1024, 128, seed=2)])
    with pytest.raises(pkg.AimaError):
        # null output pointer reaches the C ABI check
        import ctypes as C
        t = (pkg._lib.U4TensorC * 1)(pkg._lib.U4TensorC(w.qweight.data_ptr(), w.scale.data_ptr(),
                                                        w.zp.data_ptr()))
        pkg._lib.call("aima_u4_matvec_multi", x.data_ptr(), 1, t, (C.c_int64 * 1)(64), 2048, 128,
                      (C.c_void_p * 1)(None), (C.c_int32 * 1)(0), None)


@pytest.mark.parametrize("experts,k,group", [(256, 8, 128), (128, 4, 128), (1000, 16, 128),
                                             (256, 8, 32), (200, 8, 256), (17, 16, 64)])
def test_router_fc_topk(pkg, dev, experts, k, group):
    """Every expert count up to 1024 and every group size."""
    router = _weight(pkg, dev, experts, 2048, group, seed=experts + group)
    x = pkg.synth.activations(1, 2048, seed=experts + 1, device=dev)
    norm = 1.0 + 0.01 * torch.randn(2048, device=dev, generator=pkg.synth.generator(7, dev))
    h = pkg.apply_rms_norm(x, norm, 1e-6)[0]
    ids, w, logits = pkg.router_fc_topk(h, router, k)
    single = pkg.matvec_u4(h, router, out_dtype=torch.float32)
    sel_ids, sel_w = pkg.select_router_topk(logits[None], k)
    torch.cuda.synchronize()
    # the logits are the matvec's, the selection is select_router_topk's, bit for bit
    assert torch.equal(logits, single)
    assert torch.equal(ids, sel_ids[0]) and torch.equal(w, sel_w[0])
    # against the oracle: logits to the matvec tolerance; the selection on the
    # oracle's logits matches wherever the k-th and (k+1)-th probabilities are
    # apart by more than the logits' rounding
    ref_logits = _oracle_matvec(router, h)
    assert_parity(logits.cpu().numpy(), ref_logits, what="router logits")
    rid, rw = oracle.router_topk_tokens(ref_logits[None].astype(np.float32), k)
    srt = np.sort(ref_logits)[::-1]
    if srt[k - 1] - srt[k] > 1e-3:
        assert np.array_equal(ids.cpu().numpy(), rid[0])
        np.testing.assert_allclose(w.cpu().numpy(), rw[0], rtol=1e-3)
