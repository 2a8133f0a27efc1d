"""The CPU baseline library (bench.py's cpu_baseline leg) computes the same
layer as the oracle, to the parity tolerance: it reassociates the oracle's
sums (scale and zero point hoisted per group) but must not change what is
computed.  Built here for this CPU with -march=native."""

import numpy as np
import pytest

import oracle
from oracle import cpu_baseline
from tests.helpers import assert_parity


@pytest.fixture(scope="module")
def base(tmp_path_factory):
    return cpu_baseline.load(str(tmp_path_factory.mktemp("cpb")))


def _u4(rng, rows, k, group=128):
    q = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (rows, k // group))) + 1e-3).astype(np.float16)
    z = rng.integers(0, 256, rows * (k // group) // 2, dtype=np.uint8)
    return q, s.view(np.uint16), z


@pytest.mark.parametrize("threads", [1, 4])
def test_matvec_matches_oracle(base, threads):
    rng = np.random.default_rng(3)
    n, k = 512, 2048
    q, s, z = _u4(rng, n, k)
    x = rng.normal(size=k).astype(np.float32)
    y = np.empty(n, np.float32)
    base.set_threads(threads)
    base.matvec(q, s, z, n, k, 128, x, y)
    ref = oracle.u4_matvec(q, s, z, n, k, x)
    assert_parity(y, ref, tol=1e-5, what="baseline matvec")


def test_layer_matches_oracle(base):
    rng = np.random.default_rng(4)
    H, I, k = 2048, 512, 8
    experts = [(_u4(rng, 2 * I, H), _u4(rng, H, I)) for _ in range(k)]
    shared = (_u4(rng, 2 * I, H), _u4(rng, H, I))
    gate_vec = (rng.normal(size=H) / np.sqrt(H)).astype(np.float16)
    norm = (1 + 0.01 * rng.normal(size=H)).astype(np.float32)
    w = rng.random(k).astype(np.float32)
    w /= w.sum()
    r = rng.normal(size=H).astype(np.float32)
    layer = base.layer(experts, shared, gate_vec.astype(np.float32), norm, H, I, 128)
    out = np.empty(H, np.float32)
    base.set_threads(4)
    base.moe_token(layer, w, 1e-6, r, out)
    # oracle: the same layer as a k-expert stack with ids 0..k-1
    gu = oracle.U4Tensor(np.stack([e[0][0] for e in experts]),
                         np.stack([e[0][1] for e in experts]),
                         np.stack([e[0][2] for e in experts]), 2 * I, H, 128)
    dn = oracle.U4Tensor(np.stack([e[1][0] for e in experts]),
                         np.stack([e[1][1] for e in experts]),
                         np.stack([e[1][2] for e in experts]), H, I, 128)
    sg = oracle.U4Tensor(shared[0][0][None], shared[0][1][None], shared[0][2][None], 2 * I, H,
                         128)
    sd = oracle.U4Tensor(shared[1][0][None], shared[1][1][None], shared[1][2][None], H, I, 128)
    mw = oracle.MoeWeights(gu, dn, sg, sd, gate_vec.view(np.uint16))
    h = oracle.rms_norm(r, norm, 1e-6)
    ref = oracle.moe_ffn_tokens(mw, h[None], np.arange(k, dtype=np.int32)[None], w[None],
                                residual=r[None], threads=4)
    assert_parity(out, ref[0], what="baseline layer")
