"""The oracle's precision models (orc_moe_ffn_tokens_model), which the
end-to-end stack tests use to measure how far two correct implementations
of a 40-layer chain drift apart through the f16 residual.  They are pinned
here: with no flag the model is the oracle layer bit for bit; the f64 model
equals an independent float64 computation from the exhaustively pinned
dequant; each device rounding point, taken alone, moves the result by no
more than its rounding bound allows; and a chain with no flag is
moe_stack_tokens' last layer."""

import numpy as np
import pytest

import oracle

H, I, E, K, T = 256, 64, 6, 4, 5


def _u4(rng, experts, rows, k, group=64, scale=0.02):
    q = rng.integers(0, 256, (experts, rows, k // 2), dtype=np.uint8)
    s = oracle.float_to_half((np.abs(rng.normal(0, scale, (experts, rows, k // group))) + 1e-3)
                             .astype(np.float32)).reshape(experts, rows, k // group)
    z = rng.integers(0, 256, (experts, rows * (k // group) // 2), dtype=np.uint8)
    return oracle.U4Tensor(q, s, z, rows, k, group)


@pytest.fixture(scope="module")
def case():
    rng = np.random.default_rng(2024)
    mw = oracle.MoeWeights(_u4(rng, E, 2 * I, H), _u4(rng, E, H, I), _u4(rng, 1, 2 * I, H),
                           _u4(rng, 1, H, I),
                           oracle.float_to_half((rng.normal(0, 1, H) / np.sqrt(H))
                                                .astype(np.float32)))
    x = oracle.f16_values(oracle.float_to_half(rng.normal(0, 1, (T, H)).astype(np.float32))
                          ).reshape(T, H)
    res = oracle.f16_values(oracle.float_to_half(rng.normal(0, 4, (T, H)).astype(np.float32))
                            ).reshape(T, H)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    return mw, x, res, ids, w


def _dense(t: oracle.U4Tensor, e: int) -> np.ndarray:
    return oracle.u4_dequant(t.qweight[e], t.scale[e], t.zp[e], t.rows, t.k, t.group
                             ).reshape(t.rows, t.k).astype(np.float64)


def _exact(mw, x, res, ids, w):
    """float64 brute force of one layer from the dequantized matrices."""
    def expert(gu, dn, e, xv):
        g = _dense(gu, e) @ xv
        n = gu.rows // 2
        a = g[:n] / (1.0 + np.exp(-g[:n])) * g[n:]
        return _dense(dn, e) @ a

    out = np.empty_like(x, dtype=np.float64)
    gv = oracle.f16_values(mw.shared_gate_vec).astype(np.float64)
    for t in range(x.shape[0]):
        xv = x[t].astype(np.float64)
        moe = sum(float(w[t, r]) * expert(mw.gate_up, mw.down, ids[t, r], xv)
                  for r in range(ids.shape[1]))
        sh = expert(mw.shared_gate_up, mw.shared_down, 0, xv)
        sig = 1.0 / (1.0 + np.exp(-(gv @ xv)))
        out[t] = res[t] + moe + sig * sh
    return out


def test_model_without_flags_is_the_oracle_layer(case):
    mw, x, res, ids, w = case
    a = oracle.moe_ffn_tokens(mw, x, ids, w, residual=res, threads=2)
    b = oracle.moe_ffn_tokens_model(mw, x, ids, w, residual=res, flags=0, threads=2)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_f64_model_matches_float64_brute_force(case):
    mw, x, res, ids, w = case
    got = oracle.moe_ffn_tokens_model(mw, x, ids, w, residual=res, flags=oracle.MODEL_F64)
    want = _exact(mw, x, res, ids, w)
    # the model rounds once, to f32, at the end
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 2 ** -23


@pytest.mark.parametrize("flag,bound", [
    (oracle.MODEL_CHUNKED, 1e-5), (oracle.MODEL_SLICED, 1e-5),
    (oracle.MODEL_ACT_F16, 2e-3), (oracle.MODEL_WEIGHT_F16, 2e-3),
    (oracle.MODEL_CONTRIB_F16, 2e-3), (oracle.MODEL_DECODE_PLAN, 2e-3),
    (oracle.MODEL_PREFILL, 2e-3)])
def test_each_rounding_point_stays_within_its_bound(case, flag, bound):
    """A plan-style order alone moves the layer by f32 rounding only; an f16
    rounding point by at most the 2e-3 layer bar.  Every flag changes the
    result (the flag is wired), and the f32 reorders stay far below f16."""
    mw, x, res, ids, w = case
    exact = _exact(mw, x, res, ids, w)
    got = oracle.moe_ffn_tokens_model(mw, x, ids, w, residual=res, flags=flag)
    base = oracle.moe_ffn_tokens(mw, x, ids, w, residual=res)
    err = np.max(np.abs(got - exact)) / np.max(np.abs(exact))
    assert err <= bound, err
    assert not np.array_equal(got, base)


def test_sliced_model_needs_eight_slices(case):
    mw, x, res, ids, w = case
    bad = oracle.MoeWeights(mw.gate_up, mw.down, mw.shared_gate_up,
                            _u4(np.random.default_rng(1), 1, H, 36, group=36),
                            mw.shared_gate_vec)
    with pytest.raises(oracle.OracleError):
        oracle.moe_ffn_tokens_model(bad, x, ids, w, residual=res, flags=oracle.MODEL_SLICED)


def test_chain_without_flags_is_moe_stack_tokens(case):
    mw, x, res, ids, w = case
    L = 3
    rng = np.random.default_rng(7)
    norms = [(1.0 + 0.01 * rng.normal(size=H)).astype(np.float32) for _ in range(L)]
    x0 = oracle.float_to_half(res.astype(np.float32)).reshape(T, H)
    idsL, wL = np.stack([ids] * L), np.stack([w] * L)
    stack = oracle.moe_stack_tokens([mw] * L, norms, x0, idsL, wL, threads=2)
    chain = oracle.moe_stack_chain_model([mw] * L, norms, x0, idsL, wL, flags=0, threads=2)
    assert np.array_equal(stack[-1], chain)
