"""Bit-exact agreement of the C oracle with the reference's own CPU code
(engine/src/gguf_loader.cpp compiled into oracle/_ref), on random inputs.

The full-layer test writes the exactly dequantized U4 weights into an F32
GGUF and runs the reference's run_qwen36_moe_ffn_layer
(gguf_loader.cpp:5654-5782); the oracle's per-token MoE FFN must reproduce
every intermediate bit for bit from the reference's ffn_norm and router
selection."""

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


def bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("seed", range(5))
def test_router_ops_bit_exact(ref, seed):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal(256).astype(np.float32) * (1 + seed)
    if seed == 3:
        logits[10:20] = logits[5]  # ties
    assert bits_equal(oracle.softmax(logits), ref.softmax(logits))
    p = oracle.softmax(logits)
    assert np.array_equal(oracle.top_k_indices(p, 8), ref.top_k_indices(p, 8))
    a = oracle.select_router_topk(logits, 8)
    b = ref.select_router_topk(logits, 8)
    assert np.array_equal(a[0], b[0]) and bits_equal(a[1], b[1]) and bits_equal(a[2], b[2])
    w = np.abs(rng.standard_normal(8)).astype(np.float32) * 1e-5
    assert bits_equal(oracle.normalize_weights(w, oracle.MIN_WEIGHT_SUM),
                      ref.normalize_weights(w, oracle.MIN_WEIGHT_SUM))


@pytest.mark.parametrize("seed", range(3))
def test_elementwise_ops_bit_exact(ref, seed):
    rng = np.random.default_rng(100 + seed)
    g = (rng.standard_normal(512) * 4).astype(np.float32)
    u = rng.standard_normal(512).astype(np.float32)
    assert bits_equal(oracle.swiglu_pair(g, u), ref.swiglu_pair(g, u))
    gu = (rng.standard_normal(9 * 2 * 64) * 3).astype(np.float32)
    assert bits_equal(oracle.swiglu_from_gate_up(gu, 64, 9), ref.swiglu_from_gate_up(gu, 64, 9))
    down = rng.standard_normal(8 * 300).astype(np.float32)
    w = rng.random(8).astype(np.float32)
    wa = oracle.apply_expert_weights(down, w, 300)
    assert bits_equal(wa, ref.apply_expert_weights(down, w, 300))
    assert bits_equal(oracle.aggregate_experts(wa, 8, 300), ref.aggregate_experts(wa, 8, 300))
    x = rng.standard_normal(2048).astype(np.float32)
    nw = (1 + 0.01 * rng.standard_normal(2048)).astype(np.float32)
    assert bits_equal(oracle.rms_norm(x, nw, 1e-6), ref.rms_norm(x, nw, 1e-6))
    for v in (-30.0, -1.5, 0.0, 0.25, 7.0, 40.0):
        assert oracle.sigmoid_scalar(v) == ref.sigmoid_scalar(v)


def _rand_u4(rng, e, rows, k, group=128):
    q = rng.integers(0, 256, (e, rows, k // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (e, rows, k // group))) + 1e-3).astype(np.float16)
    z = rng.integers(0, 256, (e, rows * (k // group) // 2), dtype=np.uint8)
    return oracle.U4Tensor(q, s.view(np.uint16), z, rows, k, group)


def _dequant(t: oracle.U4Tensor):
    return np.stack([oracle.u4_dequant(t.qweight[e], t.scale[e], t.zp[e], t.rows, t.k, t.group)
                     for e in range(t.experts)])


def test_matvec_bit_exact(ref, tmp_path):
    rng = np.random.default_rng(7)
    t = _rand_u4(rng, 1, 96, 512)
    x = rng.standard_normal(512).astype(np.float16).astype(np.float32)
    y = oracle.u4_matvec(t.qweight[0], t.scale[0], t.zp[0], 96, 512, x)
    yr = ref.matvec_f32(_dequant(t)[0], x, tmp_path)
    assert bits_equal(y, yr)


@pytest.mark.parametrize("seed", [0, 1])
def test_moe_ffn_layer_bit_exact(ref, tmp_path, seed):
    rng = np.random.default_rng(1000 + seed)
    H, I, E = 256, 128, 16
    gate_up = _rand_u4(rng, E, 2 * I, H)
    down = _rand_u4(rng, E, H, I)
    sgu = _rand_u4(rng, 1, 2 * I, H)
    sd = _rand_u4(rng, 1, H, I)
    gate_vec = (rng.standard_normal(H) / 16).astype(np.float16)
    router = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    norm_w = (1 + 0.01 * rng.standard_normal(H)).astype(np.float32)
    residual = rng.standard_normal(H).astype(np.float16).astype(np.float32)
    r = ref.moe_ffn_layer_f32(tmp_path, _dequant(gate_up), _dequant(down), _dequant(sgu)[0],
                              _dequant(sd)[0], router, gate_vec.astype(np.float32), norm_w,
                              residual, 1e-6)
    mw = oracle.MoeWeights(gate_up, down, sgu, sd, gate_vec.view(np.uint16))
    # router: oracle on the reference's logits
    ids, _, nw = oracle.select_router_topk(r["router_logits"], 8)
    assert np.array_equal(ids, r["ids"]) and bits_equal(nw, r["normalized_weights"])
    assert bits_equal(oracle.rms_norm(residual, norm_w, 1e-6), r["ffn_norm"])
    o = oracle.moe_ffn_token_detail(mw, r["ffn_norm"], residual, r["ids"],
                                    r["normalized_weights"])
    for name in ("selected_gate_up", "selected_swiglu", "selected_down", "moe_out",
                 "shared_down", "ffn_out", "residual"):
        assert bits_equal(o[name], r[name]), name
    assert o["shared_gate"][1] == r["shared_gate_sigmoid"][0]
    # the batched token path gives the same residual
    t = oracle.moe_ffn_tokens(mw, r["ffn_norm"][None], r["ids"][None],
                              r["normalized_weights"][None], residual=residual[None])
    assert bits_equal(t[0], r["residual"])


def test_q4k_unpack_matches_reference_decode(ref, tmp_path):
    """oracle.q4k_unpack against the reference's own decode_q4_k_block (through
    decode_tensor_row on a GGUF Q4_K tensor): its codes, f32 scales and mins
    rebuild every reference value exactly as d1 * q - m1, and its f16 scales
    are those f32 scales rounded to nearest even.  Random blocks, including
    f16 subnormal and large d / dmin and every 6-bit scale / min."""
    rng = np.random.default_rng(12)
    rows, cols = 24, 512
    raw = rng.integers(0, 256, (rows, cols // 256, 144), dtype=np.uint8)
    d = np.concatenate([rng.uniform(-2, 2, rows * 2 - 6), [6e-8, -6e-8, 3e-5, 1e-3, 60000.0, 0.0]])
    dm = rng.uniform(-0.5, 0.5, rows * 2)
    raw[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, 2, 2)
    raw[:, :, 2:4] = dm.astype(np.float16).view(np.uint8).reshape(rows, 2, 2)
    vals = ref.decode_q4k_rows(raw, rows, cols, str(tmp_path / "q4k.gguf"))
    codes, s16, mins, s32 = oracle.q4k_unpack(raw, rows, cols, f32_scale=True)
    q = np.empty((rows, cols), np.float32)
    q[:, 0::2] = codes & 15
    q[:, 1::2] = codes >> 4
    rebuilt = np.repeat(s32, 32, axis=1) * q - np.repeat(mins, 32, axis=1)
    assert rebuilt.dtype == np.float32
    assert np.array_equal(rebuilt.view(np.uint32), vals.view(np.uint32))
    assert np.array_equal(s16, s32.astype(np.float16).view(np.uint16))


def test_q4s_dequant_matches_reference_decode_when_scale_is_f16_exact(ref, tmp_path):
    """oracle.q4s_dequant (the scale-and-min form the Q4_K-derived matvec
    consumes) against the reference's decode_q4_k_block: with d a power of
    two and the 6-bit scales small, d * sc is exact in f16, so the prepacked
    f16 scale loses nothing and every dequantized value equals the
    reference's d1 * q - m1 bit for bit."""
    rng = np.random.default_rng(21)
    rows, cols = 16, 512
    raw = rng.integers(0, 256, (rows, cols // 256, 144), dtype=np.uint8)
    d = np.ldexp(1.0, rng.integers(-12, -2, rows * 2)) * rng.choice([-1.0, 1.0], rows * 2)
    dm = rng.uniform(-0.25, 0.25, rows * 2)
    raw[:, :, 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, 2, 2)
    raw[:, :, 2:4] = dm.astype(np.float16).view(np.uint8).reshape(rows, 2, 2)
    vals = ref.decode_q4k_rows(raw, rows, cols, str(tmp_path / "q4s.gguf"))
    codes, s16, mins, s32 = oracle.q4k_unpack(raw, rows, cols, f32_scale=True)
    assert np.array_equal(oracle.half_to_float(s16).reshape(s32.shape), s32)  # the precondition
    w = oracle.q4s_dequant(codes, s16, mins, rows, cols)
    assert np.array_equal(w.view(np.uint32), vals.view(np.uint32))
