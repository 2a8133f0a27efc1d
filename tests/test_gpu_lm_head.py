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


@pytest.mark.parametrize("n", [1, 100, 1024, 1025, 4096, 4097, 70001, 248320, 1048576])
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


def _crowded(n, k, dev, seed):
    """Values whose best keys crowd into few 16-lane rows of each block: the
    positions a block's rows k // 2 .. 15 read (p % 256 >= 16 * (k // 2),
    for chunks that start at multiples of 256) hold -1 - |noise|, the rest
    10 + noise.  The threshold (the k-th best row best) then admits
    thousands of survivors, the selection's per-wave fallback."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    p = torch.arange(n, device=dev)
    noise = torch.randn(n, generator=g, device=dev)
    low = (p % 256) >= 16 * max(k // 2, 1)
    return torch.where(low, -1.0 - noise.abs(), 10.0 + noise)


@pytest.mark.parametrize("n", [4096, 8192, 65536, 300000])
@pytest.mark.parametrize("k", [2, 8, 16])
def test_topk_crowded_rows(pkg, dev, n, k):
    v = _crowded(n, k, dev, n + k)
    ids, vals = pkg.topk_f32(v, k)
    torch.cuda.synchronize()
    ref_i, ref_v = oracle.lm_head_topk(v.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ref_i)
    assert np.array_equal(vals.cpu().numpy(), ref_v)


@pytest.mark.parametrize("k", [8, 16])
def test_topk_signed_zeros(pkg, dev, k):
    """+0 and -0 are equal values (the lower index first) and each pick's
    value keeps its own sign bit."""
    n = 70001
    g = torch.Generator(device=dev)
    g.manual_seed(k)
    v = -1.0 - torch.rand(n, generator=g, device=dev)
    zp = torch.randperm(n, generator=g, device=dev)[:40]
    sign = torch.randint(0, 2, (40,), generator=g, device=dev).float() * 2 - 1
    v[zp] = 0.0 * sign  # -0.0 where sign is -1
    ids, vals = pkg.topk_f32(v, k)
    torch.cuda.synchronize()
    ref_i, _ = oracle.lm_head_topk(v.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ref_i)
    assert ids.cpu().tolist() == sorted(zp.cpu().tolist())[:k]
    want = v[ids.long()].cpu().numpy().view(np.int32)
    assert np.array_equal(vals.cpu().numpy().view(np.int32), want)
    assert (want == np.int32(-2**31)).any() and (want == 0).any()


def test_lm_head_topk_crowded_rows(pkg, dev):
    """The one-launch head (chunks of 2,048 at n = 65,536) with logits whose
    best crowd into few rows of every selection block."""
    n, K = 65536, 2048
    for k in (8, 16):
        scales = _crowded(n, k, "cpu", 7 + k)
        w = _structured_head(pkg, dev, n, K, scales)
        x = torch.full((K,), 0.25, dtype=torch.float16, device=dev)
        _check_head(pkg, dev, w, x, k)


@pytest.mark.parametrize("k", [1, 8, 16])
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


# ---------------------------------------------------------------------------
# LM-head top-k: the matvec into the logits, then one selection launch whose
# blocks each store their picks and whose block 0 merges them (the launch
# epoch lives in the workspace header)
# ---------------------------------------------------------------------------

def _structured_head(pkg, dev, n, K, scales, group=128):
    """U4 head whose logits are 15 * s_row * sum(x) (q = 15, z = 0 everywhere,
    one f16 scale per row repeated over its groups), so their order and ties
    follow `scales`."""
    G = K // group
    q = torch.full((n, K // 2), 0xFF, dtype=torch.uint8, device=dev)
    zp = torch.zeros(((n * G + 1) // 2,), dtype=torch.uint8, device=dev)
    sc = scales.to(torch.float16).reshape(n, 1).expand(n, G).contiguous().to(dev)
    return pkg.U4Weight(q, sc, zp, n, K, group)


def _check_head(pkg, dev, w, x, k, ws=None):
    ids, vals, logits = pkg.lm_head_topk(x, w, k, ws=ws)
    single = pkg.matvec_u4(x, w, out_dtype=torch.float32)
    torch.cuda.synchronize()
    # the fused matvec's logits are the plain matvec's bit for bit (NaN too)
    assert torch.equal(logits.view(torch.int32), single.view(torch.int32))
    ref_i, ref_v = oracle.lm_head_topk(logits.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), ref_i), (ids.cpu().numpy(), ref_i)
    assert np.array_equal(vals.cpu().numpy(), ref_v)
    return ids, vals


@pytest.mark.parametrize("order", ["rising", "falling", "flat"])
@pytest.mark.parametrize("k", [1, 8, 16])
def test_lm_head_topk_ordered_and_tied(pkg, dev, order, k):
    """Rising logits make every block beat the threshold of the blocks before
    it (the longest candidate list: k per block, merged in many chunks);
    falling ones stop the list after the first blocks; flat ones tie every
    row (lowest indices win).  f16 scales repeat, so ties occur throughout."""
    n, K = 100_000, 2048
    ramp = torch.linspace(0.01, 2.0, n)
    scales = {"rising": ramp, "falling": ramp.flip(0), "flat": torch.full((n,), 0.5)}[order]
    w = _structured_head(pkg, dev, n, K, scales)
    x = torch.full((K,), 0.25, dtype=torch.float16, device=dev)
    ids, _ = _check_head(pkg, dev, w, x, k)
    if order == "flat":
        assert ids.cpu().tolist() == list(range(k))


@pytest.mark.parametrize("K", [128, 512, 2048, 8192])
@pytest.mark.parametrize("n,k", [(5, 5), (700, 16), (33333, 8)])
def test_lm_head_topk_shapes(pkg, dev, K, n, k):
    """Every block geometry (512 rows per block at K = 128 down to 16 at
    K = 8192), partial last blocks and n = k; at K = 2048 the one-launch
    head with one selection block (n <= 4096) and with several."""
    gen = pkg.synth.generator(K + n + k, dev)
    w = pkg.synth.u4_weight(1, n, K, 128, gen, dev)
    x = pkg.synth.activations(1, K, K + n, dev)[0]
    _check_head(pkg, dev, w, x, k)


def test_lm_head_topk_nan_and_infinite_rows(pkg, dev):
    """NaN logits are never chosen (with at least k numbers present); +inf
    rows lead; -inf rows rank after every finite value."""
    n, K = 50_000, 2048
    scales = torch.linspace(0.01, 1.0, n)
    scales[7::97] = float("nan")
    scales[40_000] = float("inf")
    scales[123] = float("inf")
    w = _structured_head(pkg, dev, n, K, scales)
    x = torch.full((K,), 0.25, dtype=torch.float16, device=dev)
    ids, vals = _check_head(pkg, dev, w, x, 8)
    assert ids[0].item() == 123 and ids[1].item() == 40_000
    xn = -x  # all logits negative: -inf rows now rank last
    _check_head(pkg, dev, w, xn, 16)


def test_lm_head_topk_zero_logits_tie(pkg, dev):
    """Zero logits (rows with a zero scale, of either sign: the matvec's sums
    start at +0, so a -0 scale still gives +0) under negative ones: the 24
    zero rows tie and the lowest indices win, across blocks far apart."""
    n, K = 40_000, 2048
    scales = torch.full((n,), -1.0)
    scales[30_000:30_020] = 0.0
    scales[9_000:9_004] = -0.0
    w = _structured_head(pkg, dev, n, K, scales)
    x = torch.full((K,), 0.25, dtype=torch.float16, device=dev)
    ids, vals = _check_head(pkg, dev, w, x, 8)
    assert ids.cpu().tolist() == [9_000, 9_001, 9_002, 9_003, 30_000, 30_001, 30_002, 30_003]
    assert (vals == 0).all()


def test_lm_head_topk_state_reused_between_calls(pkg, dev):
    """The workspace keeps a launch counter that every call advances, and the
    picks it leaves behind stay in place: back-to-back calls with different
    inputs, a different k, and top-k calls of another size on the same
    workspace in between all select exactly."""
    ws = pkg.Workspace(dev)
    gen = pkg.synth.generator(11, dev)
    w = pkg.synth.u4_weight(1, 248320, 2048, 128, gen, dev)
    for seed, k in ((1, 8), (2, 8), (3, 16), (4, 1)):
        x = pkg.synth.activations(1, 2048, seed, dev)[0]
        _check_head(pkg, dev, w, x, k, ws=ws)
        v = torch.randn(300000, device=dev)
        ids, vals = pkg.topk_f32(v, 8, ws=ws)
        torch.cuda.synchronize()
        ref_i, _ = oracle.lm_head_topk(v.cpu().numpy(), 8)
        assert np.array_equal(ids.cpu().numpy(), ref_i)
    assert ws.error_bits() == 0


@pytest.mark.parametrize("group", [32, 64, 256])
def test_lm_head_topk_one_launch_groups(pkg, dev, group):
    """The one-launch head (K = 2048) with every other quantization group
    size: logits bit-identical to the plain matvec, picks the oracle's."""
    n = 70001
    gen = pkg.synth.generator(group + 5, dev)
    w = pkg.synth.u4_weight(1, n, 2048, group, gen, dev)
    x = pkg.synth.activations(1, 2048, group + 6, dev)[0]
    _check_head(pkg, dev, w, x, 8)


@pytest.mark.parametrize("n", [700, 4096, 4097])
def test_lm_head_topk_small_vocab_reused(pkg, dev, n):
    """The one-launch head with one selection block advances the launch
    counter itself (no merge does): calls on one workspace with new inputs
    each select from their own logits, never the tagged logits an earlier
    call left in place (n = 4097 takes two selection blocks and the merge)."""
    ws = pkg.Workspace(dev)
    gen = pkg.synth.generator(n, dev)
    w = pkg.synth.u4_weight(1, n, 2048, 128, gen, dev)
    for seed in range(4):
        x = pkg.synth.activations(1, 2048, 50 + seed, dev)[0]
        _check_head(pkg, dev, w, x, 8, ws=ws)
    assert ws.error_bits() == 0


def _s64(v: int) -> int:
    """A 64-bit pattern as the signed value torch.int64 holds."""
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >= (1 << 63) else v


def test_lm_head_topk_foreign_data_in_pick_region(pkg, dev):
    """A pick is taken only when both of its words carry this launch's 32-bit
    tags, whatever the pick region held before the call: a real MoE decode's
    data written through the same workspace, words that carry the next
    launch's 11-bit epoch in bits 53..63 (what a one-word, 11-bit tag would
    have accepted), and value words carrying the next launch's full tag
    next to index words that do not."""
    ws = pkg.Workspace(dev)
    gen = pkg.synth.generator(12, dev)
    w = pkg.synth.u4_weight(1, 248320, 2048, 128, gen, dev)
    layer = pkg.synth.moe_layer(hidden=2048, inter=512, experts=16, seed=13, device=dev)
    need = max(pkg.ops.size_query("aima_topk_workspace_size", 248320, 16), 1 << 20)
    buf = ws.get(need)
    g = torch.Generator(device=dev)
    g.manual_seed(14)
    for rep, k in enumerate((8, 16, 8, 4)):
        h = pkg.synth.activations(1, 2048, 20 + rep, dev)[0]
        ids = torch.randperm(16, device=dev)[:8].to(torch.int32)
        wts = torch.full((8,), 0.125, device=dev)
        pkg.run_moe_ffn_layer(layer, h, ids, wts, residual=h, ws=ws)  # foreign data
        torch.cuda.synchronize()
        buf = ws.buf
        launch = int(buf[132:136].view(torch.int32).item()) & 0xffffffff
        words = buf[256:].view(torch.int64)
        low = torch.randint(0, 1 << 30, (words.numel(),), generator=g, device=dev)
        epoch11 = _s64((1 + launch % 2047) << 53)
        if rep == 1:
            words.copy_(low | epoch11)
        elif rep == 2:
            words.copy_(low | epoch11)
            words[0::2] = low[0::2] | _s64(launch << 32)
        x = pkg.synth.activations(1, 2048, 30 + rep, dev)[0]
        _check_head(pkg, dev, w, x, k, ws=ws)
    assert ws.error_bits() == 0
