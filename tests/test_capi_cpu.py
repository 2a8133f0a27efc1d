"""The C-ABI library on a host without a GPU: it loads, exports every entry
point the header declares, binds to torch's HIP runtime, and rejects bad
arguments with the documented error codes before launching anything."""

import ctypes as C
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aima_u4moe.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(aima_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "aima_u4_matvec" in names and "aima_moe_grouped_prefill" in names
    assert len(names) >= 16


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg._lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(pkg._lib.SIGNATURES)


def test_library_shares_torch_hip_runtime(pkg):
    pkg._lib.lib()
    maps = open("/proc/self/maps").read()
    hip = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(hip) == 1, hip


def test_version_and_error_paths(pkg):
    L = pkg._lib.lib()
    assert L.aima_version() == 102
    rc = L.aima_u4_matvec(None, None, None, None, 4, 2048, 128, None, 0, None)
    assert rc == pkg._lib.AIMA_E_INVALID
    assert b"null pointer" in L.aima_last_error()
    # fake but aligned device pointers: validation happens before any launch
    p = C.c_void_p(1 << 20)
    rc = L.aima_u4_matvec(p, p, p, p, 4, 3000, 128, p, 0, None)
    assert rc == pkg._lib.AIMA_E_INVALID  # k not a multiple of group
    rc = L.aima_u4_matvec(p, p, p, p, 4, 2048, 100, p, 0, None)
    assert rc == pkg._lib.AIMA_E_INVALID  # bad group
    rc = L.aima_u4_matvec(p, p, p, p, 4, 3072, 128, p, 0, None)
    assert rc == pkg._lib.AIMA_E_UNSUPPORTED  # K not a power of two
    rc = L.aima_u4_matvec(p, C.c_void_p((1 << 20) + 4), p, p, 4, 2048, 128, p, 0, None)
    assert rc == pkg._lib.AIMA_E_INVALID  # misaligned qweight
    rc = L.aima_router_topk(p, 4, 256, 17, 1e-4, p, p, None)
    assert rc == pkg._lib.AIMA_E_INVALID  # k > 16


def _fake_layer(pkg, H=2048, I=512, E=256, group=128):
    p = 1 << 20
    t = pkg._lib.U4TensorC(p, p, p)
    return pkg._lib.MoeLayerC(t, t, t, t, p, p, H, I, I, E, group)


def test_workspace_sizes(pkg):
    L = pkg._lib
    lc = _fake_layer(pkg)
    dec = L.size_query("aima_moe_decode_workspace_size", C.byref(lc), 8)
    assert dec >= 256 + 9 * 512 * 2
    pre = L.size_query("aima_moe_prefill_workspace_size", C.byref(lc), 2048, 8)
    # act f16 [A+T][I] + contributions f16 [A+T][H] dominate
    assert pre >= (16384 + 2048) * (512 * 2 + 2048 * 2)
    stack = L.size_query("aima_moe_stack_prefill_workspace_size", C.byref(lc), 2048, 8)
    assert stack >= pre + 3 * 2048 * 2048 * 2
    sched = L.size_query("aima_grouped_schedule_workspace_size", 2048, 8, 256)
    assert 0 < sched < pre


def test_layer_validation(pkg):
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    bad_group = _fake_layer(pkg, group=64)
    rc = lib.aima_moe_grouped_prefill(C.byref(bad_group), p, None, 16, p, p, 8, p, p, 1 << 30,
                                      None)
    assert rc == L.AIMA_E_UNSUPPORTED
    lc = _fake_layer(pkg)
    rc = lib.aima_moe_grouped_prefill(C.byref(lc), p, None, 16, p, p, 8, p, p, 16, None)
    assert rc == L.AIMA_E_WORKSPACE
    rc = lib.aima_moe_ffn_decode(C.byref(lc), p, None, p, p, 300, p, p, 1 << 20, None)
    assert rc == L.AIMA_E_INVALID  # k > experts
    odd = _fake_layer(pkg, H=3000)
    rc = lib.aima_moe_ffn_decode(C.byref(odd), p, None, p, p, 8, p, p, 1 << 30, None)
    assert rc in (L.AIMA_E_INVALID, L.AIMA_E_UNSUPPORTED)
    rc = lib.aima_moe_stack_decode(C.byref(lc), 0, 1e-6, p, p, p, 8, p, p, 1 << 30, None)
    assert rc == L.AIMA_E_INVALID


def test_python_layer_rejects_cpu_tensors(pkg):
    layer = pkg.synth.moe_layer(hidden=256, inter=128, experts=8, seed=0, device="cpu")
    x = torch.zeros(256, dtype=torch.float16)
    ids = torch.zeros(8, dtype=torch.int32)
    w = torch.zeros(8, dtype=torch.float32)
    with pytest.raises(ValueError):
        pkg.run_moe_ffn_layer(layer, x, ids, w)
    with pytest.raises(ValueError):
        pkg.matvec_u4(x, layer.shared_gate_up)


def test_u4_weight_validation(pkg):
    q = torch.zeros((4, 64), dtype=torch.uint8)
    s = torch.zeros((4, 1), dtype=torch.float16)
    z = torch.zeros(2, dtype=torch.uint8)
    pkg.U4Weight(q, s, z, rows=4, k=128, group=128)
    with pytest.raises(ValueError):
        pkg.U4Weight(q, s, z, rows=4, k=256, group=128)
    with pytest.raises(TypeError):
        pkg.U4Weight(q, s.float(), z, rows=4, k=128, group=128)


def test_synthetic_distributions(pkg):
    layer = pkg.synth.moe_layer(hidden=256, inter=128, experts=4, seed=3, device="cpu")
    s = layer.gate_up.scale.float()
    assert float(s.min()) >= 1e-3 - 1e-6 and 0.01 < float(s.mean()) < 0.03
    q = layer.gate_up.qweight
    lo, hi = (q & 15).float().mean().item(), (q >> 4).float().mean().item()
    assert 7.0 < lo < 8.0 and 7.0 < hi < 8.0
    b = pkg.synth.zipf_bias(256, 1.1, seed=2, device="cpu")
    p = torch.exp(b.double())
    assert abs(float(p.sum()) - 1.0) < 1e-6  # f32 log-probabilities
    assert float(p.max() / p.min()) > 400  # 256^1.1 ~ 446


def test_new_entry_point_validation(pkg):
    """The multi-output FC, router FC, top-k, LM head, ingestion and routed
    stack entry points reject bad arguments before any launch."""
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    t = L.U4TensorC(1 << 20, 1 << 20, 1 << 20)
    tens = (L.U4TensorC * 5)(*([t] * 5))
    ns = (C.c_int64 * 5)(*([64] * 5))
    ys = (C.c_void_p * 5)(*([1 << 20] * 5))
    dts = (C.c_int32 * 5)(*([0] * 5))
    assert lib.aima_u4_matvec_multi(p, 0, tens, ns, 2048, 128, ys, dts, None) == L.AIMA_E_INVALID
    assert lib.aima_u4_matvec_multi(p, 5, tens, ns, 2048, 128, ys, dts, None) == L.AIMA_E_INVALID
    bad_dt = (C.c_int32 * 5)(*([7] * 5))
    assert lib.aima_u4_matvec_multi(p, 2, tens, ns, 2048, 128, ys, bad_dt, None) == L.AIMA_E_INVALID
    assert lib.aima_u4_matvec_multi(p, 2, tens, ns, 3072, 128, ys, dts, None) == \
        L.AIMA_E_UNSUPPORTED  # K not a power of two
    assert lib.aima_router_fc_topk(p, C.byref(t), 2000, 2048, 128, 8, 1e-4, p, p, p, None) == \
        L.AIMA_E_INVALID  # experts > 1024
    assert lib.aima_router_fc_topk(p, C.byref(t), 256, 2048, 128, 17, 1e-4, p, p, p, None) == \
        L.AIMA_E_INVALID  # k > 16
    sz = C.c_size_t(0)
    assert lib.aima_topk_workspace_size(1 << 21, 8, C.byref(sz)) == L.AIMA_E_INVALID
    assert lib.aima_topk_workspace_size(248320, 8, C.byref(sz)) == L.AIMA_OK and sz.value > 0
    assert lib.aima_topk_f32(p, 100, 0, p, p, None, 0, None) == L.AIMA_E_INVALID
    assert lib.aima_topk_f32(p, 248320, 8, p, p, None, 0, None) == L.AIMA_E_INVALID  # no workspace
    assert lib.aima_u4_lm_head_topk(p, p, p, p, 248320, 2048, 128, 8, p, p, p, None, 0, None) == \
        L.AIMA_E_INVALID  # workspace too small
    assert lib.aima_u4_group_major_to_rows(p, p, 3, 3, p, p, None) == L.AIMA_E_INVALID  # odd n*G
    assert lib.aima_u4_rows_to_group_major(None, p, 4, 4, p, p, None) == L.AIMA_E_INVALID
    assert lib.aima_q4k_unpack(p, 4, 300, p, p, p, None) == L.AIMA_E_INVALID  # cols % 256
    lc = _fake_layer(pkg)
    rt = (L.U4TensorC * 1)(t)
    assert lib.aima_moe_stack_decode_routed(C.byref(lc), rt, 1, 1e-6, p, 8, 1e-4, p, p, p, p, 16,
                                            None) == L.AIMA_E_WORKSPACE
    assert lib.aima_moe_stack_decode_routed(C.byref(lc), rt, 1, 1e-6, p, 8, 0.0, p, p, p, p,
                                            1 << 30, None) == L.AIMA_E_INVALID


def test_prefill_rejects_batches_past_the_offset_limit(pkg):
    """tokens * (k + 1) * inter must stay below 2^30 f16 elements (32-bit byte
    offsets in the grouped GEMM): 233,017 tokens at k = 8, inter = 512 is the
    first batch refused."""
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    lc = _fake_layer(pkg)
    for T in (233017, 233018, 1 << 20):
        rc = lib.aima_moe_grouped_prefill(C.byref(lc), p, None, T, p, p, 8, p, p, 1 << 40, None)
        assert rc == L.AIMA_E_INVALID, T
        assert b"2^30" in lib.aima_last_error()


def test_run_layer_entry_validation(pkg):
    """aima_moe_grouped_prefill_ex (RunLayer's contract) checks its options,
    the top-k stride and the split tensors before any launch."""
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    lc = _fake_layer(pkg)
    opt = L.PrefillOptionsC()
    opt.output_mode = L.AIMA_PREFILL_ROUTED_F32

    def call(layer=lc, o=opt, residual=None, topk=p, ws_bytes=1 << 40):
        return lib.aima_moe_grouped_prefill_ex(C.byref(layer), p, residual, 64, topk, p, 8, p,
                                               C.byref(o), p, ws_bytes, None)

    assert call(ws_bytes=16) == L.AIMA_E_WORKSPACE  # everything else valid
    opt.topk_stride = 28  # < 4 * k
    assert call() == L.AIMA_E_INVALID and b"topk_stride" in lib.aima_last_error()
    opt.topk_stride = 34  # not a multiple of 4
    assert call() == L.AIMA_E_INVALID
    opt.topk_stride = 48
    assert call(ws_bytes=16) == L.AIMA_E_WORKSPACE
    assert call(topk=C.c_void_p((1 << 20) + 2)) == L.AIMA_E_INVALID  # misaligned ids
    assert call(residual=p) == L.AIMA_E_INVALID  # routed output takes no residual
    bad = L.PrefillOptionsC()
    bad.output_mode = 5
    assert call(o=bad) == L.AIMA_E_INVALID
    bad.output_mode, bad.input_f32 = 0, 2
    assert call(o=bad) == L.AIMA_E_INVALID
    # routed-only needs no shared expert tensors
    noshared = _fake_layer(pkg)
    noshared.shared_gate_up = L.U4TensorC(None, None, None)
    noshared.shared_down = L.U4TensorC(None, None, None)
    noshared.shared_gate_vec = None
    assert call(layer=noshared, ws_bytes=16) == L.AIMA_E_WORKSPACE
    full = L.PrefillOptionsC()
    assert call(layer=noshared, o=full) == L.AIMA_E_INVALID
    # a split up tensor must be complete
    half = _fake_layer(pkg)
    half.up = L.U4TensorC(1 << 20, None, 1 << 20)
    assert call(layer=half) == L.AIMA_E_INVALID
    assert lib.aima_moe_ffn_decode(C.byref(half), p, None, p, p, 8, p, p, 1 << 30, None) == \
        L.AIMA_E_INVALID
    ok_split = _fake_layer(pkg)
    ok_split.up = L.U4TensorC(1 << 20, 1 << 20, 1 << 20)
    ok_split.shared_up = L.U4TensorC(1 << 20, 1 << 20, 1 << 20)
    assert call(layer=ok_split, ws_bytes=16) == L.AIMA_E_WORKSPACE


def test_stack_prefill_requires_aligned_norm(pkg):
    """The fused combine reads the next layer's norm weights as 16-byte
    vectors, so the stack entry checks their alignment."""
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    lc = _fake_layer(pkg)
    lc.norm_weight = (1 << 20) + 4
    rc = lib.aima_moe_stack_prefill(C.byref(lc), 1, 1e-6, p, 64, p, p, 8, p, p, 1 << 40, None)
    assert rc == L.AIMA_E_INVALID and b"norm_weight" in lib.aima_last_error()


def test_prefill_workspace_views(pkg):
    """The views point into the workspace, in its layout order, without
    overlapping, and end inside the size the size query reports."""
    L = pkg._lib
    lc = _fake_layer(pkg)
    T, k = 2048, 8
    size = L.size_query("aima_moe_prefill_workspace_size", C.byref(lc), T, k)
    base = 1 << 30
    v = L.PrefillViewsC()
    L.call("aima_moe_prefill_workspace_views", C.byref(lc), T, k, C.c_void_p(base), C.byref(v))
    A = T * k
    spans = [(v.offsets, 256 * 4), (v.tiles, 16), (v.token_map, A * 4), (v.inverse_map, A * 4),
             (v.compact_weights, A * 4), (v.swiglu, (A + T) * 512 * 2),
             (v.contributions, (A + T) * 2048 * 2)]
    end = base
    for ptr, n in spans:
        assert ptr >= end and ptr % 256 == 0
        end = ptr + n
    assert end <= base + size
    assert base <= v.tile_count < v.offsets


def _tiles_needed(counts, T, bm=256):
    """Tile records the schedule writes: per expert with rows, its full 256-row
    tiles and one remainder tile; the shared expert's T rows likewise."""
    n = sum(c // bm + (1 if c % bm else 0) for c in counts)
    return n + T // bm + (1 if T % bm else 0)


@pytest.mark.parametrize("T,k,E", [(1, 8, 256), (7, 8, 256), (2048, 8, 256), (300, 16, 1024),
                                   (16384, 8, 256), (33, 1, 4)])
def test_prefill_workspace_holds_every_tile(pkg, T, k, E):
    """The tile array of the prefill workspace (carved by the library's own
    layout, read back through aima_moe_prefill_workspace_views) has room for
    the tile records of any routing: uniform, concentrated on k experts,
    spread one row per expert, and Zipf-skewed, with the group sizes taken
    from the oracle's schedule (the checker)."""
    import numpy as np

    import oracle

    L = pkg._lib
    lc = _fake_layer(pkg, E=E)
    size = L.size_query("aima_moe_prefill_workspace_size", C.byref(lc), T, k)
    base = 1 << 30
    v = L.PrefillViewsC()
    L.call("aima_moe_prefill_workspace_views", C.byref(lc), T, k, C.c_void_p(base), C.byref(v))
    capacity = (v.token_map - v.tiles) // 16
    assert base + size >= v.contributions + (T * k + T) * 2048 * 2
    rng = np.random.default_rng(T * 31 + k * 7 + E)
    zipf = 1.0 / np.arange(1, E + 1) ** 1.1
    routings = {
        "uniform": np.stack([rng.permutation(E)[:k] for _ in range(T)]),
        "concentrated": np.tile(np.arange(k), (T, 1)),
        "spread": np.arange(T * k).reshape(T, k) % E,
        "zipf": np.stack([rng.choice(E, size=k, replace=False, p=zipf / zipf.sum())
                          for _ in range(T)]),
    }
    for name, ids in routings.items():
        ids = ids.astype(np.int32)
        assert all(len(set(r)) == k for r in ids.tolist())  # no expert twice per token
        s = oracle.build_grouped_schedule(ids, E)
        ends = s["offsets"].astype(np.int64)
        counts = np.diff(np.concatenate([[0], ends]))
        assert counts.sum() == T * k
        need = _tiles_needed(counts.tolist(), T)
        assert need <= capacity, (name, need, capacity)


def test_dequant_f16_validation(pkg):
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    assert lib.aima_u4_dequant_f16(p, p, p, 4, 256, 128, None, None) == L.AIMA_E_INVALID
    assert lib.aima_u4_dequant_f16(p, p, p, 4, 256, 100, p, None) == L.AIMA_E_INVALID
    assert lib.aima_u4_dequant_f16(p, p, p, 4, 256, 128, C.c_void_p((1 << 20) + 8), None) == \
        L.AIMA_E_INVALID  # out must be 16-byte aligned


def test_split_layout_round_trip(pkg):
    """to_split() keeps every gate and up row, scale and zero point."""
    layer = pkg.synth.moe_layer(hidden=256, inter=128, experts=4, seed=5, device="cpu")
    sp = layer.to_split()
    assert sp.split and sp.inter == 128 and sp.shared_inter == 128
    G = 2
    q = layer.gate_up.qweight
    assert torch.equal(sp.gate_up.qweight, q[:, :128]) and torch.equal(sp.up.qweight, q[:, 128:])
    assert torch.equal(sp.up.scale, layer.gate_up.scale[:, 128:])

    def nibbles(z, rows):
        z = z.reshape(z.shape[0] if z.dim() > 1 else 1, -1)
        return torch.stack([z & 15, z >> 4], -1).reshape(z.shape[0], rows, G)

    zc = nibbles(layer.gate_up.zp, 256)
    assert torch.equal(nibbles(sp.gate_up.zp, 128), zc[:, :128])
    assert torch.equal(nibbles(sp.up.zp, 128), zc[:, 128:])
    zs = nibbles(layer.shared_gate_up.zp, 256)
    assert torch.equal(nibbles(sp.shared_up.zp, 128), zs[:, 128:])
    assert sp.expert_bytes() == layer.expert_bytes()
    c = sp.c()
    assert c.up.qweight == sp.up.qweight.data_ptr() and layer.c().up.qweight is None


def test_router_gemm_validation(pkg):
    """The batched router rejects shapes its GEMM does not implement before
    any launch (hidden % 16, 16-byte alignment)."""
    L = pkg._lib
    lib = L.lib()
    p = C.c_void_p(1 << 20)
    odd = C.c_void_p((1 << 20) + 4)
    args = lambda x, H: (x, 1, 64, H, p, 256, 8, C.c_float(6.1e-5), p, p, p, None, 0, None)
    assert lib.aima_router_gemm_topk(*args(p, 2040)) == L.AIMA_E_INVALID
    assert lib.aima_router_gemm_topk(*args(odd, 2048)) == L.AIMA_E_INVALID
