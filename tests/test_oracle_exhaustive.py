"""Exhaustive and closed-form pins of the oracle's integer/byte arithmetic:
f16 conversion, U4 nibble unpack, U4 dequant over every (q, z, scale), and
f64 brute-force bounds for the f32 matvec."""

import numpy as np
import pytest

import oracle


def test_half_to_float_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.half_to_float(bits)
    exp = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(exp)
    assert np.array_equal(got[finite].view(np.uint32), exp[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(exp)]))
    assert np.array_equal(np.isinf(got), np.isinf(exp))


def test_float_to_half_rne():
    rng = np.random.default_rng(1)
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    hv = halves.view(np.float16).astype(np.float32)
    hv = hv[np.isfinite(hv)]
    # every representable value, the midpoints between neighbours (ties) and
    # values one f32 ulp either side of each midpoint
    s = np.sort(np.unique(hv))
    mid = ((s[:-1].astype(np.float64) + s[1:]) / 2).astype(np.float32)
    cand = np.concatenate([
        hv, mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf)),
        rng.standard_normal(200000).astype(np.float32) * np.float32(1000),
        rng.standard_normal(200000).astype(np.float32) * np.float32(1e-5),
        np.array([65504, 65519.99, 65520, 70000, -65520, 1e-8, 2.0 ** -25, 2.0 ** -24,
                  3 * 2.0 ** -26], np.float32)])
    got = oracle.float_to_half(cand)
    exp = cand.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)


def test_u4_unpack_all_bytes():
    b = np.arange(256, dtype=np.uint32).astype(np.uint8)
    codes = oracle.u4_unpack(b)
    assert np.array_equal(codes[0::2], b & 0x0F)  # low nibble = even index
    assert np.array_equal(codes[1::2], b >> 4)


@pytest.mark.slow
def test_u4_dequant_exhaustive():
    """Every finite f16 scale x every (q, z): f32(q - z) * f32(s), bit-exact."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    sv = bits.view(np.float16)
    scales = bits[np.isfinite(sv)]                 # 63488 patterns incl. +-0, subnormals
    n = scales.size
    k, group = 512, 32                             # 16 groups: z_g = g
    q = np.tile(np.arange(16, dtype=np.uint8), k // 16)
    packed_row = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    qweight = np.broadcast_to(packed_row, (n, k // 2)).copy()
    scale = np.repeat(scales[:, None], k // group, axis=1)
    zl = np.tile(np.arange(16, dtype=np.uint8), n)           # flat [n*16] zero points
    zp = (zl[0::2] | (zl[1::2] << 4)).astype(np.uint8)
    got = oracle.u4_dequant(qweight, scale, zp, n, k, group)
    z = np.repeat(np.arange(16, dtype=np.int32), group)       # z per column
    qz = (q.astype(np.int32) - z).astype(np.float32)
    exp = qz[None, :] * scales.view(np.float16).astype(np.float32)[:, None]
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def _rand_u4(rng, n, k, group):
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = (np.abs(rng.normal(0, 0.02, (n, k // group))) + 1e-3).astype(np.float16).view(np.uint16)
    z = rng.integers(0, 256, ((n * (k // group) + 1) // 2,), dtype=np.uint8)
    return q, s, z


def _dequant_np(q, s, z, n, k, group):
    codes = np.empty((n, k), np.int64)
    codes[:, 0::2] = q & 0x0F
    codes[:, 1::2] = q >> 4
    zl = np.empty(z.size * 2, np.int64)
    zl[0::2] = z & 0x0F
    zl[1::2] = z >> 4
    zz = zl[: n * (k // group)].reshape(n, k // group)
    sc = s.view(np.float16).astype(np.float64)
    return (codes - np.repeat(zz, group, axis=1)) * np.repeat(sc, group, axis=1)


@pytest.mark.parametrize("n,k,group", [(64, 256, 128), (33, 512, 64), (7, 2048, 128),
                                       (5, 128, 32)])
def test_dequant_matches_numpy(n, k, group):
    rng = np.random.default_rng(n * 131 + k)
    q, s, z = _rand_u4(rng, n, k, group)
    got = oracle.u4_dequant(q, s, z, n, k, group)
    exp = _dequant_np(q, s, z, n, k, group).astype(np.float32)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("n,k,group", [(64, 256, 128), (16, 2048, 128), (9, 512, 64)])
def test_matvec_brute_force_bound(n, k, group):
    """|y - y_f64| <= gamma_K * sum|w x| (sequential f32 summation bound)."""
    rng = np.random.default_rng(k + n)
    q, s, z = _rand_u4(rng, n, k, group)
    x = rng.standard_normal(k).astype(np.float16).astype(np.float32)
    y = oracle.u4_matvec(q, s, z, n, k, x, group=group)
    w = _dequant_np(q, s, z, n, k, group)
    exact = w @ x.astype(np.float64)
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    bound = gamma * (np.abs(w) @ np.abs(x.astype(np.float64))) + 1e-30
    assert np.all(np.abs(y - exact) <= bound)
    # a dropped zero point lands far outside the bound
    zl = np.zeros_like(z)
    y0 = oracle.u4_matvec(q, s, zl, n, k, x, group=group)
    assert not np.all(np.abs(y0 - exact) <= bound)


def test_matvec_threads_identical():
    rng = np.random.default_rng(5)
    q, s, z = _rand_u4(rng, 300, 512, 128)
    x = rng.standard_normal(512).astype(np.float32)
    a = oracle.u4_matvec(q, s, z, 300, 512, x, threads=1)
    b = oracle.u4_matvec(q, s, z, 300, 512, x, threads=7)
    assert np.array_equal(a, b)


def test_gpu_dot_trick_emulated():
    """The decode kernels' dot2 formulation (common.h XChunk): with f16 pairs
    (1024+q, x) and (1024+16q, x), sum (q - z) x = a1 + a16/16 - bias - z*xsum.
    Emulated here in f64 to pin the algebra (the bit tricks are exact)."""
    rng = np.random.default_rng(3)
    for _ in range(200):
        q = rng.integers(0, 16, 32)
        z = int(rng.integers(0, 16))
        x = rng.standard_normal(32).astype(np.float16).astype(np.float64)
        even, odd = np.arange(0, 32, 2), np.arange(1, 32, 2)
        a1 = np.sum((1024 + q[even]) * x[even])
        a16 = np.sum((1024 + 16 * q[odd]) * x[odd])
        bias = 1024 * x[even].sum() + 64 * x[odd].sum()
        got = a1 + a16 / 16 - bias - z * x.sum()
        exp = np.sum((q - z) * x)
        assert abs(got - exp) <= 1e-9 * (1 + np.sum(np.abs((q - z) * x)))
        # the bit patterns: 0x6400 | q is f16 1024+q; 0x6400 | (q << 4) is 1024+16q
        for qq in range(16):
            assert np.uint16(0x6400 | qq).view(np.float16) == 1024 + qq
            assert np.uint16(0x6400 | (qq << 4)).view(np.float16) == 1024 + 16 * qq
