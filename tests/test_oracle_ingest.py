"""CPU: the oracle's weight-ingestion conversions.  Group-major order is
pinned by a hand-computed case, element-wise transposition and the round
trip; the Q4_K unpack by an independent encoder of the super-block format
(6-bit scale/min packing and code layout of GGUF Q4_K) whose values must come
back unchanged."""

import numpy as np
import pytest

import oracle


def test_group_major_hand_case():
    scale = np.array([10, 11, 12, 13], np.uint16)  # [n=2][groups=2]: (0,0) (0,1) (1,0) (1,1)
    zp = np.array([0x21, 0x43], np.uint8)          # nibbles 1, 2, 3, 4 in row-major order
    assert np.array_equal(oracle.group_major_scale(scale, 2, 2), [[10, 12], [11, 13]])
    # group-major nibble order: (g0,n0)=1 (g0,n1)=3 (g1,n0)=2 (g1,n1)=4
    assert np.array_equal(oracle.group_major_zero_point(zp, 2, 2), [0x31, 0x42])


@pytest.mark.parametrize("n,groups", [(7, 6), (1024, 16), (33, 2)])
def test_group_major_round_trip(n, groups):
    rng = np.random.default_rng(n * groups)
    scale = rng.integers(0, 1 << 15, n * groups).astype(np.uint16)
    codes = rng.integers(0, 16, n * groups).astype(np.uint8)
    zp = oracle.u4_pack(codes)
    sg = oracle.group_major_scale(scale, n, groups)
    zg = oracle.group_major_zero_point(zp, n, groups)
    gcodes = oracle.u4_nibbles(zg, n * groups).reshape(groups, n)
    for _ in range(50):
        r, g = rng.integers(0, n), rng.integers(0, groups)
        assert sg[g, r] == scale[r * groups + g] and gcodes[g, r] == codes[r * groups + g]
    s2, z2 = oracle.rows_from_group_major(sg, zg, n, groups)
    assert np.array_equal(s2.reshape(-1), scale) and np.array_equal(z2, zp)


def _encode_q4k(d, dmin, sc, mn, q):
    """One super-block from d, dmin (f16), 6-bit sc[8], mn[8] and codes q[256]."""
    packed = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            packed[j] = sc[j]
            packed[j + 4] = mn[j]
        else:
            packed[j + 4] = (sc[j] & 0x0F) | ((mn[j] & 0x0F) << 4)
            packed[j - 4] |= (sc[j] >> 4) << 6
            packed[j] |= (mn[j] >> 4) << 6
    qs = np.zeros(128, np.uint8)
    for s in range(4):
        for i in range(32):
            qs[32 * s + i] = q[64 * s + i] | (q[64 * s + 32 + i] << 4)
    head = np.array([d, dmin], np.float16).view(np.uint8)
    return np.concatenate([head, packed, qs])


@pytest.mark.parametrize("rows,cols", [(3, 256), (5, 1024)])
def test_q4k_unpack_recovers_encoded_values(rows, cols):
    rng = np.random.default_rng(rows + cols)
    bpr = cols // 256
    d = rng.uniform(1e-3, 2e-2, (rows, bpr)).astype(np.float16)
    dmin = rng.uniform(1e-3, 2e-2, (rows, bpr)).astype(np.float16)
    sc = rng.integers(0, 64, (rows, bpr, 8))
    mn = rng.integers(0, 64, (rows, bpr, 8))
    q = rng.integers(0, 16, (rows, bpr, 256))
    raw = np.concatenate([_encode_q4k(d[r, b], dmin[r, b], sc[r, b], mn[r, b], q[r, b])
                          for r in range(rows) for b in range(bpr)])
    codes, scale, mins = oracle.q4k_unpack(raw, rows, cols)
    assert np.array_equal(oracle.u4_nibbles(codes, rows * cols).reshape(rows, cols),
                          q.reshape(rows, cols))
    exp_scale = (d.astype(np.float32)[:, :, None] * sc.astype(np.float32)).astype(np.float16)
    exp_min = dmin.astype(np.float32)[:, :, None] * mn.astype(np.float32)
    assert np.array_equal(scale, exp_scale.reshape(rows, -1).view(np.uint16))
    assert np.array_equal(mins, exp_min.reshape(rows, -1))


def test_q4s_dequant_with_zero_mins_is_the_u4_dequant():
    """With every min 0 the scale-and-min form is the U4 form with zero
    points 0 at group 32: oracle.q4s_dequant equals oracle.u4_dequant (pinned
    bit-exact against the reference) bit for bit; a constant min m then
    subtracts m after the product, rounding once more."""
    rng = np.random.default_rng(5)
    n, k = 7, 256
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scale = (rng.standard_normal((n, k // 32)) * 0.02).astype(np.float16).view(np.uint16)
    zero_m = np.zeros((n, k // 32), np.float32)
    zp = np.zeros((n * (k // 32) + 1) // 2, np.uint8)
    w0 = oracle.q4s_dequant(codes, scale, zero_m, n, k)
    u4 = oracle.u4_dequant(codes, scale, zp, n, k, group=32)
    assert np.array_equal(w0.view(np.uint32), u4.reshape(n, k).view(np.uint32))
    m = np.float32(0.0123)
    w1 = oracle.q4s_dequant(codes, scale, np.full((n, k // 32), m, np.float32), n, k)
    assert np.array_equal(w1, (u4.reshape(n, k) - m).astype(np.float32))
