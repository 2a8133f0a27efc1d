"""GPU: the weight-ingestion kernels bit-exact against the oracle."""

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,groups", [(4096, 16), (1001, 64), (7, 2)])
def test_group_major_conversions(pkg, dev, n, groups):
    rng = np.random.default_rng(n + groups)
    scale = rng.integers(0, 1 << 15, n * groups).astype(np.uint16)
    zp = oracle.u4_pack(rng.integers(0, 16, n * groups).astype(np.uint8))
    s_t = torch.from_numpy(scale.view(np.float16)).to(dev)
    z_t = torch.from_numpy(zp).to(dev)
    sg, zg = pkg.u4_rows_to_group_major(s_t, z_t, n, groups)
    s2, z2 = pkg.u4_group_major_to_rows(sg, zg, n, groups)
    torch.cuda.synchronize()
    assert np.array_equal(sg.cpu().numpy().view(np.uint16), oracle.group_major_scale(scale, n, groups))
    assert np.array_equal(zg.cpu().numpy(), oracle.group_major_zero_point(zp, n, groups))
    assert np.array_equal(s2.cpu().numpy().view(np.uint16).reshape(-1), scale)
    assert np.array_equal(z2.cpu().numpy(), zp)


@pytest.mark.parametrize("rows,cols", [(64, 2048), (3, 512)])
def test_q4k_unpack(pkg, dev, rows, cols):
    rng = np.random.default_rng(rows * cols)
    bpr = cols // 256
    raw = rng.integers(0, 256, (rows, bpr, 144)).astype(np.uint8)
    # finite f16 d and dmin
    raw[:, :, 0:4] = rng.uniform(-0.05, 0.05, (rows, bpr, 2)).astype(np.float16).view(np.uint8) \
        .reshape(rows, bpr, 4)
    q, sc, mn = pkg.q4k_unpack(torch.from_numpy(raw.reshape(-1)).to(dev), rows, cols)
    torch.cuda.synchronize()
    rq, rsc, rmn = oracle.q4k_unpack(raw, rows, cols)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(sc.cpu().numpy().view(np.uint16), rsc)
    assert np.array_equal(mn.cpu().numpy(), rmn)
