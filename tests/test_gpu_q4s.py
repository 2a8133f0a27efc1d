"""GPU parity for the matvec over the Q4_K-derived scale-and-min form
(aima_q4s_matvec): against the oracle's dequantize-then-dot restatement, and
end to end from raw Q4_K super-blocks through the device unpack."""

import numpy as np
import pytest
import torch

import oracle
from tests.helpers import assert_parity, f16_to_f32

pytestmark = pytest.mark.gpu


def _synth(n, k, seed, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    codes = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, generator=g, device=dev)
    scale = (torch.rand((n, k // 32), generator=g, device=dev) * 0.02 + 1e-3).half()
    mins = torch.rand((n, k // 32), generator=g, device=dev) * 0.1
    return codes, scale, mins


@pytest.mark.parametrize("n,k", [(4096, 2048), (1000, 128), (300, 512), (513, 8192)])
@pytest.mark.parametrize("out", [torch.float32, torch.float16])
def test_q4s_matvec_matches_oracle(pkg, dev, n, k, out):
    codes, scale, mins = _synth(n, k, n + k, dev)
    x = pkg.synth.activations(1, k, n, dev)[0]
    y = pkg.q4s_matvec(x, codes, scale, mins, out_dtype=out)
    torch.cuda.synchronize()
    ref = oracle.q4s_matvec(codes.cpu().numpy(), scale.cpu().numpy().view(np.uint16),
                            mins.cpu().numpy(), n, k, f16_to_f32(x))
    got = y.float().cpu().numpy()
    assert_parity(got, ref, what=f"q4s_matvec n={n} k={k} {out}")


def test_q4s_matvec_from_q4k_blocks(pkg, dev):
    """Raw Q4_K blocks -> device unpack -> q4s matvec, against the oracle's
    unpack + dequantize + dot."""
    rng = np.random.default_rng(8)
    rows, cols = 1024, 2048
    raw = rng.integers(0, 256, (rows, cols // 256, 144), dtype=np.uint8)
    raw[:, :, 0:2] = rng.uniform(1e-4, 2e-3, (rows, cols // 256)).astype(np.float16) \
        .view(np.uint8).reshape(rows, cols // 256, 2)
    raw[:, :, 2:4] = rng.uniform(1e-4, 2e-3, (rows, cols // 256)).astype(np.float16) \
        .view(np.uint8).reshape(rows, cols // 256, 2)
    q, sc, mn = pkg.q4k_unpack(torch.from_numpy(raw.reshape(-1)).to(dev), rows, cols)
    x = pkg.synth.activations(1, cols, 3, dev)[0]
    y = pkg.q4s_matvec(x, q, sc, mn)
    torch.cuda.synchronize()
    rc, rs, rm = oracle.q4k_unpack(raw, rows, cols)
    ref = oracle.q4s_matvec(rc, rs, rm, rows, cols, f16_to_f32(x))
    assert_parity(y.cpu().numpy(), ref, what="q4k blocks -> q4s matvec")


def test_q4s_matvec_rejects_bad_k(pkg, dev):
    codes, scale, mins = _synth(8, 96 * 2, 1, dev)
    with pytest.raises(pkg.AimaError):
        pkg.q4s_matvec(pkg.synth.activations(1, 192, 1, dev)[0], codes, scale, mins)
