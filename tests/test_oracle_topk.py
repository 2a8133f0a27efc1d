"""CPU: the oracle's LM-head top-k against a literal restatement of the
reference's per-block insertion (q4x8_matvec.cl:997-1015) and a sequential
merge, on small inputs with many ties."""

import numpy as np
import pytest

import oracle


def _insertion_topk(values, k, block):
    """Pure-Python loops: per 256-row block, the reference's insertion into
    best[0..k); then one more insertion pass over the block lists in order."""
    def insert(best, cand_v, cand_i):
        pos = 0
        while pos < k and best[pos][0] >= cand_v:
            pos += 1
        if pos < k:
            best.insert(pos, (cand_v, cand_i))
            del best[k:]
    parts = []
    for b0 in range(0, len(values), block):
        best = [(-np.inf, -1)] * k
        best = list(best)
        for i in range(b0, min(len(values), b0 + block)):
            insert(best, float(values[i]), i)
        parts.extend(best)
    final = [(-np.inf, -1)] * k
    final = list(final)
    for v, i in parts:
        if i >= 0:
            insert(final, v, i)
    return np.array([i for _, i in final], np.int32), np.array([v for v, _ in final], np.float32)


@pytest.mark.parametrize("n,k,levels", [(10, 3, 4), (300, 8, 5), (1000, 8, 3), (777, 16, 50),
                                        (513, 1, 2), (2000, 8, 1000)])
def test_lm_head_topk_matches_insertion(n, k, levels):
    rng = np.random.default_rng(n + k)
    v = rng.integers(0, levels, n).astype(np.float32) - levels / 2  # many ties
    got_i, got_v = oracle.lm_head_topk(v, k)
    ref_i, ref_v = _insertion_topk(v, k, 256)
    assert np.array_equal(got_i, ref_i) and np.array_equal(got_v, ref_v)
    # and the definition: value descending, lower index first among equals
    order = np.lexsort((np.arange(n), -v))[:k]
    assert np.array_equal(got_i, order.astype(np.int32))
