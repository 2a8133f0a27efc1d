"""The oracle's grouped schedule (BuildGroupedSchedule restatement,
grouped_s8_u4_prefill_runtime.cpp:231-346) against its invariants and a
brute-force construction, plus the error cases the reference throws on."""

import numpy as np
import pytest

import oracle


def brute_schedule(ids, experts):
    T, k = ids.shape
    pairs = sorted(((int(ids[t, r]), t, r) for t in range(T) for r in range(k)))
    token_map = np.array([t for _, t, _ in pairs], np.int32)
    inverse = np.empty(T * k, np.int32)
    for row, (_, t, r) in enumerate(pairs):
        inverse[t * k + r] = row
    counts = np.bincount(ids.reshape(-1), minlength=experts)
    return np.cumsum(counts).astype(np.int32), token_map, inverse


def topk_ids(rng, T, E, k):
    return np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)


@pytest.mark.parametrize("T,E,k", [(1, 16, 8), (37, 16, 8), (256, 256, 8), (100, 64, 6),
                                   (5, 8, 8)])
def test_schedule_matches_brute_force(T, E, k):
    rng = np.random.default_rng(T * 7 + E)
    ids = topk_ids(rng, T, E, k)
    w = rng.random((T, k)).astype(np.float32)
    s = oracle.build_grouped_schedule(ids, E, w)
    offsets, token_map, inverse = brute_schedule(ids, E)
    assert np.array_equal(s["offsets"], offsets)
    assert np.array_equal(s["token_map"], token_map)
    assert np.array_equal(s["inverse_map"], inverse)
    # invariants: offsets monotone ending at T*k; inverse is a permutation;
    # each sorted row carries its (token, rank)'s router weight
    assert s["offsets"][-1] == T * k and np.all(np.diff(s["offsets"]) >= 0)
    assert np.array_equal(np.sort(s["inverse_map"]), np.arange(T * k))
    assert np.array_equal(s["compact_weights"][s["inverse_map"]], w.reshape(-1))
    assert np.array_equal(s["token_map"][s["inverse_map"]], np.repeat(np.arange(T), k))
    counts = np.diff(np.concatenate([[0], s["offsets"]]))
    assert s["active_experts"] == int(np.sum(counts > 0))
    assert s["max_group"] == int(counts.max())


def test_schedule_rejects_bad_ids():
    ids = np.array([[0, 1, 2, 3], [4, 5, 6, 4]], np.int32)  # duplicate in token 1
    with pytest.raises(oracle.OracleError):
        oracle.build_grouped_schedule(ids, 8)
    ids = np.array([[0, 1, 2, 8]], np.int32)  # out of range
    with pytest.raises(oracle.OracleError):
        oracle.build_grouped_schedule(ids, 8)
    ids = np.array([[0, 1, -1, 3]], np.int32)
    with pytest.raises(oracle.OracleError):
        oracle.build_grouped_schedule(ids, 8)
