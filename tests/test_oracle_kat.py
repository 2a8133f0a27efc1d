"""Known-answer tests of the CPU oracle, ported from the reference self test
(engine/tests/self_test.cpp:1082-1251).  Each check also runs against the
reference's own compiled code (oracle/_ref) when it was built."""

import numpy as np
import pytest

import oracle


IMPLS = [("oracle", lambda: oracle)] + (
    [("ref", lambda: oracle.Ref())] if oracle.ref_available() else [])


@pytest.mark.parametrize("name,get", IMPLS)
def test_rms_norm_kat(name, get):
    m = get()
    out = m.rms_norm([3.0, 4.0], [1.0, 2.0], 0.0)  # self_test.cpp:1082-1088
    assert abs(out[0] - 0.84852815) < 1e-6 and abs(out[1] - 2.2627418) < 1e-6


@pytest.mark.parametrize("name,get", IMPLS)
def test_swiglu_kat(name, get):
    m = get()
    out = m.swiglu_from_gate_up([1.0, -2.0, 3.0, 4.0, -1.0, 2.0, 0.5, -0.5], 2, 2)
    exp = [2.1931758, -0.9536231, -0.13447072, -0.8807971]  # self_test.cpp:1136-1144
    assert np.max(np.abs(out - np.array(exp, np.float32))) < 1e-6
    pair = m.swiglu_pair([1.0, -2.0], [3.0, 4.0])  # self_test.cpp:1236-1242
    assert abs(pair[0] - 2.1931758) < 1e-6 and abs(pair[1] - -0.9536231) < 1e-6


@pytest.mark.parametrize("name,get", IMPLS)
def test_sigmoid_kat(name, get):
    assert abs(get().sigmoid_scalar(0.0) - 0.5) < 1e-7  # self_test.cpp:1146


@pytest.mark.parametrize("name,get", IMPLS)
def test_softmax_topk_kat(name, get):
    m = get()
    p = m.softmax([1.0, 2.0])  # self_test.cpp:1203-1207
    assert abs(p[0] + p[1] - 1.0) < 1e-6 and p[1] > p[0]
    # tie -> lower index, self_test.cpp:1208-1211
    assert list(m.top_k_indices([0.1, 0.3, 0.3, 0.2], 2)) == [1, 2]


@pytest.mark.parametrize("name,get", IMPLS)
def test_normalize_weights_kat(name, get):
    m = get()
    assert list(m.normalize_weights([0.25, 0.75], 1e-6)) == [0.25, 0.75]
    c = m.normalize_weights([1e-8, 1e-8], 1e-4)  # clamp, self_test.cpp:1216-1224
    assert abs(c[0] - 1e-4) < 1e-10 and abs(c[1] - 1e-4) < 1e-10


@pytest.mark.parametrize("name,get", IMPLS)
def test_select_router_topk_kat(name, get):
    ids, w, nw = get().select_router_topk([0.0, 1.0, 2.0], 2, 1e-6)  # :1225-1235
    assert list(ids) == [2, 1]
    assert abs(nw[0] + nw[1] - 1.0) < 1e-6


@pytest.mark.parametrize("name,get", IMPLS)
def test_expert_weights_aggregate_kat(name, get):
    m = get()
    weighted = m.apply_expert_weights([1.0, 2.0, 3.0, 4.0], [0.25, 0.5], 2)  # :1243-1251
    assert list(weighted) == [0.25, 0.5, 1.5, 2.0]
    assert list(m.aggregate_experts(weighted, 2, 2)) == [1.75, 2.5]


def _u4_from_int_matrix(w: np.ndarray):
    """Encode a small non-negative integer matrix exactly: q = w, z = 0, s = 1."""
    n, k = w.shape
    assert w.min() >= 0 and w.max() <= 15
    q = w.astype(np.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    g = k // 32
    scale = np.full((n, g), 0x3C00, np.uint16)  # f16 1.0
    zp = np.zeros((n * g + 1) // 2, np.uint8)
    return packed, scale, zp


def _pad_x(vals):
    x = np.zeros(32, np.float32)
    x[: len(vals)] = vals
    return x


def test_matvec_orientation_kat():
    """self_test.cpp:1094-1101: [[1,2],[3,4],[5,6]] . [10,20] = [50,110,170],
    embedded in K=32 columns (the U4 layout needs K % 32 == 0 here)."""
    w = np.zeros((3, 32), np.int64)
    w[:, :2] = [[1, 2], [3, 4], [5, 6]]
    q, s, z = _u4_from_int_matrix(w)
    y = oracle.u4_matvec(q, s, z, 3, 32, _pad_x([10.0, 20.0]), group=32)
    assert list(y) == [50.0, 110.0, 170.0]


EXPERTS = np.zeros((2, 3, 32), np.int64)
EXPERTS[0, :, :2] = [[1, 2], [3, 4], [5, 6]]
EXPERTS[1, :, :2] = [[7, 8], [9, 10], [11, 12]]


def test_expert_matvec_orientation_kat():
    """self_test.cpp:1107-1116: ids {1, 0} with input [10, 20] give expert 1's
    rows then expert 0's: [230, 290, 350, 50, 110, 170]."""
    outs = []
    for e in (1, 0):
        q, s, z = _u4_from_int_matrix(EXPERTS[e])
        outs.append(oracle.u4_matvec(q, s, z, 3, 32, _pad_x([10.0, 20.0]), group=32))
    assert list(np.concatenate(outs)) == [230.0, 290.0, 350.0, 50.0, 110.0, 170.0]


def test_expert_matvec_per_expert_input_kat():
    """self_test.cpp:1117-1134: per-expert inputs [10,20] (expert 1) and
    [1,1] (expert 0) give [230, 290, 350, 3, 7, 11]."""
    outs = []
    for e, x in ((1, [10.0, 20.0]), (0, [1.0, 1.0])):
        q, s, z = _u4_from_int_matrix(EXPERTS[e])
        outs.append(oracle.u4_matvec(q, s, z, 3, 32, _pad_x(x), group=32))
    assert list(np.concatenate(outs)) == [230.0, 290.0, 350.0, 3.0, 7.0, 11.0]
