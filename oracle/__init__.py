"""CPU oracle for the U4 MoE expert hot path -- TEST INFRASTRUCTURE ONLY.

Python bindings over ``liborc_u4moe.so`` (the C restatement in
``u4moe_oracle.c``) and, when it was built, ``_ref/libiq36_ref.so`` (the
reference engine's own ``engine/src/gguf_loader.cpp`` behind a small shim).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only as the checker or the timed CPU
baseline.  The product library never calls it and has no CPU fallback.

Arrays are numpy; the U4 layout is the boundary layout documented in the C
file: ``qweight u8[N][K/2]`` (low nibble = even k), ``scale f16[N][K/g]``,
``zp`` u4 packed over the flat ``[N*G]`` index (low nibble = even).
"""

from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liborc_u4moe.so")
REF_PATH = os.path.join(_HERE, "_ref", "libiq36_ref.so")

MIN_WEIGHT_SUM = 6.103515625e-5  # gguf_loader.cpp:5665

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = C.c_int64


class OracleError(RuntimeError):
    pass


def build(ref: bool = True) -> None:
    """Compile the oracle (and the reference shim when the reference exists)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE, "all"], check=True)
    if ref and os.path.isdir("/root/reference/engine/src"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build(ref=False)
        L = C.CDLL(LIB_PATH)
        L.orc_half_to_float.restype = C.c_float
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_float_to_half.restype = C.c_uint16
        L.orc_float_to_half.argtypes = [C.c_float]
        L.orc_half_to_float_array.argtypes = [_u16p, _i64, _f32p]
        L.orc_float_to_half_array.argtypes = [_f32p, _i64, _u16p]
        L.orc_u4_unpack.argtypes = [_u8p, _i64, _u8p]
        L.orc_u4_dequant.argtypes = [_u8p, _u16p, _u8p, _i64, _i64, _i64, _f32p]
        L.orc_u4_matvec.argtypes = [_u8p, _u16p, _u8p, _i64, _i64, _i64, _f32p, _f32p, _i64]
        L.orc_sigmoid_scalar.restype = C.c_float
        L.orc_sigmoid_scalar.argtypes = [C.c_float]
        L.orc_softmax.argtypes = [_f32p, _i64, _f32p]
        L.orc_top_k.argtypes = [_f32p, _i64, _i64, _i32p]
        L.orc_normalize_weights.argtypes = [_f32p, _i64, C.c_float, _f32p]
        L.orc_select_router_topk.argtypes = [_f32p, _i64, _i64, C.c_float, _i32p, _f32p, _f32p]
        L.orc_router_topk_tokens.argtypes = [_f32p, _i64, _i64, _i64, C.c_float, _i32p, _f32p]
        L.orc_swiglu_pair.argtypes = [_f32p, _f32p, _i64, _f32p]
        L.orc_swiglu_from_gate_up.argtypes = [_f32p, _i64, _i64, _f32p]
        L.orc_apply_expert_weights.argtypes = [_f32p, _f32p, _i64, _i64, _f32p]
        L.orc_aggregate_experts.argtypes = [_f32p, _i64, _i64, _f32p]
        L.orc_rms_norm.argtypes = [_f32p, _f32p, _i64, C.c_float, _f32p]
        L.orc_moe_ffn_token_detail.argtypes = [C.c_void_p] * 16
        L.orc_moe_ffn_tokens.argtypes = [C.c_void_p, _i64, C.c_void_p, C.c_void_p,
                                         C.c_void_p, C.c_void_p, _i64, C.c_void_p, _i64]
        L.orc_moe_routed_tokens.argtypes = [C.c_void_p, _i64, C.c_void_p, C.c_void_p,
                                            C.c_void_p, _i64, C.c_void_p, _i64]
        L.orc_moe_ffn_decode_threaded.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p,
                                                  C.c_void_p, C.c_void_p, _i64,
                                                  C.c_void_p, _i64]
        L.orc_moe_ffn_tokens_model.argtypes = [C.c_void_p, _i64, C.c_void_p, C.c_void_p,
                                               C.c_void_p, C.c_void_p, _i64, C.c_int,
                                               C.c_void_p, _i64]
        L.orc_build_grouped_schedule.argtypes = [_i32p, _i64, _i64, _i64, _f32p, _i32p,
                                                 _i32p, _i32p, _f32p, C.c_void_p,
                                                 C.c_void_p]
        _lib = L
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise OracleError(f"{what} failed with oracle code {rc}")


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------------------
# half precision
# --------------------------------------------------------------------------

def half_to_float(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    out = np.empty(bits.size, np.float32)
    lib().orc_half_to_float_array(bits, bits.size, out)
    return out


def float_to_half(values: np.ndarray) -> np.ndarray:
    values = _f32(values).reshape(-1)
    out = np.empty(values.size, np.uint16)
    lib().orc_float_to_half_array(values, values.size, out)
    return out


def f16_values(bits: np.ndarray) -> np.ndarray:
    """f32 values of an array of f16 bit patterns (any shape)."""
    bits = np.asarray(bits)
    return half_to_float(bits).reshape(bits.shape)


# --------------------------------------------------------------------------
# U4 layout
# --------------------------------------------------------------------------

@dataclass
class U4Tensor:
    """A stack of ``experts`` U4 matrices of shape [rows][k] (numpy, host)."""

    qweight: np.ndarray  # u8 [experts, rows, k//2]
    scale: np.ndarray    # u16 (f16 bits) [experts, rows, k//group]
    zp: np.ndarray       # u8 [experts, rows*(k//group)//2]
    rows: int
    k: int
    group: int = 128

    @property
    def experts(self) -> int:
        return int(self.qweight.shape[0])

    def expert(self, e: int) -> "U4Tensor":
        return U4Tensor(self.qweight[e:e + 1], self.scale[e:e + 1], self.zp[e:e + 1],
                        self.rows, self.k, self.group)


class _Tensor(C.Structure):
    _fields_ = [("qweight", C.c_void_p), ("scale", C.c_void_p), ("zp", C.c_void_p),
                ("rows", C.c_int64), ("k", C.c_int64), ("group", C.c_int64),
                ("experts", C.c_int64)]


class _Moe(C.Structure):
    _fields_ = [("gate_up", _Tensor), ("down", _Tensor), ("shared_gate_up", _Tensor),
                ("shared_down", _Tensor), ("shared_gate_vec", C.c_void_p),
                ("hidden", C.c_int64), ("inter", C.c_int64), ("shared_inter", C.c_int64)]


def _ctensor(t: U4Tensor) -> _Tensor:
    for a, dt in ((t.qweight, np.uint8), (t.scale, np.uint16), (t.zp, np.uint8)):
        assert a.dtype == dt and a.flags.c_contiguous
    return _Tensor(t.qweight.ctypes.data, t.scale.ctypes.data, t.zp.ctypes.data,
                   t.rows, t.k, t.group, t.experts)


@dataclass
class MoeWeights:
    """One MoE FFN layer: routed experts, one shared expert, shared gate."""

    gate_up: U4Tensor          # rows = 2*inter (gate rows first), k = hidden
    down: U4Tensor             # rows = hidden, k = inter
    shared_gate_up: U4Tensor   # experts = 1
    shared_down: U4Tensor      # experts = 1
    shared_gate_vec: np.ndarray  # u16 f16 bits [hidden]

    @property
    def hidden(self) -> int:
        return self.gate_up.k

    @property
    def inter(self) -> int:
        return self.gate_up.rows // 2

    @property
    def shared_inter(self) -> int:
        return self.shared_gate_up.rows // 2

    def _c(self):
        gate = f16_values(self.shared_gate_vec).astype(np.float32)
        s = _Moe(_ctensor(self.gate_up), _ctensor(self.down), _ctensor(self.shared_gate_up),
                 _ctensor(self.shared_down), gate.ctypes.data, self.hidden, self.inter,
                 self.shared_inter)
        return s, gate  # keep gate alive


def u4_unpack(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(packed.size * 2, np.uint8)
    lib().orc_u4_unpack(packed, packed.size, out)
    return out


def u4_dequant(qweight, scale, zp, n: int, k: int, group: int = 128) -> np.ndarray:
    out = np.empty((n, k), np.float32)
    _check(lib().orc_u4_dequant(np.ascontiguousarray(qweight, np.uint8).reshape(-1),
                                np.ascontiguousarray(scale, np.uint16).reshape(-1),
                                np.ascontiguousarray(zp, np.uint8).reshape(-1),
                                n, k, group, out.reshape(-1)), "u4_dequant")
    return out


def u4_matvec(qweight, scale, zp, n: int, k: int, x: np.ndarray, group: int = 128,
              threads: int = 1) -> np.ndarray:
    """y[n] = sum_k w[n][k] x[k] in f32 (sequential), x given as f32 values."""
    y = np.empty(n, np.float32)
    _check(lib().orc_u4_matvec(np.ascontiguousarray(qweight, np.uint8).reshape(-1),
                               np.ascontiguousarray(scale, np.uint16).reshape(-1),
                               np.ascontiguousarray(zp, np.uint8).reshape(-1),
                               n, k, group, _f32(x).reshape(-1), y, threads), "u4_matvec")
    return y


# --------------------------------------------------------------------------
# router and MoE glue
# --------------------------------------------------------------------------

def sigmoid_scalar(v: float) -> float:
    return float(lib().orc_sigmoid_scalar(v))


def softmax(logits) -> np.ndarray:
    logits = _f32(logits).reshape(-1)
    out = np.empty_like(logits)
    _check(lib().orc_softmax(logits, logits.size, out), "softmax")
    return out


def top_k_indices(values, k: int) -> np.ndarray:
    values = _f32(values).reshape(-1)
    out = np.empty(k, np.int32)
    _check(lib().orc_top_k(values, values.size, k, out), "top_k")
    return out


def lm_head_topk(values, k: int = 8, block: int = 256):
    """Top-k of an LM head's logits as the reference builds it
    (engine/gpu/opencl/q4x8_matvec.cl:973-1021): every block of 256 rows
    keeps its best k by insertion -- a candidate moves past every kept value
    >= itself, so an earlier index stays ahead of an equal later value -- and
    the per-block lists merge under the same order.  A stable sort on the
    negated values reproduces each insertion.  Returns (ids int32 [k],
    values f32 [k]); NaNs sort last."""
    v = _f32(values).reshape(-1)
    cand_v, cand_i = [], []
    for b0 in range(0, v.size, block):
        seg = v[b0:b0 + block]
        order = np.argsort(-seg, kind="stable")[:k]
        cand_v.append(seg[order])
        cand_i.append(order.astype(np.int64) + b0)
    cv = np.concatenate(cand_v)
    ci = np.concatenate(cand_i)
    top = np.argsort(-cv, kind="stable")[:k]
    return ci[top].astype(np.int32), cv[top].astype(np.float32)


def u4_nibbles(packed, count: int) -> np.ndarray:
    """Packed u4 stream (low nibble = even index) -> count codes."""
    p = np.asarray(packed, np.uint8).reshape(-1)
    out = np.empty(p.size * 2, np.uint8)
    out[0::2] = p & 0x0F
    out[1::2] = p >> 4
    return out[:count]


def u4_pack(codes) -> np.ndarray:
    c = np.asarray(codes, np.uint8).reshape(-1)
    if c.size % 2:
        c = np.concatenate([c, np.zeros(1, np.uint8)])
    return (c[0::2] & 0x0F) | ((c[1::2] & 0x0F) << 4)


def group_major_scale(scale, n: int, groups: int) -> np.ndarray:
    """f16 scale [n][groups] -> [groups][n]
    (tools/intel_qwen36_openvino_fixed_fc.py:218-229)."""
    return np.ascontiguousarray(np.asarray(scale, np.uint16).reshape(n, groups).T)


def group_major_zero_point(zp, n: int, groups: int) -> np.ndarray:
    """u4 zero points over [n][groups] -> packed over [groups][n]
    (tools/intel_qwen36_openvino_fixed_fc.py:241-265)."""
    logical = u4_nibbles(zp, n * groups).reshape(n, groups)
    return u4_pack(np.ascontiguousarray(logical.T))


def rows_from_group_major(scale_gm, zp_gm, n: int, groups: int):
    """Inverse of group_major_scale / group_major_zero_point."""
    scale = np.ascontiguousarray(np.asarray(scale_gm, np.uint16).reshape(groups, n).T)
    zp = u4_pack(np.ascontiguousarray(u4_nibbles(zp_gm, n * groups).reshape(groups, n).T))
    return scale, zp


Q4K_VALUES = 256
Q4K_BYTES = 144


def q4k_scale_min(packed12, j: int):
    """6-bit scale and min of sub-block j from the 12 packed bytes of a Q4_K
    super-block (tools/intel-qwen36-openvino-moe-micro-prepack.py:76-88)."""
    q = [int(v) for v in packed12]
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def q4k_unpack(raw, rows: int, cols: int, f32_scale: bool = False):
    """Q4_K [rows][cols] -> (codes u8 [rows][cols/2] boundary packing, scale
    f16 bits [rows][cols/32] = f16(d * sc), min f32 [rows][cols/32] = dmin * m)
    (tools/intel-qwen36-openvino-moe-micro-prepack.py:91-124; row-major).
    With f32_scale, a fourth output: the f32 scale d * sc before the f16
    rounding (the d1 / d2 of the reference's decode_q4_k_block,
    gguf_loader.cpp:1011-1040)."""
    bpr = cols // Q4K_VALUES
    b = np.asarray(raw, np.uint8).reshape(rows, bpr, Q4K_BYTES)
    codes = np.empty((rows, cols), np.uint8)
    qs = b[:, :, 16:]
    for s in range(4):
        seg = qs[:, :, 32 * s:32 * s + 32]
        for blk in range(bpr):
            base = blk * Q4K_VALUES + 64 * s
            codes[:, base:base + 32] = seg[:, blk] & 0x0F
            codes[:, base + 32:base + 64] = seg[:, blk] >> 4
    d = b[:, :, 0:2].copy().view("<f2").reshape(rows, bpr).astype(np.float32)
    dmin = b[:, :, 2:4].copy().view("<f2").reshape(rows, bpr).astype(np.float32)
    sc = np.empty((rows, bpr, 8), np.float32)
    mn = np.empty((rows, bpr, 8), np.float32)
    for r in range(rows):
        for blk in range(bpr):
            for j in range(8):
                s6, m6 = q4k_scale_min(b[r, blk, 4:16], j)
                sc[r, blk, j] = np.float32(d[r, blk]) * np.float32(s6)
                mn[r, blk, j] = np.float32(dmin[r, blk]) * np.float32(m6)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    scale = sc.reshape(rows, bpr * 8).astype(np.float16).view(np.uint16)
    if f32_scale:
        return packed, scale, mn.reshape(rows, bpr * 8), sc.reshape(rows, bpr * 8)
    return packed, scale, mn.reshape(rows, bpr * 8)


def q4s_dequant(codes, scale_bits, mins, n: int, k: int) -> np.ndarray:
    """The scale-and-min form (q4k_unpack's output) -> f32 weights
    value = f32(scale) * q - min, per 32-wide group
    (tools/intel-qwen36-openvino-moe-micro-prepack.py:91-124: the prepacked
    scale = d * sc rounded to f16, min = dmin * m in f32)."""
    q = u4_nibbles(codes, n * k).reshape(n, k).astype(np.float32)
    s = half_to_float(np.asarray(scale_bits, np.uint16).reshape(-1)).reshape(n, k // 32)
    m = np.asarray(mins, np.float32).reshape(n, k // 32)
    return (q * np.repeat(s, 32, axis=1)).astype(np.float32) - np.repeat(m, 32, axis=1)


def q4s_matvec(codes, scale_bits, mins, n: int, k: int, x) -> np.ndarray:
    """y = q4s_dequant(...) . x, the products and sum in float64."""
    w = q4s_dequant(codes, scale_bits, mins, n, k).astype(np.float64)
    return (w @ _f32(x).reshape(-1).astype(np.float64)).astype(np.float32)


def normalize_weights(w, min_weight_sum: float) -> np.ndarray:
    w = _f32(w).reshape(-1)
    out = np.empty_like(w)
    _check(lib().orc_normalize_weights(w, w.size, min_weight_sum, out), "normalize_weights")
    return out


def select_router_topk(logits, k: int = 8, min_weight_sum: float = MIN_WEIGHT_SUM):
    """Returns (expert_ids int32[k], weights f32[k], normalized_weights f32[k])."""
    logits = _f32(logits).reshape(-1)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    nw = np.empty(k, np.float32)
    _check(lib().orc_select_router_topk(logits, logits.size, k, min_weight_sum, ids, w, nw),
           "select_router_topk")
    return ids, w, nw


def router_topk_tokens(logits, k: int = 8, min_weight_sum: float = MIN_WEIGHT_SUM):
    """logits f32 [T][E] -> (ids int32 [T][k], normalized weights f32 [T][k])."""
    logits = _f32(logits)
    T, E = logits.shape
    ids = np.empty((T, k), np.int32)
    nw = np.empty((T, k), np.float32)
    _check(lib().orc_router_topk_tokens(logits.reshape(-1), T, E, k, min_weight_sum,
                                        ids.reshape(-1), nw.reshape(-1)), "router_topk")
    return ids, nw


def swiglu_pair(gate, up) -> np.ndarray:
    gate, up = _f32(gate).reshape(-1), _f32(up).reshape(-1)
    out = np.empty_like(gate)
    _check(lib().orc_swiglu_pair(gate, up, gate.size, out), "swiglu_pair")
    return out


def swiglu_from_gate_up(gate_up, inter: int, experts: int) -> np.ndarray:
    gate_up = _f32(gate_up).reshape(-1)
    out = np.empty(inter * experts, np.float32)
    _check(lib().orc_swiglu_from_gate_up(gate_up, inter, experts, out), "swiglu_from_gate_up")
    return out


def apply_expert_weights(down, w, hidden: int) -> np.ndarray:
    down, w = _f32(down).reshape(-1), _f32(w).reshape(-1)
    out = np.empty_like(down)
    _check(lib().orc_apply_expert_weights(down, w, w.size, hidden, out), "apply_expert_weights")
    return out


def aggregate_experts(weighted, experts: int, hidden: int) -> np.ndarray:
    weighted = _f32(weighted).reshape(-1)
    out = np.empty(hidden, np.float32)
    _check(lib().orc_aggregate_experts(weighted, experts, hidden, out), "aggregate_experts")
    return out


def rms_norm(x, weight, eps: float) -> np.ndarray:
    x, weight = _f32(x).reshape(-1), _f32(weight).reshape(-1)
    out = np.empty_like(x)
    _check(lib().orc_rms_norm(x, weight, x.size, eps, out), "rms_norm")
    return out


def rms_norm_rows(x, weight, eps: float) -> np.ndarray:
    x = _f32(x)
    return np.stack([rms_norm(row, weight, eps) for row in x.reshape(-1, x.shape[-1])]
                    ).reshape(x.shape)


def moe_ffn_token_detail(mw: MoeWeights, x, residual, ids, w) -> dict:
    """One token with every intermediate (names follow Qwen36MoeFfnLayerResult)."""
    H, I, IS = mw.hidden, mw.inter, mw.shared_inter
    x = _f32(x).reshape(-1)
    res = None if residual is None else _f32(residual).reshape(-1)
    ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
    w = _f32(w).reshape(-1)
    k = ids.size
    o = {"residual": np.empty(H, np.float32), "selected_gate_up": np.empty(k * 2 * I, np.float32),
         "selected_swiglu": np.empty(k * I, np.float32), "selected_down": np.empty(k * H, np.float32),
         "moe_out": np.empty(H, np.float32), "shared_gate_up": np.empty(2 * IS, np.float32),
         "shared_swiglu": np.empty(IS, np.float32), "shared_down": np.empty(H, np.float32),
         "shared_gate": np.empty(2, np.float32), "ffn_out": np.empty(H, np.float32)}
    cs, keep = mw._c()
    rc = lib().orc_moe_ffn_token_detail(
        C.addressof(cs), x.ctypes.data, None if res is None else res.ctypes.data,
        ids.ctypes.data, w.ctypes.data, k, o["residual"].ctypes.data,
        o["selected_gate_up"].ctypes.data, o["selected_swiglu"].ctypes.data,
        o["selected_down"].ctypes.data, o["moe_out"].ctypes.data,
        o["shared_gate_up"].ctypes.data, o["shared_swiglu"].ctypes.data,
        o["shared_down"].ctypes.data, o["shared_gate"].ctypes.data, o["ffn_out"].ctypes.data)
    del keep
    _check(rc, "moe_ffn_token_detail")
    return o


def moe_ffn_tokens(mw: MoeWeights, x, ids, w, residual=None, threads: int = 8) -> np.ndarray:
    """Per-token MoE FFN over T tokens.  x/residual f32 [T][H]; ids/w [T][k]."""
    x = _f32(x)
    T = x.shape[0]
    ids = np.ascontiguousarray(ids, np.int32)
    w = _f32(w)
    res = None if residual is None else _f32(residual)
    out = np.empty((T, mw.hidden), np.float32)
    cs, keep = mw._c()
    rc = lib().orc_moe_ffn_tokens(C.addressof(cs), T, x.ctypes.data,
                                  None if res is None else res.ctypes.data, ids.ctypes.data,
                                  w.ctypes.data, ids.shape[1], out.ctypes.data, threads)
    del keep
    _check(rc, "moe_ffn_tokens")
    return out


def moe_routed_tokens(mw: MoeWeights, x, ids, w, threads: int = 8) -> np.ndarray:
    """Routed sum only, sum_r w_r * down_r(swiglu(gate_up_r x)), per token:
    the output of the reference's grouped RunLayer
    (grouped_s8_u4_prefill_runtime.hpp:100-121) with the CPU arithmetic of
    apply_expert_weights / aggregate_experts (gguf_loader.cpp:3773-3819)."""
    x = _f32(x)
    T = x.shape[0]
    ids = np.ascontiguousarray(ids, np.int32)
    w = _f32(w)
    out = np.empty((T, mw.hidden), np.float32)
    cs, keep = mw._c()
    rc = lib().orc_moe_routed_tokens(C.addressof(cs), T, x.ctypes.data, ids.ctypes.data,
                                     w.ctypes.data, ids.shape[1], out.ctypes.data, threads)
    del keep
    _check(rc, "moe_routed_tokens")
    return out


def moe_ffn_decode_threaded(mw: MoeWeights, x, ids, w, residual=None,
                            threads: int = 8) -> np.ndarray:
    """One token, row-parallel matvecs (the reference CPU decode pattern)."""
    x = _f32(x).reshape(-1)
    ids = np.ascontiguousarray(ids, np.int32).reshape(-1)
    w = _f32(w).reshape(-1)
    res = None if residual is None else _f32(residual).reshape(-1)
    out = np.empty(mw.hidden, np.float32)
    cs, keep = mw._c()
    rc = lib().orc_moe_ffn_decode_threaded(C.addressof(cs), x.ctypes.data,
                                           None if res is None else res.ctypes.data,
                                           ids.ctypes.data, w.ctypes.data, ids.size,
                                           out.ctypes.data, threads)
    del keep
    _check(rc, "moe_ffn_decode_threaded")
    return out


# Precision models (u4moe_oracle.c, orc_moe_ffn_tokens_model): the same layer
# with other rounding points and summation orders, used only to measure how
# far two correct implementations of a layer stack drift apart through the
# f16 residual.  Never a parity reference.
MODEL_ACT_F16 = 1       # SwiGLU rounded to f16 before the down matvec
MODEL_SLICED = 2        # persistent decode order: sum over x of (w_x d_x + sigma shared_x)
MODEL_CHUNKED = 4       # dot products as 32-element chunk sums + pairwise tree
MODEL_WEIGHT_F16 = 8    # dequantized weights rounded to f16 (prefill MFMA operand)
MODEL_CONTRIB_F16 = 16  # prefill combine: f16 contribution rows, fma with sigma
MODEL_F64 = 32          # f64 arithmetic (exact up to the f16 h and r roundings)
MODEL_DECODE_PLAN = MODEL_ACT_F16 | MODEL_SLICED | MODEL_CHUNKED
MODEL_PREFILL = MODEL_ACT_F16 | MODEL_CHUNKED | MODEL_WEIGHT_F16 | MODEL_CONTRIB_F16


def moe_ffn_tokens_model(mw: MoeWeights, x, ids, w, residual=None, flags: int = 0,
                         threads: int = 8) -> np.ndarray:
    """moe_ffn_tokens under a precision model (flags = 0: bit-identical)."""
    x = _f32(x)
    T = x.shape[0]
    ids = np.ascontiguousarray(ids, np.int32)
    w = _f32(w)
    res = None if residual is None else _f32(residual)
    out = np.empty((T, mw.hidden), np.float32)
    cs, keep = mw._c()
    rc = lib().orc_moe_ffn_tokens_model(C.addressof(cs), T, x.ctypes.data,
                                        None if res is None else res.ctypes.data,
                                        ids.ctypes.data, w.ctypes.data, ids.shape[1], int(flags),
                                        out.ctypes.data, threads)
    del keep
    _check(rc, "moe_ffn_tokens_model")
    return out


def rms_norm_rows_model(x, weight, eps: float, flags: int = 0) -> np.ndarray:
    """RMSNorm under a precision model: flags = 0 is rms_norm_rows; with
    MODEL_F64 the sum of squares and scaling are f64; with MODEL_CHUNKED the
    sum of squares is numpy's pairwise f32 sum (another f32 order)."""
    x = _f32(x)
    if not flags & (MODEL_F64 | MODEL_CHUNKED):
        return rms_norm_rows(x, weight, eps)
    wt = _f32(weight).reshape(-1)
    if flags & MODEL_F64:
        xd = x.astype(np.float64)
        scale = 1.0 / np.sqrt(np.mean(xd * xd, axis=-1, keepdims=True) + eps)
        return (xd * scale * wt.astype(np.float64)).astype(np.float32)
    ss = np.sum(x * x, axis=-1, keepdims=True, dtype=np.float32)
    scale = np.float32(1.0) / np.sqrt(ss / np.float32(x.shape[-1]) + np.float32(eps))
    return ((x * scale) * wt).astype(np.float32)


def moe_stack_chain_model(layers, norm_weights, x0_bits, ids, w, eps: float = 1e-6,
                          flags: int = 0, threads: int = 8):
    """moe_stack_tokens' chain under a precision model: per layer
    h = f16(rms_norm(r)), r = f16(r + ffn(h)).  Returns the last r (f16 bits)."""
    r = np.ascontiguousarray(x0_bits, np.uint16)
    for L, mw in enumerate(layers):
        rf = f16_values(r)
        h = f16_values(float_to_half(rms_norm_rows_model(rf, norm_weights[L], eps, flags))
                       .reshape(rf.shape))
        o = moe_ffn_tokens_model(mw, h, ids[L], w[L], residual=rf, flags=flags, threads=threads)
        r = float_to_half(o).reshape(o.shape)
    return r


def build_grouped_schedule(ids, experts: int, router_weights=None) -> dict:
    """ids int32 [T][k] -> schedule dict (offsets are exclusive ends per expert)."""
    ids = np.ascontiguousarray(ids, np.int32)
    T, k = ids.shape
    A = T * k
    w = _f32(np.zeros(A) if router_weights is None else router_weights).reshape(-1)
    offsets = np.empty(experts, np.int32)
    token_map = np.empty(A, np.int32)
    inverse_map = np.empty(A, np.int32)
    compact = np.empty(A, np.float32)
    active = C.c_int64()
    mx = C.c_int64()
    _check(lib().orc_build_grouped_schedule(ids.reshape(-1), T, k, experts, w, offsets,
                                            token_map, inverse_map, compact,
                                            C.byref(active), C.byref(mx)),
           "build_grouped_schedule")
    return {"offsets": offsets, "token_map": token_map, "inverse_map": inverse_map,
            "compact_weights": compact, "active_experts": active.value,
            "max_group": mx.value}


def moe_stack_tokens(layers, norm_weights, x0_bits, ids, w, eps: float = 1e-6,
                     threads: int = 8, start_layer: int = 0):
    """Config-4 semantics for a set of tokens through ``len(layers)`` layers.

    Per layer L: h = f16(rms_norm(r_L)); r_{L+1} = f16(r_L + ffn(h)), where
    r_0 = ``x0_bits`` (f16 bits [T][H]); ids/w are [L][T][k].  Returns the
    f16 bits of every layer's output, shape [L][T][H].
    """
    r = np.ascontiguousarray(x0_bits, np.uint16)
    outs = []
    for li, mw in enumerate(layers):
        L = start_layer + li
        rf = f16_values(r)
        h = f16_values(float_to_half(rms_norm_rows(rf, norm_weights[L], eps)).reshape(rf.shape))
        o = moe_ffn_tokens(mw, h, ids[L], w[L], residual=rf, threads=threads)
        r = float_to_half(o).reshape(o.shape)
        outs.append(r)
    return np.stack(outs)


# --------------------------------------------------------------------------
# reference shim (oracle/_ref), when built
# --------------------------------------------------------------------------

class Ref:
    """The reference's own CPU ops (engine/src/gguf_loader.cpp), via _ref."""

    def __init__(self, path: str = REF_PATH):
        L = C.CDLL(path)
        L.ref_last_error.restype = C.c_char_p
        L.ref_sigmoid_scalar.restype = C.c_float
        L.ref_sigmoid_scalar.argtypes = [C.c_float]
        L.ref_softmax.argtypes = [_f32p, _i64, _f32p]
        L.ref_top_k.argtypes = [_f32p, _i64, _i64, _i32p]
        L.ref_normalize_weights.argtypes = [_f32p, _i64, C.c_float, _f32p]
        L.ref_select_router_topk.argtypes = [_f32p, _i64, _i64, C.c_float, _i32p, _f32p, _f32p]
        L.ref_swiglu_pair.argtypes = [_f32p, _f32p, _i64, _f32p]
        L.ref_swiglu_from_gate_up.argtypes = [_f32p, _i64, _i64, _f32p]
        L.ref_apply_expert_weights.argtypes = [_f32p, _f32p, _i64, _i64, _f32p]
        L.ref_aggregate_experts.argtypes = [_f32p, _i64, _i64, _f32p]
        L.ref_rms_norm.argtypes = [_f32p, _f32p, _i64, C.c_float, _f32p]
        L.ref_matvec_f32.argtypes = [C.c_char_p, _f32p, _i64, _i64, _f32p, _f32p]
        L.ref_moe_ffn_layer_f32.argtypes = [C.c_char_p, _i64, _i64, _i64, _i64] + \
            [_f32p] * 8 + [C.c_float] + [C.c_void_p] * 12
        L.ref_decode_q4k_rows.argtypes = [C.c_char_p, _u8p, _i64, _i64, _f32p]
        self.L = L

    def _check(self, rc, what):
        if rc != 0:
            raise OracleError(f"reference {what}: {self.L.ref_last_error().decode()}")

    def sigmoid_scalar(self, v):
        return float(self.L.ref_sigmoid_scalar(v))

    def decode_q4k_rows(self, raw, rows: int, cols: int, path: str):
        """The reference's Q4_K decode (decode_q4_k_block via decode_tensor_row)
        of a raw [rows][cols] tensor -> f32 [rows][cols]."""
        raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
        out = np.empty((rows, cols), np.float32)
        self._check(self.L.ref_decode_q4k_rows(path.encode(), raw, rows, cols, out),
                    "decode_q4k_rows")
        return out

    def softmax(self, logits):
        logits = _f32(logits).reshape(-1)
        out = np.empty_like(logits)
        self._check(self.L.ref_softmax(logits, logits.size, out), "softmax")
        return out

    def top_k_indices(self, values, k):
        values = _f32(values).reshape(-1)
        out = np.empty(k, np.int32)
        self._check(self.L.ref_top_k(values, values.size, k, out), "top_k")
        return out

    def normalize_weights(self, w, m):
        w = _f32(w).reshape(-1)
        out = np.empty_like(w)
        self._check(self.L.ref_normalize_weights(w, w.size, m, out), "normalize")
        return out

    def select_router_topk(self, logits, k=8, m=MIN_WEIGHT_SUM):
        logits = _f32(logits).reshape(-1)
        ids = np.empty(k, np.int32)
        w = np.empty(k, np.float32)
        nw = np.empty(k, np.float32)
        self._check(self.L.ref_select_router_topk(logits, logits.size, k, m, ids, w, nw),
                    "select_router_topk")
        return ids, w, nw

    def swiglu_pair(self, g, u):
        g, u = _f32(g).reshape(-1), _f32(u).reshape(-1)
        out = np.empty_like(g)
        self._check(self.L.ref_swiglu_pair(g, u, g.size, out), "swiglu_pair")
        return out

    def swiglu_from_gate_up(self, gu, inter, experts):
        gu = _f32(gu).reshape(-1)
        out = np.empty(inter * experts, np.float32)
        self._check(self.L.ref_swiglu_from_gate_up(gu, inter, experts, out), "swiglu")
        return out

    def apply_expert_weights(self, down, w, hidden):
        down, w = _f32(down).reshape(-1), _f32(w).reshape(-1)
        out = np.empty_like(down)
        self._check(self.L.ref_apply_expert_weights(down, w, w.size, hidden, out), "weights")
        return out

    def aggregate_experts(self, weighted, experts, hidden):
        weighted = _f32(weighted).reshape(-1)
        out = np.empty(hidden, np.float32)
        self._check(self.L.ref_aggregate_experts(weighted, experts, hidden, out), "aggregate")
        return out

    def rms_norm(self, x, w, eps):
        x, w = _f32(x).reshape(-1), _f32(w).reshape(-1)
        out = np.empty_like(x)
        self._check(self.L.ref_rms_norm(x, w, x.size, eps, out), "rms_norm")
        return out

    def matvec_f32(self, w, x, tmpdir):
        w = _f32(w)
        x = _f32(x).reshape(-1)
        y = np.empty(w.shape[0], np.float32)
        path = os.path.join(str(tmpdir), "ref_matvec.gguf").encode()
        self._check(self.L.ref_matvec_f32(path, w.reshape(-1), w.shape[0], w.shape[1], x, y),
                    "matvec")
        return y

    def moe_ffn_layer_f32(self, tmpdir, gate_up, down, sh_gate_up, sh_down, router,
                          sh_gate, norm_w, residual, eps):
        E, I2, H = gate_up.shape
        I = I2 // 2
        IS = sh_gate_up.shape[0] // 2
        o = {"ffn_norm": np.empty(H, np.float32), "router_logits": np.empty(E, np.float32),
             "ids": np.empty(8, np.int32), "normalized_weights": np.empty(8, np.float32),
             "selected_gate_up": np.empty(8 * 2 * I, np.float32),
             "selected_swiglu": np.empty(8 * I, np.float32),
             "selected_down": np.empty(8 * H, np.float32), "moe_out": np.empty(H, np.float32),
             "shared_gate_sigmoid": np.empty(1, np.float32),
             "shared_down": np.empty(H, np.float32), "ffn_out": np.empty(H, np.float32),
             "residual": np.empty(H, np.float32)}
        path = os.path.join(str(tmpdir), "ref_moe_layer.gguf").encode()
        args = [_f32(a).reshape(-1) for a in (gate_up, down, sh_gate_up, sh_down, router,
                                              sh_gate, norm_w, residual)]
        rc = self.L.ref_moe_ffn_layer_f32(
            path, H, I, IS, E, *args, eps,
            *[o[n].ctypes.data for n in ("ffn_norm", "router_logits", "ids",
                                          "normalized_weights", "selected_gate_up",
                                          "selected_swiglu", "selected_down", "moe_out",
                                          "shared_gate_sigmoid", "shared_down", "ffn_out",
                                          "residual")])
        self._check(rc, "moe_ffn_layer")
        return o


def ref_available() -> bool:
    return os.path.exists(REF_PATH)
