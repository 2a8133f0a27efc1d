"""Host API of the U4 MoE hot path (PyTorch tensors in, PyTorch tensors out).

Each function validates shapes on the host, then calls one C-ABI entry point
on torch's current HIP stream.  Names mirror the reference interfaces they
replace:

* ``matvec_u4``            <- ``iq36_fixed_fc1`` / ``matvec_tensor``
* ``apply_rms_norm``       <- ``apply_rms_norm`` (gguf_loader.hpp:355-357)
* ``select_router_topk``   <- ``select_router_topk`` (gguf_loader.hpp:371-373)
* ``run_moe_ffn_layer``    <- ``run_qwen36_moe_ffn_layer``'s expert part
  (gguf_loader.hpp:519-524, gguf_loader.cpp:5711-5780)
* ``ffn_layer_trace``      <- ``run_qwen36_moe_ffn_layer`` with its
  ``Qwen36MoeFfnLayerResult`` / ``RouterTopKSelection`` records
  (gguf_loader.hpp:138-161)
* ``grouped_moe_prefill``  <- ``GroupedS8U4PrefillRuntime::RunLayer`` /
  ``MOE3GemmFusedCompressed``
* ``build_grouped_schedule`` <- ``BuildGroupedSchedule``
  (grouped_s8_u4_prefill_runtime.cpp:231-346)

Errors: invalid arguments raise ``ValueError``/``TypeError`` before launch;
a failing C call raises ``AimaError``.  Out-of-range or duplicated expert ids
are flagged in the workspace error word on the device (the reference throws
``std::out_of_range`` / ``runtime_error``); ``Workspace.check()`` reads it.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from . import _lib
from ._lib import MoeLayerC, call, size_query
from .layout import MoeLayerWeights, U4Weight

MIN_WEIGHT_SUM = 6.103515625e-5  # gguf_loader.cpp:5665


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("tensors must live on the GPU (no CPU path)")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


class Workspace:
    """Caller-owned scratch for the entry points that need it (grown on demand)."""

    def __init__(self, device=None):
        self.device = torch.device("cuda") if device is None else torch.device(device)
        self.buf: Optional[torch.Tensor] = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)
            if self.buf.data_ptr() % 256:
                raise RuntimeError("workspace allocation is not 256-byte aligned")
        return self.buf

    def error_bits(self) -> int:
        """Read and clear the device error word (synchronizes the stream)."""
        if self.buf is None:
            return 0
        out = C.c_uint32(0)
        call("aima_workspace_error", self.buf.data_ptr(), C.byref(out), _stream())
        return int(out.value)

    def check(self) -> None:
        bits = self.error_bits()
        if bits & _lib.AIMA_DEVERR_EXPERT_RANGE:
            raise IndexError("expert id out of range")
        if bits & _lib.AIMA_DEVERR_EXPERT_DUPLICATE:
            raise ValueError("expert id duplicated within a token")


_default_ws: dict = {}
# the device top-k keeps its launch counter and picks in its own workspace
# (other entry points' data never sits under its pick slots)
_default_topk_ws: dict = {}


def _ws(ws: Optional[Workspace], device, pool: Optional[dict] = None) -> Workspace:
    if ws is not None:
        return ws
    pool = _default_ws if pool is None else pool
    key = str(device)
    if key not in pool:
        pool[key] = Workspace(device)
    return pool[key]


# ---------------------------------------------------------------------------
# U4 matrix ops
# ---------------------------------------------------------------------------

def u4_dequant(w: U4Weight) -> torch.Tensor:
    """Exact dequantization f32(q - z) * f32(s) -> float32 [experts*rows, k]."""
    _require_cuda(w.qweight)
    n = w.experts * w.rows
    out = torch.empty((n, w.k), dtype=torch.float32, device=w.qweight.device)
    call("aima_u4_dequant", w.qweight.data_ptr(), w.scale.data_ptr(), w.zp.data_ptr(), n, w.k,
         w.group, out.data_ptr(), _stream())
    return out


def u4_dequant_f16(w: U4Weight) -> torch.Tensor:
    """f16(f32(q - z) * f32(s)) -> float16 [experts*rows, k]: the weight
    operand the grouped prefill GEMM feeds its MFMAs, by the same routine."""
    _require_cuda(w.qweight)
    n = w.experts * w.rows
    out = torch.empty((n, w.k), dtype=torch.float16, device=w.qweight.device)
    call("aima_u4_dequant_f16", w.qweight.data_ptr(), w.scale.data_ptr(), w.zp.data_ptr(), n,
         w.k, w.group, out.data_ptr(), _stream())
    return out


def matvec_u4(x: torch.Tensor, w: U4Weight, out_dtype=torch.float16) -> torch.Tensor:
    """y = W x for a batch-1 float16 activation x [k]; f32 accumulate."""
    _require_cuda(x, w.qweight)
    if x.dtype != torch.float16 or x.numel() != w.k or not x.is_contiguous():
        raise ValueError("x must be a contiguous float16 vector of length k")
    if out_dtype not in (torch.float16, torch.float32):
        raise ValueError("out_dtype must be float16 or float32")
    n = w.experts * w.rows
    y = torch.empty(n, dtype=out_dtype, device=x.device)
    call("aima_u4_matvec", x.data_ptr(), w.qweight.data_ptr(), w.scale.data_ptr(),
         w.zp.data_ptr(), n, w.k, w.group, y.data_ptr(),
         _lib.AIMA_OUT_F32 if out_dtype == torch.float32 else _lib.AIMA_OUT_F16, _stream())
    return y


def matvec_u4_multi(x: torch.Tensor, weights: Sequence[U4Weight],
                    out_dtypes: Optional[Sequence] = None):
    """Multi-output fixed FC (iq36_fixed_fc3/4): [W_j x for each W_j] in one launch.

    All matrices share k and group; out_dtypes per output (float16 default).
    """
    _require_cuda(x, *[w.qweight for w in weights])
    count = len(weights)
    if not 1 <= count <= _lib.AIMA_MAX_MULTI_OUT:
        raise ValueError(f"1 to {_lib.AIMA_MAX_MULTI_OUT} weight matrices")
    k, group = weights[0].k, weights[0].group
    if any(w.k != k or w.group != group for w in weights):
        raise ValueError("every matrix needs the same k and group")
    if x.dtype != torch.float16 or x.numel() != k or not x.is_contiguous():
        raise ValueError("x must be a contiguous float16 vector of length k")
    dts = list(out_dtypes) if out_dtypes is not None else [torch.float16] * count
    if len(dts) != count or any(d not in (torch.float16, torch.float32) for d in dts):
        raise ValueError("one out dtype per matrix, float16 or float32")
    ys = [torch.empty(w.experts * w.rows, dtype=d, device=x.device) for w, d in zip(weights, dts)]
    tens = (_lib.U4TensorC * count)(*[_lib.U4TensorC(w.qweight.data_ptr(), w.scale.data_ptr(),
                                                      w.zp.data_ptr()) for w in weights])
    ns = (C.c_int64 * count)(*[w.experts * w.rows for w in weights])
    yp = (C.c_void_p * count)(*[y.data_ptr() for y in ys])
    od = (C.c_int32 * count)(*[_lib.AIMA_OUT_F32 if d == torch.float32 else _lib.AIMA_OUT_F16
                               for d in dts])
    call("aima_u4_matvec_multi", x.data_ptr(), count, tens, ns, k, group, yp, od, _stream())
    return ys


def router_fc_topk(h: torch.Tensor, router: U4Weight, expert_used_count: int = 8,
                   min_weight_sum: float = MIN_WEIGHT_SUM):
    """Routing of one token on the device: logits = router · h (U4 FC, f32),
    then select_router_topk.  Returns (ids int32 [k], weights float32 [k],
    logits float32 [experts]) (gguf_loader.cpp:5708-5711)."""
    _require_cuda(h, router.qweight)
    if h.dtype != torch.float16 or h.numel() != router.k or not h.is_contiguous():
        raise ValueError("h must be a contiguous float16 vector of length hidden")
    E = router.experts * router.rows
    k = int(expert_used_count)
    if k <= 0 or k > E:
        raise ValueError("top-k count must be in [1, experts]")
    logits = torch.empty(E, dtype=torch.float32, device=h.device)
    ids = torch.empty(k, dtype=torch.int32, device=h.device)
    w = torch.empty(k, dtype=torch.float32, device=h.device)
    t = _lib.U4TensorC(router.qweight.data_ptr(), router.scale.data_ptr(), router.zp.data_ptr())
    call("aima_router_fc_topk", h.data_ptr(), C.byref(t), E, router.k, router.group, k,
         float(min_weight_sum), logits.data_ptr(), ids.data_ptr(), w.data_ptr(), _stream())
    return ids, w, logits


def router_gemm_topk(hidden_states: torch.Tensor, router_weight: torch.Tensor,
                     expert_used_count: int = 8, min_weight_sum: float = MIN_WEIGHT_SUM,
                     ws: Optional[Workspace] = None):
    """Routing of a batch of tokens on the device (the grouped prefill's
    native router, grouped_s8_u4_prefill_runtime.cpp:1085-1101): logits =
    hidden_states [T, H] (float32 or float16) . router_weight [E, H]^T
    (float32), then select_router_topk per token.  Returns (ids int32
    [T, k], weights float32 [T, k], logits float32 [T, E])."""
    _require_cuda(hidden_states, router_weight)
    if hidden_states.dim() != 2 or hidden_states.dtype not in (torch.float32, torch.float16):
        raise ValueError("hidden_states must be float32 or float16 [tokens, hidden]")
    if router_weight.dtype != torch.float32 or router_weight.dim() != 2 or \
            router_weight.shape[1] != hidden_states.shape[1]:
        raise ValueError("router_weight must be float32 [experts, hidden]")
    x = hidden_states.contiguous()
    wt = router_weight.contiguous()
    T, H = x.shape
    E = wt.shape[0]
    k = int(expert_used_count)
    f32 = 1 if x.dtype == torch.float32 else 0
    dev = x.device
    logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    ids = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), dtype=torch.float32, device=dev)
    need = size_query("aima_router_gemm_workspace_size", T, H, f32)
    buf = _ws(ws, dev).get(need) if need else None
    call("aima_router_gemm_topk", x.data_ptr(), f32, T, H, wt.data_ptr(), E, k,
         float(min_weight_sum), logits.data_ptr(), ids.data_ptr(), w.data_ptr(),
         _ptr(buf), 0 if buf is None else buf.numel(), _stream())
    return ids, w, logits


def u4_group_major_to_rows(scale_gm: torch.Tensor, zp_gm: torch.Tensor, n: int, groups: int):
    """Group-major scale f16 [groups][n] and zero points (packed over the
    group-major flat index) -> the boundary row-major order."""
    _require_cuda(scale_gm, zp_gm)
    if scale_gm.dtype != torch.float16 or zp_gm.dtype != torch.uint8:
        raise TypeError("scale must be float16 and zero points uint8")
    if scale_gm.numel() != n * groups or zp_gm.numel() != (n * groups + 1) // 2:
        raise ValueError("scale / zero-point sizes do not match n * groups")
    scale = torch.empty(n * groups, dtype=torch.float16, device=scale_gm.device)
    zp = torch.empty((n * groups + 1) // 2, dtype=torch.uint8, device=scale_gm.device)
    call("aima_u4_group_major_to_rows", scale_gm.contiguous().data_ptr(),
         zp_gm.contiguous().data_ptr(), n, groups, scale.data_ptr(), zp.data_ptr(), _stream())
    return scale.reshape(n, groups), zp


def u4_rows_to_group_major(scale: torch.Tensor, zp: torch.Tensor, n: int, groups: int):
    """Boundary row-major scale / zero points -> the group-major package order
    (tools/intel_qwen36_openvino_fixed_fc.py:218-265)."""
    _require_cuda(scale, zp)
    if scale.dtype != torch.float16 or zp.dtype != torch.uint8:
        raise TypeError("scale must be float16 and zero points uint8")
    if scale.numel() != n * groups or zp.numel() != (n * groups + 1) // 2:
        raise ValueError("scale / zero-point sizes do not match n * groups")
    scale_gm = torch.empty(n * groups, dtype=torch.float16, device=scale.device)
    zp_gm = torch.empty((n * groups + 1) // 2, dtype=torch.uint8, device=scale.device)
    call("aima_u4_rows_to_group_major", scale.contiguous().data_ptr(), zp.contiguous().data_ptr(),
         n, groups, scale_gm.data_ptr(), zp_gm.data_ptr(), _stream())
    return scale_gm.reshape(groups, n), zp_gm


def q4k_unpack(blocks: torch.Tensor, rows: int, cols: int):
    """GGUF Q4_K [rows][cols] (144-byte super-blocks) -> (codes uint8
    [rows][cols/2] in the boundary packing, scale float16 [rows][cols/32],
    min float32 [rows][cols/32]); value = scale * q - min."""
    _require_cuda(blocks)
    if blocks.dtype != torch.uint8 or cols % 256 or blocks.numel() != rows * (cols // 256) * 144:
        raise ValueError("blocks must be uint8 [rows][cols/256][144]")
    dev = blocks.device
    q = torch.empty((rows, cols // 2), dtype=torch.uint8, device=dev)
    sc = torch.empty((rows, cols // 32), dtype=torch.float16, device=dev)
    mn = torch.empty((rows, cols // 32), dtype=torch.float32, device=dev)
    call("aima_q4k_unpack", blocks.contiguous().data_ptr(), rows, cols, q.data_ptr(), sc.data_ptr(),
         mn.data_ptr(), _stream())
    return q, sc, mn


def q4s_matvec(x: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor, mins: torch.Tensor,
               out_dtype=torch.float32) -> torch.Tensor:
    """Matvec over q4k_unpack's output (codes uint8 [n, k/2], scale float16
    [n, k/32], mins float32 [n, k/32]): y = sum (scale * q - min) * x."""
    _require_cuda(x, codes, scale, mins)
    n, k = codes.shape[0], codes.shape[1] * 2
    if x.dtype != torch.float16 or x.numel() != k or not x.is_contiguous():
        raise ValueError("x must be a contiguous float16 vector of length k")
    if codes.dtype != torch.uint8 or scale.dtype != torch.float16 or mins.dtype != torch.float32:
        raise TypeError("codes uint8, scale float16, mins float32")
    if scale.shape != (n, k // 32) or mins.shape != (n, k // 32):
        raise ValueError("scale and mins must be [n, k/32]")
    y = torch.empty(n, dtype=out_dtype, device=x.device)
    call("aima_q4s_matvec", x.data_ptr(), codes.contiguous().data_ptr(),
         scale.contiguous().data_ptr(), mins.contiguous().data_ptr(), n, k, y.data_ptr(),
         _lib.AIMA_OUT_F32 if out_dtype == torch.float32 else _lib.AIMA_OUT_F16, _stream())
    return y


def topk_f32(values: torch.Tensor, k: int, ws: Optional[Workspace] = None):
    """Top-k of a float32 vector on the device: (ids int32 [k], values float32
    [k]), value descending, lower index first among equal values."""
    _require_cuda(values)
    if values.dtype != torch.float32 or values.dim() != 1 or not values.is_contiguous():
        raise ValueError("values must be a contiguous float32 vector")
    n = values.numel()
    ws = _ws(ws, values.device, _default_topk_ws)
    buf = ws.get(size_query("aima_topk_workspace_size", n, int(k)))
    ids = torch.empty(int(k), dtype=torch.int32, device=values.device)
    out = torch.empty(int(k), dtype=torch.float32, device=values.device)
    call("aima_topk_f32", values.data_ptr(), n, int(k), ids.data_ptr(), out.data_ptr(),
         buf.data_ptr(), buf.numel(), _stream())
    return ids, out


def lm_head_topk(x: torch.Tensor, w: U4Weight, k: int = 8, ws: Optional[Workspace] = None):
    """U4 LM head with top-k (q4x8_matvec.cl:973-1021): returns (ids int32 [k],
    values float32 [k], logits float32 [rows])."""
    _require_cuda(x, w.qweight)
    if x.dtype != torch.float16 or x.numel() != w.k or not x.is_contiguous():
        raise ValueError("x must be a contiguous float16 vector of length k")
    n = w.experts * w.rows
    ws = _ws(ws, x.device, _default_topk_ws)
    buf = ws.get(size_query("aima_topk_workspace_size", n, int(k)))
    logits = torch.empty(n, dtype=torch.float32, device=x.device)
    ids = torch.empty(int(k), dtype=torch.int32, device=x.device)
    vals = torch.empty(int(k), dtype=torch.float32, device=x.device)
    call("aima_u4_lm_head_topk", x.data_ptr(), w.qweight.data_ptr(), w.scale.data_ptr(),
         w.zp.data_ptr(), n, w.k, w.group, int(k), logits.data_ptr(), ids.data_ptr(),
         vals.data_ptr(), buf.data_ptr(), buf.numel(), _stream())
    return ids, vals, logits


def apply_rms_norm(x: torch.Tensor, weight: torch.Tensor, epsilon: float) -> torch.Tensor:
    """Row-wise RMSNorm of float16 x [rows, hidden] with float32 weight -> float16."""
    _require_cuda(x, weight)
    if x.dtype != torch.float16 or weight.dtype != torch.float32:
        raise TypeError("x must be float16 and weight float32")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    if weight.numel() != x2.shape[1]:
        raise ValueError("RMSNorm input and weight sizes differ")
    out = torch.empty_like(x2)
    call("aima_rmsnorm", x2.data_ptr(), weight.data_ptr(), x2.shape[0], x2.shape[1],
         float(epsilon), out.data_ptr(), _stream())
    return out.reshape(x.shape)


def select_router_topk(logits: torch.Tensor, expert_used_count: int = 8,
                       min_weight_sum: float = MIN_WEIGHT_SUM):
    """Router logits float32 [..., E] -> (ids int32 [..., k], weights float32 [..., k])."""
    _require_cuda(logits)
    if logits.dtype != torch.float32:
        raise TypeError("router logits must be float32")
    E = logits.shape[-1]
    l2 = logits.reshape(-1, E).contiguous()
    k = int(expert_used_count)
    if k <= 0 or k > E:
        raise ValueError("top-k count must be in [1, experts]")
    ids = torch.empty((l2.shape[0], k), dtype=torch.int32, device=logits.device)
    w = torch.empty((l2.shape[0], k), dtype=torch.float32, device=logits.device)
    call("aima_router_topk", l2.data_ptr(), l2.shape[0], E, k, float(min_weight_sum),
         ids.data_ptr(), w.data_ptr(), _stream())
    return ids.reshape(*logits.shape[:-1], k), w.reshape(*logits.shape[:-1], k)


# ---------------------------------------------------------------------------
# MoE FFN
# ---------------------------------------------------------------------------

def _check_route(ids: torch.Tensor, w: torch.Tensor, rows: int) -> int:
    if ids.dtype != torch.int32 or w.dtype != torch.float32:
        raise TypeError("expert ids must be int32 and weights float32")
    if ids.shape != w.shape or ids.numel() % max(rows, 1):
        raise ValueError("expert ids and weights must have matching [rows, k] shapes")
    if not ids.is_contiguous() or not w.is_contiguous():
        raise ValueError("expert ids and weights must be contiguous")
    return ids.numel() // max(rows, 1)


def run_moe_ffn_layer(layer: MoeLayerWeights, x: torch.Tensor, ids: torch.Tensor,
                      weights: torch.Tensor, residual: Optional[torch.Tensor] = None,
                      ws: Optional[Workspace] = None) -> torch.Tensor:
    """One token: f16(residual + sum_r w_r down_r(swiglu(gate_up_r x)) + shared)."""
    _require_cuda(x, ids, weights, residual)
    H = layer.hidden
    if x.dtype != torch.float16 or x.numel() != H or not x.is_contiguous():
        raise ValueError("x must be a contiguous float16 [hidden] vector")
    if residual is not None and (residual.dtype != torch.float16 or residual.numel() != H):
        raise ValueError("residual must be float16 [hidden]")
    k = _check_route(ids, weights, 1)
    lc = layer.c()
    ws = _ws(ws, x.device)
    buf = ws.get(size_query("aima_moe_decode_workspace_size", C.byref(lc), k))
    out = torch.empty(H, dtype=torch.float16, device=x.device)
    call("aima_moe_ffn_decode", C.byref(lc), x.data_ptr(), _ptr(residual), ids.data_ptr(),
         weights.data_ptr(), k, out.data_ptr(), buf.data_ptr(), buf.numel(), _stream())
    return out


@dataclass
class RouterTopKSelection:
    """``RouterTopKSelection`` (gguf_loader.hpp:138-142), as device tensors."""
    expert_ids: torch.Tensor          # int32 [k]
    weights: torch.Tensor             # float32 [k] softmax probabilities of the picks
    normalized_weights: torch.Tensor  # float32 [k]


@dataclass
class DecodeRoutes:
    """What a routed DecodePlan run chose for every layer of the token."""
    expert_ids: torch.Tensor  # int32 [L, k], rank order
    weights: torch.Tensor     # float32 [L, k] normalized router weights
    logits: torch.Tensor      # float32 [L, E] router logits


@dataclass
class Qwen36MoeFfnLayerResult:
    """``Qwen36MoeFfnLayerResult`` (gguf_loader.hpp:144-161), as device
    tensors: every intermediate of one decode FFN layer (ffn_layer_trace)."""
    ffn_norm: torch.Tensor                # float16 [H] (the decode kernels' input)
    router_logits: torch.Tensor           # float32 [E]
    router: RouterTopKSelection
    selected_gate_up: torch.Tensor        # float32 [k * 2I] gate rows, then up rows, per pick
    selected_swiglu: torch.Tensor         # float16 [k * I]
    selected_down: torch.Tensor           # float32 [k * H]
    weighted_selected_down: torch.Tensor  # float32 [k * H]
    moe_out: torch.Tensor                 # float32 [H]
    shared_gate: torch.Tensor             # float32 [1]
    shared_gate_sigmoid: torch.Tensor     # float32 [1]
    shared_gate_up: torch.Tensor          # float32 [2I]
    shared_swiglu: torch.Tensor           # float16 [I]
    shared_down: torch.Tensor             # float32 [H]
    shared_gated: torch.Tensor            # float32 [H]
    ffn_out: torch.Tensor                 # float32 [H]
    residual: torch.Tensor                # float16 [H] (the layer's output)


def ffn_layer_trace(layer: MoeLayerWeights, router: U4Weight, residual: torch.Tensor,
                    epsilon: float = 1e-6, expert_used_count: int = 8,
                    min_weight_sum: float = MIN_WEIGHT_SUM,
                    ws: Optional[Workspace] = None) -> Qwen36MoeFfnLayerResult:
    """One decode FFN layer from its residual input with every intermediate,
    the counterpart of run_qwen36_moe_ffn_layer (gguf_loader.cpp:5654-5782):
    RMSNorm, router FC and selection, the two decode kernels (their own
    gate/up rows, activations, per-pick down rows and shared gate captured)
    and the rank-order sums.  A debugging path; the fast paths do not keep
    these."""
    _require_cuda(residual, router.qweight)
    H, I, E = layer.hidden, layer.inter, layer.experts
    if residual.dtype != torch.float16 or residual.numel() != H or not residual.is_contiguous():
        raise ValueError("residual must be a contiguous float16 [hidden] vector")
    if layer.norm_weight is None:
        raise ValueError("the layer needs its norm weight")
    if router.experts * router.rows != E or router.k != H or router.group != layer.group:
        raise ValueError("router must be U4 [experts][hidden] with the layer's group")
    k = int(expert_used_count)
    dev = residual.device

    def f32(n):
        return torch.empty(n, dtype=torch.float32, device=dev)

    def f16(n):
        return torch.empty(n, dtype=torch.float16, device=dev)

    r = Qwen36MoeFfnLayerResult(
        ffn_norm=f16(H), router_logits=f32(E),
        router=RouterTopKSelection(torch.empty(k, dtype=torch.int32, device=dev), f32(k), f32(k)),
        selected_gate_up=f32(k * 2 * I), selected_swiglu=f16(k * I), selected_down=f32(k * H),
        weighted_selected_down=f32(k * H), moe_out=f32(H), shared_gate=f32(1),
        shared_gate_sigmoid=f32(1), shared_gate_up=f32(2 * I), shared_swiglu=f16(I),
        shared_down=f32(H), shared_gated=f32(H), ffn_out=f32(H), residual=f16(H))
    t = _lib.FfnTraceC(
        r.ffn_norm.data_ptr(), r.router_logits.data_ptr(), r.router.expert_ids.data_ptr(),
        r.router.weights.data_ptr(), r.router.normalized_weights.data_ptr(),
        r.selected_gate_up.data_ptr(), r.selected_swiglu.data_ptr(), r.selected_down.data_ptr(),
        r.weighted_selected_down.data_ptr(), r.moe_out.data_ptr(), r.shared_gate.data_ptr(),
        r.shared_gate_sigmoid.data_ptr(), r.shared_gate_up.data_ptr(), r.shared_swiglu.data_ptr(),
        r.shared_down.data_ptr(), r.shared_gated.data_ptr(), r.ffn_out.data_ptr(),
        r.residual.data_ptr())
    lc = layer.c()
    rt = _lib.U4TensorC(router.qweight.data_ptr(), router.scale.data_ptr(), router.zp.data_ptr())
    ws = _ws(ws, dev)
    buf = ws.get(size_query("aima_moe_ffn_layer_trace_workspace_size", C.byref(lc), k))
    call("aima_moe_ffn_layer_trace", C.byref(lc), C.byref(rt), residual.data_ptr(),
         float(epsilon), k, float(min_weight_sum), C.byref(t), buf.data_ptr(), buf.numel(),
         _stream())
    return r


def moe_decode_gate_up(layer: MoeLayerWeights, x: torch.Tensor, ids: torch.Tensor,
                       act: Optional[torch.Tensor] = None,
                       sigma: Optional[torch.Tensor] = None,
                       error_word: Optional[torch.Tensor] = None, layer_c=None):
    """Decode phase 1: SwiGLU activations f16 [k+1, I] (shared expert last) and
    the shared gate sigmoid (float32 [1])."""
    _require_cuda(x, ids)
    k = ids.numel()
    dev = x.device
    if act is None:
        act = torch.empty((k + 1, layer.inter), dtype=torch.float16, device=dev)
    if sigma is None:
        sigma = torch.empty(1, dtype=torch.float32, device=dev)
    if error_word is None:
        error_word = torch.zeros(1, dtype=torch.int32, device=dev)
    lc = layer.c() if layer_c is None else layer_c
    call("aima_moe_decode_gate_up", C.byref(lc), x.data_ptr(), ids.data_ptr(), k,
         act.data_ptr(), sigma.data_ptr(), error_word.data_ptr(), _stream())
    return act, sigma


def moe_decode_down(layer: MoeLayerWeights, act: torch.Tensor, sigma: torch.Tensor,
                    ids: torch.Tensor, weights: torch.Tensor,
                    residual: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None, layer_c=None) -> torch.Tensor:
    """Decode phase 2: f16(residual + sum_r w_r down_r act_r + sigma * shared)."""
    _require_cuda(act, sigma, ids, weights, residual)
    k = _check_route(ids, weights, 1)
    if out is None:
        out = torch.empty(layer.hidden, dtype=torch.float16, device=act.device)
    lc = layer.c() if layer_c is None else layer_c
    call("aima_moe_decode_down", C.byref(lc), act.data_ptr(), sigma.data_ptr(), ids.data_ptr(),
         weights.data_ptr(), k, _ptr(residual), out.data_ptr(), _stream())
    return out


def grouped_moe_prefill(layer: MoeLayerWeights, x: torch.Tensor, ids: torch.Tensor,
                        weights: torch.Tensor, residual: Optional[torch.Tensor] = None,
                        ws: Optional[Workspace] = None) -> torch.Tensor:
    """T tokens: x float16 [T, H], ids int32 [T, k], weights float32 [T, k] -> f16 [T, H]."""
    _require_cuda(x, ids, weights, residual)
    if x.dtype != torch.float16 or x.dim() != 2 or x.shape[1] != layer.hidden:
        raise ValueError("x must be float16 [tokens, hidden]")
    x = x.contiguous()
    T = x.shape[0]
    k = _check_route(ids, weights, T)
    if residual is not None:
        if residual.shape != x.shape or residual.dtype != torch.float16:
            raise ValueError("residual must match x")
        residual = residual.contiguous()
    lc = layer.c()
    ws = _ws(ws, x.device)
    buf = ws.get(size_query("aima_moe_prefill_workspace_size", C.byref(lc), T, k))
    out = torch.empty_like(x)
    call("aima_moe_grouped_prefill", C.byref(lc), x.data_ptr(), _ptr(residual), T,
         ids.data_ptr(), weights.data_ptr(), k, out.data_ptr(), buf.data_ptr(), buf.numel(),
         _stream())
    return out


def grouped_moe_prefill_routed(layer: MoeLayerWeights, hidden_states: torch.Tensor,
                               topk: torch.Tensor, router_weights: torch.Tensor,
                               topk_stride: Optional[int] = None, expert_used_count: int = 8,
                               ws: Optional[Workspace] = None, stage_events=None,
                               capture_f32: Optional[dict] = None) -> torch.Tensor:
    """GroupedS8U4PrefillRuntime::RunLayer's operation: the f32 routed sum
    out[t] = sum_r f16(w[t][r] * down_r(f16(swiglu(gate_up_r x_t)))) (no
    shared expert, no residual).

    hidden_states: float32 or float16 [T, H]; topk: int32 ids with token t's
    ``expert_used_count`` ids at byte offset t * topk_stride (a 2-D [T, >= k]
    tensor uses its row stride; a flat int32 or uint8 buffer needs
    ``topk_stride``); router_weights: float32 [T * k] (or [T, k]).
    stage_events: optional five torch.cuda.Event recorded around the stages.
    capture_f32: a dict that receives "swiglu_f32" [T*k, I] and
    "contributions_f32" [T*k, H] (schedule order, before f16 rounding).
    """
    _require_cuda(hidden_states, topk, router_weights)
    if hidden_states.dtype not in (torch.float32, torch.float16) or hidden_states.dim() != 2 \
            or hidden_states.shape[1] != layer.hidden:
        raise ValueError("hidden_states must be float32 or float16 [tokens, hidden]")
    x = hidden_states.contiguous()
    T = x.shape[0]
    k = int(expert_used_count)
    if topk.dtype == torch.uint8:
        if topk_stride is None:
            raise ValueError("a byte top-k buffer needs topk_stride")
        stride = int(topk_stride)
    elif topk.dtype == torch.int32:
        if topk.dim() == 2:
            if topk.stride(1) != 1 or topk.shape[1] < k:
                raise ValueError("top-k rows must be contiguous with at least k ids")
            stride = int(topk_stride) if topk_stride is not None else topk.stride(0) * 4
        else:
            stride = int(topk_stride) if topk_stride is not None else k * 4
    else:
        raise TypeError("topk must be int32 (or uint8 bytes)")
    if stride < 4 * k or stride % 4:
        raise ValueError("topk_stride must be a multiple of 4 and at least 4 * k bytes")
    # the reference's check: (T - 1) * stride + k ids must lie inside the payload
    # (grouped_s8_u4_prefill_runtime.cpp:234-236)
    need = (T - 1) * stride + k * 4
    avail = topk.untyped_storage().nbytes() - topk.storage_offset() * topk.element_size()
    if avail < need:
        raise ValueError("top-k payload is truncated")
    if router_weights.dtype != torch.float32 or router_weights.numel() != T * k:
        raise ValueError("router_weights must be float32 with tokens * k values")
    rw = router_weights.contiguous()
    lc = layer.c()
    ws = _ws(ws, x.device)
    buf = ws.get(size_query("aima_moe_prefill_workspace_size", C.byref(lc), T, k))
    out = torch.empty((T, layer.hidden), dtype=torch.float32, device=x.device)
    opt = _lib.PrefillOptionsC()
    opt.output_mode = _lib.AIMA_PREFILL_ROUTED_F32
    opt.input_f32 = 1 if x.dtype == torch.float32 else 0
    opt.topk_stride = stride
    if stage_events is not None:
        if len(stage_events) != 5:
            raise ValueError("five stage events")
        for i, e in enumerate(stage_events):
            if e is not None and not e.cuda_event:
                e.record(torch.cuda.current_stream())  # torch creates its events lazily
            opt.stage_events[i] = e.cuda_event if e is not None else None
    if capture_f32 is not None:
        capture_f32["swiglu_f32"] = torch.empty((T * k, layer.inter), dtype=torch.float32,
                                                device=x.device)
        capture_f32["contributions_f32"] = torch.empty((T * k, layer.hidden),
                                                       dtype=torch.float32, device=x.device)
        opt.swiglu_f32 = capture_f32["swiglu_f32"].data_ptr()
        opt.contributions_f32 = capture_f32["contributions_f32"].data_ptr()
    call("aima_moe_grouped_prefill_ex", C.byref(lc), x.data_ptr(), None, T, topk.data_ptr(),
         rw.data_ptr(), k, out.data_ptr(), C.byref(opt), buf.data_ptr(), buf.numel(), _stream())
    return out


def moe_3gemm_fused_compressed(hidden_states: torch.Tensor, routing_logits: torch.Tensor,
                               layer: MoeLayerWeights, expert_used_count: int = 8,
                               min_weight_sum: float = MIN_WEIGHT_SUM,
                               include_shared: bool = False,
                               residual: Optional[torch.Tensor] = None,
                               ws: Optional[Workspace] = None):
    """MOE3GemmFusedCompressed(hidden, routing_logits, gate_*, up_*, down_*)
    (engine/openvino/iq36-fixed-fc-moe-router-compat.patch:31-56): the
    routes are selected on the device from the f32 logits [T, E] (the
    select_router_topk rule) and the grouped layer runs on them.  Returns
    (out, ids int32 [T, k], weights float32 [T, k]); out is the f32 routed
    sum [T, H] (the op's output), or with ``include_shared`` the f16 block
    output with the sigmoid-gated shared expert (+ ``residual``).
    ``layer`` holds the gate and up projections either concatenated or
    split (``layer.to_split()``, the op's separate gate_* / up_* inputs)."""
    _require_cuda(hidden_states, routing_logits, residual)
    x = hidden_states.contiguous()
    if x.dim() != 2 or x.shape[1] != layer.hidden or x.dtype not in (torch.float16,
                                                                       torch.float32):
        raise ValueError("hidden_states must be float16 or float32 [tokens, hidden]")
    T = x.shape[0]
    k = int(expert_used_count)
    if routing_logits.dtype != torch.float32 or tuple(routing_logits.shape) != (T, layer.experts) \
            or not routing_logits.is_contiguous():
        raise ValueError("routing_logits must be contiguous float32 [tokens, experts]")
    if include_shared and x.dtype != torch.float16:
        raise ValueError("the full block output takes float16 hidden states")
    if residual is not None and not include_shared:
        raise ValueError("a residual needs include_shared")
    lc = layer.c()
    ws = _ws(ws, x.device)
    buf = ws.get(size_query("aima_moe_prefill_workspace_size", C.byref(lc), T, k))
    ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
    w = torch.empty((T, k), dtype=torch.float32, device=x.device)
    opt = _lib.PrefillOptionsC()
    opt.output_mode = _lib.AIMA_PREFILL_FULL_F16 if include_shared else _lib.AIMA_PREFILL_ROUTED_F32
    opt.input_f32 = 1 if x.dtype == torch.float32 else 0
    out = torch.empty((T, layer.hidden), dtype=torch.float16 if include_shared else torch.float32,
                      device=x.device)
    call("aima_moe_grouped_prefill_logits", C.byref(lc), x.data_ptr(), _ptr(residual), T,
         routing_logits.data_ptr(), k, float(min_weight_sum), ids.data_ptr(), w.data_ptr(),
         out.data_ptr(), C.byref(opt), buf.data_ptr(), buf.numel(), _stream())
    return out, ids, w


def prefill_workspace_views(layer: MoeLayerWeights, tokens: int, k: int, ws: Workspace,
                            with_shared: bool = True) -> dict:
    """Tensor views of the intermediates the last prefill call left in ``ws``
    (schedule, unweighted f16 SwiGLU rows and router-weighted f16 down
    contributions, in schedule order; aliases of the workspace, valid until
    its next use)."""
    if ws.buf is None:
        raise ValueError("workspace was never used")
    lc = layer.c()
    v = _lib.PrefillViewsC()
    call("aima_moe_prefill_workspace_views", C.byref(lc), int(tokens), int(k), ws.buf.data_ptr(),
         C.byref(v))
    base = ws.buf.data_ptr()
    A = tokens * k
    rows = A + (tokens if with_shared else 0)

    def view(ptr, n, dtype):
        off = ptr - base
        esz = torch.tensor([], dtype=dtype).element_size()
        return ws.buf[off:off + n * esz].view(dtype)

    return {"offsets": view(v.offsets, layer.experts, torch.int32),
            "token_map": view(v.token_map, A, torch.int32),
            "inverse_map": view(v.inverse_map, A, torch.int32),
            "compact_weights": view(v.compact_weights, A, torch.float32),
            "swiglu": view(v.swiglu, rows * layer.inter,
                           torch.float16).reshape(rows, layer.inter),
            "contributions": view(v.contributions, rows * layer.hidden,
                                  torch.float16).reshape(rows, layer.hidden),
            "tile_count": view(v.tile_count, 1, torch.int32)}


def build_grouped_schedule(ids: torch.Tensor, router_weights: torch.Tensor, experts: int,
                           ws: Optional[Workspace] = None) -> dict:
    """Device BuildGroupedSchedule: offsets [E], token_map/inverse_map/compact_weights [T*k]."""
    _require_cuda(ids, router_weights)
    if ids.dim() != 2:
        raise ValueError("ids must be [tokens, k]")
    T, k = ids.shape
    _check_route(ids, router_weights, T)
    dev = ids.device
    A = T * k
    ws = _ws(ws, dev)
    buf = ws.get(size_query("aima_grouped_schedule_workspace_size", T, k, experts))
    out = {"offsets": torch.empty(experts, dtype=torch.int32, device=dev),
           "token_map": torch.empty(A, dtype=torch.int32, device=dev),
           "inverse_map": torch.empty(A, dtype=torch.int32, device=dev),
           "compact_weights": torch.empty(A, dtype=torch.float32, device=dev)}
    call("aima_grouped_schedule", ids.data_ptr(), router_weights.data_ptr(), T, k, experts,
         out["offsets"].data_ptr(), out["token_map"].data_ptr(), out["inverse_map"].data_ptr(),
         out["compact_weights"].data_ptr(), buf.data_ptr(), buf.numel(), _stream())
    return out


def _layers_c(layers: Sequence[MoeLayerWeights]):
    arr = (MoeLayerC * len(layers))()
    for i, l in enumerate(layers):
        if l.norm_weight is None:
            raise ValueError("stack layers need norm_weight")
        arr[i] = l.c()
    return arr


def moe_stack_decode(layers: Sequence[MoeLayerWeights], residual: torch.Tensor,
                     ids: torch.Tensor, weights: torch.Tensor, epsilon: float = 1e-6,
                     ws: Optional[Workspace] = None, out: Optional[torch.Tensor] = None,
                     layers_c=None) -> torch.Tensor:
    """len(layers) layers for one token; ids/weights [L, k]; residual f16 [H]."""
    _require_cuda(residual, ids, weights)
    L = len(layers)
    H = layers[0].hidden
    if residual.dtype != torch.float16 or residual.numel() != H:
        raise ValueError("residual must be float16 [hidden]")
    k = _check_route(ids, weights, L)
    arr = _layers_c(layers) if layers_c is None else layers_c
    ws = _ws(ws, residual.device)
    buf = ws.get(size_query("aima_moe_decode_workspace_size", C.byref(arr[0]), k))
    if out is None:
        out = torch.empty(H, dtype=torch.float16, device=residual.device)
    call("aima_moe_stack_decode", arr, L, float(epsilon), residual.data_ptr(), ids.data_ptr(),
         weights.data_ptr(), k, out.data_ptr(), buf.data_ptr(), buf.numel(), _stream())
    return out


def moe_stack_decode_routed(layers: Sequence[MoeLayerWeights], routers: Sequence[U4Weight],
                            residual: torch.Tensor, expert_used_count: int = 8,
                            epsilon: float = 1e-6, min_weight_sum: float = MIN_WEIGHT_SUM,
                            ws: Optional[Workspace] = None):
    """True decode of one token: every layer routes from its own normalized
    input (router U4 FC [experts][hidden], then select_router_topk).
    Returns (out f16 [H], ids int32 [L, k], weights float32 [L, k])."""
    _require_cuda(residual, *[r.qweight for r in routers])
    L = len(layers)
    if len(routers) != L:
        raise ValueError("one router per layer")
    H = layers[0].hidden
    if residual.dtype != torch.float16 or residual.numel() != H:
        raise ValueError("residual must be float16 [hidden]")
    for lay, r in zip(layers, routers):
        if r.experts * r.rows != lay.experts or r.k != H or r.group != lay.group:
            raise ValueError("router must be [experts][hidden] at the layer's group")
    k = int(expert_used_count)
    arr = _layers_c(layers)
    rt = (_lib.U4TensorC * L)(*[_lib.U4TensorC(r.qweight.data_ptr(), r.scale.data_ptr(),
                                                r.zp.data_ptr()) for r in routers])
    ws = _ws(ws, residual.device)
    buf = ws.get(size_query("aima_moe_decode_workspace_size", C.byref(arr[0]), k))
    out = torch.empty(H, dtype=torch.float16, device=residual.device)
    ids = torch.empty((L, k), dtype=torch.int32, device=residual.device)
    w = torch.empty((L, k), dtype=torch.float32, device=residual.device)
    call("aima_moe_stack_decode_routed", arr, rt, L, float(epsilon), residual.data_ptr(), k,
         float(min_weight_sum), ids.data_ptr(), w.data_ptr(), out.data_ptr(), buf.data_ptr(),
         buf.numel(), _stream())
    return out, ids, w


def moe_stack_prefill(layers: Sequence[MoeLayerWeights], x: torch.Tensor, ids: torch.Tensor,
                      weights: torch.Tensor, epsilon: float = 1e-6,
                      ws: Optional[Workspace] = None, out: Optional[torch.Tensor] = None,
                      layers_c=None) -> torch.Tensor:
    """len(layers) layers for T tokens; x f16 [T, H]; ids/weights [L, T, k]."""
    _require_cuda(x, ids, weights)
    L = len(layers)
    if x.dtype != torch.float16 or x.dim() != 2:
        raise ValueError("x must be float16 [tokens, hidden]")
    x = x.contiguous()
    T = x.shape[0]
    if ids.dim() != 3 or ids.shape[0] != L or ids.shape[1] != T:
        raise ValueError("ids must be [layers, tokens, k]")
    k = ids.shape[2]
    _check_route(ids, weights, L * T)
    arr = _layers_c(layers) if layers_c is None else layers_c
    ws = _ws(ws, x.device)
    buf = ws.get(size_query("aima_moe_stack_prefill_workspace_size", C.byref(arr[0]), T, k))
    if out is None:
        out = torch.empty_like(x)
    call("aima_moe_stack_prefill", arr, L, float(epsilon), x.data_ptr(), T, ids.data_ptr(),
         weights.data_ptr(), k, out.data_ptr(), buf.data_ptr(), buf.numel(), _stream())
    return out


class DecodePlan:
    """Resident whole-stack decode: every layer of one token in one launch.

    Mirrors the reference's resident native loop: ``DecodePlan(layers, k)``
    uploads the layer table once; ``run`` executes RMSNorm -> MoE FFN ->
    residual for every layer in a single persistent kernel (graph-capturable,
    no allocation).  Routing comes from ``router_logits`` [L, E] (the
    select_router_topk rule) or from ``ids``/``weights`` [L, k].  With
    ``routers`` (one U4 router [experts][hidden] per layer, experts <= 256)
    ``run(residual, routers=...)`` is true decode: every layer routes from its
    own normalized input inside the same launch, as run_qwen36_moe_ffn_layer
    does (gguf_loader.cpp:5704-5711); the chosen ids, weights and logits can
    be captured through ``route_out``.
    Raises AimaError(AIMA_E_UNSUPPORTED) for shapes outside the specialization
    (hidden 2048, inter 512, k <= 8); ``moe_stack_decode`` covers those.
    ``run`` is asynchronous: its output is valid only if ``check()`` (or
    ``error_bits()``) afterwards reports no device error -- a wait that hit
    its spin limit leaves ``out`` unwritten.
    """

    def __init__(self, layers: Sequence[MoeLayerWeights], k: int = 8,
                 routers: Optional[Sequence[U4Weight]] = None):
        self.layers = list(layers)  # keep the weights alive
        self.k = int(k)
        self.hidden = self.layers[0].hidden
        self._arr = _layers_c(self.layers)
        h = C.c_void_p(0)
        call("aima_moe_decode_plan_create", self._arr, len(self.layers), self.k, C.byref(h))
        self._h = h
        self.routers = None
        if routers is not None:
            self.set_routers(routers)

    def set_routers(self, routers: Sequence[U4Weight]) -> None:
        """Registers one router per layer for true decode (setup time: waits
        for the device, then uploads the router rows into the plan)."""
        if self._h is None:
            raise RuntimeError("decode plan was closed")
        routers = list(routers)
        L = len(self.layers)
        if len(routers) != L:
            raise ValueError("one router per layer")
        _require_cuda(*[r.qweight for r in routers])
        for lay, r in zip(self.layers, routers):
            if r.experts * r.rows != lay.experts or r.k != lay.hidden or r.group != lay.group:
                raise ValueError("router must be [experts][hidden] at the layer's group")
        rt = (_lib.U4TensorC * L)(*[_lib.U4TensorC(r.qweight.data_ptr(), r.scale.data_ptr(),
                                                    r.zp.data_ptr()) for r in routers])
        call("aima_moe_decode_plan_set_routers", self._h, rt)
        self.routers = routers  # keep the router weights alive

    def run(self, residual: torch.Tensor, router_logits: Optional[torch.Tensor] = None,
            ids: Optional[torch.Tensor] = None, weights: Optional[torch.Tensor] = None,
            epsilon: float = 1e-6, min_weight_sum: float = MIN_WEIGHT_SUM,
            out: Optional[torch.Tensor] = None,
            routers: Optional[Sequence[U4Weight]] = None,
            route_out: Optional[DecodeRoutes] = None) -> torch.Tensor:
        """One token through every layer.  ``routers``: route each layer on
        the device from its own normalized input (registered on first use;
        pass the same list again for the fast path).  ``route_out``: a
        DecodeRoutes (``plan.route_buffers()``) that the routed run fills."""
        if self._h is None:
            raise RuntimeError("decode plan was closed")
        _require_cuda(residual, router_logits, ids, weights, out)
        L = len(self.layers)
        if residual.dtype != torch.float16 or residual.numel() != self.hidden or \
                not residual.is_contiguous() or residual.data_ptr() % 16:
            raise ValueError("residual must be a contiguous, 16-byte aligned float16 [hidden]")
        if routers is not None or route_out is not None:
            if router_logits is not None or ids is not None or weights is not None:
                raise ValueError("routers and router_logits / ids are exclusive")
            if routers is not None and (self.routers is None or len(routers) != L or any(
                    a is not b for a, b in zip(routers, self.routers))):
                self.set_routers(routers)
            if self.routers is None:
                raise ValueError("no routers registered")
            return self._run_routed(residual, epsilon, min_weight_sum, out, route_out)
        if router_logits is not None:
            if router_logits.dtype != torch.float32 or router_logits.dim() != 2 or \
                    router_logits.shape[0] != L or not router_logits.is_contiguous():
                raise ValueError("router_logits must be contiguous float32 [layers, experts]")
            if router_logits.shape[1] != self.layers[0].experts:
                raise ValueError("router_logits width must equal the expert count")
        else:
            if ids is None or weights is None:
                raise ValueError("need router_logits or ids + weights")
            if _check_route(ids, weights, L) != self.k:
                raise ValueError("ids/weights must be [layers, k]")
        if out is None:
            out = torch.empty(self.hidden, dtype=torch.float16, device=residual.device)
        elif out.dtype != torch.float16 or out.numel() != self.hidden or not out.is_contiguous():
            raise ValueError("out must be a contiguous float16 [hidden]")
        call("aima_moe_decode_plan_run", self._h, float(epsilon), residual.data_ptr(),
             _ptr(router_logits), _ptr(ids), _ptr(weights), float(min_weight_sum),
             out.data_ptr(), _stream())
        return out

    def route_buffers(self, device=None) -> DecodeRoutes:
        """Empty [L, k] ids / weights and [L, E] logits for ``route_out``."""
        L, E = len(self.layers), self.layers[0].experts
        dev = device if device is not None else self.layers[0].norm_weight.device
        return DecodeRoutes(
            expert_ids=torch.empty((L, self.k), dtype=torch.int32, device=dev),
            weights=torch.empty((L, self.k), dtype=torch.float32, device=dev),
            logits=torch.empty((L, E), dtype=torch.float32, device=dev))

    def _run_routed(self, residual, epsilon, min_weight_sum, out, route_out):
        L, E = len(self.layers), self.layers[0].experts
        if out is None:
            out = torch.empty(self.hidden, dtype=torch.float16, device=residual.device)
        elif out.dtype != torch.float16 or out.numel() != self.hidden or not out.is_contiguous():
            raise ValueError("out must be a contiguous float16 [hidden]")
        ids_p = w_p = lg_p = None
        if route_out is not None:
            ids, w, lg = route_out.expert_ids, route_out.weights, route_out.logits
            _require_cuda(ids, w, lg)
            if ids.dtype != torch.int32 or tuple(ids.shape) != (L, self.k) or \
                    not ids.is_contiguous():
                raise ValueError("route_out.expert_ids must be contiguous int32 [layers, k]")
            if w.dtype != torch.float32 or tuple(w.shape) != (L, self.k) or \
                    not w.is_contiguous():
                raise ValueError("route_out.weights must be contiguous float32 [layers, k]")
            if lg.dtype != torch.float32 or tuple(lg.shape) != (L, E) or \
                    not lg.is_contiguous():
                raise ValueError("route_out.logits must be contiguous float32 [layers, experts]")
            ids_p, w_p, lg_p = ids.data_ptr(), w.data_ptr(), lg.data_ptr()
        call("aima_moe_decode_plan_run_routed", self._h, float(epsilon), residual.data_ptr(),
             float(min_weight_sum), ids_p, w_p, lg_p, out.data_ptr(), _stream())
        return out

    def error_bits(self) -> int:
        out = C.c_uint32(0)
        call("aima_moe_decode_plan_error", self._h, C.byref(out), _stream())
        return int(out.value)

    def check(self) -> None:
        bits = self.error_bits()
        if bits & _lib.AIMA_DEVERR_TIMEOUT:
            raise RuntimeError("persistent decode wait timed out")
        if bits & _lib.AIMA_DEVERR_EXPERT_RANGE:
            raise IndexError("expert id out of range")

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            call("aima_moe_decode_plan_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
