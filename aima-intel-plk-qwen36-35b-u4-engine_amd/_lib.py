"""ctypes binding of libaima_u4moe.so (the C ABI in include/aima_u4moe.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime
PyTorch already loaded (both carry the soname ``libamdhip64.so.7``); device
pointers and streams from torch are then valid inside the library.  There is
no CPU fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes as C
import os

import torch  # noqa: F401  (loads the HIP runtime before the library)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaima_u4moe.so")

AIMA_OK = 0
AIMA_E_INVALID = -1
AIMA_E_RANGE = -2
AIMA_E_HIP = -3
AIMA_E_WORKSPACE = -4
AIMA_E_UNSUPPORTED = -5
AIMA_DEVERR_EXPERT_RANGE = 1
AIMA_DEVERR_EXPERT_DUPLICATE = 2
AIMA_DEVERR_TIMEOUT = 4
AIMA_OUT_F16 = 0
AIMA_OUT_F32 = 1
AIMA_MAX_MULTI_OUT = 4
AIMA_PREFILL_FULL_F16 = 0
AIMA_PREFILL_ROUTED_F32 = 1

# Every symbol the header declares, with (restype, argtypes).
_vp = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float
_szp = C.POINTER(C.c_size_t)


class U4TensorC(C.Structure):
    _fields_ = [("qweight", _vp), ("scale", _vp), ("zp", _vp)]


class MoeLayerC(C.Structure):
    _fields_ = [("gate_up", U4TensorC), ("down", U4TensorC), ("shared_gate_up", U4TensorC),
                ("shared_down", U4TensorC), ("shared_gate_vec", _vp), ("norm_weight", _vp),
                ("hidden", _i32), ("inter", _i32), ("shared_inter", _i32),
                ("experts", _i32), ("group", _i32), ("up", U4TensorC),
                ("shared_up", U4TensorC)]


class PrefillOptionsC(C.Structure):
    _fields_ = [("output_mode", _i32), ("input_f32", _i32), ("topk_stride", _i64),
                ("stage_events", _vp * 5), ("swiglu_f32", _vp), ("contributions_f32", _vp)]


class PrefillViewsC(C.Structure):
    _fields_ = [("offsets", _vp), ("token_map", _vp), ("inverse_map", _vp),
                ("compact_weights", _vp), ("swiglu", _vp), ("contributions", _vp),
                ("tiles", _vp), ("tile_count", _vp)]


class FfnTraceC(C.Structure):
    _fields_ = [(name, _vp) for name in (
        "ffn_norm", "router_logits", "expert_ids", "router_weights", "normalized_weights",
        "selected_gate_up", "selected_swiglu", "selected_down", "weighted_selected_down",
        "moe_out", "shared_gate", "shared_gate_sigmoid", "shared_gate_up", "shared_swiglu",
        "shared_down", "shared_gated", "ffn_out", "residual")]


_LP = C.POINTER(MoeLayerC)

SIGNATURES = {
    "aima_last_error": (C.c_char_p, []),
    "aima_version": (C.c_int, []),
    "aima_u4_dequant": (C.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _vp, _vp]),
    "aima_u4_dequant_f16": (C.c_int, [_vp, _vp, _vp, _i64, _i64, _i32, _vp, _vp]),
    "aima_u4_matvec": (C.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp, _i32, _vp]),
    "aima_rmsnorm": (C.c_int, [_vp, _vp, _i64, _i64, _f32, _vp, _vp]),
    "aima_router_topk": (C.c_int, [_vp, _i64, _i32, _i32, _f32, _vp, _vp, _vp]),
    "aima_u4_matvec_multi": (C.c_int, [_vp, _i32, C.POINTER(U4TensorC), C.POINTER(_i64), _i64,
                                       _i32, C.POINTER(_vp), C.POINTER(_i32), _vp]),
    "aima_router_fc_topk": (C.c_int, [_vp, C.POINTER(U4TensorC), _i32, _i64, _i32, _i32, _f32,
                                      _vp, _vp, _vp, _vp]),
    "aima_router_gemm_workspace_size": (C.c_int, [_i64, _i64, _i32, _szp]),
    "aima_router_gemm_topk": (C.c_int, [_vp, _i32, _i64, _i64, _vp, _i32, _i32, _f32, _vp, _vp,
                                        _vp, _vp, C.c_size_t, _vp]),
    "aima_u4_group_major_to_rows": (C.c_int, [_vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "aima_u4_rows_to_group_major": (C.c_int, [_vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "aima_q4k_unpack": (C.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "aima_q4s_matvec": (C.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    "aima_topk_workspace_size": (C.c_int, [_i64, _i32, _szp]),
    "aima_topk_f32": (C.c_int, [_vp, _i64, _i32, _vp, _vp, _vp, C.c_size_t, _vp]),
    "aima_u4_lm_head_topk": (C.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _vp,
                                       _vp, C.c_size_t, _vp]),
    "aima_moe_decode_workspace_size": (C.c_int, [_LP, _i32, _szp]),
    "aima_moe_ffn_decode": (C.c_int, [_LP, _vp, _vp, _vp, _vp, _i32, _vp, _vp, C.c_size_t,
                                      _vp]),
    "aima_moe_ffn_layer_trace_workspace_size": (C.c_int, [_LP, _i32, _szp]),
    "aima_moe_ffn_layer_trace": (C.c_int, [_LP, C.POINTER(U4TensorC), _vp, _f32, _i32, _f32,
                                           C.POINTER(FfnTraceC), _vp, C.c_size_t, _vp]),
    "aima_moe_decode_gate_up": (C.c_int, [_LP, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "aima_moe_decode_down": (C.c_int, [_LP, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp]),
    "aima_moe_prefill_workspace_size": (C.c_int, [_LP, _i64, _i32, _szp]),
    "aima_moe_grouped_prefill": (C.c_int, [_LP, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _vp,
                                           C.c_size_t, _vp]),
    "aima_moe_grouped_prefill_ex": (C.c_int, [_LP, _vp, _vp, _i64, _vp, _vp, _i32, _vp,
                                              C.POINTER(PrefillOptionsC), _vp, C.c_size_t, _vp]),
    "aima_moe_grouped_prefill_logits": (C.c_int, [_LP, _vp, _vp, _i64, _vp, _i32, _f32, _vp,
                                                  _vp, _vp, C.POINTER(PrefillOptionsC), _vp,
                                                  C.c_size_t, _vp]),
    "aima_moe_prefill_workspace_views": (C.c_int, [_LP, _i64, _i32, _vp,
                                                   C.POINTER(PrefillViewsC)]),
    "aima_grouped_schedule_workspace_size": (C.c_int, [_i64, _i32, _i32, _szp]),
    "aima_grouped_schedule": (C.c_int, [_vp, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                        C.c_size_t, _vp]),
    "aima_moe_stack_decode": (C.c_int, [_LP, _i32, _f32, _vp, _vp, _vp, _i32, _vp, _vp,
                                        C.c_size_t, _vp]),
    "aima_moe_stack_decode_routed": (C.c_int, [_LP, C.POINTER(U4TensorC), _i32, _f32, _vp, _i32,
                                               _f32, _vp, _vp, _vp, _vp, C.c_size_t, _vp]),
    "aima_moe_stack_decode_routed_noalloc": (C.c_int, [_LP, C.POINTER(U4TensorC), _i32, _f32, _vp,
                                                       _i32, _f32, _vp, _vp, _vp, _vp, _vp]),
    "aima_moe_stack_prefill_workspace_size": (C.c_int, [_LP, _i64, _i32, _szp]),
    "aima_moe_stack_prefill": (C.c_int, [_LP, _i32, _f32, _vp, _i64, _vp, _vp, _i32, _vp, _vp,
                                         C.c_size_t, _vp]),
    "aima_workspace_error": (C.c_int, [_vp, C.POINTER(C.c_uint32), _vp]),
    "aima_moe_decode_plan_create": (C.c_int, [_LP, _i32, _i32, C.POINTER(_vp)]),
    "aima_moe_decode_plan_run": (C.c_int, [_vp, _f32, _vp, _vp, _vp, _vp, _f32, _vp, _vp]),
    "aima_moe_decode_plan_set_routers": (C.c_int, [_vp, C.POINTER(U4TensorC)]),
    "aima_moe_decode_plan_run_routed": (C.c_int, [_vp, _f32, _vp, _f32, _vp, _vp, _vp, _vp, _vp]),
    "aima_moe_decode_plan_error": (C.c_int, [_vp, C.POINTER(C.c_uint32), _vp]),
    "aima_moe_decode_plan_destroy": (C.c_int, [_vp]),
}


class AimaError(RuntimeError):
    """A non-zero return code from the C ABI."""

    def __init__(self, code: int, what: str, message: str):
        super().__init__(f"{what}: {message} (code {code})")
        self.code = code
        self.message = message


_lib = None


def lib():
    """Load the library (once).  Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != AIMA_OK:
        raise AimaError(rc, what, lib().aima_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def size_query(name: str, *args) -> int:
    out = C.c_size_t(0)
    call(name, *args, C.byref(out))
    return int(out.value)
