"""Resident grouped-prefill runtime with the reference runtime's contract.

Mirrors ``iq36::GroupedS8U4PrefillRuntime``
(engine/include/intel_qwen36/grouped_s8_u4_prefill_runtime.hpp:62-162):
``LoadLayer`` makes a layer resident and returns a handle, ``RunLayer`` runs
warmup + timed repeats of the complete grouped layer and returns the output
with min/median/mean timings and per-stage times
(grouped_s8_u4_prefill_runtime.cpp:1375-1432).

The input record keeps the reference field names (hidden_states, topk,
topk_stride, router_weights, warmup, repeat, capture_intermediates) and the
output is RunLayer's: the f32 routed sum ``sum_r w_r * down_r(...)`` per
token.  ``include_shared=True`` (an extension) returns instead the complete
f16 block output with the sigmoid-gated shared expert and an optional
residual.  Differences: the weights are already U4 tensors on the device (no
prep directory), inputs are device tensors, the schedule is always built on
the device (the reference's ``device_schedule``), and timing uses HIP events
on the current stream.  Intermediates come from the last timed repeat's own
workspace, not from a second run.  ``native_router`` routes the tokens on the
device from the hidden states with the layer's f32 router (one GEMM and the
top-k selection, inside each timed repeat) as the reference runtime's native
router does.
"""

from __future__ import annotations

import statistics
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

from . import ops
from .layout import MoeLayerWeights

# stage_us[i]: native router (0 without it), schedule, gate/up GEMM + SwiGLU,
# down GEMM, combine
STAGES = ("router", "schedule", "gate_up", "down", "combine")


@dataclass
class GroupedU4PrefillInput:
    hidden_states: torch.Tensor          # float32 or float16 [T, H]
    topk: torch.Tensor                   # int32 ids [T, >= k] (or bytes, with topk_stride)
    router_weights: torch.Tensor         # float32 [T * k] (or [T, k])
    topk_stride: int = 0                 # bytes between tokens' id rows (0: from topk)
    expert_used_count: int = 8
    warmup: int = 0
    repeat: int = 1
    capture_intermediates: bool = False
    include_shared: bool = False         # extension: f16 routed + shared (+ residual)
    residual: Optional[torch.Tensor] = None
    # route every token on the device from hidden_states with the layer's
    # resident f32 router (LoadLayer(..., router_weight=...)); topk and
    # router_weights are then ignored (grouped_s8_u4_prefill_runtime.hpp:80-83)
    native_router: bool = False


@dataclass
class GroupedU4PrefillTiming:
    """RunLayer's timing record (grouped_s8_u4_prefill_runtime.hpp:86-98).

    input_upload_us: host -> device copy of host hidden states (0 when they
    are already on the device); schedule_prepare_us: host work on the
    schedule's inputs before the run (moving host top-k rows and router
    weights to the device, repacking strided rows; 0 for dense device inputs
    and for the native router); device_schedule_us: the device schedule
    (count, scan, scatter kernels), median over the timed repeats from the
    stage events; schedule_upload_us equals it and schedule_setup_us is
    prepare + upload, as in the reference's device-schedule path
    (grouped_s8_u4_prefill_runtime.cpp:1165-1168).  The samples include the
    device schedule (it runs inside every repeat), so complete_minimum_us is
    minimum_us + schedule_prepare_us (the reference adds its setup to
    samples that exclude it, :1428-1429)."""
    stage_us: List[float] = field(default_factory=lambda: [0.0] * len(STAGES))
    samples_us: List[float] = field(default_factory=list)
    minimum_us: float = 0.0
    median_us: float = 0.0
    mean_us: float = 0.0
    input_upload_us: float = 0.0
    schedule_prepare_us: float = 0.0
    schedule_upload_us: float = 0.0
    schedule_setup_us: float = 0.0
    device_schedule_us: float = 0.0
    complete_minimum_us: float = 0.0


@dataclass
class GroupedU4PrefillRun:
    output: torch.Tensor
    # intermediates (capture_intermediates), in schedule order, as the
    # reference's run record (grouped_s8_u4_prefill_runtime.hpp:101-107):
    grouped_swiglu_f16: Optional[torch.Tensor] = None          # silu(g) * u, [rows][I]
    grouped_swiglu_f32: Optional[torch.Tensor] = None          # same, before f16 rounding
    grouped_contributions_f16: Optional[torch.Tensor] = None   # w_r * down, [rows][H]
    grouped_contributions_f32: Optional[torch.Tensor] = None   # same, before f16 rounding
    inverse_map: Optional[torch.Tensor] = None
    token_map: Optional[torch.Tensor] = None
    offsets: Optional[torch.Tensor] = None
    active_experts: int = 0
    max_group_size: int = 0
    gateup_work_tile_count: int = 0
    device_schedule: bool = True
    native_router: bool = False
    timing: GroupedU4PrefillTiming = field(default_factory=GroupedU4PrefillTiming)


class GroupedU4PrefillRuntime:
    def __init__(self, device=None):
        self.device = torch.device("cuda") if device is None else torch.device(device)
        self._layers: Dict[int, MoeLayerWeights] = {}
        self._routers: Dict[int, torch.Tensor] = {}
        self._next = 1
        self._ws = ops.Workspace(self.device)
        self._stats = {"layer_load_count": 0, "layer_count": 0, "run_count": 0,
                       "resident_weight_bytes": 0, "device_schedule_run_count": 0,
                       "native_router_run_count": 0}

    def LoadLayer(self, weights: MoeLayerWeights,
                  router_weight: Optional[torch.Tensor] = None) -> int:
        """router_weight: the layer's f32 router [experts, hidden] for
        native_router runs (the reference's layer router_weights path)."""
        if weights.gate_up.qweight.device.type != "cuda":
            weights = _to_device(weights, self.device)
        handle = self._next
        self._next += 1
        self._layers[handle] = weights
        if router_weight is not None:
            if router_weight.dtype != torch.float32 or \
                    tuple(router_weight.shape) != (weights.experts, weights.hidden):
                raise ValueError("router_weight must be float32 [experts, hidden]")
            self._routers[handle] = router_weight.to(self.device).contiguous()
            self._stats["resident_weight_bytes"] += router_weight.numel() * 4
        self._stats["layer_load_count"] += 1
        self._stats["layer_count"] = len(self._layers)
        self._stats["resident_weight_bytes"] += (weights.gate_up.nbytes + weights.down.nbytes +
                                                 (weights.up.nbytes if weights.split else 0) +
                                                 weights.shared_bytes())
        return handle

    def _layer(self, handle: int) -> MoeLayerWeights:
        if handle not in self._layers:
            raise KeyError("unknown grouped prefill layer handle")
        return self._layers[handle]

    def RunLayer(self, handle: int, inp: GroupedU4PrefillInput) -> GroupedU4PrefillRun:
        layer = self._layer(handle)
        if inp.warmup < 0 or inp.repeat <= 0:
            raise ValueError("grouped prefill warmup/repeat are invalid")
        # host inputs are copied to the device first, as the reference's
        # WriteBuffer calls (timed with the host clock, copies complete)
        input_upload_us = schedule_prepare_us = 0.0
        x = inp.hidden_states
        if x.device.type != "cuda":
            t0 = time.perf_counter()
            x = x.to(self.device).contiguous()
            torch.cuda.synchronize(self.device)
            input_upload_us = (time.perf_counter() - t0) * 1e6
        topk_in, rw_in = inp.topk, inp.router_weights
        if not inp.native_router and (topk_in.device.type != "cuda" or
                                      rw_in.device.type != "cuda"):
            t0 = time.perf_counter()
            topk_in = topk_in.to(self.device)
            rw_in = rw_in.to(self.device)
            torch.cuda.synchronize(self.device)
            schedule_prepare_us = (time.perf_counter() - t0) * 1e6
        if x.dim() != 2 or x.shape[1] != layer.hidden:
            raise ValueError("grouped prefill hidden-state count mismatch")
        T, k = x.shape[0], int(inp.expert_used_count)
        router = None
        if inp.native_router:
            if handle not in self._routers:
                raise ValueError("native_router needs a layer loaded with its router weight")
            if inp.include_shared:
                raise ValueError("native_router runs return the routed sum")
            router = self._routers[handle]
        elif rw_in.numel() != T * k:
            raise ValueError("grouped prefill router weight count mismatch")
        stride = inp.topk_stride or None
        if inp.include_shared:
            if topk_in.dtype != torch.int32 or topk_in.shape != (T, k) or stride:
                raise ValueError("include_shared takes dense int32 top-k [T, k]")
            if x.dtype != torch.float16:
                raise ValueError("include_shared takes float16 hidden states")

        # events: router start, then the prefill call's own five
        stage_events = [torch.cuda.Event(enable_timing=True) for _ in range(len(STAGES) + 1)]

        def execute(events=None, capture=None):
            if inp.include_shared:
                return ops.grouped_moe_prefill(layer, x, topk_in,
                                               rw_in.reshape(T, k),
                                               residual=inp.residual, ws=self._ws)
            topk, rw, st = topk_in, rw_in, stride
            if events is not None:
                events[0].record(torch.cuda.current_stream())
            if router is not None:
                topk, rw, _ = ops.router_gemm_topk(x, router, k, ws=self._ws)
                rw, st = rw.reshape(-1), None
            return ops.grouped_moe_prefill_routed(layer, x, topk, rw, topk_stride=st,
                                                  expert_used_count=k, ws=self._ws,
                                                  stage_events=None if events is None
                                                  else events[1:], capture_f32=capture)

        for _ in range(inp.warmup):
            execute()
        stream = torch.cuda.current_stream()
        samples, stages = [], []
        out = None
        # the last timed repeat also writes the f32 intermediates (as the
        # reference's kernels write theirs next to the f16 ones)
        capture = {} if inp.capture_intermediates and not inp.include_shared else None
        for i in range(inp.repeat):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(stream)
            out = execute(None if inp.include_shared else stage_events,
                          capture if i == inp.repeat - 1 else None)
            end.record(stream)
            end.synchronize()
            samples.append(start.elapsed_time(end) * 1000.0)
            if not inp.include_shared:
                stages.append([stage_events[i].elapsed_time(stage_events[i + 1]) * 1000.0
                               for i in range(len(STAGES))])
        self._ws.check()
        srt = sorted(samples)
        timing = GroupedU4PrefillTiming(samples_us=samples, minimum_us=srt[0],
                                        median_us=srt[len(srt) // 2],
                                        mean_us=statistics.fmean(samples))
        if stages:
            timing.stage_us = [statistics.median(s[i] for s in stages) for i in range(len(STAGES))]
        timing.input_upload_us = input_upload_us
        timing.schedule_prepare_us = schedule_prepare_us
        timing.device_schedule_us = timing.stage_us[1]
        timing.schedule_upload_us = timing.device_schedule_us
        timing.schedule_setup_us = timing.schedule_prepare_us + timing.schedule_upload_us
        timing.complete_minimum_us = timing.minimum_us + timing.schedule_prepare_us
        run = GroupedU4PrefillRun(output=out, timing=timing, native_router=router is not None)
        if inp.capture_intermediates:
            # the last repeat's schedule and intermediates, still in the workspace
            v = ops.prefill_workspace_views(layer, T, k, self._ws, with_shared=inp.include_shared)
            counts = torch.diff(v["offsets"], prepend=torch.zeros(1, dtype=torch.int32,
                                                                  device=self.device))
            run.inverse_map = v["inverse_map"].clone()
            run.token_map = v["token_map"].clone()
            run.offsets = v["offsets"].clone()
            run.grouped_swiglu_f16 = v["swiglu"].clone()
            run.grouped_contributions_f16 = v["contributions"].clone()
            if capture:
                run.grouped_swiglu_f32 = capture["swiglu_f32"]
                run.grouped_contributions_f32 = capture["contributions_f32"]
            run.gateup_work_tile_count = int(v["tile_count"].item()) * (layer.inter // 128)
            run.active_experts = int((counts > 0).sum().item())
            run.max_group_size = int(counts.max().item())
        self._stats["run_count"] += 1
        self._stats["device_schedule_run_count"] += 1
        if router is not None:
            self._stats["native_router_run_count"] += 1
        return run

    def stats(self) -> dict:
        return dict(self._stats)


def _to_device(w: MoeLayerWeights, device) -> MoeLayerWeights:
    return MoeLayerWeights(w.gate_up.to(device), w.down.to(device), w.shared_gate_up.to(device),
                           w.shared_down.to(device), w.shared_gate_vec.to(device),
                           None if w.norm_weight is None else w.norm_weight.to(device),
                           None if w.up is None else w.up.to(device),
                           None if w.shared_up is None else w.shared_up.to(device))
