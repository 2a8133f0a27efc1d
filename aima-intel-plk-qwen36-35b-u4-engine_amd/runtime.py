"""Resident grouped-prefill runtime with the reference runtime's contract.

Mirrors ``iq36::GroupedS8U4PrefillRuntime``
(engine/include/intel_qwen36/grouped_s8_u4_prefill_runtime.hpp:137-162):
``LoadLayer`` makes a layer resident and returns a handle, ``RunLayer`` runs
warmup + timed repeats of the complete grouped layer and returns the output
with min/median/mean timings (grouped_s8_u4_prefill_runtime.cpp:1375-1432).
The input record keeps the reference field names (hidden_states, topk,
router_weights, warmup, repeat, capture_intermediates).  Differences: the
weights are already U4 tensors on the device (no prep directory), inputs are
device tensors, and timing uses HIP events on the current stream.
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

from . import ops
from .layout import MoeLayerWeights


@dataclass
class GroupedU4PrefillInput:
    hidden_states: torch.Tensor          # float16 [T, H]
    topk: torch.Tensor                   # int32 [T, k]
    router_weights: torch.Tensor         # float32 [T, k]
    residual: Optional[torch.Tensor] = None
    warmup: int = 0
    repeat: int = 1
    capture_intermediates: bool = False


@dataclass
class GroupedU4PrefillTiming:
    samples_us: List[float] = field(default_factory=list)
    minimum_us: float = 0.0
    median_us: float = 0.0
    mean_us: float = 0.0


@dataclass
class GroupedU4PrefillRun:
    output: torch.Tensor
    inverse_map: Optional[torch.Tensor] = None
    token_map: Optional[torch.Tensor] = None
    offsets: Optional[torch.Tensor] = None
    active_experts: int = 0
    max_group_size: int = 0
    timing: GroupedU4PrefillTiming = field(default_factory=GroupedU4PrefillTiming)


class GroupedU4PrefillRuntime:
    def __init__(self, device=None):
        self.device = torch.device("cuda") if device is None else torch.device(device)
        self._layers: Dict[int, MoeLayerWeights] = {}
        self._next = 1
        self._ws = ops.Workspace(self.device)
        self._stats = {"layer_load_count": 0, "layer_count": 0, "run_count": 0,
                       "resident_weight_bytes": 0}

    def LoadLayer(self, weights: MoeLayerWeights) -> int:
        if weights.gate_up.qweight.device.type != "cuda":
            weights = _to_device(weights, self.device)
        handle = self._next
        self._next += 1
        self._layers[handle] = weights
        self._stats["layer_load_count"] += 1
        self._stats["layer_count"] = len(self._layers)
        self._stats["resident_weight_bytes"] += (weights.gate_up.nbytes + weights.down.nbytes +
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
        T = inp.hidden_states.shape[0]
        if inp.topk.shape[0] != T or inp.router_weights.shape != inp.topk.shape:
            raise ValueError("grouped prefill top-k / router weight shape mismatch")

        def execute():
            return ops.grouped_moe_prefill(layer, inp.hidden_states, inp.topk, inp.router_weights,
                                           residual=inp.residual, ws=self._ws)

        for _ in range(inp.warmup):
            execute()
        stream = torch.cuda.current_stream()
        samples = []
        out = None
        for _ in range(inp.repeat):
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(stream)
            out = execute()
            end.record(stream)
            end.synchronize()
            samples.append(start.elapsed_time(end) * 1000.0)
        self._ws.check()
        srt = sorted(samples)
        run = GroupedU4PrefillRun(output=out, timing=GroupedU4PrefillTiming(
            samples_us=samples, minimum_us=srt[0], median_us=srt[len(srt) // 2],
            mean_us=statistics.fmean(samples)))
        if inp.capture_intermediates:
            sched = ops.build_grouped_schedule(inp.topk, inp.router_weights, layer.experts)
            counts = torch.diff(sched["offsets"], prepend=torch.zeros(1, dtype=torch.int32,
                                                                      device=self.device))
            run.inverse_map = sched["inverse_map"]
            run.token_map = sched["token_map"]
            run.offsets = sched["offsets"]
            run.active_experts = int((counts > 0).sum().item())
            run.max_group_size = int(counts.max().item())
        self._stats["run_count"] += 1
        return run

    def stats(self) -> dict:
        return dict(self._stats)


def _to_device(w: MoeLayerWeights, device) -> MoeLayerWeights:
    return MoeLayerWeights(w.gate_up.to(device), w.down.to(device), w.shared_gate_up.to(device),
                           w.shared_down.to(device), w.shared_gate_vec.to(device),
                           None if w.norm_weight is None else w.norm_weight.to(device))
