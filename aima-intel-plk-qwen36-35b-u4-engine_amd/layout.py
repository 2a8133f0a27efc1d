"""Device-resident U4 weights in the boundary layout.

U4 matrix W[N][K], group size g (tools/intel_qwen36_openvino_fixed_fc.py:107-144,
241-265; engine/openvino/custom/iq36_fixed_fc_multi_output.cl:118-127):

* ``qweight`` uint8 [N][K/2]: low nibble = even k, high nibble = odd k
* ``scale``   float16 [N][K/g]
* ``zp``      uint8, u4 over the flat [N*(K/g)] index, low nibble = even

An expert stack puts E such matrices back to back (leading dimension E).  A
routed gate/up stack has 2*I rows per expert, gate rows first
(engine/src/gguf_loader.cpp:4654-4660).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from ._lib import MoeLayerC, U4TensorC


@dataclass
class U4Weight:
    """One U4 matrix ([rows][k]) or an expert stack ([experts][rows][k])."""

    qweight: torch.Tensor
    scale: torch.Tensor
    zp: torch.Tensor
    rows: int
    k: int
    group: int = 128

    def __post_init__(self):
        e = self.experts
        g = self.k // self.group
        if self.k % self.group or self.k % 2:
            raise ValueError("k must be a multiple of group (and even)")
        if self.qweight.dtype != torch.uint8 or self.zp.dtype != torch.uint8:
            raise TypeError("qweight and zp must be uint8")
        if self.scale.dtype != torch.float16:
            raise TypeError("scale must be float16")
        if self.qweight.numel() != e * self.rows * self.k // 2:
            raise ValueError("qweight has the wrong size")
        if self.scale.numel() != e * self.rows * g:
            raise ValueError("scale has the wrong size")
        if self.zp.numel() != e * ((self.rows * g + 1) // 2):
            raise ValueError("zp has the wrong size")
        for t in (self.qweight, self.scale, self.zp):
            if not t.is_contiguous():
                raise ValueError("U4 tensors must be contiguous")

    @property
    def experts(self) -> int:
        return int(self.qweight.shape[0]) if self.qweight.dim() == 3 else 1

    @property
    def groups(self) -> int:
        return self.k // self.group

    @property
    def nbytes(self) -> int:
        return self.qweight.numel() + 2 * self.scale.numel() + self.zp.numel()

    def expert_bytes(self) -> int:
        """Bytes streamed for one expert: N*K/2 + N*K/g*2 + N*K/g/2."""
        return self.nbytes // self.experts

    def c(self) -> U4TensorC:
        return U4TensorC(self.qweight.data_ptr(), self.scale.data_ptr(), self.zp.data_ptr())

    def to(self, device) -> "U4Weight":
        return U4Weight(self.qweight.to(device), self.scale.to(device), self.zp.to(device),
                        self.rows, self.k, self.group)


@dataclass
class MoeLayerWeights:
    """One MoE FFN layer: routed expert stacks, the shared expert, its gate."""

    gate_up: U4Weight                  # E x [2I][H]
    down: U4Weight                     # E x [H][I]
    shared_gate_up: U4Weight           # [2I][H]
    shared_down: U4Weight              # [H][I]
    shared_gate_vec: torch.Tensor      # float16 [H]
    norm_weight: Optional[torch.Tensor] = None  # float32 [H] (RMSNorm before the layer)

    def __post_init__(self):
        H, I = self.hidden, self.inter
        if self.gate_up.rows != 2 * I or self.down.rows != H or self.down.k != I:
            raise ValueError("routed expert shapes disagree")
        if self.shared_gate_up.k != H or self.shared_down.rows != H:
            raise ValueError("shared expert shapes disagree")
        if self.shared_down.k != self.shared_gate_up.rows // 2:
            raise ValueError("shared down K must equal shared intermediate")
        if self.gate_up.experts != self.down.experts:
            raise ValueError("gate/up and down expert counts differ")
        if self.shared_gate_vec.dtype != torch.float16 or self.shared_gate_vec.numel() != H:
            raise ValueError("shared_gate_vec must be float16 [hidden]")
        if self.norm_weight is not None and (self.norm_weight.dtype != torch.float32
                                             or self.norm_weight.numel() != H):
            raise ValueError("norm_weight must be float32 [hidden]")

    @property
    def hidden(self) -> int:
        return self.gate_up.k

    @property
    def inter(self) -> int:
        return self.gate_up.rows // 2

    @property
    def shared_inter(self) -> int:
        return self.shared_gate_up.rows // 2

    @property
    def experts(self) -> int:
        return self.gate_up.experts

    @property
    def group(self) -> int:
        return self.gate_up.group

    def expert_bytes(self) -> int:
        """Weight bytes of one routed expert (gate/up + down)."""
        return self.gate_up.expert_bytes() + self.down.expert_bytes()

    def shared_bytes(self) -> int:
        return self.shared_gate_up.nbytes + self.shared_down.nbytes

    def c(self) -> MoeLayerC:
        return MoeLayerC(self.gate_up.c(), self.down.c(), self.shared_gate_up.c(),
                         self.shared_down.c(), self.shared_gate_vec.data_ptr(),
                         self.norm_weight.data_ptr() if self.norm_weight is not None else None,
                         self.hidden, self.inter, self.shared_inter, self.experts, self.group)
