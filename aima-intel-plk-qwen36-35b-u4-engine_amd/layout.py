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
    """One MoE FFN layer: routed expert stacks, the shared expert, its gate.

    Gate and up come in either boundary form: concatenated (``gate_up`` =
    E x [2I][H], gate rows first; ``up`` is None) or split, the operands of
    OpenVINO's MOE3GemmFusedCompressed (``gate_up`` = the gate projection
    E x [I][H] and ``up`` = E x [I][H]; likewise ``shared_up``).
    """

    gate_up: U4Weight                  # E x [2I][H], or the gate E x [I][H] when split
    down: U4Weight                     # E x [H][I]
    shared_gate_up: U4Weight           # [2I][H], or the shared gate [I][H] when split
    shared_down: U4Weight              # [H][I]
    shared_gate_vec: torch.Tensor      # float16 [H]
    norm_weight: Optional[torch.Tensor] = None  # float32 [H] (RMSNorm before the layer)
    up: Optional[U4Weight] = None      # E x [I][H] (split form)
    shared_up: Optional[U4Weight] = None  # [I][H] (split form)

    def __post_init__(self):
        H, I = self.hidden, self.inter
        if (self.up is None) != (self.shared_up is None):
            raise ValueError("split form needs both up and shared_up")
        if self.up is not None:
            if (self.up.rows != self.gate_up.rows or self.up.k != H or
                    self.up.experts != self.gate_up.experts or self.up.group != self.group or
                    self.shared_up.rows != self.shared_gate_up.rows or self.shared_up.k != H):
                raise ValueError("split up tensors must match the gate tensors")
        if self.down.rows != H or self.down.k != I:
            raise ValueError("routed expert shapes disagree")
        if self.shared_gate_up.k != H or self.shared_down.rows != H:
            raise ValueError("shared expert shapes disagree")
        if self.shared_down.k != self.shared_inter:
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
    def split(self) -> bool:
        return self.up is not None

    @property
    def inter(self) -> int:
        return self.gate_up.rows if self.split else self.gate_up.rows // 2

    @property
    def shared_inter(self) -> int:
        return self.shared_gate_up.rows if self.split else self.shared_gate_up.rows // 2

    @property
    def experts(self) -> int:
        return self.gate_up.experts

    @property
    def group(self) -> int:
        return self.gate_up.group

    def expert_bytes(self) -> int:
        """Weight bytes of one routed expert (gate/up + down)."""
        up = self.up.expert_bytes() if self.split else 0
        return self.gate_up.expert_bytes() + up + self.down.expert_bytes()

    def shared_bytes(self) -> int:
        up = self.shared_up.nbytes if self.split else 0
        return self.shared_gate_up.nbytes + up + self.shared_down.nbytes

    def c(self) -> MoeLayerC:
        none = U4TensorC(None, None, None)
        return MoeLayerC(self.gate_up.c(), self.down.c(), self.shared_gate_up.c(),
                         self.shared_down.c(), self.shared_gate_vec.data_ptr(),
                         self.norm_weight.data_ptr() if self.norm_weight is not None else None,
                         self.hidden, self.inter, self.shared_inter, self.experts, self.group,
                         self.up.c() if self.split else none,
                         self.shared_up.c() if self.split else none)

    def to_split(self) -> "MoeLayerWeights":
        """The same layer in the split form (copies of the gate and up rows)."""
        if self.split:
            return self
        gate, up = _split_rows(self.gate_up, self.inter)
        sgate, sup = _split_rows(self.shared_gate_up, self.shared_inter)
        return MoeLayerWeights(gate, self.down, sgate, self.shared_down, self.shared_gate_vec,
                               self.norm_weight, up, sup)


def _split_rows(w: U4Weight, inter: int):
    """Concatenated [E][2I][K] -> (gate [E][I][K], up [E][I][K]) U4 tensors."""
    e, G = w.experts, w.groups
    q = w.qweight.reshape(e, 2 * inter, w.k // 2)
    s = w.scale.reshape(e, 2 * inter, G)
    # zero points: nibbles over the flat [rows * G] index of each expert
    zb = w.zp.reshape(e, -1)
    nib = torch.stack([zb & 0xF, zb >> 4], dim=-1).reshape(e, 2 * inter, G)
    out = []
    for h in range(2):
        n = nib[:, h * inter:(h + 1) * inter].reshape(e, -1)
        zp = (n[:, 0::2] | (n[:, 1::2] << 4)).to(torch.uint8)
        qq = q[:, h * inter:(h + 1) * inter].contiguous()
        ss = s[:, h * inter:(h + 1) * inter].contiguous()
        if w.qweight.dim() == 2:
            qq, ss, zp = qq[0], ss[0], zp[0]
        out.append(U4Weight(qq.contiguous(), ss.contiguous(), zp.contiguous(), inter, w.k,
                            w.group))
    return out
