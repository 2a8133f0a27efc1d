"""Seeded synthetic inputs for the benchmark configurations (no checkpoints).

Distributions follow the benchmark definition: packed codes q and zero points
z uniform in [0, 15] (uniform random bytes give independent uniform nibbles),
scale s = f16(|N(0, 0.02)| + 1e-3), activations f16(N(0, 1)), router logits
f32 N(0, 1), optional Zipf(s) expert popularity bias b_e = ln p_e with
p_e ~ rank_e^-s over a seeded permutation of ranks, RMSNorm weight
1 + N(0, 0.01), shared-expert gate vector f16(N(0, 1) / sqrt(hidden)).
``scale_log2=(lo, hi)`` draws the scales log-uniformly from [2^lo, 2^hi]
instead (parity cases for small scales: below 2^-14 they are f16
subnormals).
Works on any torch device; generation on the GPU is used for the large
configurations (the 40-layer stack is ~17 GB of U4 weights).
"""

from __future__ import annotations

import math

import torch

from .layout import MoeLayerWeights, U4Weight


def generator(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=torch.device(device))
    g.manual_seed(int(seed))
    return g


def u4_weight(experts: int, rows: int, k: int, group: int, gen: torch.Generator,
              device, scale_log2=None) -> U4Weight:
    G = k // group
    shape = (experts, rows, k // 2) if experts > 1 else (rows, k // 2)
    qweight = torch.randint(0, 256, shape, dtype=torch.uint8, generator=gen, device=device)
    zshape = (experts, (rows * G + 1) // 2) if experts > 1 else ((rows * G + 1) // 2,)
    zp = torch.randint(0, 256, zshape, dtype=torch.uint8, generator=gen, device=device)
    sshape = (experts, rows, G) if experts > 1 else (rows, G)
    if scale_log2 is None:
        scale = (torch.randn(sshape, generator=gen, device=device) * 0.02).abs_().add_(1e-3)
    else:
        lo, hi = scale_log2
        u = torch.rand(sshape, generator=gen, device=device)
        scale = torch.exp2(lo + (hi - lo) * u)
    return U4Weight(qweight, scale.to(torch.float16), zp, rows, k, group)


def u4_expert_stack(experts: int, rows: int, k: int, group: int, gen, device,
                    scale_log2=None) -> U4Weight:
    """Like u4_weight but always with a leading expert dimension."""
    w = u4_weight(max(experts, 2), rows, k, group, gen, device, scale_log2) if experts == 1 \
        else u4_weight(experts, rows, k, group, gen, device, scale_log2)
    if experts == 1:
        w = U4Weight(w.qweight[:1].contiguous(), w.scale[:1].contiguous(), w.zp[:1].contiguous(),
                     rows, k, group)
    return w


def moe_layer(hidden: int = 2048, inter: int = 512, experts: int = 256, group: int = 128,
              seed: int = 0, device="cuda", shared_inter: int = None,
              with_norm: bool = True, scale_log2=None, split: bool = False) -> MoeLayerWeights:
    """A seeded layer; ``split`` returns the same weights in the split
    gate / up form (MOE3GemmFusedCompressed's operands)."""
    device = torch.device(device)
    gen = generator(seed, device)
    si = inter if shared_inter is None else shared_inter
    gate_up = u4_expert_stack(experts, 2 * inter, hidden, group, gen, device, scale_log2)
    down = u4_expert_stack(experts, hidden, inter, group, gen, device, scale_log2)
    sgu = u4_weight(1, 2 * si, hidden, group, gen, device, scale_log2)
    sd = u4_weight(1, hidden, si, group, gen, device, scale_log2)
    gate_vec = (torch.randn(hidden, generator=gen, device=device) /
                math.sqrt(hidden)).to(torch.float16)
    norm = None
    if with_norm:
        norm = 1.0 + 0.01 * torch.randn(hidden, generator=gen, device=device)
    layer = MoeLayerWeights(gate_up, down, sgu, sd, gate_vec, norm)
    return layer.to_split() if split else layer


def activations(tokens: int, hidden: int, seed: int, device="cuda") -> torch.Tensor:
    gen = generator(seed, device)
    return torch.randn((tokens, hidden), generator=gen, device=device).to(torch.float16)


def router_logits(tokens: int, experts: int, seed: int, device="cuda",
                  zipf_s: float = None) -> torch.Tensor:
    gen = generator(seed, device)
    logits = torch.randn((tokens, experts), generator=gen, device=device)
    if zipf_s is not None:
        logits = logits + zipf_bias(experts, zipf_s, seed, device)
    return logits


def zipf_bias(experts: int, s: float, seed: int, device="cuda") -> torch.Tensor:
    """b_e = ln p_e, p_e proportional to rank_e^-s, ranks a seeded permutation."""
    gen = generator(seed + 7919, "cpu")
    ranks = torch.randperm(experts, generator=gen) + 1
    p = ranks.double().pow(-s)
    p = p / p.sum()
    return torch.log(p).float().to(device)
