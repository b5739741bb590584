"""Seeded synthetic MoE weights and inputs, generated on the device.

Every tensor is one stream of the counter-based generator
(``moe.fill_normal_``), so any host can regenerate any element from
(seed, stream id, index) alone.  Weights are ~N(0, 0.02) and hidden states
~N(0, 1), the shapes of one Qwen3.6-35B-A3B sparse MoE block.
"""

from __future__ import annotations

import torch

from .moe import EXPERTS, HIDDEN, INNER, ExpertBank, LayerWeights, fill_normal_

STREAM_BANK = 1000
STREAM_ROUTER = 2000
STREAM_SHARED_GATE_PROJ = 3000
STREAM_SHARED_UP_PROJ = 4000
STREAM_SHARED_DOWN_PROJ = 5000
STREAM_SHARED_EXPERT_GATE = 6000
STREAM_NORM = 7000
STREAM_HIDDEN = 9000
WEIGHT_SIGMA = 0.02


def _tensor(shape, device, seed, stream, sigma):
    return fill_normal_(torch.empty(shape, dtype=torch.bfloat16, device=device), seed, stream, sigma)


class SyntheticModel:
    """``layers`` sparse MoE blocks: resident experts, routers, shared experts
    and (optionally) RMSNorm weights, all seeded."""

    def __init__(self, layers: int = 1, device="cuda", seed: int = 0, *, shared: bool = True,
                 norm: str | None = None, eps: float = 1e-6):
        self.seed = seed
        self.device = torch.device(device)
        self.bank = ExpertBank(layers, self.device).fill_normal(seed, STREAM_BANK, WEIGHT_SIGMA)
        self.layers = []
        for layer in range(layers):
            weights = LayerWeights(
                router=_tensor((EXPERTS, HIDDEN), device, seed, STREAM_ROUTER + layer, WEIGHT_SIGMA),
                expert_ptrs=self.bank.expert_ptrs(layer), eps=eps)
            if shared:
                weights.shared_gate_proj = _tensor((INNER, HIDDEN), device, seed, STREAM_SHARED_GATE_PROJ + layer,
                                                   WEIGHT_SIGMA)
                weights.shared_up_proj = _tensor((INNER, HIDDEN), device, seed, STREAM_SHARED_UP_PROJ + layer,
                                                 WEIGHT_SIGMA)
                weights.shared_down_proj = _tensor((HIDDEN, INNER), device, seed, STREAM_SHARED_DOWN_PROJ + layer,
                                                   WEIGHT_SIGMA)
                weights.shared_expert_gate = _tensor((HIDDEN,), device, seed, STREAM_SHARED_EXPERT_GATE + layer,
                                                     WEIGHT_SIGMA)
            if norm == "zeros":
                weights.norm_weight = torch.zeros(HIDDEN, dtype=torch.bfloat16, device=device)
            elif norm == "normal":
                weights.norm_weight = _tensor((HIDDEN,), device, seed, STREAM_NORM + layer, WEIGHT_SIGMA)
            self.layers.append(weights)

    def hidden(self, tokens: int, step: int = 0, sigma: float = 1.0) -> torch.Tensor:
        return _tensor((tokens, HIDDEN), self.device, self.seed, STREAM_HIDDEN + step, sigma)


STREAM_MIXER = 20000  # + 16 * layer + field
STREAM_MIXER_HIDDEN = 40000


class SyntheticMixers:
    """``layers`` Gated DeltaNet mixers of the 35B shape (the model's 30
    linear-attention layers) with decode states, all seeded: projections
    ~N(0, 0.02), conv1d ~N(0, 0.3), A_log 1.5 + N(0, 0.5), dt_bias
    ~N(0, 0.5), norm 1 + N(0, 0.1); conv states ~N(0, 1) and recurrent
    states ~N(0, 0.05) in ``state_dtype``."""

    def __init__(self, layers: int = 30, device="cuda", seed: int = 0, state_dtype=torch.float32):
        from .delta import CONV_DIM, CONV_TAPS, HEAD_WIDTH, VALUE_HEADS, DeltaMixer

        self.seed = seed
        self.device = torch.device(device)
        self.mixers, self.conv, self.state = [], [], []
        for layer in range(layers):
            base = STREAM_MIXER + 16 * layer

            def t(shape, field, sigma, shift=0.0):
                x = _tensor(shape, device, seed, base + field, sigma)
                return x.add_(shift) if shift else x

            self.mixers.append(DeltaMixer(
                in_proj_qkv=t((CONV_DIM, HIDDEN), 0, WEIGHT_SIGMA), in_proj_z=t((VALUE_HEADS * HEAD_WIDTH, HIDDEN), 1, WEIGHT_SIGMA),
                in_proj_b=t((VALUE_HEADS, HIDDEN), 2, WEIGHT_SIGMA), in_proj_a=t((VALUE_HEADS, HIDDEN), 3, WEIGHT_SIGMA),
                conv1d=t((CONV_DIM, CONV_TAPS), 4, 0.3), A_log=t((VALUE_HEADS,), 5, 0.5, 1.5),
                dt_bias=t((VALUE_HEADS,), 6, 0.5), norm=t((HEAD_WIDTH,), 7, 0.1, 1.0),
                out_proj=t((HIDDEN, VALUE_HEADS * HEAD_WIDTH), 8, WEIGHT_SIGMA)))
            self.conv.append(t((CONV_DIM, CONV_TAPS), 9, 1.0))
            self.state.append(t((VALUE_HEADS, HEAD_WIDTH, HEAD_WIDTH), 10, 0.05).to(state_dtype))

    def hidden(self, tokens: int, step: int = 0, sigma: float = 1.0) -> torch.Tensor:
        return _tensor((tokens, HIDDEN), self.device, self.seed, STREAM_MIXER_HIDDEN + step, sigma)
