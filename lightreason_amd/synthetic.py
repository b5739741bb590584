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


def _mixer(device, seed: int, base: int, state_dtype):
    """One seeded Gated DeltaNet mixer of the 35B shape (streams base ..
    base + 10) with its conv and recurrent states."""
    from .delta import CONV_DIM, CONV_TAPS, HEAD_WIDTH, VALUE_HEADS, DeltaMixer

    def t(shape, field, sigma, shift=0.0):
        x = _tensor(shape, device, seed, base + field, sigma)
        return x.add_(shift) if shift else x

    mixer = DeltaMixer(
        in_proj_qkv=t((CONV_DIM, HIDDEN), 0, WEIGHT_SIGMA), in_proj_z=t((VALUE_HEADS * HEAD_WIDTH, HIDDEN), 1, WEIGHT_SIGMA),
        in_proj_b=t((VALUE_HEADS, HIDDEN), 2, WEIGHT_SIGMA), in_proj_a=t((VALUE_HEADS, HIDDEN), 3, WEIGHT_SIGMA),
        conv1d=t((CONV_DIM, CONV_TAPS), 4, 0.3), A_log=t((VALUE_HEADS,), 5, 0.5, 1.5),
        dt_bias=t((VALUE_HEADS,), 6, 0.5), norm=t((HEAD_WIDTH,), 7, 0.1, 1.0),
        out_proj=t((HIDDEN, VALUE_HEADS * HEAD_WIDTH), 8, WEIGHT_SIGMA))
    conv = t((CONV_DIM, CONV_TAPS), 9, 1.0)
    state = t((VALUE_HEADS, HEAD_WIDTH, HEAD_WIDTH), 10, 0.05).to(state_dtype)
    return mixer, conv, state


class SyntheticMixers:
    """``layers`` Gated DeltaNet mixers of the 35B shape (the model's 30
    linear-attention layers) with decode states, all seeded: projections
    ~N(0, 0.02), conv1d ~N(0, 0.3), A_log 1.5 + N(0, 0.5), dt_bias
    ~N(0, 0.5), norm 1 + N(0, 0.1); conv states ~N(0, 1) and recurrent
    states ~N(0, 0.05) in ``state_dtype``."""

    def __init__(self, layers: int = 30, device="cuda", seed: int = 0, state_dtype=torch.float32):
        self.seed = seed
        self.device = torch.device(device)
        self.mixers, self.conv, self.state = [], [], []
        for layer in range(layers):
            mixer, conv, state = _mixer(device, seed, STREAM_MIXER + 16 * layer, state_dtype)
            self.mixers.append(mixer)
            self.conv.append(conv)
            self.state.append(state)

    def hidden(self, tokens: int, step: int = 0, sigma: float = 1.0) -> torch.Tensor:
        return _tensor((tokens, HIDDEN), self.device, self.seed, STREAM_MIXER_HIDDEN + step, sigma)


STREAM_DECODER_NORM = 50000    # + layer: input_layernorm weights
STREAM_DECODER_MIXER = 60000   # + 16 * layer + field
STREAM_DECODER_ATTN = 80000    # + 16 * layer + field
STREAM_DECODER_HIDDEN = 90000
ROPE_THETA = 10000.0


class SyntheticDecoder:
    """``layers`` decoder layers of the 35B model (layer l full attention
    when (l + 1) % 4 == 0, else Gated DeltaNet; then the MoE block), all
    seeded: the MoE blocks of SyntheticModel (shared experts, post-attention
    RMSNorm weights ~N(0, 0.02)), input RMSNorm weights ~N(0, 0.02), the
    mixers of SyntheticMixers, attention projections ~N(0, 0.02) with q/k
    norms ~N(0, 0.1), key and value caches of ``capacity`` positions whose
    first ``context`` rows are ~N(0, 1).  ``moe`` reuses the MoE blocks of an
    existing SyntheticModel.  ``stack`` is the DecoderStack."""

    def __init__(self, layers: int, device="cuda", seed: int = 0, *, context: int = 4096,
                 capacity: int | None = None, state_dtype=torch.float32, eps: float = 1e-6,
                 moe: SyntheticModel | None = None):
        from .attention import HEAD_DIM, HEADS, KV_HEADS, AttentionDecode
        from .decoder import DecoderLayer, DecoderStack, is_full_attention

        self.seed = seed
        self.device = torch.device(device)
        self.context = context
        self.capacity = capacity if capacity is not None else context + 16
        if moe is None:
            moe = SyntheticModel(layers, device, seed, shared=True, norm="normal", eps=eps)
        elif len(moe.layers) < layers or any(ly.norm_weight is None or ly.shared_down_proj is None
                                             for ly in moe.layers[:layers]):
            raise ValueError("moe must hold at least `layers` blocks with shared experts and RMSNorm weights")
        self.moe = moe
        self.layers = []
        for l in range(layers):
            norm = _tensor((HIDDEN,), device, seed, STREAM_DECODER_NORM + l, WEIGHT_SIGMA)
            if is_full_attention(l):
                base = STREAM_DECODER_ATTN + 16 * l
                attn = AttentionDecode(
                    q_proj=_tensor((HEADS * 2 * HEAD_DIM, HIDDEN), device, seed, base, WEIGHT_SIGMA),
                    k_proj=_tensor((KV_HEADS * HEAD_DIM, HIDDEN), device, seed, base + 1, WEIGHT_SIGMA),
                    v_proj=_tensor((KV_HEADS * HEAD_DIM, HIDDEN), device, seed, base + 2, WEIGHT_SIGMA),
                    o_proj=_tensor((HIDDEN, HEADS * HEAD_DIM), device, seed, base + 3, WEIGHT_SIGMA),
                    q_norm=_tensor((HEAD_DIM,), device, seed, base + 4, 0.1),
                    k_norm=_tensor((HEAD_DIM,), device, seed, base + 5, 0.1), eps=eps)
                caches = []
                for field in (6, 7):
                    c = torch.zeros((KV_HEADS, self.capacity, HEAD_DIM), dtype=torch.bfloat16, device=device)
                    for g in range(KV_HEADS):
                        fill_normal_(c[g, :context], seed, base + field + 8 * g, 1.0)
                    caches.append(c)
                self.layers.append(DecoderLayer(input_norm=norm, moe=self.moe.layers[l], attention=attn,
                                                k_cache=caches[0], v_cache=caches[1], eps=eps))
            else:
                mixer, conv, state = _mixer(device, seed, STREAM_DECODER_MIXER + 16 * l, state_dtype)
                self.layers.append(DecoderLayer(input_norm=norm, moe=self.moe.layers[l], mixer=mixer,
                                                conv_state=conv, state=state, eps=eps))
        self.stack = DecoderStack(self.layers, self.device)

    def hidden(self, tokens: int, step: int = 0, sigma: float = 1.0) -> torch.Tensor:
        return _tensor((tokens, HIDDEN), self.device, self.seed, STREAM_DECODER_HIDDEN + step, sigma)

    def rope(self, tokens: int, start: int):
        """cos, sin [tokens, 64] bf16 of positions start .. start + tokens - 1
        (the rotary embedding of the attention's 64 rotated dims)."""
        pos = torch.arange(start, start + tokens, device=self.device, dtype=torch.float32)
        inv = 1.0 / (ROPE_THETA ** (torch.arange(0, 64, 2, device=self.device, dtype=torch.float32) / 64))
        ang = torch.cat([pos[:, None] * inv[None], pos[:, None] * inv[None]], dim=1)
        return ang.cos().to(torch.bfloat16).contiguous(), ang.sin().to(torch.bfloat16).contiguous()
