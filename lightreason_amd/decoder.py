"""The 35B decoder step for decode and speculative-verify blocks of 1..16
positions, every part native.  Per layer ([HF] Qwen3_5MoeDecoderLayer.forward
855-877):

* the input RMSNorm, the Gated DeltaNet mixer (3 of every 4 layers) or the
  full attention (every 4th layer), and the residual add, as one call
  (``lrmoe_delta_mixer_step`` / ``lrmoe_attn_decode_step``, which norm the
  rows inside the mixer or projection launch and add the residual in the
  output launch; ``fused=False`` runs ``lrmoe_add_rmsnorm`` around
  ``lrmoe_delta_mixer`` / ``lrmoe_attn_decode`` instead, with the same bits),
* the MoE block with its post-attention RMSNorm and residual
  (``lrmoe_moe_layer``).

The reference verifies a drafter's block with one forward of the stock
Transformers model (edge35b/dflash_probe.py:119-121, adaptive width at
:144-148), with its MoE blocks patched (expert_stream.patch_experts) and the
linear-attention recurrence replaced (delta_decode.fused_delta); here the
whole step is native, and ``VerifyPass`` captures it once per width as one
HIP graph.

``DecoderStack.step`` runs a block eagerly on the caches (attention caches
hold ``length`` positions before it, the mixers' states are advanced in
place).  ``VerifyPass(stack, widths, length)`` captures one graph per width
over static buffers: a replay reads the block from ``hidden``, the rotary
rows from ``cos``/``sin`` and the cache length from a device word
(``lrmoe_attn_decode_step`` with ``length_dev``), appends at positions ``length ..`` of every
attention cache and advances every mixer state.  ``verify(..., length=n)``
sets that word before the replay, so the same graphs serve a cache that
grows between verify blocks.

There is no CPU path: the calls raise when liblrmoe.so is missing.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native
from .attention import AttentionDecode
from .delta import DeltaMixer, check_mixer_status
from .moe import DECODE_MAX_TOKENS, HIDDEN, TOPK, LayerWeights, Workspace, moe_layer

FULL_ATTENTION_INTERVAL = 4  # layer l is full attention when (l + 1) % 4 == 0 (the 35B config's layer_types)


def is_full_attention(layer: int) -> bool:
    return (layer + 1) % FULL_ATTENTION_INTERVAL == 0


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def add_rmsnorm(x: torch.Tensor, *, add: torch.Tensor | None = None, norm: torch.Tensor | None = None,
                eps: float = 1e-6, sum_out: torch.Tensor | None = None,
                norm_out: torch.Tensor | None = None):
    """``lrmoe_add_rmsnorm`` on [T, 2048] bf16 rows: s = bf16(x + add) (x
    when add is None) into ``sum_out``, RMSNorm(s) with ``norm`` [2048] into
    ``norm_out``.  Outputs that are None but needed are allocated.  Returns
    (sum_out, norm_out)."""
    T = x.shape[0]
    if x.dim() != 2 or x.shape[1] != HIDDEN or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError(f"x must be contiguous bf16 [T, {HIDDEN}], got {tuple(x.shape)} {x.dtype}")
    for name, t in (("add", add), ("sum_out", sum_out), ("norm_out", norm_out)):
        if t is not None and (t.shape != x.shape or t.dtype != torch.bfloat16 or not t.is_contiguous()
                              or t.device != x.device):
            raise ValueError(f"{name} must be contiguous bf16 {tuple(x.shape)} on {x.device}")
    if norm is not None and (norm.shape != (HIDDEN,) or norm.dtype != torch.bfloat16 or norm.device != x.device):
        raise ValueError(f"norm must be bf16 [{HIDDEN}] on {x.device}")
    if add is not None and sum_out is None:
        sum_out = torch.empty_like(x)
    if norm is not None and norm_out is None:
        norm_out = torch.empty_like(x)
    _native.call("lrmoe_add_rmsnorm", x.data_ptr(), None if add is None else add.data_ptr(), T,
                 None if norm is None else norm.data_ptr(), float(eps),
                 None if sum_out is None else sum_out.data_ptr(), None if norm_out is None else norm_out.data_ptr(),
                 _stream(x.device))
    return sum_out, norm_out


@dataclass
class DecoderLayer:
    """One decoder layer: ``input_norm`` [2048] (input_layernorm), the mixer
    -- ``mixer`` with its ``conv_state`` [8192, 4] and ``state`` [32, 128,
    128], or ``attention`` with its ``k_cache``/``v_cache`` [2, capacity,
    256] -- and the MoE block ``moe`` whose ``norm_weight`` is the
    post-attention layernorm."""

    input_norm: torch.Tensor
    moe: LayerWeights
    mixer: DeltaMixer | None = None
    conv_state: torch.Tensor | None = None
    state: torch.Tensor | None = None
    attention: AttentionDecode | None = None
    k_cache: torch.Tensor | None = None
    v_cache: torch.Tensor | None = None
    eps: float = 1e-6

    def check(self) -> None:
        if (self.mixer is None) == (self.attention is None):
            raise ValueError("a decoder layer has either a Gated DeltaNet mixer or a full attention")
        if self.moe.norm_weight is None:
            raise ValueError("the MoE block needs its post-attention RMSNorm weight")
        if self.mixer is not None and (self.conv_state is None or self.state is None):
            raise ValueError("a mixer layer needs its conv and recurrent states")
        if self.attention is not None and (self.k_cache is None or self.v_cache is None):
            raise ValueError("an attention layer needs its key and value caches")


class StepBuffers:
    """Device buffers of one width's step: per layer (``trace``) or shared,
    the normed rows ``n``, the mixer outputs ``mix``, the post-mixer residual
    ``h2`` and the layer outputs ``h`` (the last layer's goes to the step's
    ``out`` when one is given); ``indices``/``weights`` [L, T, 8] receive
    every MoE block's routes."""

    def __init__(self, layers: int, tokens: int, device, trace: bool = False):
        rows = dict(dtype=torch.bfloat16, device=device)
        k = layers if trace else 1
        self.trace = trace
        self.n = torch.empty((k, tokens, HIDDEN), **rows)
        self.mix = torch.empty((k, tokens, HIDDEN), **rows)
        self.h2 = torch.empty((k, tokens, HIDDEN), **rows)
        self.h = torch.empty((layers if trace else 2, tokens, HIDDEN), **rows)
        self.indices = torch.empty((layers, tokens, TOPK), dtype=torch.int64, device=device)
        self.weights = torch.empty((layers, tokens, TOPK), **rows)

    def at(self, l: int):
        i = l if self.trace else 0
        return self.n[i], self.mix[i], self.h2[i], self.h[l if self.trace else l % 2]


class DecoderStack:
    """A stack of decoder layers sharing one MoE workspace (sized for 16
    tokens, so that captured graphs keep its address)."""

    def __init__(self, layers, device=None):
        self.layers = list(layers)
        if not self.layers:
            raise ValueError("DecoderStack needs at least one layer")
        for layer in self.layers:
            layer.check()
        self.device = torch.device(device) if device is not None else self.layers[0].input_norm.device
        self.workspace = Workspace(self.device, DECODE_MAX_TOKENS)

    def step(self, hidden: torch.Tensor, length, cos: torch.Tensor | None = None,
             sin: torch.Tensor | None = None, *, buffers: StepBuffers | None = None,
             out: torch.Tensor | None = None, fused: bool = True) -> torch.Tensor:
        """One cached forward of T = hidden.shape[0] (1..16) positions after
        ``length`` cached positions (an int, or a one-element int32 device
        tensor read by the attention kernels when they run); cos, sin [T, 64]
        bf16 (the rotary rows of the new positions) are needed when the stack
        has attention layers.  Returns the last layer's output [T, 2048] bf16
        (``out`` if given).

        ``fused`` (default) runs each layer's input norm and residual add
        inside its mixer or attention launches (``layer_step``; the normed
        rows are stored only for traced buffers); ``fused=False`` runs them as
        ``lrmoe_add_rmsnorm`` launches around the plain steps, with the same
        bits."""
        T = hidden.shape[0]
        if not 1 <= T <= DECODE_MAX_TOKENS or hidden.shape != (T, HIDDEN) or hidden.dtype != torch.bfloat16:
            raise ValueError(f"hidden must be bf16 [T, {HIDDEN}] with 1 <= T <= {DECODE_MAX_TOKENS}")
        if buffers is None:
            buffers = StepBuffers(len(self.layers), T, self.device)
        h = hidden
        last = len(self.layers) - 1
        for l, layer in enumerate(self.layers):
            n, mix, h2, h_out = buffers.at(l)
            if l == last and out is not None:
                h_out = out
            if layer.mixer is None and (cos is None or sin is None):
                raise ValueError("an attention layer needs the rotary rows cos and sin")
            if fused:
                n_out = n if buffers.trace else None
                if layer.mixer is not None:
                    layer.mixer.layer_step(h, layer.input_norm, layer.eps, layer.conv_state, layer.state, out=mix,
                                           sum_out=h2, norm_out=n_out)
                else:
                    layer.attention.layer_step(h, layer.input_norm, layer.eps, cos, sin, layer.k_cache,
                                               layer.v_cache, length, out=mix, sum_out=h2, norm_out=n_out)
            else:
                add_rmsnorm(h, norm=layer.input_norm, eps=layer.eps, norm_out=n)
                if layer.mixer is not None:
                    layer.mixer.step(n, layer.conv_state, layer.state, out=mix)
                else:
                    layer.attention.step(n, cos, sin, layer.k_cache, layer.v_cache, length, out=mix)
                add_rmsnorm(h, add=mix, sum_out=h2)
            moe_layer(h2, layer.moe, out=h_out, indices=buffers.indices[l], weights=buffers.weights[l],
                      workspace=self.workspace)
            h = h_out
        return h

    def check_status(self) -> None:
        """Raise for the last steps' status words (reads the device): a
        timed-out wait of the MoE or mixer kernels (RuntimeError), bad routes
        (ValueError)."""
        self.workspace.check("decoder step")
        if any(layer.mixer is not None for layer in self.layers):
            check_mixer_status(self.device, "decoder step")


class VerifyPass:
    """The whole decoder step captured once per width in ``widths`` (1..16)
    as one HIP graph, for verify blocks after ``length`` cached positions.
    ``verify(hidden, cos, sin, length=n)`` copies the block in, sets the
    cache length (when given; else the last one stays), replays the width's
    graph and returns its static output (valid until the next verify of that
    width); ``buffers(width)`` gives that width's StepBuffers (per layer when
    ``trace``).  Every replay advances the mixers' states and rewrites
    positions ``length .. length + width - 1`` of the attention caches.  The
    attention steps read the length from a device word, and their positions
    are split into chunks sized for the caches' capacity."""

    def __init__(self, stack: DecoderStack, widths, length: int, *, trace: bool = False):
        self.stack = stack
        self.widths = sorted(set(int(w) for w in widths))
        if not self.widths or self.widths[0] < 1 or self.widths[-1] > DECODE_MAX_TOKENS:
            raise ValueError(f"verify widths must lie in 1..{DECODE_MAX_TOKENS}")
        device = stack.device
        caps = [layer.k_cache.shape[1] for layer in stack.layers if layer.attention is not None]
        self.capacity = min(caps) if caps else None
        self.length_dev = torch.zeros(1, dtype=torch.int32, device=device)
        self.length = 0
        self.set_length(length, self.widths[-1])
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs = {}
        L = len(stack.layers)
        capture_stream = torch.cuda.Stream(device)
        capture_stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(capture_stream):
            for w in self.widths:
                static = dict(hidden=torch.zeros((w, HIDDEN), dtype=torch.bfloat16, device=device),
                              cos=torch.zeros((w, 64), dtype=torch.bfloat16, device=device),
                              sin=torch.zeros((w, 64), dtype=torch.bfloat16, device=device),
                              out=torch.empty((w, HIDDEN), dtype=torch.bfloat16, device=device),
                              buffers=StepBuffers(L, w, device, trace))

                def run(static=static):
                    stack.step(static["hidden"], self.length_dev, static["cos"], static["sin"],
                               buffers=static["buffers"], out=static["out"])

                run()  # eager once: any one-time set-up happens outside the capture
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.pool, stream=capture_stream):
                    run()
                self.graphs[w] = (graph, static)
        torch.cuda.current_stream(device).wait_stream(capture_stream)

    def set_length(self, length: int, width: int | None = None) -> None:
        """The cache length the next replays read (checked against the
        caches' capacity for ``width`` new positions, default the widest)."""
        length = int(length)
        width = self.widths[-1] if width is None else int(width)
        if length < 0 or (self.capacity is not None and length + width > self.capacity):
            raise ValueError(f"length {length} + {width} positions exceeds the cache capacity {self.capacity}")
        self.length_dev.fill_(length)
        self.length = length

    def verify(self, hidden: torch.Tensor, cos: torch.Tensor | None = None, sin: torch.Tensor | None = None, *,
               length: int | None = None, check: bool = True) -> torch.Tensor:
        width = hidden.shape[0]
        entry = self.graphs.get(width)
        if entry is None:
            raise ValueError(f"no verify graph of width {width} (captured: {self.widths})")
        if length is not None:
            self.set_length(length, width)
        elif self.capacity is not None and self.length + width > self.capacity:
            raise ValueError(f"length {self.length} + {width} positions exceeds the cache capacity {self.capacity}")
        graph, static = entry
        static["hidden"].copy_(hidden)
        if cos is not None:
            static["cos"].copy_(cos)
        if sin is not None:
            static["sin"].copy_(sin)
        graph.replay()
        if check:
            self.stack.check_status()
        return static["out"]

    def buffers(self, width: int) -> StepBuffers:
        return self.graphs[width][1]["buffers"]
