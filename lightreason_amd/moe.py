"""Torch-facing host API over liblrmoe.so: routing, bucketing, experts, layers.

Tensors stay on the GPU; every call enqueues HIP work on torch's current
stream and returns without a host synchronisation (graph-capturable), except
where a docstring says it reads a device value.

Expert weights live in an :class:`ExpertBank`: one HBM allocation holding
``layers x 256`` experts in the packed pair layout (per expert: gate_up
[1024, 2048] then down [2048, 512], 6 MiB), plus a per-layer device table of
(gate_up, down) addresses that the kernels index by expert id.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _native

HIDDEN = 2048
INNER = 512
EXPERTS = 256
TOPK = 8
DECODE_MAX_TOKENS = 16  # token counts of the one-launch decode layer and chain
EXPERT_ELEMENTS = 3 * INNER * HIDDEN
GATE_UP_ELEMENTS = 2 * INNER * HIDDEN
EXPERT_BYTES = 2 * EXPERT_ELEMENTS


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _check(tensor: torch.Tensor, name: str, dtype: torch.dtype, shape=None, device=None) -> None:
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if tensor.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {tensor.dtype}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor")
    if device is not None and tensor.device != device:
        raise ValueError(f"{name} is on {tensor.device}, expected {device}")
    if shape is not None and tuple(tensor.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(tensor.shape)}")


def _opt(tensor):
    return None if tensor is None else tensor.data_ptr()


class Workspace:
    """Zero-initialised device scratch for lrmoe calls on one stream.

    Grows (reallocates) when a call needs more; size it up front with
    ``max_tokens`` so that captured graphs keep a fixed address."""

    def __init__(self, device, max_tokens: int = 16):
        self.device = torch.device(device)
        self.buffer = None
        self.max_tokens = 0
        self.ensure(max_tokens)

    def ensure(self, tokens: int) -> "Workspace":
        if tokens > self.max_tokens or self.buffer is None:
            need = _native.workspace_bytes(max(tokens, 1))
            self.buffer = torch.zeros(need, dtype=torch.uint8, device=self.device)
            self.max_tokens = max(tokens, 1)
        return self

    @property
    def ptr(self) -> int:
        return self.buffer.data_ptr()

    @property
    def nbytes(self) -> int:
        return self.buffer.numel()

    def status(self) -> int:
        """Route status bits of the last call (reads the device: synchronises)."""
        word = self.buffer[_native.WS_STATUS_OFFSET:_native.WS_STATUS_OFFSET + 4]
        return int(word.view(torch.int32).item())


_workspaces: dict = {}


def default_workspace(device, tokens: int) -> Workspace:
    device = torch.device(device)
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None:
        ws = _workspaces[key] = Workspace(device, max(tokens, 16))
    return ws.ensure(tokens)


# ---- generator --------------------------------------------------------------

def fill_normal_(tensor: torch.Tensor, seed: int, stream_id: int, sigma: float, first: int = 0) -> torch.Tensor:
    """Fill a bf16 device tensor with the counter-based ~N(0, sigma) generator
    (element i depends only on seed, stream_id and first + i)."""
    if tensor.dtype != torch.bfloat16 or not tensor.is_contiguous() or tensor.device.type != "cuda":
        raise ValueError("fill_normal_ needs a contiguous bf16 device tensor")
    _native.call("lrmoe_fill_normal_bf16", tensor.data_ptr(), tensor.numel(), seed & (2**64 - 1),
                 stream_id & (2**64 - 1), float(sigma), int(first), _stream(tensor.device))
    return tensor


# ---- expert storage -----------------------------------------------------------

class ExpertBank:
    """``layers x 256`` routed experts resident in one HBM allocation."""

    def __init__(self, layers: int, device="cuda", *, experts: int = EXPERTS):
        self.layers = layers
        self.experts = experts
        self.device = torch.device(device)
        self.bank = torch.empty((layers, experts, EXPERT_ELEMENTS), dtype=torch.bfloat16, device=self.device)
        base = self.bank.data_ptr()
        e = torch.arange(experts, dtype=torch.int64)
        tables = []
        for layer in range(layers):
            start = base + (layer * experts + e) * EXPERT_BYTES
            tables.append(torch.stack([start, start + 2 * GATE_UP_ELEMENTS], dim=1))
        self.tables = torch.stack(tables).to(self.device)

    def expert_ptrs(self, layer: int) -> torch.Tensor:
        """Device int64 [256, 2]: (gate_up, down) addresses of each expert."""
        return self.tables[layer]

    def gate_up(self, layer: int) -> torch.Tensor:
        """Strided [256, 1024, 2048] view in Transformers' gate_up_proj layout."""
        view = self.bank[layer]
        return view.as_strided((self.experts, 2 * INNER, HIDDEN), (EXPERT_ELEMENTS, HIDDEN, 1))

    def down(self, layer: int) -> torch.Tensor:
        """Strided [256, 2048, 512] view in Transformers' down_proj layout."""
        view = self.bank[layer]
        return view.as_strided((self.experts, HIDDEN, INNER), (EXPERT_ELEMENTS, INNER, 1), GATE_UP_ELEMENTS)

    def expert(self, layer: int, expert: int):
        row = self.bank[layer, expert]
        return row[:GATE_UP_ELEMENTS].view(2 * INNER, HIDDEN), row[GATE_UP_ELEMENTS:].view(HIDDEN, INNER)

    def load(self, layer: int, gate_up: torch.Tensor, down: torch.Tensor) -> None:
        """Copy Transformers-layout experts ([E,1024,2048], [E,2048,512]) in."""
        self.gate_up(layer).copy_(gate_up)
        self.down(layer).copy_(down)

    def fill_normal(self, seed: int, stream_base: int = 1000, sigma: float = 0.02) -> "ExpertBank":
        """Layer l is one generator stream (stream_base + l) over its
        256 x 3,145,728 packed elements."""
        for layer in range(self.layers):
            fill_normal_(self.bank[layer], seed, stream_base + layer, sigma)
        return self

    @property
    def nbytes(self) -> int:
        return self.bank.numel() * 2


@dataclass
class LayerWeights:
    """Everything one sparse MoE block reads besides the routed experts."""

    router: torch.Tensor                       # [256, 2048] bf16
    expert_ptrs: torch.Tensor                  # [256, 2] int64 device addresses
    shared_gate_proj: torch.Tensor | None = None   # [512, 2048]
    shared_up_proj: torch.Tensor | None = None     # [512, 2048]
    shared_down_proj: torch.Tensor | None = None   # [2048, 512]
    shared_expert_gate: torch.Tensor | None = None  # [2048] (Linear(2048, 1).weight flattened)
    norm_weight: torch.Tensor | None = None    # [2048] RMSNorm weight (scale 1 + w)
    eps: float = 1e-6

    def check(self, device) -> None:
        _check(self.router, "router", torch.bfloat16, (EXPERTS, HIDDEN), device)
        _check(self.expert_ptrs, "expert_ptrs", torch.int64, (EXPERTS, 2), device)
        shared = (self.shared_gate_proj, self.shared_up_proj, self.shared_down_proj, self.shared_expert_gate)
        if any(t is not None for t in shared):
            if any(t is None for t in shared):
                raise ValueError("give all four shared-expert tensors or none")
            _check(self.shared_gate_proj, "shared_gate_proj", torch.bfloat16, (INNER, HIDDEN), device)
            _check(self.shared_up_proj, "shared_up_proj", torch.bfloat16, (INNER, HIDDEN), device)
            _check(self.shared_down_proj, "shared_down_proj", torch.bfloat16, (HIDDEN, INNER), device)
            _check(self.shared_expert_gate, "shared_expert_gate", torch.bfloat16, (HIDDEN,), device)
        if self.norm_weight is not None:
            _check(self.norm_weight, "norm_weight", torch.bfloat16, (HIDDEN,), device)


# ---- the hot path ---------------------------------------------------------------

def route_topk(hidden: torch.Tensor, router: torch.Tensor | None, *, logits_in: torch.Tensor | None = None,
               norm_weight=None, eps: float = 1e-6, shared_expert_gate=None, workspace: Workspace | None = None):
    """Router softmax/top-8/renormalise.  Give ``router`` [256,2048] or
    ``logits_in`` [T,256].  Returns (indices [T,8] int64, weights [T,8] bf16,
    logits [T,256] bf16, shared_gate [T] bf16 or None, normed [T,2048] bf16 or
    None)."""
    tokens = hidden.shape[0]
    device = hidden.device
    _check(hidden, "hidden", torch.bfloat16, (tokens, HIDDEN))
    if (router is None) == (logits_in is None):
        raise ValueError("give exactly one of router and logits_in")
    if router is not None:
        _check(router, "router", torch.bfloat16, (EXPERTS, HIDDEN), device)
    else:
        _check(logits_in, "logits_in", torch.bfloat16, (tokens, EXPERTS), device)
    ws = workspace.ensure(tokens) if workspace is not None else default_workspace(device, tokens)
    indices = torch.empty((tokens, TOPK), dtype=torch.int64, device=device)
    weights = torch.empty((tokens, TOPK), dtype=torch.bfloat16, device=device)
    logits = torch.empty((tokens, EXPERTS), dtype=torch.bfloat16, device=device)
    sg = torch.empty(tokens, dtype=torch.bfloat16, device=device) if shared_expert_gate is not None else None
    normed = torch.empty_like(hidden) if norm_weight is not None else None
    _native.call("lrmoe_route_topk", hidden.data_ptr(), tokens, _opt(router), _opt(logits_in), _opt(norm_weight),
                 float(eps),
                 _opt(shared_expert_gate), logits.data_ptr(), indices.data_ptr(), weights.data_ptr(), _opt(sg),
                 _opt(normed), ws.ptr, ws.nbytes, _stream(device))
    return indices, weights, logits, sg, normed


def bucket(indices: torch.Tensor, workspace: Workspace | None = None) -> dict:
    """Device-side token-to-expert bucketing of indices [T, 8] (int64)."""
    tokens = indices.shape[0]
    device = indices.device
    _check(indices, "indices", torch.int64, (tokens, TOPK))
    ws = workspace.ensure(tokens) if workspace is not None else default_workspace(device, tokens)
    i32 = dict(dtype=torch.int32, device=device)
    out = dict(expert=torch.full((EXPERTS,), -1, **i32), offset=torch.zeros(EXPERTS + 1, **i32),
               pair_token=torch.empty(TOPK * tokens, **i32), pair_slot=torch.empty(TOPK * tokens, **i32),
               route_pair=torch.empty((tokens, TOPK), **i32), unique=torch.zeros(1, **i32),
               status=torch.zeros(1, **i32))
    _native.call("lrmoe_bucket", indices.data_ptr(), tokens, out["expert"].data_ptr(), out["offset"].data_ptr(),
                 out["pair_token"].data_ptr(), out["pair_slot"].data_ptr(), out["route_pair"].data_ptr(),
                 out["unique"].data_ptr(), out["status"].data_ptr(), ws.ptr, ws.nbytes, _stream(device))
    return out


def moe_experts(hidden: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor, expert_ptrs: torch.Tensor, *,
                out: torch.Tensor | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """Routed experts for given routes (the Transformers experts forward):
    hidden [T,2048] bf16, indices [T,8] int64, weights [T,8] bf16 -> [T,2048]."""
    tokens = hidden.shape[0]
    device = hidden.device
    _check(hidden, "hidden", torch.bfloat16, (tokens, HIDDEN))
    _check(indices, "indices", torch.int64, (tokens, TOPK), device)
    _check(weights, "weights", torch.bfloat16, (tokens, TOPK), device)
    _check(expert_ptrs, "expert_ptrs", torch.int64, (EXPERTS, 2), device)
    ws = workspace.ensure(tokens) if workspace is not None else default_workspace(device, tokens)
    if out is None:
        out = torch.empty_like(hidden)
    else:
        _check(out, "out", torch.bfloat16, (tokens, HIDDEN), device)
    _native.call("lrmoe_moe_experts", hidden.data_ptr(), tokens, indices.data_ptr(), weights.data_ptr(),
                 expert_ptrs.data_ptr(), out.data_ptr(), ws.ptr, ws.nbytes, _stream(device))
    return out


def moe_layer(hidden: torch.Tensor, layer: LayerWeights, *, out: torch.Tensor | None = None,
              indices: torch.Tensor | None = None, weights: torch.Tensor | None = None,
              logits_in: torch.Tensor | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """Whole sparse MoE block (router, experts, shared expert); with
    ``layer.norm_weight`` the decoder MLP half: hidden + MoE(RMSNorm(hidden)).
    ``logits_in`` [T,256] replaces the router GEMV (top-k runs on it)."""
    tokens = hidden.shape[0]
    device = hidden.device
    _check(hidden, "hidden", torch.bfloat16, (tokens, HIDDEN))
    layer.check(device)
    if logits_in is not None:
        _check(logits_in, "logits_in", torch.bfloat16, (tokens, EXPERTS), device)
    ws = workspace.ensure(tokens) if workspace is not None else default_workspace(device, tokens)
    if out is None:
        out = torch.empty_like(hidden)
    router = None if logits_in is not None else layer.router.data_ptr()
    _native.call("lrmoe_moe_layer", hidden.data_ptr(), tokens, router, _opt(logits_in), layer.expert_ptrs.data_ptr(),
                 _opt(layer.shared_gate_proj), _opt(layer.shared_up_proj), _opt(layer.shared_down_proj),
                 _opt(layer.shared_expert_gate), _opt(layer.norm_weight), float(layer.eps), out.data_ptr(),
                 _opt(indices), _opt(weights), ws.ptr, ws.nbytes, _stream(device))
    return out


def chain_table(layers) -> "C.Array":
    """Host layer table of lrmoe_moe_chain: per layer the router, the expert
    address table, the shared expert's gate/up/down projections and gate row
    (0 when absent) and the RMSNorm weight (0 for none)."""
    table = (C.c_int64 * (_native.CHAIN_PTRS * len(layers)))()
    for l, w in enumerate(layers):
        row = [w.router.data_ptr(), w.expert_ptrs.data_ptr(), _opt(w.shared_gate_proj), _opt(w.shared_up_proj),
               _opt(w.shared_down_proj), _opt(w.shared_expert_gate), _opt(w.norm_weight), 0]
        for i, v in enumerate(row):
            table[_native.CHAIN_PTRS * l + i] = v or 0
    return table


def moe_chain(hidden: torch.Tensor, layers, *, out: torch.Tensor | None = None, indices: torch.Tensor | None = None,
              weights: torch.Tensor | None = None, workspace: Workspace | None = None) -> torch.Tensor:
    """Decode (T <= 16) through a stack of MoE layers in persistent launches
    of up to 48 layers each: h = moe_layer(h, layer) for every layer in
    order, with results identical to those successive calls.  ``indices`` /
    ``weights``, when given, receive every layer's routes ([L, T, 8])."""
    tokens = hidden.shape[0]
    device = hidden.device
    layers = list(layers)
    _check(hidden, "hidden", torch.bfloat16, (tokens, HIDDEN))
    if not 0 < tokens <= DECODE_MAX_TOKENS:
        raise ValueError(f"moe_chain takes 1..{DECODE_MAX_TOKENS} tokens, got {tokens}")
    if not layers:
        raise ValueError("moe_chain needs at least one layer")
    for w in layers:
        w.check(device)
    eps = {float(w.eps) for w in layers}
    if len(eps) != 1:
        raise ValueError("all layers of a chain use one RMSNorm eps")
    if indices is not None:
        _check(indices, "indices", torch.int64, (len(layers), tokens, TOPK), device)
    if weights is not None:
        _check(weights, "weights", torch.bfloat16, (len(layers), tokens, TOPK), device)
    ws = workspace.ensure(tokens) if workspace is not None else default_workspace(device, tokens)
    if out is None:
        out = torch.empty_like(hidden)
    else:
        _check(out, "out", torch.bfloat16, (tokens, HIDDEN), device)
    step = _native.CHAIN_MAX_LAYERS
    groups = [layers[i:i + step] for i in range(0, len(layers), step)]
    # Stacks longer than one call pass their rows between calls through two
    # scratch buffers; the last call writes `out`.
    inner = [torch.empty_like(hidden) for _ in range(min(len(groups) - 1, 2))]
    src = hidden
    for g, group in enumerate(groups):
        dst = out if g == len(groups) - 1 else inner[g % 2]
        first = g * step
        table = chain_table(group)  # held until the call returns (the launch copies it)
        _native.call("lrmoe_moe_chain", src.data_ptr(), tokens, len(group), C.addressof(table),
                     float(layers[0].eps), dst.data_ptr(),
                     None if indices is None else indices[first].data_ptr(),
                     None if weights is None else weights[first].data_ptr(), ws.ptr, ws.nbytes, _stream(device))
        src = dst
    return out


def gather(descriptors, destinations, sizes, src, dst, count, *, max_copies: int, experts: int, stripes: int = 64,
           threads: int = 256, keep_in_l2: bool = False, status: torch.Tensor | None = None) -> None:
    """Raw BF16 row gather (see include/lrmoe.h lrmoe_gather)."""
    device = destinations.device
    _native.call("lrmoe_gather", descriptors.data_ptr(), destinations.data_ptr(), sizes.data_ptr(), src.data_ptr(),
                 dst.data_ptr(), count.data_ptr(), int(experts), int(destinations.numel()), int(max_copies),
                 int(stripes), int(threads), int(bool(keep_in_l2)), _opt(status), _stream(device))
