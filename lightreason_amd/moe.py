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

    def check(self, what: str = "lrmoe call") -> int:
        """Raise for the last call's status (reads the device: synchronises):
        RuntimeError when a bounded wait of the decode kernel expired (its
        outputs are invalid: some of its workgroups were kept off the GPU),
        ValueError for bad routes (an expert id outside [0, 256) or a token
        routed twice to one expert).  Returns the status word otherwise."""
        return check_status(self.status(), what)


def check_status(status: int, what: str = "lrmoe call") -> int:
    """The mapping of Workspace.check: status bits to exceptions."""
    if status & _native.STATUS_TIMEOUT:
        raise RuntimeError(f"{what}: a cross-workgroup wait timed out; the outputs are invalid (the decode kernel "
                           "needs every workgroup resident: is another kernel running on the device?)")
    if status & (_native.STATUS_BAD_EXPERT | _native.STATUS_REPEATED_EXPERT):
        raise ValueError(f"{what}: routes hold an expert id outside [0, 256) or repeat an expert within a token")
    return status


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


# ---- lossless BF16 tile codec --------------------------------------------------

CODEC_TILE = 256
CODEC_TILE_BYTES = 384
CODEC_MISFIT = 255
CODEC_GU_PACKED = 2 * INNER * (HIDDEN // CODEC_TILE) * CODEC_TILE_BYTES   # 3 MiB
CODEC_DN_PACKED = HIDDEN * (INNER // CODEC_TILE) * CODEC_TILE_BYTES       # 1.5 MiB
CODEC_GU_BASES = 2 * INNER * (HIDDEN // CODEC_TILE)                        # 8 KiB
CODEC_DN_BASES = HIDDEN * (INNER // CODEC_TILE)                            # 4 KiB
# One expert's block: packed gate_up, packed down, their bases, and room for
# the 16-byte base loads that read past the last row.
CODEC_EXPERT_BYTES = (CODEC_GU_PACKED + CODEC_DN_PACKED + CODEC_GU_BASES + CODEC_DN_BASES + 256 + 4095) // 4096 * 4096


def codec_pack(w: torch.Tensor, packed: torch.Tensor, bases: torch.Tensor,
               misfit: torch.Tensor | None = None) -> None:
    """Pack a [rows, cols] bf16 matrix (cols a multiple of 256; row stride
    cols) into tile-codec form: ``packed`` uint8 [rows * cols / 256 * 384],
    ``bases`` uint8 [rows * cols / 256]; ``misfit`` (int64 [1]) is increased
    by the number of tiles that do not fit (lrmoe_codec_pack)."""
    rows, cols = w.shape
    if w.dtype != torch.bfloat16 or w.stride() != (cols, 1):
        raise ValueError("codec_pack takes a row-contiguous bf16 matrix")
    tiles = rows * cols // CODEC_TILE
    if packed.numel() < tiles * CODEC_TILE_BYTES or bases.numel() < tiles:
        raise ValueError("codec_pack output buffers are too small")
    _native.call("lrmoe_codec_pack", w.data_ptr(), rows, cols, packed.data_ptr(), bases.data_ptr(), _opt(misfit),
                 _stream(w.device))


def codec_unpack(packed: torch.Tensor, bases: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=packed.device)
    _native.call("lrmoe_codec_unpack", packed.data_ptr(), bases.data_ptr(), rows, cols, out.data_ptr(),
                 _stream(packed.device))
    return out


def _reference_tile_order(device):
    """Byte positions, in lrmoe_codec_pack's tile, of the reference tile
    layout's bytes (value k: low byte k, code nibble k of bytes 256..383)."""
    k = torch.arange(CODEC_TILE, device=device)
    g, s, j = (k >> 3) & 3, k >> 5, k & 7
    low_at = 64 * (s >> 1) + 16 * g + 8 * (s & 1) + j
    code_at = 256 + 64 * (s >> 2) + 16 * g + 4 * (s & 3) + (j & 3)
    return low_at, code_at, 4 * (j >> 2)


def pack_tiles_reference_order(w: torch.Tensor):
    """A [rows, cols] bf16 matrix in the reference's tile-codec layout
    (edge35b/cpu_bf16_reads.h:16-52; decoded by lrmoe_gather_tiles): returns
    (packed uint8 [tiles, 384], bases uint8 [tiles], tiles that do not fit).
    lrmoe_codec_pack on the device, then its bytes rearranged."""
    rows, cols = w.shape
    tiles = rows * cols // CODEC_TILE
    ours = torch.empty((tiles, CODEC_TILE_BYTES), dtype=torch.uint8, device=w.device)
    bases = torch.empty(tiles, dtype=torch.uint8, device=w.device)
    misfit = torch.zeros(1, dtype=torch.int64, device=w.device)
    codec_pack(w, ours.view(-1), bases, misfit)
    low_at, code_at, shift = _reference_order_cached(w.device)
    codes = (ours[:, code_at] >> shift.to(torch.uint8)) & 15
    packed = torch.cat([ours[:, low_at], codes[:, 0::2] | (codes[:, 1::2] << 4)], dim=1)
    return packed, bases, int(misfit.item())


_ORDER = {}


def _reference_order_cached(device):
    key = str(device)
    if key not in _ORDER:
        _ORDER[key] = _reference_tile_order(device)
    return _ORDER[key]


def pack_escape_row(w: torch.Tensor):
    """A bf16 row (any shape, flattened) in the gather's escape-codec format
    (edge35b/bf16_expert_codec.py:27-55; decoded by lrmoe_gather): returns
    (packed uint8, base, escapes).  base starts the first window of 16
    consecutive exponents holding the most values; per value one
    sign|fraction byte and a 4-bit exponent delta, then the escapes' sorted
    int32 indices and raw bits."""
    bits = w.reshape(-1).view(torch.int16).to(torch.int32) & 0xFFFF
    n = bits.numel()
    exponent = (bits >> 7) & 255
    counts = torch.bincount(exponent, minlength=256)
    upto = torch.cat([counts.new_zeros(1), torch.cumsum(counts, 0)])
    inside = upto[16:] - upto[:-16]
    base = int(torch.argmax(inside).item())   # torch.argmax returns the first maximum
    delta = exponent - base
    escaped = torch.nonzero((delta < 0) | (delta >= 16)).reshape(-1)
    escapes = escaped.numel()
    sf = ((bits & 0x7F) | ((bits >> 8) & 0x80)).to(torch.uint8)
    nib = (delta & 15).to(torch.uint8)
    deltas = nib[0::2] | (nib[1::2] << 4)
    index_bytes = escaped.to(torch.int32).view(torch.uint8)
    value_bytes = bits[escaped].to(torch.int16).view(torch.uint8)
    return torch.cat([sf, deltas, index_bytes, value_bytes]), base, escapes


CODEC_TABLE_COLUMNS = _native.CODEC_TABLE_COLUMNS   # 4 addresses + 48 bytes of per-(item, wave) raw flags


def codec_unit_flags(gu_bases: torch.Tensor, dn_bases: torch.Tensor) -> torch.Tensor:
    """Raw flags of the decode kernel's (item, wave) units from an expert's
    tile bases: byte i (0..31) for gate/up item i, byte 32 + i (0..15) for
    down item i; bit w is set when a tile read by wave w of that item does
    not fit the codec.  Gate/up item i, wave w reads tiles 2(w%4), 2(w%4)+1
    of gate rows and up rows 16i + 8(w/4) .. +7; down item i, wave w reads
    both tiles of down rows 128i + 16w .. +15.  Leading dimensions of the
    bases ([..., 8192] and [..., 4096]) are kept: the result is [..., 48]."""
    lead = gu_bases.shape[:-1]
    gu = gu_bases.reshape(*lead, 2, 32, 2, 8, 4, 2) == CODEC_MISFIT   # [gate/up, item, w/4, row, w%4, tile]
    a = gu.any(dim=-1).any(dim=-2).any(dim=-4)                         # [item, w/4, w%4]
    a = a.reshape(*lead, 32, 8).to(torch.int32)
    dn = (dn_bases.reshape(*lead, 16, 8, 16, 2) == CODEC_MISFIT).any(dim=-1).any(dim=-1).to(torch.int32)
    weights = 1 << torch.arange(8, dtype=torch.int32, device=a.device)   # bit w for wave w
    return torch.cat([(a * weights).sum(dim=-1), (dn * weights).sum(dim=-1)], dim=-1).to(torch.uint8)


class CodecBank:
    """Tile-codec copies of an ExpertBank's experts (and of each layer's
    shared expert) for the decode kernel.  ``tables[l]`` is a device int64
    [257, 10] table per expert (row 256 the shared expert): the addresses of
    the packed gate_up, packed down, gate_up bases and down bases, then 48
    bytes of raw flags (codec_unit_flags).  A wave whose unit has a tile that
    does not fit (its exponent fields span more than 8 values) reads that
    unit's raw rows; an all-zero row reads the whole expert raw."""

    def __init__(self, bank: ExpertBank, shared=None):
        """``shared``: per layer (gate_proj [512,2048], up_proj [512,2048],
        down_proj [2048,512]) or None."""
        self.layers = bank.layers
        self.device = bank.device
        slots = EXPERTS + 1
        self.blob = torch.zeros((bank.layers, slots, CODEC_EXPERT_BYTES), dtype=torch.uint8, device=self.device)
        misfit = torch.zeros((bank.layers, slots), dtype=torch.int64, device=self.device)
        present = torch.ones((bank.layers, slots), dtype=torch.bool)
        for layer in range(bank.layers):
            for e in range(EXPERTS):
                gate_up, down = bank.expert(layer, e)
                self._pack(layer, e, gate_up[:INNER], gate_up[INNER:], down, misfit[layer, e:e + 1])
            if shared is not None and shared[layer] is not None:
                g, u, d = shared[layer]
                self._pack(layer, EXPERTS, g, u, d, misfit[layer, EXPERTS:EXPERTS + 1])
            else:
                present[layer, EXPERTS] = False
        self.misfit = misfit.cpu()   # tiles that do not fit, per expert
        gu0 = CODEC_GU_PACKED + CODEC_DN_PACKED
        dn0 = gu0 + CODEC_GU_BASES
        flags = codec_unit_flags(self.blob[:, :, gu0:gu0 + CODEC_GU_BASES],
                                 self.blob[:, :, dn0:dn0 + CODEC_DN_BASES]).cpu()      # [L, 257, 48]
        bits = (flags[present].to(torch.int32).unsqueeze(-1) >> torch.arange(8, dtype=torch.int32)) & 1
        self.raw_units = int(bits.sum())
        self.units = bits.numel()
        base = self.blob.data_ptr()
        tables = torch.zeros((bank.layers, slots, CODEC_TABLE_COLUMNS), dtype=torch.int64)
        tables[:, :, 4:] = flags.cpu().view(torch.int64).view(bank.layers, slots, 6)
        for layer in range(bank.layers):
            for e in range(slots):
                if not present[layer, e]:
                    tables[layer, e] = 0
                    continue
                start = base + (layer * slots + e) * CODEC_EXPERT_BYTES
                tables[layer, e, :4] = torch.tensor([start, start + CODEC_GU_PACKED, start + gu0, start + dn0])
        self.tables = tables.to(self.device)

    def _pack(self, layer, e, gate, up, down, misfit):
        block = self.blob[layer, e]
        gu_packed = block[:CODEC_GU_PACKED]
        dn_packed = block[CODEC_GU_PACKED:CODEC_GU_PACKED + CODEC_DN_PACKED]
        gu_bases = block[CODEC_GU_PACKED + CODEC_DN_PACKED:CODEC_GU_PACKED + CODEC_DN_PACKED + CODEC_GU_BASES]
        dn_bases = block[CODEC_GU_PACKED + CODEC_DN_PACKED + CODEC_GU_BASES:
                         CODEC_GU_PACKED + CODEC_DN_PACKED + CODEC_GU_BASES + CODEC_DN_BASES]
        half_packed, half_bases = CODEC_GU_PACKED // 2, CODEC_GU_BASES // 2
        codec_pack(gate, gu_packed[:half_packed], gu_bases[:half_bases], misfit)
        codec_pack(up, gu_packed[half_packed:], gu_bases[half_bases:], misfit)
        codec_pack(down, dn_packed, dn_bases, misfit)

    def table(self, layer: int) -> torch.Tensor:
        return self.tables[layer]

    @property
    def packed_fraction(self) -> float:
        """Share of the (item, wave) units read from the codec form."""
        return 1.0 - self.raw_units / max(self.units, 1)

    @property
    def nbytes(self) -> int:
        return self.blob.numel()


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
    codec: torch.Tensor | None = None          # [257, 10] int64 tile-codec table (CodecBank.table), or None

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
        if self.codec is not None:
            _check(self.codec, "codec", torch.int64, (EXPERTS + 1, CODEC_TABLE_COLUMNS), device)


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
                out: torch.Tensor | None = None, workspace: Workspace | None = None,
                check: bool = False) -> torch.Tensor:
    """Routed experts for given routes (the Transformers experts forward):
    hidden [T,2048] bf16, indices [T,8] int64, weights [T,8] bf16 -> [T,2048].
    ``check`` reads the status word after the call (a host sync) and raises
    as Workspace.check does."""
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
    if check:
        ws.check("moe_experts")
    return out


def moe_layer(hidden: torch.Tensor, layer: LayerWeights, *, out: torch.Tensor | None = None,
              indices: torch.Tensor | None = None, weights: torch.Tensor | None = None,
              logits_in: torch.Tensor | None = None, workspace: Workspace | None = None,
              check: bool = False) -> torch.Tensor:
    """Whole sparse MoE block (router, experts, shared expert); with
    ``layer.norm_weight`` the decoder MLP half: hidden + MoE(RMSNorm(hidden)).
    ``logits_in`` [T,256] replaces the router GEMV (top-k runs on it).
    ``check`` reads the status word after the call (a host sync) and raises
    as Workspace.check does."""
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
                 _opt(layer.codec),
                 _opt(layer.shared_gate_proj), _opt(layer.shared_up_proj), _opt(layer.shared_down_proj),
                 _opt(layer.shared_expert_gate), _opt(layer.norm_weight), float(layer.eps), out.data_ptr(),
                 _opt(indices), _opt(weights), ws.ptr, ws.nbytes, _stream(device))
    if check:
        ws.check("moe_layer")
    return out


def chain_table(layers) -> "C.Array":
    """Host layer table of lrmoe_moe_chain: per layer the router, the expert
    address table, the shared expert's gate/up/down projections and gate row
    (0 when absent) and the RMSNorm weight (0 for none)."""
    table = (C.c_int64 * (_native.CHAIN_PTRS * len(layers)))()
    for l, w in enumerate(layers):
        row = [w.router.data_ptr(), w.expert_ptrs.data_ptr(), _opt(w.shared_gate_proj), _opt(w.shared_up_proj),
               _opt(w.shared_down_proj), _opt(w.shared_expert_gate), _opt(w.norm_weight), _opt(w.codec)]
        for i, v in enumerate(row):
            table[_native.CHAIN_PTRS * l + i] = v or 0
    return table


def moe_chain(hidden: torch.Tensor, layers, *, out: torch.Tensor | None = None, indices: torch.Tensor | None = None,
              weights: torch.Tensor | None = None, workspace: Workspace | None = None,
              check: bool = False) -> torch.Tensor:
    """Decode (T <= 16) through a stack of MoE layers in persistent launches
    of up to 48 layers each: h = moe_layer(h, layer) for every layer in
    order, with results identical to those successive calls.  ``indices`` /
    ``weights``, when given, receive every layer's routes ([L, T, 8]).
    ``check`` reads the status word after each launch (a host sync) and
    raises as Workspace.check does."""
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
        if check:
            ws.check(f"moe_chain layers {first}..{first + len(group) - 1}")
        src = dst
    return out


def gather(descriptors, destinations, sizes, src, dst, count, *, max_copies: int, experts: int, stripes: int = 64,
           threads: int = 256, keep_in_l2: bool = False, status: torch.Tensor | None = None) -> None:
    """Raw BF16 row gather (see include/lrmoe.h lrmoe_gather)."""
    device = destinations.device
    _native.call("lrmoe_gather", descriptors.data_ptr(), destinations.data_ptr(), sizes.data_ptr(), src.data_ptr(),
                 dst.data_ptr(), count.data_ptr(), int(experts), int(destinations.numel()), int(max_copies),
                 int(stripes), int(threads), int(bool(keep_in_l2)), _opt(status), _stream(device))
