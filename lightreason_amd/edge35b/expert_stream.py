"""The plugin point: run a Transformers model's routed experts on liblrmoe.

Mirrors edge35b/expert_stream.py, whose ``patch_experts`` (457-526) replaces
``Qwen3_5MoeExperts.forward`` with ``_Layer.forward(hidden [T,H],
top_k_index [T,8] int64, top_k_weights [T,8] bf16) -> [T,H]`` (383-454) and
whose ``ExpertPool`` (60-174) moves expert rows from host memory into a
device LRU.  On MI355X every expert of every layer is resident in HBM
(40 x 256 x 6 MiB = 60 GiB of 288 GB), so :class:`ExpertPool` here is a
*resident* pool: ``_expert`` returns views of the HBM banks, nothing is
transferred, and the transfer modes of the reference (dense, selected,
cached, packed, ...) all run the same device kernels.  There is no CPU
expert path: the ``cpu`` and ``hybrid`` modes, whose cold experts ran on the
host, also run every expert on the GPU.

Two ways in:

* :func:`patch_experts` -- the reference's context manager, same arguments;
* :func:`register_experts_implementation` -- Transformers' own registry
  (``ExpertsInterface.register``): set ``config._experts_implementation``
  to the registered name and the model dispatches here.
"""

from __future__ import annotations

import threading
from contextlib import contextmanager
from dataclasses import asdict, dataclass

import torch

from .. import moe
from ..moe import EXPERTS, HIDDEN, INNER, TOPK

MODES = ("dense", "selected", "cached", "packed", "scheduled", "grouped", "pipelined",
         "fused", "batched", "cpu", "seeded", "hybrid")
PACKED_ROWS = 8
SCHEDULED_TOP_K = 8


@dataclass
class TransferStats:
    """Counter names of edge35b/expert_stream.py:37-57.  With resident
    experts the transfer counters stay zero; every lookup is a cache hit."""

    layer_calls: int = 0
    dense_layer_calls: int = 0
    selected_layer_calls: int = 0
    cached_layer_calls: int = 0
    packed_layer_calls: int = 0
    scheduled_layer_calls: int = 0
    prefill_cache_bypasses: int = 0
    prefill_packed_bypasses: int = 0
    prefill_scheduled_bypasses: int = 0
    scheduled_router_d2h_bytes: int = 0
    packed_router_d2h_bytes: int = 0
    packed_reuse_fences: int = 0
    packed_h2d_copies: int = 0
    routing_scalar_reads: int = 0
    transferred_bytes: int = 0
    transferred_expert_rows: int = 0
    cache_hits: int = 0
    cache_misses: int = 0
    cache_evictions: int = 0
    peak_cached_bytes: int = 0
    cpu_expert_rows: int = 0


class ExpertPool:
    """Resident expert pool on one device, used from one thread and stream
    (edge35b/expert_stream.py:60-174 keeps the same rule).

    ``capacity_bytes`` and ``non_blocking`` are accepted for signature
    compatibility; residency makes them moot.  Experts given as host tensors
    are copied into HBM once, when their layer is adapted."""

    def __init__(self, device="cuda:0", *, capacity_bytes=0, non_blocking=True):
        if type(capacity_bytes) is not int or capacity_bytes < 0:
            raise ValueError("capacity_bytes must be a nonnegative integer")
        if type(non_blocking) is not bool:
            raise ValueError("non_blocking must be a boolean")
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError("The resident expert pool needs a GPU device")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = device
        self._torch = torch
        self._capacity_bytes = capacity_bytes
        self._non_blocking = non_blocking
        self._rows: dict = {}
        self._resident_bytes = 0
        self._schedule_slots = None
        self._owner = None
        self._attached = False
        self.cache_multi_token = True
        self.grouped_verifier = True
        self.hybrid_verifier = False
        self.packed_hybrid = False
        self.packed_workspace = None
        self.cpu_block = None
        self.hybrid_reuse_window = None
        self.stats = TransferStats()
        self._workspaces: dict = {}

    # -- reference surface ----------------------------------------------------
    def snapshot(self) -> dict:
        return {**asdict(self.stats), "capacity_bytes": self._capacity_bytes,
                "cached_bytes": self._resident_bytes, "cached_rows": 0, "non_blocking": self._non_blocking,
                "packed_pinned_bytes": 0, "packed_setup_s": 0.0, "resident_bytes": self._resident_bytes}

    def reset_stats(self) -> None:
        self.stats = TransferStats(peak_cached_bytes=self._resident_bytes)

    def clear(self) -> None:
        """Nothing is cached beyond residency; kept for the reference API."""

    def _check_context(self) -> None:
        owner = (threading.get_ident(), torch.cuda.current_stream(self.device).cuda_stream)
        if self._owner is None:
            self._owner = owner
        elif owner != self._owner:
            raise RuntimeError("Use the pool on its original thread and stream")

    @staticmethod
    def _row_key(layer, index):
        return (id(layer), index)

    def _expert(self, layer, index, *, cached=True, copy=None):
        """(gate_up [1024, 2048], down [2048, 512]) views of a resident expert."""
        if not 0 <= int(index) < layer.gate_up.shape[0]:
            raise IndexError(f"expert {index} out of range")
        self.stats.cache_hits += 1
        return layer.gate_up[index], layer.down[index]

    # -- resident storage -----------------------------------------------------
    def workspace(self, tokens: int) -> moe.Workspace:
        key = torch.cuda.current_stream(self.device).cuda_stream
        ws = self._workspaces.get(key)
        if ws is None:
            ws = self._workspaces[key] = moe.Workspace(self.device, max(16, tokens))
        return ws.ensure(tokens)

    def make_resident(self, tensor: torch.Tensor) -> torch.Tensor:
        """The tensor itself when it is on the pool device with contiguous
        rows (any expert stride, e.g. a packed-pair bank view); otherwise a
        contiguous copy in HBM, made once."""
        if tensor.device == self.device and tensor.stride()[1:] == (tensor.shape[2], 1):
            return tensor
        resident = tensor.detach().to(self.device).contiguous()
        self._resident_bytes += resident.numel() * resident.element_size()
        self.stats.peak_cached_bytes = max(self.stats.peak_cached_bytes, self._resident_bytes)
        return resident


def expert_table(layer) -> torch.Tensor:
    """Device int64 [256, 2] of (gate_up, down) addresses for a layer whose
    ``gate_up`` [256, 1024, 2048] and ``down`` [256, 2048, 512] are device
    bf16 tensors with unit stride in the last dimension (the expert stride
    may be anything, e.g. a packed-pair bank).  Cached on the layer."""
    table = getattr(layer, "expert_ptrs", None)
    if table is not None:
        return table
    gate_up, down = layer.gate_up, layer.down
    if (tuple(gate_up.shape) != (EXPERTS, 2 * INNER, HIDDEN) or tuple(down.shape) != (EXPERTS, HIDDEN, INNER)
            or gate_up.dtype != torch.bfloat16 or down.dtype != torch.bfloat16):
        raise ValueError("expert tensors must be bf16 gate_up [256,1024,2048] and down [256,2048,512]")
    if gate_up.device.type != "cuda" or down.device != gate_up.device:
        raise ValueError("expert tensors must be resident on the GPU")
    if gate_up.stride()[1:] != (HIDDEN, 1) or down.stride()[1:] != (INNER, 1):
        raise ValueError("expert rows must be contiguous")
    key = (gate_up.data_ptr(), gate_up.stride(0), down.data_ptr(), down.stride(0))
    cached = getattr(layer, "_lrmoe_table", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    e = torch.arange(EXPERTS, dtype=torch.int64, device=gate_up.device)
    table = torch.stack([gate_up.data_ptr() + e * (2 * gate_up.stride(0)),
                         down.data_ptr() + e * (2 * down.stride(0))], dim=1).contiguous()
    layer._lrmoe_table = (key, table)
    return table


def raise_on_bad_routes(workspace: moe.Workspace, message: str) -> None:
    """Reads the device status of the last call (a host sync): ValueError
    with the reference's message for bad routes, RuntimeError when a
    bounded wait of the decode kernel expired (the outputs are invalid)."""
    status = workspace.status()
    if status & moe._native.STATUS_TIMEOUT:
        moe.check_status(status, "experts forward")
    if status & (moe._native.STATUS_BAD_EXPERT | moe._native.STATUS_REPEATED_EXPERT):
        raise ValueError(message)


def _is_silu(act_fn) -> bool:
    probe = torch.tensor([-3.0, -0.5, 0.0, 0.75, 4.0])
    try:
        got = act_fn(probe)
    except Exception:  # noqa: BLE001 -- any failure means "not SiLU"
        return False
    return isinstance(got, torch.Tensor) and torch.allclose(got, torch.nn.functional.silu(probe), atol=1e-6)


class _Layer:
    """One experts module bound to the resident pool
    (edge35b/expert_stream.py:325-454).  The module's gate_up_proj and
    down_proj become resident device tensors; the module itself is not
    modified apart from its forward while patched."""

    def __init__(self, name, module, pool: ExpertPool, mode: str):
        self.name = name
        self.module = module
        self.pool = pool
        self.mode = mode
        self.act_fn = module.act_fn
        self.decode_step = 0
        self.last_route: dict = {}
        if "forward" in vars(module):
            raise ValueError(f"{name}: expert forwards must have no existing patches")
        dims = (module.num_experts, module.hidden_dim, module.intermediate_dim)
        if dims != (EXPERTS, HIDDEN, INNER):
            raise ValueError(f"{name}: the kernels are built for 256 experts, hidden 2048, intermediate 512; "
                             f"got {dims}")
        for source, shape in ((module.gate_up_proj, (EXPERTS, 2 * INNER, HIDDEN)),
                              (module.down_proj, (EXPERTS, HIDDEN, INNER))):
            if source.dtype != torch.bfloat16 or tuple(source.shape) != shape or source.requires_grad:
                raise ValueError(f"{name}: expected frozen BF16 expert parameters of shape {shape}")
        if not _is_silu(self.act_fn):
            raise ValueError(f"{name}: the expert activation must be SiLU")
        self.gate_up = pool.make_resident(module.gate_up_proj.detach())
        self.down = pool.make_resident(module.down_proj.detach())
        self.row_bytes = 2 * (2 * INNER * HIDDEN + HIDDEN * INNER)
        self.expert_ptrs = None
        self.expert_ptrs = expert_table(self)

    def forward(self, hidden_states, top_k_index, top_k_weights):
        pool = self.pool
        pool._check_context()
        if torch.is_grad_enabled():
            raise RuntimeError("Run the patched experts under torch.no_grad() or torch.inference_mode()")
        if (hidden_states.ndim != 2 or hidden_states.device != pool.device or top_k_index.device != pool.device
                or top_k_weights.device != pool.device):
            raise ValueError(f"{self.name}: routed states and indices must be on the pool device")
        pool.stats.layer_calls += 1
        tokens = hidden_states.shape[0]
        if tokens == 1 and self.mode in ("fused", "batched"):
            from .fused_experts import fused_forward

            return fused_forward(self, hidden_states, top_k_index, top_k_weights,
                                 torch_projections=self.mode == "batched")
        if 2 <= tokens <= 16 and pool.grouped_verifier:
            from .block_experts import grouped_block

            return grouped_block(self, hidden_states, top_k_index, top_k_weights)
        from .pipeline import routed_forward

        return routed_forward(self, hidden_states, top_k_index, top_k_weights)


def _expert_modules(model):
    for name, module in model.named_modules():
        if all(hasattr(module, a) for a in ("gate_up_proj", "down_proj", "num_experts", "act_fn")):
            yield name, module


@contextmanager
def patch_experts(model, *, mode, pool):
    """Route every experts module of ``model`` (Transformers
    ``Qwen3_5MoeExperts`` or any module with ``gate_up_proj``, ``down_proj``,
    ``num_experts`` and ``act_fn``) through liblrmoe, then restore the
    original forwards (edge35b/expert_stream.py:457-526)."""
    if mode not in MODES:
        raise ValueError(f"Choose an expert transfer mode from {MODES}")
    if pool._attached:
        raise RuntimeError("The pool already has active expert forwards")
    layers = [_Layer(name, module, pool, mode) for name, module in _expert_modules(model)]
    if not layers:
        raise ValueError("No experts modules found")
    pool._check_context()
    pool._attached = True
    installed = []
    try:
        for layer in layers:
            layer.module.forward = layer.forward
            installed.append(layer)
        yield pool
    finally:
        for layer in reversed(installed):
            del layer.module.forward
        pool._attached = False


def register_experts_implementation(name: str = "lrmoe", *, pool: ExpertPool | None = None, mode: str = "fused"):
    """Register liblrmoe in Transformers' ExpertsInterface under ``name``.
    A model whose ``config._experts_implementation == name`` then calls
    ``fn(module, hidden_states, top_k_index, top_k_weights)`` for its experts;
    each module is adapted to the resident pool on first use."""
    from transformers.integrations.moe import ExpertsInterface

    if mode not in MODES:
        raise ValueError(f"Choose an expert transfer mode from {MODES}")
    state = {"pool": pool}

    def experts_forward(module, hidden_states, top_k_index, top_k_weights):
        layer = getattr(module, "_lrmoe_layer", None)
        if layer is None:
            if state["pool"] is None:
                state["pool"] = ExpertPool(hidden_states.device)
            layer = _Layer(type(module).__name__, module, state["pool"], mode)
            module._lrmoe_layer = layer
        return layer.forward(hidden_states, top_k_index, top_k_weights)

    ExpertsInterface.register(name, experts_forward)
    return experts_forward
