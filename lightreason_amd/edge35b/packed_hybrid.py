"""Table-driven single-token experts (edge35b/packed_hybrid.py) on liblrmoe.

The reference splits the 8 routes into GPU-cached ("hot") experts, run by
two ``_matvec`` launches, and host ("cold") experts run by the AVX2 library,
then ``_combine``s both (packed_hybrid.py:13-85).  With every expert resident
in HBM all routes are hot, so the cold half is always empty; the table keeps
its 4-column layout (gate_up address, down address, router slot, cold row
= -1) so that ``_combine`` and ``packed_native`` callers see the same
protocol.  The table is built on the device (sort of the 8 routes by expert
id), so ``packed_forward`` needs no host read of the routes.
"""

from __future__ import annotations

import torch

from .. import _native, moe
from ._grid import GridKernel, pointer, stream_of
from .expert_stream import expert_table
from .fused_experts import _matvec


def _launch_combine(grid, Table, Hot, Cold, Router, Out, WIDTH, BLOCK):
    if int(WIDTH) != moe.HIDDEN or grid[0] * int(BLOCK) < moe.HIDDEN:
        raise ValueError("_combine: WIDTH must be 2048 and the grid must cover it")
    if Table.numel() < 4 * moe.TOPK or Hot.numel() < moe.TOPK * moe.HIDDEN or Out.numel() < moe.HIDDEN:
        raise ValueError("_combine: Table, Hot or Out too small for 8 routes")
    if Router.numel() < moe.TOPK or Cold.numel() < moe.TOPK * moe.HIDDEN:
        raise ValueError("_combine: Router or Cold too small for 8 routes")
    _native.call("lrmoe_ordered_sum", pointer(Table, torch.int64, "Table"), pointer(Hot, torch.bfloat16, "Hot"),
                 pointer(Cold, torch.bfloat16, "Cold"), pointer(Router, torch.bfloat16, "Router"),
                 pointer(Out, torch.bfloat16, "Out"), 4, stream_of(Out))


_combine = GridKernel("_combine", _launch_combine)


class Workspace:
    """Device buffers of one single-token expert pass (packed_hybrid.py:30-43,
    minus the pinned host staging that resident experts do not need)."""

    def __init__(self, device):
        device = torch.device(device)
        bf16 = dict(dtype=torch.bfloat16, device=device)
        self.device = device
        self.device_table = torch.zeros((8, 4), dtype=torch.int64, device=device)
        self.valid = torch.ones(8, dtype=torch.bool, device=device)
        self.gate_up = torch.empty((8, 2 * moe.INNER), **bf16)
        self.active = torch.empty((8, moe.INNER), **bf16)
        self.hot_results = torch.empty((8, moe.HIDDEN), **bf16)
        self.cold_results = torch.zeros((8, moe.HIDDEN), **bf16)

    def build_table(self, layer, indices: torch.Tensor) -> None:
        """Rows in ascending expert order: (gate_up, down, slot, -1); rows of
        out-of-range experts get null addresses (skipped by _matvec) and a
        False in ``valid``.  Device ops only."""
        ids = indices.reshape(-1)[:8]
        experts, slots = torch.sort(ids, stable=True)
        ok = (experts >= 0) & (experts < moe.EXPERTS)
        addresses = expert_table(layer)[experts.clamp(0, moe.EXPERTS - 1)] * ok[:, None]
        self.device_table[:, :2].copy_(addresses)
        self.device_table[:, 2].copy_(slots)
        self.device_table[:, 3].fill_(-1)
        self.valid.copy_(ok)

    def hot(self, hidden: torch.Tensor) -> None:
        """Gate/up matvec, SwiGLU, down matvec of the 8 table rows."""
        _matvec[(128, 8)](self.device_table, hidden, self.gate_up, 2048, 1024, 0, 8, True, 4, num_warps=8)
        _native.call("lrmoe_swiglu_rows", self.gate_up.data_ptr(), self.active.data_ptr(), 8, stream_of(hidden))
        _matvec[(256, 8)](self.device_table, self.active, self.hot_results, 512, 2048, 1, 8, False, 4, num_warps=4)


def packed_forward(layer, hidden, indices, weights, *, validate=True):
    """out [1, 2048]: the 8 routes' experts combined in ascending expert order
    (bf16 product with the router weight, bf16 running sum from zero).
    ``validate`` raises ValueError for an expert id outside [0, 256) (one
    device read); ``validate=False`` is free of host synchronisation."""
    if hidden.shape != (1, moe.HIDDEN) or indices.shape != (1, 8) or weights.shape != (1, 8):
        raise ValueError("Packed decode requires one token and eight routes")
    pool = layer.pool
    if pool.packed_workspace is None:
        pool.packed_workspace = Workspace(hidden.device)
    work = pool.packed_workspace
    layer.decode_step += 1
    work.build_table(layer, indices)
    work.hot(hidden.contiguous())
    result = torch.empty_like(hidden)
    _combine[(8,)](work.device_table, work.hot_results, work.cold_results, weights.contiguous(), result, 2048, 256,
                   enable_fp_fusion=False)
    if validate and not bool(work.valid.all()):
        raise ValueError("Packed decode requires in-range expert IDs")
    return result
