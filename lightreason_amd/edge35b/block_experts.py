"""Grouped verification of 2-16 target positions (edge35b/block_experts.py).

``_project`` and ``_combine`` keep the reference kernels' grid protocol
(block_experts.py:12-49) on liblrmoe.  ``grouped_block`` keeps the guards of
block_experts.py:89-95 and replaces the host-side route grouping (102-121)
and the two projections + combine with the device decode path: bucketing,
one gate/up pass that streams each unique expert once for all of its
tokens, and a down pass with the ordered combine fused in.
"""

from __future__ import annotations

import torch

from .. import _native, moe
from ._grid import GridKernel, pointer, stream_of
from .expert_stream import expert_table, raise_on_bad_routes

ROWS = 16


def _launch_project(grid, Pointers, Routes, X, Y, IN, OUT, DOWN, ROWS_, COLS, REDUCE):
    experts, col_blocks, depth = grid
    IN, OUT, COLS = int(IN), int(OUT), int(COLS)
    if depth != 1 or int(ROWS_) != ROWS or col_blocks * COLS != OUT:
        raise ValueError("_project: ROWS must be 16 and the grid must cover OUT columns exactly")
    if Pointers.numel() < 2 * experts or Routes.numel() < experts * ROWS or Y.numel() < experts * ROWS * OUT:
        raise ValueError("_project: Pointers, Routes or Y smaller than the grid needs")
    if DOWN and X.numel() < experts * ROWS * IN:
        raise ValueError("_project: X smaller than the grid needs")
    _native.call("lrmoe_project", pointer(Pointers, torch.int64, "Pointers"), pointer(Routes, torch.int32, "Routes"),
                 pointer(X, torch.bfloat16, "X"), pointer(Y, torch.bfloat16, "Y"), IN, OUT, int(bool(DOWN)), experts,
                 stream_of(Y))


def _launch_combine(grid, Inverse, X, Cold, Router, Out, WIDTH, ROWS_, TILE, HYBRID):
    tokens, tiles, depth = grid
    if depth != 1 or int(WIDTH) != moe.HIDDEN or int(ROWS_) != ROWS or tiles * int(TILE) != moe.HIDDEN:
        raise ValueError("_combine: WIDTH 2048, ROWS 16, and the grid must cover WIDTH")
    if Inverse.numel() < tokens * moe.TOPK * 3 or Router.numel() < tokens * moe.TOPK or Out.numel() < tokens * moe.HIDDEN:
        raise ValueError("_combine: Inverse, Router or Out smaller than the grid needs")
    cold = pointer(Cold, torch.bfloat16, "Cold") if HYBRID else None
    _native.call("lrmoe_block_combine", pointer(Inverse, torch.int32, "Inverse"), pointer(X, torch.bfloat16, "X"),
                 cold, pointer(Router, torch.bfloat16, "Router"), pointer(Out, torch.bfloat16, "Out"), tokens,
                 int(bool(HYBRID)), stream_of(Out))


_project = GridKernel("_project", _launch_project)
_combine = GridKernel("_combine", _launch_combine)


def grouped_block(layer, hidden, indices, weights, *, validate=True):
    """out [T, 2048] for 2 <= T <= 16 positions: per token, its 8 routes in
    ascending expert order, bf16(expert(hidden[t]) * w) accumulated in bf16.

    ``validate`` raises ValueError for routes outside [0, 256) or a token
    routed twice to one expert (one device read after the launches);
    ``validate=False`` leaves them to the workspace status bits (no sync)."""
    count, width = hidden.shape
    if not 2 <= count <= 16 or width != 2048 or indices.shape != (count, 8):
        raise ValueError("Grouped expert verification needs 2–16 Qwen3.6 target positions")
    if not hidden.is_contiguous() or not weights.is_contiguous():
        raise ValueError("Grouped expert verification requires contiguous target activations")
    ws = layer.pool.workspace(count)
    out = moe.moe_experts(hidden, indices.contiguous(), weights, expert_table(layer), workspace=ws)
    if validate:
        raise_on_bad_routes(ws, "Grouped expert verification requires distinct in-range routes per position")
    return out
