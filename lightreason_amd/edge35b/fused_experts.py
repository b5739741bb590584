"""Single-token experts (edge35b/fused_experts.py) on liblrmoe.

``_matvec`` and ``_ordered_sum`` keep the reference kernels' grid protocol
(``_matvec[(g0, g1)](table, x, result, K, N, WEIGHT_COLUMN, BLOCK_ROWS,
SHARED_X, STRIDE=3, num_warps=...)``, fused_experts.py:8-37) for callers that
build their own tables (packed_hybrid, packed_native).  ``fused_forward``
keeps the reference's guards (40-50) but schedules on the device: no
``.tolist()`` of the routes, one fused decode launch sequence
(bucketing + gate/up/SwiGLU + down/combine).
"""

from __future__ import annotations

import torch

from .. import _native, moe
from ._grid import GridKernel, pointer, stream_of
from .expert_stream import expert_table, raise_on_bad_routes

_ROUTE_ERROR = "Fused expert decode requires eight distinct valid routes"


def _launch_matvec(grid, table, x, result, K, N, WEIGHT_COLUMN, BLOCK_ROWS, SHARED_X, STRIDE=3):
    rows, experts, depth = grid
    K, N, column, stride = int(K), int(N), int(WEIGHT_COLUMN), int(STRIDE)
    if depth != 1 or rows * int(BLOCK_ROWS) < N:
        raise ValueError("_matvec: the grid must cover all N rows of every expert")
    if table.numel() < stride * experts:
        raise ValueError("_matvec: table is smaller than the grid's experts")
    if x.numel() < (K if SHARED_X else experts * K) or result.numel() < experts * N:
        raise ValueError("_matvec: x or result is smaller than the grid needs")
    _native.call("lrmoe_matvec", pointer(table, torch.int64, "table"), pointer(x, torch.bfloat16, "x"),
                 pointer(result, torch.bfloat16, "result"), K, N, column, int(bool(SHARED_X)), stride, experts,
                 stream_of(result))


def _launch_ordered_sum(grid, table, values, weights, out, HIDDEN, BLOCK):
    if int(HIDDEN) != moe.HIDDEN or grid[0] * int(BLOCK) < moe.HIDDEN:
        raise ValueError("_ordered_sum: HIDDEN must be 2048 and the grid must cover it")
    if table.numel() < 3 * moe.TOPK or values.numel() < moe.TOPK * moe.HIDDEN or out.numel() < moe.HIDDEN:
        raise ValueError("_ordered_sum: table, values or out too small for 8 routes")
    if weights.numel() < moe.TOPK:
        raise ValueError("_ordered_sum: weights must hold the 8 router slots")
    _native.call("lrmoe_ordered_sum", pointer(table, torch.int64, "table"), pointer(values, torch.bfloat16, "values"),
                 None, pointer(weights, torch.bfloat16, "weights"), pointer(out, torch.bfloat16, "out"), 3,
                 stream_of(out))


_matvec = GridKernel("_matvec", _launch_matvec)
_ordered_sum = GridKernel("_ordered_sum", _launch_ordered_sum)


def _check_single_token(layer, hidden, indices, weights) -> None:
    if (hidden.shape != (1, 2048) or indices.shape != (1, 8) or weights.shape != (1, 8)
            or hidden.dtype != torch.bfloat16 or weights.dtype != torch.bfloat16
            or not hidden.is_contiguous() or not weights.is_contiguous()
            or layer.gate_up.shape[1:] != (1024, 2048) or layer.down.shape[1:] != (2048, 512)):
        raise ValueError("Fused expert decode requires the single-token 35B route shape")
    if layer.module.num_experts != moe.EXPERTS:
        raise ValueError("Fused expert decode requires 256 experts")


def fused_forward(layer, hidden, indices, weights, *, torch_projections=False, validate=True):
    """out [1, 2048] = sum over the 8 routes, ascending expert id, of
    bf16(expert(hidden) * weight), accumulated in bf16 from zero.

    ``validate`` (default, the reference's behaviour) raises ValueError when
    the routes are not eight distinct experts in range; that reads one device
    word after the launches.  ``validate=False`` makes the call free of host
    synchronisation (graph-capturable); bad routes then only set the
    workspace status bits and yield zeros.  ``torch_projections=True`` is the
    reference's ``batched`` ablation: the projections run as torch batched
    products (scheduled on the device), the combine on liblrmoe."""
    _check_single_token(layer, hidden, indices, weights)
    if indices.dtype != torch.int64:
        raise ValueError("Fused expert decode requires int64 routes")
    if torch_projections:
        return _torch_projection_forward(layer, hidden, indices, weights)
    ws = layer.pool.workspace(1)
    out = moe.moe_experts(hidden, indices.contiguous(), weights, expert_table(layer), workspace=ws)
    if validate:
        raise_on_bad_routes(ws, _ROUTE_ERROR)
    return out


def _torch_projection_forward(layer, hidden, indices, weights):
    """The ``batched`` ablation: the expert projections as torch products
    instead of the decode kernel (the reference runs one torch linear per
    expert from a host-side schedule).  Here the schedule stays on the
    device: the eight routes are sorted there and checked with one device
    read (the same ValueError), the selected experts' weights are gathered
    with ``index_select`` into one batched product for gate/up and one for
    down, SwiGLU is the module's ``act_fn`` on bf16 tensors, and the ordered
    combine is the ``_ordered_sum`` shim over a device-built table."""
    experts, slots = torch.sort(indices.reshape(moe.TOPK), stable=True)
    valid = (experts[0] >= 0) & (experts[-1] < moe.EXPERTS) & (experts[1:] != experts[:-1]).all()
    if not bool(valid):
        raise ValueError(_ROUTE_ERROR)
    column = hidden.reshape(1, moe.HIDDEN, 1).expand(moe.TOPK, moe.HIDDEN, 1).contiguous()
    products = torch.bmm(layer.gate_up.index_select(0, experts).contiguous(), column).squeeze(2)
    gate, up = products.split(moe.INNER, dim=1)
    act = (layer.act_fn(gate) * up).unsqueeze(2).contiguous()
    projected = torch.bmm(layer.down.index_select(0, experts).contiguous(), act).squeeze(2).contiguous()
    addresses = expert_table(layer).index_select(0, experts)
    table = torch.cat((addresses, slots.unsqueeze(1)), dim=1).contiguous()
    result = torch.empty_like(hidden)
    _ordered_sum[(8,)](table, projected, weights, result, 2048, 256, enable_fp_fusion=False)
    return result
