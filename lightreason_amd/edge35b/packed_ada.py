"""The packed gate/SiLU kernel (edge35b/packed_ada.py, packed_ada.cu) on
liblrmoe.  ``load_gate()`` returns ``launch(table, hidden, active)``:
for the 8 rows of a 4-column table whose gate_up address is non-zero,
active[e, r] = bf16(bf16(silu(bf16(g))) * bf16(u)) with g, u the fp32 dot
products of gate row r and up row r with hidden (packed_ada.cu:13-40).
The reference compiles for sm_89 at first use; here the kernel is part of
liblrmoe.so (gfx950) and the loader checks the device instead."""

from __future__ import annotations

from functools import lru_cache

import torch

from .. import _native, moe
from ._grid import pointer, stream_of


@lru_cache(maxsize=1)
def load_gate():
    try:
        _native.device_check()
    except _native.NativeError as exc:
        raise RuntimeError("The packed gate kernel is built for gfx950 (MI355X)") from exc

    def launch(table, hidden, active):
        if table.numel() < 4 * moe.TOPK or hidden.numel() < moe.HIDDEN or active.numel() < moe.TOPK * moe.INNER:
            raise ValueError("packed gate: table [8,4], hidden [2048] and active [8,512] expected")
        _native.call("lrmoe_gate_silu", pointer(table, torch.int64, "table"), pointer(hidden, torch.bfloat16, "hidden"),
                     pointer(active, torch.bfloat16, "active"), 4, moe.TOPK, stream_of(active))

    return launch
