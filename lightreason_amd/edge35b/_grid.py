"""Grid-indexable launch objects with the reference kernels' call protocol.

The reference launches its Triton kernels as ``kernel[grid](*args, **meta)``
(e.g. edge35b/packed_hybrid.py:71-74, packed_native.py:49-52,
block_experts.py:130-133).  :class:`GridKernel` keeps that protocol and runs
the matching liblrmoe entry point on torch's current stream instead.
Meta-parameters that only steer the reference's code generation
(``num_warps``, ``num_stages``, ``enable_fp_fusion``) are accepted and have
no effect: the HIP kernels fix their own launch shape, and their arithmetic
never contracts a multiply-add that the reference rounds separately.
"""

from __future__ import annotations

import torch

_CODEGEN_META = frozenset({"num_warps", "num_stages", "num_ctas", "enable_fp_fusion", "maxnreg"})


class GridKernel:
    def __init__(self, name: str, launch):
        self.__name__ = name
        self._launch = launch

    def __getitem__(self, grid):
        if callable(grid):
            raise TypeError(f"{self.__name__}: give the launch grid as a tuple of ints")
        dims = tuple(int(g) for g in (grid if isinstance(grid, (tuple, list)) else (grid,)))
        if not 1 <= len(dims) <= 3 or any(g <= 0 for g in dims):
            raise ValueError(f"{self.__name__}: invalid grid {grid!r}")
        dims = dims + (1,) * (3 - len(dims))

        def launch(*args, **meta):
            unknown = set(meta) - _CODEGEN_META
            if unknown:
                raise TypeError(f"{self.__name__}: unexpected arguments {sorted(unknown)}")
            return self._launch(dims, *args)

        return launch

    def __repr__(self) -> str:
        return f"<GridKernel {self.__name__} (liblrmoe)>"


def pointer(tensor, dtype: torch.dtype, name: str) -> int:
    """Device address of a contiguous device tensor of ``dtype``."""
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a device tensor")
    if tensor.device.type != "cuda":
        raise ValueError(f"{name} must be a device tensor")
    if tensor.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {tensor.dtype}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return tensor.data_ptr()


def stream_of(tensor: torch.Tensor) -> int:
    return torch.cuda.current_stream(tensor.device).cuda_stream
