"""The reference runner's expert-path modules (package ``edge35b``) on
liblrmoe: same module names, functions, arguments and error types, backed
by the gfx950 kernels.  ``install_as_edge35b()`` makes ``import edge35b.X``
resolve here, for code written against the reference package."""

from __future__ import annotations

import importlib
import sys

MODULES = ("expert_stream", "fused_experts", "block_experts", "pipeline", "packed_hybrid", "packed_ada",
           "packed_native", "native_bf16_gather")


def install_as_edge35b() -> None:
    package = sys.modules[__name__]
    sys.modules.setdefault("edge35b", package)
    for module in MODULES:
        sys.modules.setdefault(f"edge35b.{module}", importlib.import_module(f"{__name__}.{module}"))
