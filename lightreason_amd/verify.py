"""Verify-width integration: speculative-verify blocks of 1-16 positions
through the MoE stack, one captured HIP graph per width, and the width
controller of the reference's DFlash verify loop.

The reference verifies a drafter's block of `count` positions with one
target forward (edge35b/dflash_probe.py:111-120), whose MoE layers take the
grouped path for 2-16 positions (edge35b/block_experts.py:89-139: routes
[T, 8], weights [T, 8], an inverse map per token), and in its adaptive mode
changes the width between blocks (dflash_probe.py:144-148).  Here a block's
MoE stack is one ``moe_chain`` launch per 48 layers (the whole decode layer
-- router, bucketing, experts, combine, shared expert, RMSNorm and residual
-- for every layer), captured once per width so that a verify pass is one
graph replay whatever width the controller picks.
"""

from __future__ import annotations

import torch

from .moe import DECODE_MAX_TOKENS, HIDDEN, TOPK, Workspace, moe_chain


class WidthController:
    """The adaptive verify width of edge35b/dflash_probe.py:144-148: start at
    ``start``; after a block verified at the full width (count == width),
    widen by ``step`` (at most ``limit``, the drafter's block size) when at
    least width - 1 positions were committed, narrow by ``step`` (at least
    ``floor``) when at most width // 2 were, and hold otherwise."""

    def __init__(self, start: int = 8, floor: int = 4, limit: int = 16, step: int = 4):
        if not 1 <= floor <= start <= limit <= DECODE_MAX_TOKENS or step < 1:
            raise ValueError(f"need 1 <= floor <= start <= limit <= {DECODE_MAX_TOKENS} and step >= 1")
        self.width, self.floor, self.limit, self.step = start, floor, limit, step

    def block(self, remaining: int) -> int:
        """Positions of the next block when `remaining` outputs are left
        under the cap (dflash_probe.py:111)."""
        return max(0, min(self.width, remaining))

    def update(self, count: int, committed: int) -> int:
        """Adjust after a block of `count` positions that committed
        `committed` outputs; returns the new width."""
        if count == self.width:
            if committed >= self.width - 1:
                self.width = min(self.width + self.step, self.limit)
            elif committed <= self.width // 2:
                self.width = max(self.floor, self.width - self.step)
        return self.width


class VerifyGraphs:
    """The MoE stack (``layers``: LayerWeights, RMSNorm + residual when they
    carry norm weights) for verify blocks of each width in ``widths``, each
    captured as one HIP graph over static buffers.  ``verify(hidden)`` copies
    a [T, 2048] block in, replays width T's graph and returns its static
    output (valid until the next verify of that width); ``routes(T)`` gives
    that replay's per-layer routes ([L, T, 8] indices and weights).  All
    widths share one workspace and run on the capturing stream in call
    order."""

    def __init__(self, layers, widths=range(1, DECODE_MAX_TOKENS + 1), device=None):
        self.layers = list(layers)
        if not self.layers:
            raise ValueError("VerifyGraphs needs at least one layer")
        self.device = torch.device(device) if device is not None else self.layers[0].router.device
        self.widths = sorted(set(int(w) for w in widths))
        if not self.widths or self.widths[0] < 1 or self.widths[-1] > DECODE_MAX_TOKENS:
            raise ValueError(f"verify widths must lie in 1..{DECODE_MAX_TOKENS}")
        self.workspace = Workspace(self.device, DECODE_MAX_TOKENS)
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs = {}
        L = len(self.layers)
        stream = torch.cuda.Stream(self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            for w in self.widths:
                static = dict(
                    hidden=torch.zeros((w, HIDDEN), dtype=torch.bfloat16, device=self.device),
                    out=torch.empty((w, HIDDEN), dtype=torch.bfloat16, device=self.device),
                    indices=torch.empty((L, w, TOPK), dtype=torch.int64, device=self.device),
                    weights=torch.empty((L, w, TOPK), dtype=torch.bfloat16, device=self.device))
                run = self._runner(static)
                run()  # eager once: any one-time setup happens outside the capture
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, pool=self.pool, stream=stream):
                    run()
                self.graphs[w] = (graph, static)
        torch.cuda.current_stream(self.device).wait_stream(stream)

    def _runner(self, static):
        def run():
            moe_chain(static["hidden"], self.layers, out=static["out"], indices=static["indices"],
                      weights=static["weights"], workspace=self.workspace)
        return run

    def verify(self, hidden: torch.Tensor, *, check: bool = True) -> torch.Tensor:
        """Replay the block's width graph.  ``check`` (default) reads the
        workspace status word afterwards (a host synchronisation) and raises
        RuntimeError when a bounded wait of the chain kernel expired (its
        outputs are invalid: another kernel kept workgroups off the GPU);
        ``check=False`` leaves the status to ``status()``."""
        width = hidden.shape[0]
        entry = self.graphs.get(width)
        if entry is None:
            raise ValueError(f"no verify graph of width {width} (captured: {self.widths})")
        if hidden.shape != (width, HIDDEN) or hidden.dtype != torch.bfloat16 or hidden.device != self.device:
            raise ValueError(f"hidden must be bf16 [{width}, {HIDDEN}] on {self.device}")
        graph, static = entry
        static["hidden"].copy_(hidden)
        graph.replay()
        if check:
            self.workspace.check("VerifyGraphs.verify")
        return static["out"]

    def routes(self, width: int):
        _, static = self.graphs[width]
        return static["indices"], static["weights"]

    def status(self) -> int:
        """Status word of the last replay (reads the device)."""
        return self.workspace.status()
