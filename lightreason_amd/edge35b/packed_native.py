"""Replay variants of the single-token table path (edge35b/packed_native.py).

``configure(pool, mode)`` swaps ``packed_hybrid.packed_forward`` for the
duration of a ``with`` block (packed_native.py:152-255).  The reference's
modes differ in how cold experts reach the CPU workers and how hot rows are
staged over PCIe; with resident experts there are neither, so the modes
reduce to:

* ``buffers`` -- eager launches into a reusable workspace;
* ``graph``, ``native``, ``overlap``, ``pinned`` -- the same launches
  captured once into a HIP graph per workspace and replayed;
* ``ada`` -- as ``graph``, with gate/up + SiLU fused into the packed gate
  kernel (packed_ada.load_gate) instead of matvec + SwiGLU.

The captured graphs read the routes and weights from fixed device buffers
(the device table is rebuilt in place before each replay), so a call never
reads the routes on the host.

``mixer_graphs(model, pool)`` keeps the reference's name and report
attribute (packed_native.py:96-149, read by native_bench.py:143-155,198).
The reference captures the eager single-token mixer into one graph per
layer and copies the live states in and out around each replay; here the
single-token step is the native Gated DeltaNet launch of
``lightreason_amd.delta.fused_delta``, which works on the live cache states
in place, so there is nothing to capture or copy.
"""

from __future__ import annotations

from contextlib import ExitStack, contextmanager

import torch

from .. import _native, delta, moe
from . import packed_hybrid
from ._grid import stream_of
from .fused_experts import _matvec

MODES = ("buffers", "graph", "native", "overlap", "pinned", "ada")


class Workspace(packed_hybrid.Workspace):
    """Fixed-address buffers for one mode (packed_native.py:14-63)."""

    def __init__(self, device, library=None):
        super().__init__(device)
        bf16 = dict(dtype=torch.bfloat16, device=self.device)
        self.hidden_gpu = torch.empty((1, moe.HIDDEN), **bf16)
        self.router = torch.empty((1, moe.TOPK), **bf16)
        self.indices = torch.zeros((1, moe.TOPK), dtype=torch.int64, device=self.device)
        self.result = torch.empty((1, moe.HIDDEN), **bf16)
        self.hot_graph = self.combine_graph = None
        self.library = library
        self.ada_gate = None

    def hot(self, hidden=None) -> None:
        hidden = self.hidden_gpu if hidden is None else hidden
        if self.ada_gate is not None:
            self.ada_gate(self.device_table, hidden, self.active)
        else:
            _matvec[(128, 8)](self.device_table, hidden, self.gate_up, 2048, 1024, 0, 8, True, 4, num_warps=8)
            _native.call("lrmoe_swiglu_rows", self.gate_up.data_ptr(), self.active.data_ptr(), 8, stream_of(hidden))
        _matvec[(256, 8)](self.device_table, self.active, self.hot_results, 512, 2048, 1, 8, False, 4, num_warps=4)

    def combine(self) -> None:
        packed_hybrid._combine[(8,)](self.device_table, self.hot_results, self.cold_results, self.router, self.result,
                                     2048, 256, enable_fp_fusion=False)

    def capture(self, operation):
        """Run ``operation`` once eagerly, then capture it into a graph."""
        operation()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            operation()
        return graph


def native_library():
    """The native library of this build (liblrmoe.so).  The reference's
    (EDGE35B_PACKED_WORKERS, packed_native.py:66-79) provides the host plan and
    CPU expert workers; here the plan is built on the device and no expert
    runs on the host."""
    return _native.library()


@contextmanager
def configure(pool, mode):
    if mode not in MODES:
        raise ValueError(f"Unknown Packed ablation: {mode}")
    replay = mode != "buffers"
    library = native_library() if mode in ("native", "overlap", "pinned", "ada") else None
    original = packed_hybrid.packed_forward
    workspaces = getattr(pool, "native_workspaces", None)
    if workspaces is None:
        workspaces = pool.native_workspaces = {}

    def forward(layer, hidden, indices, weights, *, validate=True):
        if hidden.shape != (1, moe.HIDDEN) or indices.shape != (1, 8) or weights.shape != (1, 8):
            raise ValueError("Packed decode requires one token and eight routes")
        work = workspaces.get(mode)
        if work is None:
            work = workspaces[mode] = Workspace(hidden.device, library)
            if mode == "ada":
                from .packed_ada import load_gate

                work.ada_gate = load_gate()
        work.hidden_gpu.copy_(hidden)
        work.router.copy_(weights)
        work.indices.copy_(indices)
        layer.decode_step += 1
        work.build_table(layer, work.indices)
        if replay:
            if work.hot_graph is None:
                work.hot_graph = work.capture(work.hot)
            work.hot_graph.replay()
            if work.combine_graph is None:
                work.combine_graph = work.capture(work.combine)
            work.combine_graph.replay()
        else:
            work.hot()
            work.combine()
        if validate and not bool(work.valid.all()):
            raise ValueError("Packed decode requires in-range expert IDs")
        return work.result

    packed_hybrid.packed_forward = forward
    try:
        yield
    finally:
        packed_hybrid.packed_forward = original


def _counting(inner, index, served):
    """A mixer forward that notes layer `index` in `served` when it gets a
    single-token cached step (the reference's capture condition,
    packed_native.py:107-109), then runs `inner`."""

    def forward(hidden_states, cache_params=None, attention_mask=None, **kwargs):
        if (hidden_states.shape[:2] == (1, 1) and cache_params is not None and attention_mask is None
                and cache_params.has_previous_state(index)):
            served.setdefault(index, "native")
        return inner(hidden_states, cache_params=cache_params, attention_mask=attention_mask, **kwargs)

    forward.lrmoe_native = True
    return forward


@contextmanager
def mixer_graphs(model, pool):
    """Single-token Gated DeltaNet steps on the native mixer for the
    duration of the block.  Enters ``delta.fused_delta(model)`` unless every
    linear-attention mixer already runs natively (an enclosing
    ``fused_delta``, as native_bench.py:138 sets up).  ``pool.mixer_graphs``
    maps each layer index whose single-token cached step ran to "native",
    the keys the reference's report counts (native_bench.py:198)."""
    served = getattr(pool, "mixer_graphs", None)
    if served is None:
        served = pool.mixer_graphs = {}
    mixers = [(i, layer.linear_attn) for i, layer in enumerate(model.model.layers) if hasattr(layer, "linear_attn")]
    restore = []
    with ExitStack() as stack:
        if not all(getattr(m.__dict__.get("forward"), "lrmoe_native", False) for _, m in mixers):
            stack.enter_context(delta.fused_delta(model))
        try:
            for index, mixer in mixers:
                restore.append((mixer, mixer.__dict__.get("forward")))
                mixer.forward = _counting(mixer.forward, index, served)
            yield
        finally:
            for mixer, previous in reversed(restore):
                if previous is None:
                    del mixer.forward
                else:
                    mixer.forward = previous
