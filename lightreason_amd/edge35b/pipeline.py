"""Multi-token (prefill) experts in the eager order (edge35b/pipeline.py).

``routed_forward`` (pipeline.py:79-110) visits experts ascending, runs each
expert on its tokens in ascending token order, scales by the router weight in
bf16 and ``index_add_``s in bf16 -- per token that is the ordered bf16
combine over its routes in ascending expert order.  Here the grouping
(``_routes``, 59-76) happens on the device and the experts run as grouped
BF16 MFMA tiles: each (expert, 16-row weight tile) is read from HBM once for
all of the expert's tokens.  The reference's ``TransferPipeline`` (9-56)
overlaps host-to-device copies of expert rows; with resident experts there
is nothing to copy, so ``pipeline`` must be None.
"""

from __future__ import annotations

from .. import moe
from .expert_stream import expert_table, raise_on_bad_routes


def routed_forward(layer, hidden_states, top_k_index, top_k_weights, *, pipeline=None, validate=True):
    if pipeline is not None:
        raise ValueError("Experts are resident in HBM: there is no transfer pipeline to overlap")
    tokens = hidden_states.shape[0]
    if tokens == 0:
        return hidden_states.new_zeros(hidden_states.shape)
    ws = layer.pool.workspace(tokens)
    out = moe.moe_experts(hidden_states.contiguous(), top_k_index.contiguous(), top_k_weights.contiguous(),
                          expert_table(layer), workspace=ws)
    if validate:
        raise_on_bad_routes(ws, "Routed experts require distinct in-range expert ids per token")
    return out
