"""Verify-width integration: the adaptive width controller (host logic, no
GPU) and the per-width captured MoE stacks (needs an MI355X).

Bar for the graphs: every width's replay gives the same output, routes and
routing weights, bit for bit, as an eager moe_chain call on the same block
(the chain itself is checked against the oracle layer by layer in
test_gpu_stack.py), across replays with new inputs and interleaved widths."""

from __future__ import annotations

import pytest
import torch

from lightreason_amd.verify import WidthController


def test_width_controller_follows_the_reference_rule():
    """edge35b/dflash_probe.py:144-148: widen by 4 after committing at least
    width - 1, narrow by 4 after at most width // 2, hold otherwise; only
    after a full-width block; bounded by 4 and the drafter's 16."""
    c = WidthController()
    assert c.width == 8 and c.block(100) == 8
    assert c.update(8, 7) == 12        # width - 1 committed: widen
    assert c.update(12, 12) == 16      # all committed: widen
    assert c.update(16, 16) == 16      # already at the drafter's block size
    assert c.update(16, 9) == 16       # 9 > 16 // 2 and < 15: hold
    assert c.update(16, 8) == 12       # at most half: narrow
    assert c.update(12, 6) == 8
    assert c.update(8, 4) == 4
    assert c.update(4, 1) == 4         # floor
    assert c.update(4, 3) == 8         # 3 >= 4 - 1: widen
    assert c.block(5) == 5             # a block cut short at the output cap...
    assert c.update(5, 5) == 8         # ...does not move the width
    assert c.block(0) == 0
    with pytest.raises(ValueError):
        WidthController(start=2, floor=4)
    with pytest.raises(ValueError):
        WidthController(limit=17)


@pytest.mark.gpu
def test_verify_graphs_equal_eager_chains(device):
    from lightreason_amd.moe import LayerWeights, Workspace, moe_chain
    from lightreason_amd.synthetic import SyntheticModel
    from lightreason_amd.verify import VerifyGraphs

    model = SyntheticModel(layers=3, device=device, seed=6262, shared=True, norm="normal")
    layers = [LayerWeights(**ly.__dict__) for ly in model.layers] * 2   # a 6-layer stack
    widths = (2, 5, 8, 16)
    graphs = VerifyGraphs(layers, widths=widths)
    ws = Workspace(device, 16)
    for rep, width in enumerate((8, 2, 16, 5, 8, 16)):
        print(f"[verify] replay {rep}: width {width}", flush=True)
        x = model.hidden(width, step=6000 + rep)
        got = graphs.verify(x).clone()
        idx_g, w_g = (t.clone() for t in graphs.routes(width))
        assert graphs.status() == 0
        idx = torch.empty((len(layers), width, 8), dtype=torch.int64, device=device)
        wts = torch.empty((len(layers), width, 8), dtype=torch.bfloat16, device=device)
        want = moe_chain(x, layers, indices=idx, weights=wts, workspace=ws)
        torch.cuda.synchronize()
        assert ws.status() == 0
        assert torch.equal(idx_g, idx)
        assert torch.equal(w_g.view(torch.int16), wts.view(torch.int16))
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    with pytest.raises(ValueError, match="no verify graph"):
        graphs.verify(model.hidden(3, step=1))
