"""Verify-width integration: the adaptive width controller (host logic, no
GPU) and the per-width captured MoE stacks (needs an MI355X).

Bar for the graphs: every width's replay gives the same output, routes and
routing weights, bit for bit, as an eager moe_chain call and as successive
moe_layer calls on the same block, and every layer of the replay matches the
oracle (routes bit-exact, outputs within the layer bar), across replays with
new inputs and interleaved widths."""

from __future__ import annotations

import numpy as np
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
def test_verify_graphs_against_oracle_per_width(device, oracle):
    """Six distinct seeded layers (routers, experts, shared experts, RMSNorm
    weights all differ) captured at widths 1, 2, 5, 8, 13 and 16, replayed
    in an interleaved order with a new block each time.  Per replay:

    - the graph's output and per-layer routes are bit-identical to an eager
      moe_chain and to successive moe_layer calls on the same block;
    - for every layer l, the oracle's block applied to that layer's input
      (layer l-1's output from the successive calls) gives the graph's
      routes and routing weights bit for bit and an output within
      helpers.assert_layer_close (1e-2 of the row's MoE magnitude plus one
      bf16 ulp);
    - the status word is clean (verify() checks it by default)."""
    from helpers import HostExperts, assert_layer_close, oracle_layer_rows, to_u16
    from lightreason_amd.moe import Workspace, moe_chain, moe_layer
    from lightreason_amd.synthetic import SyntheticModel
    from lightreason_amd.verify import VerifyGraphs

    model = SyntheticModel(layers=6, device=device, seed=6262, shared=True, norm="normal")
    layers = model.layers
    L = len(layers)
    widths = (1, 2, 5, 8, 13, 16)
    graphs = VerifyGraphs(layers, widths=widths)
    ws = Workspace(device, 16)
    host = [HostExperts(model.bank, l) for l in range(L)]
    for rep, width in enumerate((8, 2, 16, 5, 1, 13, 8, 16)):
        print(f"[verify] replay {rep}: width {width}", flush=True)
        x = model.hidden(width, step=6000 + rep)
        got = graphs.verify(x).clone()
        idx_g, w_g = (t.clone() for t in graphs.routes(width))
        idx = torch.empty((L, width, 8), dtype=torch.int64, device=device)
        wts = torch.empty((L, width, 8), dtype=torch.bfloat16, device=device)
        want = moe_chain(x, layers, indices=idx, weights=wts, workspace=ws)
        inputs = [x]
        for layer in layers:
            inputs.append(moe_layer(inputs[-1], layer, workspace=ws))
        torch.cuda.synchronize()
        assert ws.status() == 0
        assert torch.equal(idx_g, idx)
        assert torch.equal(w_g.view(torch.int16), wts.view(torch.int16))
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        assert torch.equal(got.view(torch.int16), inputs[-1].view(torch.int16))
        idx_h, w_h = idx_g.cpu().numpy(), to_u16(w_g)
        for l, layer in enumerate(layers):
            xb = to_u16(inputs[l])
            ref, o_idx, o_w = oracle_layer_rows(oracle, layer, xb, host[l])
            np.testing.assert_array_equal(idx_h[l], o_idx, err_msg=f"width {width} layer {l} routes")
            np.testing.assert_array_equal(w_h[l], o_w, err_msg=f"width {width} layer {l} weights")
            assert_layer_close(to_u16(inputs[l + 1]), ref, xb, what=f"width {width} layer {l}")
    with pytest.raises(ValueError, match="no verify graph"):
        graphs.verify(model.hidden(3, step=1))
