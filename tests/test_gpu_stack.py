"""The 40-layer decode stack (one lrmoe_moe_chain launch) against the oracle,
layer by layer, on an MI355X.

Workload: 40 distinct seeded layers (seed 2026: routers, experts, shared
experts and RMSNorm weights all differ per layer), h <- h + MoE_l(RMSNorm_l(h))
with eps 1e-6, T = 1 and T = 16, the first layer's input model.hidden(T,
step=100): the decode stack the benchmark times, 60 GiB of experts resident.

Bar:
  - the chain's output and every layer's routes are bit-identical to 40
    successive moe_layer calls on the same workspace (same arithmetic, same
    order);
  - for every layer l, the oracle's block applied to that layer's input
    (the output of layer l-1, taken from the successive calls) gives the
    same routes bit for bit and an output within helpers.assert_layer_close
    (1e-2 of the row's MoE magnitude plus one bf16 ulp).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import HostExperts, assert_layer_close, oracle_layer_rows, to_u16

pytestmark = pytest.mark.gpu

LAYERS = 40
SEED = 2026


@pytest.fixture(scope="module")
def stack40(device):
    from lightreason_amd.synthetic import SyntheticModel

    model = SyntheticModel(layers=LAYERS, device=device, seed=SEED, shared=True, norm="normal")
    torch.cuda.synchronize()
    yield model
    del model
    torch.cuda.empty_cache()


@pytest.mark.parametrize("tokens", [1, 16])
def test_chain_40_layers_against_oracle(stack40, oracle, tokens):
    from lightreason_amd.moe import Workspace, moe_chain, moe_layer

    layers = stack40.layers
    x = stack40.hidden(tokens, step=100)
    ws = Workspace(x.device, tokens)
    print(f"[stack] T={tokens}: chain of {LAYERS} layers", flush=True)
    idx_c = torch.empty((LAYERS, tokens, 8), dtype=torch.int64, device=x.device)
    w_c = torch.empty((LAYERS, tokens, 8), dtype=torch.bfloat16, device=x.device)
    out_c = moe_chain(x, layers, indices=idx_c, weights=w_c, workspace=ws)
    torch.cuda.synchronize()
    assert ws.status() == 0
    inputs = [x]
    idx_s = torch.empty_like(idx_c)
    w_s = torch.empty_like(w_c)
    for l, layer in enumerate(layers):
        inputs.append(moe_layer(inputs[-1], layer, indices=idx_s[l], weights=w_s[l], workspace=ws))
    torch.cuda.synchronize()
    assert ws.status() == 0
    assert torch.equal(idx_c, idx_s), "chain routes differ from successive layers"
    assert torch.equal(w_c.view(torch.int16), w_s.view(torch.int16)), "chain weights differ"
    assert torch.equal(out_c.view(torch.int16), inputs[-1].view(torch.int16)), "chain output differs"
    idx_c, w_c = idx_c.cpu().numpy(), to_u16(w_c)
    for l, layer in enumerate(layers):
        xb = to_u16(inputs[l])
        want, o_idx, o_w = oracle_layer_rows(oracle, layer, xb, HostExperts(stack40.bank, l))
        np.testing.assert_array_equal(idx_c[l], o_idx, err_msg=f"layer {l} routes")
        np.testing.assert_array_equal(w_c[l], o_w, err_msg=f"layer {l} weights")
        assert_layer_close(to_u16(inputs[l + 1]), want, xb, what=f"T={tokens} layer {l}")
