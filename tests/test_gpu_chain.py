"""Decode layers chained in one persistent launch (lrmoe_moe_chain) vs the
same layers called one at a time (lrmoe_moe_layer, itself checked against
the oracle in test_gpu_parity.py), on an MI355X.

Bar: the chain's output and every layer's routing indices and weights are
bit-identical to the successive single-layer calls, since each layer runs
the same arithmetic in the same order; the first layer's routes also match
the oracle bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import to_u16

pytestmark = pytest.mark.gpu

SEED = 5151


@pytest.fixture(scope="module")
def stack(device):
    """Three distinct synthetic layers (routers, experts, shared experts and
    RMSNorm weights all differ per layer)."""
    from lightreason_amd.synthetic import SyntheticModel

    return SyntheticModel(layers=3, device=device, seed=SEED, shared=True, norm="normal")


def _layers(stack, norm: bool, count: int):
    from lightreason_amd.moe import LayerWeights

    out = []
    for l in range(count):
        base = stack.layers[l % len(stack.layers)]
        out.append(LayerWeights(**{**base.__dict__, "norm_weight": base.norm_weight if norm else None}))
    return out


def _successive(x, layers, ws):
    """The chain's meaning: one moe_layer call per layer."""
    from lightreason_amd.moe import moe_layer

    tokens = x.shape[0]
    idx = torch.empty((len(layers), tokens, 8), dtype=torch.int64, device=x.device)
    wts = torch.empty((len(layers), tokens, 8), dtype=torch.bfloat16, device=x.device)
    h = x
    for l, layer in enumerate(layers):
        h = moe_layer(h, layer, indices=idx[l], weights=wts[l], workspace=ws)
    return h, idx, wts


def _chain(x, layers, ws):
    from lightreason_amd.moe import moe_chain

    tokens = x.shape[0]
    idx = torch.empty((len(layers), tokens, 8), dtype=torch.int64, device=x.device)
    wts = torch.empty((len(layers), tokens, 8), dtype=torch.bfloat16, device=x.device)
    out = moe_chain(x, layers, indices=idx, weights=wts, workspace=ws)
    return out, idx, wts


def _assert_same(got, want, what):
    out_g, idx_g, w_g = got
    out_w, idx_w, w_w = want
    assert torch.equal(idx_g, idx_w), f"{what}: routes differ"
    assert torch.equal(w_g.view(torch.int16), w_w.view(torch.int16)), f"{what}: routing weights differ"
    diff = (out_g.view(torch.int16) != out_w.view(torch.int16)).sum().item()
    assert diff == 0, f"{what}: {diff} output values differ"


@pytest.mark.parametrize("tokens", [1, 8, 16])
@pytest.mark.parametrize("count,norm", [(1, True), (3, True), (3, False)])
def test_chain_equals_successive_layers(stack, oracle, tokens, count, norm):
    from lightreason_amd.moe import Workspace

    layers = _layers(stack, norm, count)
    x = stack.hidden(tokens, step=100 + tokens)
    ws = Workspace(x.device, tokens)
    print(f"chain T={tokens} layers={count} norm={norm}", flush=True)
    want = _successive(x, layers, ws)
    got = _chain(x, layers, ws)
    torch.cuda.synchronize()
    _assert_same(got, want, f"T={tokens} L={count}")
    assert ws.status() == 0
    # The first layer's routes against the oracle.
    xb = to_u16(x)
    xin = oracle.rmsnorm(xb, to_u16(layers[0].norm_weight), layers[0].eps) if norm else xb
    _, o_idx, o_w = oracle.route(xin, to_u16(layers[0].router))
    np.testing.assert_array_equal(got[1][0].cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(got[2][0]), o_w)
    # Later layers see different inputs: their routes differ from layer 0's.
    if count > 1:
        assert not torch.equal(got[1][0], got[1][1])


def test_chain_interleaved_with_single_layers_and_longer_than_one_launch(stack):
    """Chains and single-layer calls share one workspace's call numbering;
    a stack longer than one launch's 48 layers is split into several."""
    from lightreason_amd.moe import Workspace, moe_chain, moe_layer

    ws = Workspace(stack.device, 16)
    layers = _layers(stack, True, 3)
    for i, tokens in enumerate((8, 1, 16, 3)):
        x = stack.hidden(tokens, step=200 + i)
        print(f"interleaved call {i} T={tokens}", flush=True)
        single = moe_layer(x, layers[i % 3], workspace=ws)
        want = _successive(x, layers[: 1 + i % 3], ws)
        got = _chain(x, layers[: 1 + i % 3], ws)
        again = moe_layer(x, layers[i % 3], workspace=ws)
        torch.cuda.synchronize()
        _assert_same(got, want, f"call {i}")
        assert torch.equal(single.view(torch.int16), again.view(torch.int16))
        assert ws.status() == 0
    tokens = 4
    long_stack = _layers(stack, True, 50)
    x = stack.hidden(tokens, step=300)
    print("50-layer stack", flush=True)
    want = _successive(x, long_stack, ws)
    got = _chain(x, long_stack, ws)
    out = moe_chain(x, long_stack, workspace=ws)
    torch.cuda.synchronize()
    _assert_same(got, want, "50 layers")
    assert torch.equal(out.view(torch.int16), got[0].view(torch.int16))
    assert ws.status() == 0


def test_chain_graph_replays(stack):
    """A captured chain replayed with new inputs between replays matches the
    eager chain every time."""
    from lightreason_amd.moe import Workspace, moe_chain

    tokens = 8
    layers = _layers(stack, True, 3)
    ws = Workspace(stack.device, tokens)
    x = stack.hidden(tokens, step=400)
    out = torch.empty_like(x)
    idx = torch.empty((3, tokens, 8), dtype=torch.int64, device=x.device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe_chain(x, layers, out=out, indices=idx, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        moe_chain(x, layers, out=out, indices=idx, workspace=ws)
    for r in range(3):
        x.copy_(stack.hidden(tokens, step=500 + r))
        torch.cuda.synchronize()
        print(f"graph replay {r}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        want_out = moe_chain(x.clone(), layers, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want_out.view(torch.int16)), f"replay {r}"
        assert ws.status() == 0
