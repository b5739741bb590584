"""HIP path vs the oracle on the same seeded inputs (needs an MI355X).

Bar: routing indices, routing weights, logits, shared-gate values, RMSNorm
outputs, bucketing plans, generator output and gathered bytes bit-exact;
expert outputs within 1e-2 of the row's max magnitude (bf16 storage, fp32
accumulation; see helpers.assert_close_bf16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import (HostExperts, assert_close_bf16, from_u16, oracle_experts, to_u16, uniform_routes,
                     zipf_routes)

pytestmark = pytest.mark.gpu

SEED = 4242


def test_generator_matches_host(device, oracle):
    from lightreason_amd.moe import fill_normal_

    for count, stream, sigma, first in ((1, 3, 1.0, 0), (1000, 7, 0.02, 0), (65537, 8, 2.5, 123456789)):
        t = fill_normal_(torch.empty(count, dtype=torch.bfloat16, device=device), 99, stream, sigma, first)
        np.testing.assert_array_equal(to_u16(t), oracle.normal_bf16((count,), 99, stream, sigma, first))


def test_bank_generator_matches_host(model, oracle):
    from lightreason_amd.moe import EXPERT_ELEMENTS
    from lightreason_amd.synthetic import STREAM_BANK

    for e in (0, 77, 255):
        got = to_u16(model.bank.bank[0, e])
        want = oracle.normal_bf16((EXPERT_ELEMENTS,), SEED, STREAM_BANK, 0.02, first=e * EXPERT_ELEMENTS)
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("tokens", [1, 3, 8, 16, 40, 300])
@pytest.mark.parametrize("norm", [False, True])
def test_route_topk_bit_exact(model, oracle, tokens, norm):
    from lightreason_amd.moe import Workspace, route_topk

    layer = model.layers[0]
    x = model.hidden(tokens, step=tokens)
    ws = Workspace(x.device, tokens)
    indices, weights, logits, sg, normed = route_topk(
        x, layer.router, norm_weight=layer.norm_weight if norm else None, eps=layer.eps,
        shared_expert_gate=layer.shared_expert_gate, workspace=ws)
    torch.cuda.synchronize()
    xb = to_u16(x)
    if norm:
        nb = oracle.rmsnorm(xb, to_u16(layer.norm_weight), layer.eps)
        np.testing.assert_array_equal(to_u16(normed), nb)
        xb = nb
    o_logits, o_idx, o_w = oracle.route(xb, to_u16(layer.router))
    np.testing.assert_array_equal(to_u16(logits), o_logits)
    np.testing.assert_array_equal(indices.cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(weights), o_w)
    np.testing.assert_array_equal(to_u16(sg), oracle.shared_gate(xb, to_u16(layer.shared_expert_gate)))
    assert ws.status() == 0


@pytest.mark.parametrize("tokens", [1, 8, 16, 64, 65, 500])
def test_bucket_bit_exact(device, oracle, tokens):
    from lightreason_amd.moe import Workspace, bucket

    idx, _ = (zipf_routes if tokens % 2 == 0 else uniform_routes)(tokens, tokens)
    plan = bucket(torch.from_numpy(idx).to(device), Workspace(device, tokens))
    torch.cuda.synchronize()
    ref = oracle.bucket(idx)
    unique = int(plan["unique"].item())
    assert int(plan["status"].item()) == 0
    assert unique == ref["unique"]
    np.testing.assert_array_equal(plan["expert"][:unique].cpu().numpy(), ref["expert"])
    np.testing.assert_array_equal(plan["offset"][:unique + 1].cpu().numpy(), ref["offset"])
    np.testing.assert_array_equal(plan["pair_token"].cpu().numpy(), ref["pair_token"])
    np.testing.assert_array_equal(plan["pair_slot"].cpu().numpy(), ref["pair_slot"])
    np.testing.assert_array_equal(plan["route_pair"].cpu().numpy(), ref["route_pair"])


@pytest.mark.parametrize("tokens", [1, 100])
def test_bucket_flags_bad_routes(device, tokens):
    from lightreason_amd.moe import Workspace, bucket

    idx, _ = uniform_routes(tokens, 5)
    idx[-1, 3] = 300
    plan = bucket(torch.from_numpy(idx).to(device), Workspace(device, tokens))
    assert int(plan["status"].item()) & 1
    idx, _ = uniform_routes(tokens, 6)
    idx[0, 7] = idx[0, 2]
    plan = bucket(torch.from_numpy(idx).to(device), Workspace(device, tokens))
    assert int(plan["status"].item()) & 2


@pytest.mark.parametrize("tokens,routes", [(1, "uniform"), (4, "uniform"), (8, "zipf"), (16, "zipf"), (33, "zipf")])
def test_moe_experts_parity(model, oracle, host_experts, tokens, routes):
    from lightreason_amd.moe import Workspace, moe_experts

    idx, wb = (zipf_routes if routes == "zipf" else uniform_routes)(tokens, 1000 + tokens)
    x = model.hidden(tokens, step=500 + tokens)
    ws = Workspace(x.device, tokens)
    out = moe_experts(x, torch.from_numpy(idx).to(x.device), from_u16(wb, x.device), model.bank.expert_ptrs(0),
                      workspace=ws)
    torch.cuda.synchronize()
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    stats = assert_close_bf16(to_u16(out), want, what=f"experts T={tokens}")
    assert stats["exact_fraction"] > 0.5


@pytest.mark.parametrize("tokens", [1, 8, 16, 24])
@pytest.mark.parametrize("norm", [False, True])
def test_moe_layer_parity(model, oracle, host_experts, tokens, norm):
    from lightreason_amd.moe import LayerWeights, Workspace, moe_layer

    base = model.layers[0]
    layer = LayerWeights(**{**base.__dict__, "norm_weight": base.norm_weight if norm else None})
    x = model.hidden(tokens, step=900 + tokens)
    ws = Workspace(x.device, tokens)
    idx_out = torch.empty((tokens, 8), dtype=torch.int64, device=x.device)
    w_out = torch.empty((tokens, 8), dtype=torch.bfloat16, device=x.device)
    out = moe_layer(x, layer, indices=idx_out, weights=w_out, workspace=ws)
    torch.cuda.synchronize()
    xb = to_u16(x)
    xin = oracle.rmsnorm(xb, to_u16(layer.norm_weight), layer.eps) if norm else xb
    _, o_idx, o_w = oracle.route(xin, to_u16(layer.router))
    np.testing.assert_array_equal(idx_out.cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(w_out), o_w)
    shared = (to_u16(layer.shared_gate_proj), to_u16(layer.shared_up_proj), to_u16(layer.shared_down_proj))
    sg = oracle.shared_gate(xin, to_u16(layer.shared_expert_gate))
    want = oracle_experts(oracle, xin, o_idx, o_w, host_experts, shared, sg, xb if norm else None)
    if norm:
        # out = bf16(h + moe): allow 1e-2 of the row's MoE magnitude plus one
        # bf16 ulp of the output for the final residual rounding.
        from helpers import bf16_f32

        got, exp_, h = bf16_f32(to_u16(out)), bf16_f32(want), bf16_f32(xb)
        moe_scale = np.abs(exp_ - h).max(axis=1, keepdims=True)
        assert np.all(np.abs(got - exp_) <= 1e-2 * moe_scale + 2.0 ** -7 * np.abs(exp_))
    else:
        assert_close_bf16(to_u16(out), want, what=f"layer T={tokens}")


def test_gather_raw_rows_graph_replay(device):
    """Mirror of the reference's resident-gather fixture
    (edge35b/test_gpu_resident_experts.py:12-57) for raw rows: sentinel -123
    slots stay untouched, count in {2, 0, 1} under graph replay with swapped
    descriptors."""
    from lightreason_amd.moe import gather

    gen = torch.Generator().manual_seed(7091)
    words = torch.randint(-32768, 32767, (2, 32, 256), generator=gen, dtype=torch.int32).to(torch.int16)
    rows = words.to(device)
    output = torch.full((4, 32, 256), -123, device=device, dtype=torch.int16)
    descriptors = torch.tensor([[[rows[0].data_ptr(), -1, 0], [rows[1].data_ptr(), -1, 0]]], device=device,
                               dtype=torch.int64)
    destinations = torch.tensor([output.data_ptr()], device=device, dtype=torch.int64)
    sizes = torch.tensor([32 * 256 * 2], device=device, dtype=torch.int64)
    ids = torch.tensor([0, 1], device=device, dtype=torch.int32)
    slots = torch.tensor([1, 3], device=device, dtype=torch.int32)
    count = torch.tensor([2], device=device, dtype=torch.int64)

    def copy():
        gather(descriptors, destinations, sizes, ids, slots, count, max_copies=2, experts=2, stripes=4)

    copy()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        copy()
    references = [words[0], words[1]]
    for n in (2, 0, 1):
        descriptors.copy_(descriptors.flip(1))
        references.reverse()
        output.fill_(-123)
        count.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        expected = torch.full((4, 32, 256), -123, dtype=torch.int16)
        for slot, ref in zip((1, 3)[:n], references[:n]):
            expected[slot] = ref
        assert torch.equal(output.cpu(), expected)


def test_gather_expert_rows_bit_exact(model, device):
    """C1 shape: gather experts of the packed bank into contiguous staging."""
    from lightreason_amd.moe import EXPERT_ELEMENTS, GATE_UP_ELEMENTS, gather

    bank = model.bank
    sel = [255, 3, 77, 128, 0, 19]
    staging_gu = torch.full((len(sel), 1024, 2048), 0x5A5A, dtype=torch.int16, device=device)
    staging_dn = torch.full((len(sel) + 1, 2048, 512), 0x5A5A, dtype=torch.int16, device=device)
    ptrs = bank.expert_ptrs(0).cpu()
    desc = torch.stack([torch.stack([ptrs[:, 0], torch.full((256,), -1), torch.zeros(256, dtype=torch.int64)], 1),
                        torch.stack([ptrs[:, 1], torch.full((256,), -1), torch.zeros(256, dtype=torch.int64)], 1)])
    desc = desc.to(device)
    destinations = torch.tensor([staging_gu.data_ptr(), staging_dn.data_ptr()], device=device)
    sizes = torch.tensor([GATE_UP_ELEMENTS * 2, (EXPERT_ELEMENTS - GATE_UP_ELEMENTS) * 2], device=device)
    src = torch.tensor(sel + [-1] * 2, dtype=torch.int32, device=device)
    dst = torch.tensor(list(range(len(sel))) + [-1] * 2, dtype=torch.int32, device=device)
    count = torch.tensor([len(sel)], device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    gather(desc, destinations, sizes, src, dst, count, max_copies=8, experts=256, stripes=64, status=status)
    torch.cuda.synchronize()
    for i, e in enumerate(sel):
        gu, dn = bank.expert(0, e)
        assert torch.equal(staging_gu[i], gu.view(torch.int16))
        assert torch.equal(staging_dn[i], dn.view(torch.int16))
    assert torch.all(staging_dn[len(sel)] == 0x5A5A)
    assert int(status.item()) == 0


def _check_layer(oracle, host_experts, layer, x, idx_out, w_out, out, what):
    xb = to_u16(x)
    _, o_idx, o_w = oracle.route(xb, to_u16(layer.router))
    np.testing.assert_array_equal(idx_out.cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(w_out), o_w)
    shared = (to_u16(layer.shared_gate_proj), to_u16(layer.shared_up_proj), to_u16(layer.shared_down_proj))
    sg = oracle.shared_gate(xb, to_u16(layer.shared_expert_gate))
    want = oracle_experts(oracle, xb, o_idx, o_w, host_experts, shared, sg)
    assert_close_bf16(to_u16(out), want, what=what)


def test_decode_layer_reuses_workspace_and_replays(model, oracle, host_experts):
    """The T <= 16 layer runs as one kernel whose cross-workgroup counters
    live in the workspace and return to zero after every call: consecutive
    calls of different sizes on one workspace, then replays of a captured
    graph with new inputs between replays, all match the oracle and leave the
    status word clear."""
    from lightreason_amd.moe import LayerWeights, Workspace, moe_layer

    layer = LayerWeights(**{**model.layers[0].__dict__, "norm_weight": None})
    device = model.device
    ws = Workspace(device, 16)
    for i, tokens in enumerate((8, 1, 16, 3, 8)):
        x = model.hidden(tokens, step=1300 + i)
        idx_out = torch.empty((tokens, 8), dtype=torch.int64, device=device)
        w_out = torch.empty((tokens, 8), dtype=torch.bfloat16, device=device)
        out = moe_layer(x, layer, indices=idx_out, weights=w_out, workspace=ws)
        torch.cuda.synchronize()
        _check_layer(oracle, host_experts, layer, x, idx_out, w_out, out, f"call {i} T={tokens}")
        assert ws.status() == 0

    tokens = 8
    x = model.hidden(tokens, step=1400)
    idx_out = torch.empty((tokens, 8), dtype=torch.int64, device=device)
    w_out = torch.empty((tokens, 8), dtype=torch.bfloat16, device=device)
    out = torch.empty_like(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe_layer(x, layer, out=out, indices=idx_out, weights=w_out, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        moe_layer(x, layer, out=out, indices=idx_out, weights=w_out, workspace=ws)
    for r in range(3):
        x.copy_(model.hidden(tokens, step=1500 + r))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check_layer(oracle, host_experts, layer, x, idx_out, w_out, out, f"replay {r}")
        assert ws.status() == 0


@pytest.mark.parametrize("tokens", [1, 8, 16])
@pytest.mark.parametrize("norm", [False, True])
def test_moe_layer_caller_logits_parity(model, oracle, host_experts, tokens, norm):
    """The headline step's routing: the decode kernel's top-8 on caller logits
    (Zipf(1.1) Gumbel logits rounded to bf16, as the T=8 verify workload
    draws them) against the oracle's top-8 of the same logits.  Indices and
    weights bit-exact; outputs within the layer bar."""
    from helpers import assert_layer_close, oracle_layer_rows
    from lightreason_amd.moe import LayerWeights, Workspace, moe_layer

    base = model.layers[0]
    layer = LayerWeights(**{**base.__dict__, "norm_weight": base.norm_weight if norm else None})
    rng = np.random.default_rng(8100 + tokens)
    ranks = rng.permutation(256) + 1
    raw = (-1.1 * np.log(ranks)[None, :] + rng.gumbel(size=(tokens, 256))).astype(np.float32)
    lg_bits = oracle.f32_to_bf16(raw)
    x = model.hidden(tokens, step=8100 + tokens)
    lg = from_u16(lg_bits, x.device)
    ws = Workspace(x.device, tokens)
    idx_out = torch.empty((tokens, 8), dtype=torch.int64, device=x.device)
    w_out = torch.empty((tokens, 8), dtype=torch.bfloat16, device=x.device)
    out = moe_layer(x, layer, indices=idx_out, weights=w_out, logits_in=lg, workspace=ws)
    torch.cuda.synchronize()
    assert ws.status() == 0
    xb = to_u16(x)
    want, o_idx, o_w = oracle_layer_rows(oracle, layer, xb, host_experts, logits_bits=lg_bits)
    np.testing.assert_array_equal(idx_out.cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(w_out), o_w)
    assert_layer_close(to_u16(out), want, xb if norm else None, what=f"caller logits T={tokens} norm={norm}")


def test_gather_t16_selection_bit_exact(model, device):
    """C1 at T=16: the unique experts of 16 tokens x 8 distinct uniform
    experts (about 102 copies, max_copies 128) gathered into staging; every
    copied byte equals its source, unused staging rows keep the sentinel."""
    from lightreason_amd.moe import EXPERT_BYTES, EXPERT_ELEMENTS, gather

    rng = np.random.default_rng(16)
    sel = sorted(set(np.concatenate([rng.choice(256, 8, replace=False) for _ in range(16)]).tolist()))
    assert 90 <= len(sel) <= 115, len(sel)
    bank = model.bank
    staging = torch.full((128, EXPERT_ELEMENTS), 0x5A5A, dtype=torch.int16, device=device)
    ptrs = bank.expert_ptrs(0).cpu()
    desc = torch.stack([ptrs[:, 0], torch.full((256,), -1), torch.zeros(256, dtype=torch.int64)], 1)[None]
    desc = desc.contiguous().to(device)
    order = rng.permutation(len(sel))             # staging slot of each copy, not in expert order
    src = torch.tensor(sel + [0] * (128 - len(sel)), dtype=torch.int32, device=device)
    dst = torch.tensor(order.tolist() + [0] * (128 - len(sel)), dtype=torch.int32, device=device)
    count = torch.tensor([len(sel)], device=device)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    gather(desc, torch.tensor([staging.data_ptr()], device=device), torch.tensor([EXPERT_BYTES], device=device),
           src, dst, count, max_copies=128, experts=256, stripes=48, status=status)
    torch.cuda.synchronize()
    for i, e in enumerate(sel):
        assert torch.equal(staging[int(order[i])], bank.bank[0, e].view(torch.int16)), (i, e)
    assert bool((staging[len(sel):] == 0x5A5A).all())
    assert int(status.item()) == 0
