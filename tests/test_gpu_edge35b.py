"""The reference-shaped module surface (lightreason_amd.edge35b) on an MI355X,
against the oracle on the same seeded inputs.

Same bar as the core parity tests: routing-order and combine arithmetic
bit-exact where the inputs are bf16 values (ordered combine), expert outputs
within helpers.assert_close_bf16 (1e-2 of the max magnitude, and per-row L2),
gathered bytes bit-exact.
"""

from __future__ import annotations

import types

import numpy as np
import pytest
import torch

from helpers import assert_close_bf16, bf16_f32, from_u16, oracle_experts, to_u16, uniform_routes, zipf_routes

pytestmark = pytest.mark.gpu


class _Module:
    num_experts = 256


@pytest.fixture(scope="module")
def layer(model, device):
    """A resident layer object with the attributes the reference's forwards
    read: pool, module.num_experts, gate_up, down, act_fn, decode_step."""
    from lightreason_amd.edge35b.expert_stream import ExpertPool

    pool = ExpertPool(device)
    return types.SimpleNamespace(pool=pool, module=_Module(), gate_up=model.bank.gate_up(0), down=model.bank.down(0),
                                 act_fn=torch.nn.functional.silu, decode_step=0, last_route={},
                                 expert_ptrs=model.bank.expert_ptrs(0))


def _routes(tokens, seed, kind="uniform"):
    return (zipf_routes if kind == "zipf" else uniform_routes)(tokens, seed)


def test_fused_forward_matches_oracle(model, layer, oracle, host_experts):
    from lightreason_amd.edge35b.fused_experts import fused_forward

    idx, wb = _routes(1, 71)
    x = model.hidden(1, step=71)
    with torch.no_grad():
        out = fused_forward(layer, x, torch.from_numpy(idx).to(x.device), from_u16(wb, x.device))
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    assert_close_bf16(to_u16(out), want, what="fused_forward")


def test_fused_forward_rejects_bad_routes(model, layer):
    from lightreason_amd.edge35b.fused_experts import fused_forward

    x = model.hidden(1, step=72)
    w = torch.full((1, 8), 0.125, dtype=torch.bfloat16, device=x.device)
    repeated = torch.tensor([[3, 9, 3, 40, 41, 42, 43, 44]], device=x.device)
    with pytest.raises(ValueError, match="eight distinct valid routes"):
        fused_forward(layer, x, repeated, w)
    outside = torch.tensor([[3, 9, 300, 40, 41, 42, 43, 44]], device=x.device)
    with pytest.raises(ValueError, match="eight distinct valid routes"):
        fused_forward(layer, x, outside, w)
    with pytest.raises(ValueError, match="single-token 35B route shape"):
        fused_forward(layer, x.float(), repeated, w)


def test_fused_forward_batched_ablation(model, layer, oracle, host_experts):
    from lightreason_amd.edge35b.fused_experts import fused_forward

    idx, wb = _routes(1, 73)
    x = model.hidden(1, step=73)
    with torch.no_grad():
        out = fused_forward(layer, x, torch.from_numpy(idx).to(x.device), from_u16(wb, x.device),
                            torch_projections=True)
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    assert_close_bf16(to_u16(out), want, what="fused_forward torch projections")


def test_matvec_shim_protocol(model, device, oracle, host_experts):
    """_matvec[(128, 8)] gate/up (shared x, stride 3) and [(256, 8)] down
    (per-expert x), as launched at fused_experts.py:60,67."""
    from lightreason_amd.edge35b.fused_experts import _matvec

    experts = [5, 17, 64, 99, 130, 201, 222, 255]
    ptrs = model.bank.expert_ptrs(0)
    table = torch.stack([ptrs[experts, 0], ptrs[experts, 1], torch.arange(8, device=device)], 1).contiguous()
    x = model.hidden(1, step=74)
    gate_up = torch.empty((8, 1024), dtype=torch.bfloat16, device=device)
    _matvec[(128, 8)](table, x, gate_up, 2048, 1024, 0, 8, True, num_warps=8)
    act = from_u16(oracle.f32_to_bf16(np.arange(8 * 512, dtype=np.float32).reshape(8, 512) % 7 / 16 - 0.2), device)
    down = torch.empty((8, 2048), dtype=torch.bfloat16, device=device)
    _matvec[(256, 8)](table, act, down, 512, 2048, 1, 8, False, num_warps=4)
    torch.cuda.synchronize()
    xf = bf16_f32(to_u16(x)[0]).astype(np.float64)
    af = bf16_f32(to_u16(act)).astype(np.float64)
    want_gu = np.empty((8, 1024), dtype=np.uint16)
    want_dn = np.empty((8, 2048), dtype=np.uint16)
    for i, e in enumerate(experts):
        gu, dn = host_experts(e)
        want_gu[i] = oracle.f32_to_bf16((bf16_f32(gu).astype(np.float64) @ xf).astype(np.float32))
        want_dn[i] = oracle.f32_to_bf16((bf16_f32(dn).astype(np.float64) @ af[i]).astype(np.float32))
    assert_close_bf16(to_u16(gate_up), want_gu, what="_matvec gate/up")
    assert_close_bf16(to_u16(down), want_dn, what="_matvec down")
    with pytest.raises(ValueError):
        _matvec[(64, 8)](table, x, gate_up, 2048, 1024, 0, 8, True)  # grid covers half the rows


def test_ordered_sum_and_combine_shims_bit_exact(device, oracle):
    """_ordered_sum (stride 3) and packed_hybrid._combine (stride 4, cold
    rows) against the oracle's ordered combine: bit-exact."""
    from lightreason_amd.edge35b.fused_experts import _ordered_sum
    from lightreason_amd.edge35b.packed_hybrid import _combine

    rng = np.random.default_rng(75)
    values = oracle.f32_to_bf16(rng.normal(0, 1, (8, 2048)).astype(np.float32))
    cold = oracle.f32_to_bf16(rng.normal(0, 1, (8, 2048)).astype(np.float32))
    slots = rng.permutation(8)
    wb = oracle.f32_to_bf16(rng.random(8).astype(np.float32))
    table3 = torch.tensor([[0, 0, int(s)] for s in slots], dtype=torch.int64, device=device)
    out = torch.empty((1, 2048), dtype=torch.bfloat16, device=device)
    _ordered_sum[(8,)](table3, from_u16(values, device), from_u16(wb[None], device), out, 2048, 256,
                       enable_fp_fusion=False)
    want = oracle.combine(values, np.arange(8, dtype=np.int32)[None], slots.astype(np.int32), wb[None])
    np.testing.assert_array_equal(to_u16(out), want)
    # stride 4: rows 1 and 6 come from cold rows 4 and 0
    cold_row = [-1, 4, -1, -1, -1, -1, 0, -1]
    table4 = torch.tensor([[0, 0, int(s), c] for s, c in zip(slots, cold_row)], dtype=torch.int64, device=device)
    _combine[(8,)](table4, from_u16(values, device), from_u16(cold, device), from_u16(wb[None], device), out, 2048,
                   256, enable_fp_fusion=False)
    mixed = values.copy()
    mixed[1], mixed[6] = cold[4], cold[0]
    want = oracle.combine(mixed, np.arange(8, dtype=np.int32)[None], slots.astype(np.int32), wb[None])
    np.testing.assert_array_equal(to_u16(out), want)


def test_packed_forward_and_configure_modes(model, layer, oracle, host_experts):
    from lightreason_amd.edge35b import packed_hybrid, packed_native

    idx, wb = _routes(1, 76)
    x = model.hidden(1, step=76)
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    indices, weights = torch.from_numpy(idx).to(x.device), from_u16(wb, x.device)
    with torch.no_grad():
        out = packed_hybrid.packed_forward(layer, x, indices, weights)
        assert_close_bf16(to_u16(out), want, what="packed_forward")
        for mode in ("buffers", "graph", "ada"):
            with packed_native.configure(layer.pool, mode):
                for step in range(3):  # graph modes: capture once, replay with new routes
                    i2, w2 = _routes(1, 760 + step)
                    x2 = model.hidden(1, step=760 + step)
                    got = packed_hybrid.packed_forward(layer, x2, torch.from_numpy(i2).to(x.device),
                                                       from_u16(w2, x.device))
                    torch.cuda.synchronize()
                    assert_close_bf16(to_u16(got), oracle_experts(oracle, to_u16(x2), i2, w2, host_experts),
                                      what=f"configure({mode}) step {step}")
        assert packed_hybrid.packed_forward.__module__ == packed_hybrid.__name__
        outside = torch.tensor([[3, 9, 300, 40, 41, 42, 43, 44]], device=x.device)
        with pytest.raises(ValueError):
            packed_hybrid.packed_forward(layer, x, outside, weights)
    with pytest.raises(ValueError):
        with packed_native.configure(layer.pool, "bogus"):
            pass


def test_packed_ada_gate(model, device, oracle, host_experts):
    from lightreason_amd.edge35b.packed_ada import load_gate

    experts = [1, 2, 30, 31, 100, 180, 181, 250]
    ptrs = model.bank.expert_ptrs(0)
    table = torch.zeros((8, 4), dtype=torch.int64, device=device)
    table[:, 0] = ptrs[experts, 0]
    table[3, 0] = 0  # a cold row: skipped, its active row untouched
    x = model.hidden(1, step=77)
    active = torch.full((8, 512), -5.0, dtype=torch.bfloat16, device=device)
    load_gate()(table, x, active)
    torch.cuda.synchronize()
    got = to_u16(active)
    xf = bf16_f32(to_u16(x)[0]).astype(np.float64)
    for i, e in enumerate(experts):
        if i == 3:
            assert (got[i] == to_u16(torch.tensor([-5.0], dtype=torch.bfloat16))[0]).all()
            continue
        gu, _ = host_experts(e)
        g = oracle.f32_to_bf16((bf16_f32(gu[:512]).astype(np.float64) @ xf).astype(np.float32))
        u = oracle.f32_to_bf16((bf16_f32(gu[512:]).astype(np.float64) @ xf).astype(np.float32))
        gf, uf = bf16_f32(g).astype(np.float64), bf16_f32(u)
        s = oracle.f32_to_bf16((gf / (1 + np.exp(-gf))).astype(np.float32))
        want = oracle.f32_to_bf16((bf16_f32(s) * uf).astype(np.float32))
        assert_close_bf16(got[i][None], want[None], what=f"packed gate row {i}")


@pytest.mark.parametrize("tokens", [2, 8, 16])
def test_grouped_block_and_shims(model, layer, oracle, host_experts, tokens, device):
    from lightreason_amd.edge35b.block_experts import _combine, _project, grouped_block

    idx, wb = _routes(tokens, 80 + tokens, "zipf")
    x = model.hidden(tokens, step=80 + tokens)
    indices, weights = torch.from_numpy(idx).to(device), from_u16(wb, device)
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    with torch.no_grad():
        out = grouped_block(layer, x, indices, weights)
    assert_close_bf16(to_u16(out), want, what=f"grouped_block T={tokens}")
    # the reference's own launch sequence (block_experts.py:102-138) through the shims
    routes = {}
    for t, row in enumerate(idx.tolist()):
        for slot, e in enumerate(row):
            routes.setdefault(e, []).append((t, slot))
    pairs, inputs, inverse = [], [], [[] for _ in range(tokens)]
    ptrs = model.bank.expert_ptrs(0).cpu()
    for e, matches in sorted(routes.items()):
        k = len(inputs)
        pairs += [int(ptrs[e, 0]), int(ptrs[e, 1])]
        inputs.append([t for t, _ in matches] + [-1] * (16 - len(matches)))
        for r, (t, slot) in enumerate(matches):
            inverse[t].append((k, r, slot))
    E = len(inputs)
    pointers = torch.tensor(pairs, dtype=torch.int64, device=device)
    inputs = torch.tensor(inputs, dtype=torch.int32, device=device)
    inverse = torch.tensor(inverse, dtype=torch.int32, device=device)
    gates = torch.empty((E, 16, 1024), dtype=torch.bfloat16, device=device)
    _project[(E, 32)](pointers, inputs, x, gates, 2048, 1024, False, 16, 32, 64)
    active = torch.empty((E, 16, 512), dtype=torch.bfloat16, device=device)
    from lightreason_amd import _native

    _native.call("lrmoe_swiglu_rows", gates.data_ptr(), active.data_ptr(), E * 16,
                 torch.cuda.current_stream().cuda_stream)
    projected = torch.empty((E, 16, 2048), dtype=torch.bfloat16, device=device)
    _project[(E, 64)](pointers, inputs, active, projected, 512, 2048, True, 16, 32, 64)
    result = torch.empty_like(x)
    _combine[(tokens, 8)](inverse, projected, projected, weights, result, 2048, 16, 256, False,
                          enable_fp_fusion=False)
    torch.cuda.synchronize()
    assert_close_bf16(to_u16(result), want, what=f"_project/_combine T={tokens}")


def test_routed_forward_prefill(model, layer, oracle, host_experts, device):
    from lightreason_amd.edge35b.pipeline import routed_forward

    tokens = 40
    idx, wb = _routes(tokens, 90, "zipf")
    x = model.hidden(tokens, step=90)
    with torch.no_grad():
        out = routed_forward(layer, x, torch.from_numpy(idx).to(device), from_u16(wb, device))
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    assert_close_bf16(to_u16(out), want, what="routed_forward T=40")
    with pytest.raises(ValueError):
        routed_forward(layer, x, torch.from_numpy(idx).to(device), from_u16(wb, device), pipeline=object())


@pytest.mark.parametrize("geometry", ["hip-8-256-default", "hip-16-128-l2", "cuda-4-256-default"])
def test_native_gather_copy(model, device, geometry):
    from lightreason_amd.edge35b.native_bf16_gather import NativeBf16Gather, expert_descriptors, select_geometry

    gather = NativeBf16Gather()
    desc = expert_descriptors(model.bank.expert_ptrs(0))
    sel = [7, 8, 100, 255, 0]
    slots = 6
    gate_dst = torch.full((slots, 1024, 2048), -123.0, dtype=torch.bfloat16, device=device)
    down_dst = torch.full((slots, 2048, 512), -123.0, dtype=torch.bfloat16, device=device)
    destinations = torch.tensor([gate_dst.data_ptr(), down_dst.data_ptr()], dtype=torch.int64, device=device)
    sizes = torch.tensor([1024 * 2048 * 2, 2048 * 512 * 2], dtype=torch.int64, device=device)
    src = torch.tensor(sel + [0, 0, 0], dtype=torch.int32, device=device)
    dst = torch.tensor([4, 0, 1, 3, 2, 5, 5, 5], dtype=torch.int32, device=device)
    count = torch.tensor([len(sel)], dtype=torch.int64, device=device)
    gather.copy(desc, destinations, sizes, src, dst, count, max_copies=8, experts=256,
                geometry=select_geometry(geometry))
    torch.cuda.synchronize()
    for row, e in enumerate(sel):
        gu, dn = model.bank.expert(0, e)
        slot = int(dst[row])
        assert torch.equal(gate_dst[slot].view(torch.int16), gu.view(torch.int16))
        assert torch.equal(down_dst[slot].view(torch.int16), dn.view(torch.int16))
    assert bool((gate_dst[5] == -123.0).all()) and bool((down_dst[5] == -123.0).all())
    assert not gather.codec_rows_seen()
    # Expert 100's gate_up as an escape-codec row (bf16_expert_codec.py):
    # decoded into its slot, and flagged.
    from oracle import oracle as O

    bits = model.bank.expert(0, 100)[0].view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    base, escapes = O.escape_window(bits)
    packed = torch.from_numpy(O.escape_pack(bits, base, escapes)).to(device)
    desc[0, 100] = torch.tensor([packed.data_ptr(), base, escapes])
    gate_dst.fill_(-123.0)
    gather.copy(desc, destinations, sizes, src, dst, count, max_copies=8, experts=256,
                geometry=select_geometry(geometry))
    torch.cuda.synchronize()
    assert gather.codec_rows_seen()
    assert torch.equal(gate_dst[1].view(torch.int16), model.bank.expert(0, 100)[0].view(torch.int16))
    # An unknown policy is refused on the host, before any launch.
    with pytest.raises(ValueError):
        gather.copy(desc, destinations, sizes, src, dst, count, max_copies=8, experts=256,
                    geometry=(4, 256, "no-such-policy"))


def _hf_experts(model, device):
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeExperts

    cfg = Qwen3_5MoeTextConfig(num_experts=256, hidden_size=2048, moe_intermediate_size=512, hidden_act="silu",
                               num_experts_per_tok=8)
    with torch.device("meta"):
        module = Qwen3_5MoeExperts(cfg)
    module.gate_up_proj = torch.nn.Parameter(model.bank.gate_up(0), requires_grad=False)
    module.down_proj = torch.nn.Parameter(model.bank.down(0), requires_grad=False)
    holder = torch.nn.Module()
    holder.experts = module
    return holder, module, cfg


def test_patch_experts_on_transformers_module(model, device, oracle, host_experts):
    from lightreason_amd.edge35b.expert_stream import ExpertPool, patch_experts

    holder, module, _ = _hf_experts(model, device)
    pool = ExpertPool(device)
    for tokens, mode in ((1, "fused"), (8, "cached"), (24, "selected")):
        idx, wb = _routes(tokens, 95 + tokens, "zipf")
        x = model.hidden(tokens, step=95 + tokens)
        with torch.no_grad(), patch_experts(holder, mode=mode, pool=pool):
            out = module(x, torch.from_numpy(idx).to(device), from_u16(wb, device))
        assert "forward" not in vars(module)
        want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
        assert_close_bf16(to_u16(out), want, what=f"patch_experts {mode} T={tokens}")
    assert pool.snapshot()["transferred_bytes"] == 0


def test_experts_interface_registration(model, device, oracle, host_experts):
    from lightreason_amd.edge35b.expert_stream import register_experts_implementation

    _, module, cfg = _hf_experts(model, device)
    register_experts_implementation("lrmoe_test")
    cfg._experts_implementation = "lrmoe_test"
    idx, wb = _routes(4, 99)
    x = model.hidden(4, step=99)
    with torch.no_grad():
        out = module(x, torch.from_numpy(idx).to(device), from_u16(wb, device))
    want = oracle_experts(oracle, to_u16(x), idx, wb, host_experts)
    assert_close_bf16(to_u16(out), want, what="ExpertsInterface lrmoe")
