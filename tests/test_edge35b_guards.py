"""Host-side behaviour of the reference-shaped surface (no GPU needed): the
guards, error types and protocol checks that fire before any kernel launch,
mirroring the reference's own argument checks (fused_experts.py:41-50,
block_experts.py:91-95, native_bf16_gather.py:17-22, packed_native.py:153-154,
expert_stream.py:465-466)."""

from __future__ import annotations

import sys
import types

import pytest
import torch

from lightreason_amd.edge35b import _grid, block_experts, expert_stream, fused_experts, native_bf16_gather, \
    packed_native


def _layer(**kw):
    base = dict(pool=None, module=types.SimpleNamespace(num_experts=256),
                gate_up=torch.empty((256, 1024, 2048), dtype=torch.bfloat16, device="meta"),
                down=torch.empty((256, 2048, 512), dtype=torch.bfloat16, device="meta"))
    base.update(kw)
    return types.SimpleNamespace(**base)


def test_fused_forward_guards():
    layer = _layer()
    x = torch.zeros((1, 2048), dtype=torch.bfloat16)
    idx = torch.zeros((1, 8), dtype=torch.int64)
    w = torch.zeros((1, 8), dtype=torch.bfloat16)
    for bad in (dict(hidden=torch.zeros((2, 2048), dtype=torch.bfloat16)),
                dict(hidden=x.float()), dict(indices=torch.zeros((1, 7), dtype=torch.int64)),
                dict(weights=w.float()), dict(hidden=torch.zeros((2048, 2), dtype=torch.bfloat16).t())):
        args = dict(hidden=x, indices=idx, weights=w)
        args.update(bad)
        with pytest.raises(ValueError, match="single-token 35B route shape"):
            fused_experts.fused_forward(layer, args["hidden"], args["indices"], args["weights"])
    with pytest.raises(ValueError, match="single-token"):
        fused_experts.fused_forward(_layer(down=torch.empty((256, 512, 2048), device="meta")), x, idx, w)


def test_grouped_block_guards():
    layer = _layer()
    w = torch.zeros((4, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="2–16"):
        block_experts.grouped_block(layer, torch.zeros((17, 2048), dtype=torch.bfloat16),
                                    torch.zeros((17, 8), dtype=torch.int64), torch.zeros((17, 8)))
    with pytest.raises(ValueError, match="2–16"):
        block_experts.grouped_block(layer, torch.zeros((4, 2048)), torch.zeros((4, 7), dtype=torch.int64), w)
    with pytest.raises(ValueError, match="contiguous"):
        block_experts.grouped_block(layer, torch.zeros((2048, 4)).t(), torch.zeros((4, 8), dtype=torch.int64), w)


def test_grid_protocol():
    calls = []
    k = _grid.GridKernel("k", lambda grid, *args: calls.append((grid, args)))
    k[(4, 8)](1, 2, num_warps=8, enable_fp_fusion=False)
    k[16](3)
    assert calls == [((4, 8, 1), (1, 2)), ((16, 1, 1), (3,))]
    with pytest.raises(TypeError):
        k[(4,)](1, bogus=1)
    with pytest.raises(TypeError):
        k[lambda meta: (1,)]
    with pytest.raises(ValueError):
        k[(0, 1)]
    with pytest.raises(ValueError):
        k[(1, 1, 1, 1)]


def test_shims_check_sizes_before_launch():
    t = torch.zeros(3 * 8, dtype=torch.int64)
    x = torch.zeros(2048, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="cover all N rows"):
        fused_experts._matvec[(64, 8)](t, x, torch.zeros(8 * 1024, dtype=torch.bfloat16), 2048, 1024, 0, 8, True)
    with pytest.raises(ValueError, match="table"):
        fused_experts._matvec[(128, 9)](t, x, torch.zeros(9 * 1024, dtype=torch.bfloat16), 2048, 1024, 0, 8, True)
    with pytest.raises(ValueError, match="device tensor"):
        fused_experts._matvec[(128, 8)](t, x, torch.zeros(8 * 1024, dtype=torch.bfloat16), 2048, 1024, 0, 8, True)
    with pytest.raises(ValueError, match="HIDDEN must be 2048"):
        fused_experts._ordered_sum[(8,)](t, x, x, x, 1024, 256)
    with pytest.raises(ValueError, match="ROWS must be 16"):
        block_experts._project[(4, 32)](t, t, x, x, 2048, 1024, False, 8, 32, 64)


def test_gather_geometries():
    g = native_bf16_gather
    assert g.select_geometry("hip-8-256-l2") == (8, 256, "l2")
    assert g.select_geometry("cuda-8-256-l2") == (8, 256, "l2")  # reference tag
    assert g.select_geometry("hip-4-256-cpu-tiles", shared=True) == (4, 256, "cpu-tiles")
    assert [g.name(x) for x in g.NATIVE_GEOMETRIES][0] == "hip-4-256-default"
    with pytest.raises(ValueError, match="Unknown"):
        g.select_geometry("hip-4-256-cpu-tiles")
    with pytest.raises(ValueError, match="Unknown"):
        g.select_geometry("hip-3-256-default")


def test_mode_validation():
    pool = expert_stream.ExpertPool("cuda:0")
    with pytest.raises(ValueError, match="transfer mode"):
        with expert_stream.patch_experts(torch.nn.Module(), mode="bogus", pool=pool):
            pass
    with pytest.raises(ValueError, match="No experts modules"):
        with expert_stream.patch_experts(torch.nn.Module(), mode="fused", pool=pool):
            pass
    with pytest.raises(ValueError, match="Unknown Packed ablation"):
        with packed_native.configure(pool, "bogus"):
            pass
    with pytest.raises(ValueError, match="GPU device"):
        expert_stream.ExpertPool("cpu")
    with pytest.raises(ValueError, match="capacity_bytes"):
        expert_stream.ExpertPool("cuda:0", capacity_bytes=-1)


def test_layer_adapter_checks_shapes_and_activation():
    pool = expert_stream.ExpertPool("cuda:0")

    def module(experts=256, hidden=2048, inner=512, act=torch.nn.functional.silu):
        m = torch.nn.Module()
        m.num_experts, m.hidden_dim, m.intermediate_dim, m.act_fn = experts, hidden, inner, act
        m.gate_up_proj = torch.nn.Parameter(torch.empty((experts, 2 * inner, hidden), dtype=torch.bfloat16,
                                                        device="meta"), requires_grad=False)
        m.down_proj = torch.nn.Parameter(torch.empty((experts, hidden, inner), dtype=torch.bfloat16, device="meta"),
                                         requires_grad=False)
        return m

    with pytest.raises(ValueError, match="256 experts"):
        expert_stream._Layer("l", module(experts=128), pool, "fused")
    with pytest.raises(ValueError, match="SiLU"):
        expert_stream._Layer("l", module(act=torch.nn.functional.gelu), pool, "fused")


def test_install_as_edge35b():
    import lightreason_amd.edge35b as pkg

    pkg.install_as_edge35b()
    import edge35b.fused_experts as fe  # noqa: F401 -- resolved through the alias

    assert sys.modules["edge35b"] is pkg
    assert fe is fused_experts
    assert sys.modules["edge35b.native_bf16_gather"] is native_bf16_gather


def _forged_workspace(status: int):
    """A workspace whose status word (byte offset WS_STATUS_OFFSET) holds
    ``status``, in host memory: what a decode call leaves behind."""
    from lightreason_amd import _native, moe

    ws = moe.Workspace.__new__(moe.Workspace)
    ws.device = torch.device("cpu")
    ws.max_tokens = 1
    ws.buffer = torch.zeros(64, dtype=torch.uint8)
    ws.buffer[_native.WS_STATUS_OFFSET:_native.WS_STATUS_OFFSET + 4].view(torch.int32)[0] = status
    return ws


def test_status_word_maps_to_errors():
    """The timeout bit (a bounded cross-workgroup wait of the decode kernel
    expired) raises RuntimeError on every checked path; bad routes raise the
    reference's ValueError; a clean word passes."""
    from lightreason_amd import _native, moe

    assert _native.STATUS_TIMEOUT == 8
    assert _forged_workspace(0).check() == 0
    assert _forged_workspace(_native.STATUS_CODEC_ROW).check() == _native.STATUS_CODEC_ROW
    with pytest.raises(RuntimeError, match="timed out"):
        _forged_workspace(_native.STATUS_TIMEOUT).check()
    with pytest.raises(RuntimeError, match="timed out"):   # timeout wins over bad routes
        _forged_workspace(_native.STATUS_TIMEOUT | _native.STATUS_BAD_EXPERT).check()
    for bits in (_native.STATUS_BAD_EXPERT, _native.STATUS_REPEATED_EXPERT):
        with pytest.raises(ValueError, match="expert id"):
            _forged_workspace(bits).check()
    # the edge35b validate=True paths (fused_forward, grouped_block,
    # routed_forward, the patched experts forward) all go through this check
    with pytest.raises(RuntimeError, match="timed out"):
        expert_stream.raise_on_bad_routes(_forged_workspace(_native.STATUS_TIMEOUT), "bad routes")
    with pytest.raises(ValueError, match="^bad routes$"):
        expert_stream.raise_on_bad_routes(_forged_workspace(_native.STATUS_REPEATED_EXPERT), "bad routes")
    expert_stream.raise_on_bad_routes(_forged_workspace(0), "bad routes")
    assert moe.check_status(0) == 0


def test_header_declares_the_timeout_bit():
    from pathlib import Path

    header = (Path(__file__).resolve().parents[1] / "include" / "lrmoe.h").read_text()
    assert "#define LRMOE_STATUS_TIMEOUT 8" in header


def test_reference_driver_imports_mixer_graphs():
    """native_bench.py:143,151 import these names from edge35b.packed_native."""
    import lightreason_amd.edge35b as pkg

    pkg.install_as_edge35b()
    from edge35b.packed_native import configure, mixer_graphs  # noqa: F401 -- the reference's import line

    assert mixer_graphs is packed_native.mixer_graphs


def _fake_model(native: bool):
    """A model shell with two linear-attention layers (indices 0 and 2) and
    one attention layer, whose mixer forwards echo their input; marked as
    already native (an enclosing fused_delta) when ``native``."""
    calls = []

    def make_forward(index):
        def forward(hidden_states, cache_params=None, attention_mask=None, **kwargs):
            calls.append(index)
            return hidden_states
        forward.lrmoe_native = native
        return forward

    layers = []
    for index in range(3):
        layer = types.SimpleNamespace()
        if index != 1:
            mixer = types.SimpleNamespace()
            mixer.forward = make_forward(index)
            layer.linear_attn = mixer
        layers.append(layer)
    return types.SimpleNamespace(model=types.SimpleNamespace(layers=layers)), calls


class _Cache:
    def has_previous_state(self, index):
        return True


def test_mixer_graphs_records_single_token_steps_and_restores():
    """Inside mixer_graphs (with the mixers already native) a single-token
    cached step of layer i is noted in pool.mixer_graphs[i]; longer blocks
    and uncached calls are not; the forwards are restored on exit."""
    model, calls = _fake_model(native=True)
    originals = [l.linear_attn.forward for l in model.model.layers if hasattr(l, "linear_attn")]
    pool = types.SimpleNamespace()
    x1 = torch.zeros((1, 1, 8))
    with packed_native.mixer_graphs(model, pool):
        assert pool.mixer_graphs == {}
        mixer0 = model.model.layers[0].linear_attn
        mixer2 = model.model.layers[2].linear_attn
        assert mixer0.forward(x1, cache_params=_Cache()) is x1
        mixer2.forward(torch.zeros((1, 4, 8)), cache_params=_Cache())   # a verify block
        mixer2.forward(x1)                                              # no cache
        assert pool.mixer_graphs == {0: "native"}
        mixer2.forward(x1, cache_params=_Cache())
    assert pool.mixer_graphs == {0: "native", 2: "native"}
    assert calls == [0, 2, 2, 2]
    assert [l.linear_attn.forward for l in model.model.layers if hasattr(l, "linear_attn")] == originals


def test_mixer_status_timeout_raises_and_clears(monkeypatch):
    """A mixer workspace whose sticky timeout bit is set (a bounded wait of a
    step expired) makes check_mixer_status, PrefixStates.commit and the end
    of fused_delta's block raise RuntimeError; the bit is cleared by the
    raise, so the next check passes."""
    from lightreason_amd import _native, delta

    cpu = torch.device("cpu")
    ws = torch.zeros(64, dtype=torch.uint8)
    off = _native.DELTA_WS_STATUS_OFFSET
    monkeypatch.setitem(delta._WORKSPACES, (cpu, 0), ws)

    def set_timeout():
        ws[off:off + 4].view(torch.int32)[0] = _native.STATUS_TIMEOUT

    assert delta.check_mixer_status(cpu) == 0
    set_timeout()
    with pytest.raises(RuntimeError, match="timed out"):
        delta.check_mixer_status(cpu)
    assert delta.check_mixer_status(cpu) == 0
    histories = delta.PrefixStates()
    histories.devices.add(cpu)
    set_timeout()
    with pytest.raises(RuntimeError, match="timed out"):
        histories.commit(None, 10, 4, 4)          # even a fully accepted block is checked
    histories.commit(None, 10, 4, 4)

    shell = types.SimpleNamespace(model=types.SimpleNamespace(layers=[types.SimpleNamespace()]))
    set_timeout()
    with pytest.raises(RuntimeError, match="timed out"):
        with delta.fused_delta(shell) as h:
            h.devices.add(cpu)
    assert delta.check_mixer_status(cpu) == 0
