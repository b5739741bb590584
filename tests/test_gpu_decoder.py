"""The whole decoder step (lightreason_amd.decoder: input RMSNorm, Gated
DeltaNet mixer or full attention, residual add, MoE block, for every layer)
captured per verify width as one HIP graph (VerifyPass), against the oracle
composition on an MI355X.

Workload: a 4-layer stack in the 35B pattern (layers 0-2 Gated DeltaNet,
layer 3 full attention; seeded weights, fp32 recurrent states, 300 cached
positions in caches of 364), widths 1, 5 and 16, each replayed twice with a
new block, then at two longer cache lengths from the same graphs (the
attention reads the length from a device word).

Bar, per replay and layer l, the oracle given the layer's own device input:
  - the normed rows equal oracle.rmsnorm bit for bit;
  - the mixer output within helpers.assert_close_bf16 (1e-2) of
    oracle.delta_mixer on the states the replay started from, its conv state
    within one bf16 unit (99% bit-identical) and its recurrent state within
    1e-2; the attention output within 1e-2 of oracle.attn_decode and the
    appended key/value rows 98% bit-identical to its rows, every element
    within two bf16 units or one unit of its row's largest (_rows_close);
  - the post-mixer residual equals bf16(h + mixer output) bit for bit;
  - the MoE block's routes equal the oracle's bit for bit and its output is
    within helpers.assert_layer_close;
and the replay's output, routes and final states equal an eager
DecoderStack.step from the same states bit for bit (the graphs' attention
chunks are sized for the capacity and the eager step's for the length: the
chunk size is the same here, and the graphs' extra chunks are empty, which
adds exact zeros to the merge)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import HostExperts, assert_close_bf16, assert_layer_close, bf16_f32, oracle_layer_rows, to_u16

pytestmark = pytest.mark.gpu

LAYERS = 4
CONTEXT = 300
CAPACITY = CONTEXT + 64
WIDTHS = (1, 5, 16)
MIXER_FIELDS = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "conv1d", "A_log", "dt_bias", "norm", "out_proj")
ATTN_FIELDS = ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")


@pytest.fixture(scope="module")
def decoder(device):
    from lightreason_amd.decoder import VerifyPass
    from lightreason_amd.synthetic import SyntheticDecoder

    model = SyntheticDecoder(LAYERS, device, seed=4321, context=CONTEXT, capacity=CAPACITY)
    vp = VerifyPass(model.stack, WIDTHS, CONTEXT, trace=True)
    torch.cuda.synchronize()
    host = [HostExperts(model.moe.bank, l) for l in range(LAYERS)]
    weights = []
    for layer in model.layers:
        if layer.mixer is not None:
            weights.append({f: to_u16(getattr(layer.mixer, f)) for f in MIXER_FIELDS})
        else:
            weights.append({f: to_u16(getattr(layer.attention, f)) for f in ATTN_FIELDS})
    yield model, vp, host, weights
    del vp, model
    torch.cuda.empty_cache()


def _snapshot(model):
    snap = []
    for layer in model.layers:
        if layer.mixer is not None:
            snap.append((layer.conv_state.clone(), layer.state.clone()))
        else:
            snap.append((layer.k_cache.clone(), layer.v_cache.clone()))
    return snap


def _restore(model, snap):
    for layer, (a, b) in zip(model.layers, snap):
        if layer.mixer is not None:
            layer.conv_state.copy_(a)
            layer.state.copy_(b)
        else:
            layer.k_cache.copy_(a)
            layer.v_cache.copy_(b)


def _rows_close(got, want, what):
    """Appended key/value rows: at least 98% bit-identical, every element
    within two bf16 units of its value or one bf16 unit (2^-8) of its row's
    largest.  A key passes through the projection, the per-head RMSNorm and
    the rotation, each rounded to bf16, so one projection ulp can become two;
    a rotated element near zero is the rounded sum of two terms as large as
    the row's elements, whose own rounding sets its error."""
    g, w = bf16_f32(got).astype(np.float64), bf16_f32(want).astype(np.float64)
    same = float((got == want).mean())
    bound = np.maximum(2.0 ** -6 * np.abs(w), 2.0 ** -8 * np.abs(w).max(axis=-1, keepdims=True))
    excess = float(np.max(np.abs(g - w) / bound))
    print(f"{what}: identical {same:.4f}, worst {excess:.2f} of the bound", flush=True)
    assert same >= 0.98 and excess <= 1.0, what


@pytest.mark.parametrize("width", WIDTHS)
def test_verify_pass_against_oracle(decoder, oracle, device, width):
    from lightreason_amd.delta import mixer_status

    model, vp, host, weights = decoder
    eps = model.layers[0].eps
    for rep in range(2):
        what = f"decoder width {width} replay {rep}"
        print(f"[case] {what}", flush=True)
        x = model.hidden(width, step=7000 + 10 * width + rep)
        cos, sin = model.rope(width, CONTEXT)
        before = _snapshot(model)
        out = vp.verify(x, cos, sin).clone()           # checks both status words
        buf = vp.buffers(width)
        after = _snapshot(model)
        torch.cuda.synchronize()
        assert mixer_status(device) == 0
        # the eager step from the same states: the same kernels, the same bits
        _restore(model, before)
        eager = model.stack.step(x, CONTEXT, cos, sin)
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), out.view(torch.int16)), f"{what}: graph != eager"
        for (a, b), (c, d) in zip(_snapshot(model), after):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                               c.view(torch.int16) if c.dtype == torch.bfloat16 else c)
            assert torch.equal(b.view(torch.int16) if b.dtype == torch.bfloat16 else b,
                               d.view(torch.int16) if d.dtype == torch.bfloat16 else d)
        _restore(model, after)
        cos_b, sin_b = to_u16(cos), to_u16(sin)
        h_in = to_u16(x)
        for l, layer in enumerate(model.layers):
            lw = f"{what} layer {l}"
            n = to_u16(buf.n[l])
            np.testing.assert_array_equal(n, oracle.rmsnorm(h_in, to_u16(layer.input_norm), eps), err_msg=lw)
            mix = to_u16(buf.mix[l])
            if layer.mixer is not None:
                conv0, state0 = before[l]
                want, want_conv, want_state, _ = oracle.delta_mixer(n, weights[l], to_u16(conv0),
                                                                    state0.cpu().numpy())
                assert_close_bf16(mix, want, what=lw + " mixer")
                conv1, state1 = after[l]
                got_conv, wconv = to_u16(conv1), want_conv
                g, w = bf16_f32(got_conv).astype(np.float64), bf16_f32(wconv).astype(np.float64)
                bound = np.maximum(2.0 ** -7 * np.maximum(np.abs(g), np.abs(w)), 1e-5 * np.abs(w).max())
                assert float((np.abs(g - w) - bound).max()) <= 0, lw + " conv state"
                assert float((got_conv == wconv).mean()) >= 0.99, lw + " conv state"
                s_got = state1.cpu().numpy().astype(np.float64)
                s_err = np.abs(s_got - want_state).max() / max(np.abs(want_state).max(), 1e-30)
                print(f"{lw}: state max rel {s_err:.2e}", flush=True)
                assert s_err <= 1e-2, lw + " recurrent state"
            else:
                kc0, vc0 = before[l]
                want, want_k, want_v = oracle.attn_decode(n, weights[l], cos_b, sin_b, to_u16(kc0), to_u16(vc0),
                                                          CONTEXT, eps=eps)
                assert_close_bf16(mix, want, what=lw + " attention")
                kc1, vc1 = after[l]
                new = slice(CONTEXT, CONTEXT + width)
                _rows_close(to_u16(kc1)[:, new], want_k[:, new], lw + " appended keys")
                _rows_close(to_u16(vc1)[:, new], want_v[:, new], lw + " appended values")
            h2 = to_u16(buf.h2[l])
            np.testing.assert_array_equal(h2, oracle.f32_to_bf16(bf16_f32(h_in) + bf16_f32(mix)), err_msg=lw)
            ref, o_idx, o_w = oracle_layer_rows(oracle, layer.moe, h2, host[l])
            np.testing.assert_array_equal(buf.indices[l].cpu().numpy(), o_idx, err_msg=lw + " routes")
            np.testing.assert_array_equal(to_u16(buf.weights[l]), o_w, err_msg=lw + " weights")
            # (the last layer writes the pass's output buffer)
            h_out = to_u16(out) if l == LAYERS - 1 else to_u16(buf.h[l])
            assert_layer_close(h_out, ref, h2, what=lw + " moe")
            h_in = h_out
        np.testing.assert_array_equal(to_u16(out), h_in)


@pytest.mark.parametrize("width", WIDTHS)
def test_verify_pass_follows_the_cache_length(decoder, oracle, width):
    """The graphs captured at CONTEXT replayed at two longer cache lengths
    (a verify loop's cache grows between blocks): output and states equal
    the eager step at that length bit for bit, and the attention layer's
    output and appended rows meet the oracle at that length."""
    model, vp, _, weights = decoder
    eps = model.layers[0].eps
    for length in (CONTEXT + width + 3, CAPACITY - 24):
        what = f"decoder width {width} at length {length}"
        print(f"[case] {what}", flush=True)
        x = model.hidden(width, step=8000 + 10 * width + length)
        cos, sin = model.rope(width, length)
        before = _snapshot(model)
        out = vp.verify(x, cos, sin, length=length).clone()
        buf = vp.buffers(width)
        after = _snapshot(model)
        _restore(model, before)
        eager = model.stack.step(x, length, cos, sin)
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), out.view(torch.int16)), f"{what}: graph != eager"
        for (a, b), (c, d) in zip(_snapshot(model), after):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                               c.view(torch.int16) if c.dtype == torch.bfloat16 else c)
            assert torch.equal(b.view(torch.int16) if b.dtype == torch.bfloat16 else b,
                               d.view(torch.int16) if d.dtype == torch.bfloat16 else d)
        _restore(model, after)
        l = LAYERS - 1  # the attention layer
        kc0, vc0 = before[l]
        n = to_u16(buf.n[l])
        want, want_k, want_v = oracle.attn_decode(n, weights[l], to_u16(cos), to_u16(sin), to_u16(kc0),
                                                  to_u16(vc0), length, eps=eps)
        assert_close_bf16(to_u16(buf.mix[l]), want, what=what + " attention")
        kc1, vc1 = after[l]
        new = slice(length, length + width)
        _rows_close(to_u16(kc1)[:, new], want_k[:, new], what + " appended keys")
        _rows_close(to_u16(vc1)[:, new], want_v[:, new], what + " appended values")
    vp.set_length(CONTEXT)


@pytest.mark.parametrize("width", (1, 16))
def test_fused_glue_equals_separate_launches(decoder, width):
    """The layer step with the input norm and residual add fused into the
    mixer and attention launches (the default) against the same step with
    them as separate lrmoe_add_rmsnorm launches, from the same states: every
    layer's normed rows, mixer output, post-mixer residual, routes and
    output, and the final states, bit for bit; and the fused step's output
    with untraced buffers (no normed rows stored)."""
    from lightreason_amd.decoder import StepBuffers

    model, _, _, _ = decoder
    print(f"[case] fused glue width {width}", flush=True)
    x = model.hidden(width, step=9100 + width)
    cos, sin = model.rope(width, CONTEXT)
    before = _snapshot(model)
    runs = []
    for fused in (True, False):
        _restore(model, before)
        buf = StepBuffers(LAYERS, width, x.device, trace=True)
        out = model.stack.step(x, CONTEXT, cos, sin, buffers=buf, fused=fused).clone()
        torch.cuda.synchronize()
        runs.append((out, buf, _snapshot(model)))
    # the fused step with untraced buffers (no normed rows stored)
    _restore(model, before)
    o3 = model.stack.step(x, CONTEXT, cos, sin, buffers=StepBuffers(LAYERS, width, x.device), fused=True).clone()
    torch.cuda.synchronize()
    (o1, b1, s1), (o2, b2, s2) = runs
    assert torch.equal(o3.view(torch.int16), o1.view(torch.int16))
    for name in ("n", "mix", "h2", "h", "weights"):
        assert torch.equal(getattr(b1, name).view(torch.int16), getattr(b2, name).view(torch.int16)), name
    assert torch.equal(b1.indices, b2.indices)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    for (a, b), (c, d) in zip(s1, s2):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           c.view(torch.int16) if c.dtype == torch.bfloat16 else c)
        assert torch.equal(b.view(torch.int16) if b.dtype == torch.bfloat16 else b,
                           d.view(torch.int16) if d.dtype == torch.bfloat16 else d)
    _restore(model, before)


def test_verify_pass_rejects_unknown_width(decoder):
    model, vp, _, _ = decoder
    with pytest.raises(ValueError, match="no verify graph"):
        vp.verify(model.hidden(3, step=1))
    with pytest.raises(ValueError, match="capacity"):
        vp.verify(model.hidden(16, step=1), length=CAPACITY - 15)
