"""Gated DeltaNet decode on the GPU against the oracle (oracle/lro.c
lro_delta_rule, lro_delta_mixer), through the C-ABI (lrmoe_delta_rule,
lrmoe_delta_mixer) and the Python surface that mirrors
edge35b/delta_decode.py.

Bars (floating point; the projections run on MFMA, whose fp32 summation
order differs from the oracle's, so a bf16 rounding can flip by one unit):
  * bf16 outputs: assert_close_bf16, rel 1e-2 (max error within 1e-2 of the
    output's magnitude and every row within 1e-2 in L2);
  * recurrent states: max |got - want| <= tol * max |want|, tol 1e-4 for an
    fp32 state from unnormalised inputs (only the summation order differs),
    else 1e-2 (a q/k/v element one bf16 unit away moves a state element by
    ~2^-8 of its update);
  * conv states: each element within one bf16 unit (2^-7 of the larger
    magnitude; at least 1e-5 of the largest entry) of the oracle's, and at
    least 99% bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import assert_close_bf16

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dev_bf16(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def _f(bits):
    from oracle import oracle as O

    return O.bf16_to_f32(bits).astype(np.float64)


def _bf(x):
    from oracle import oracle as O

    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def _state_close(got, want, tol, what):
    g = _f(got) if got.dtype == np.uint16 else got.astype(np.float64)
    w = _f(want) if want.dtype == np.uint16 else want.astype(np.float64)
    assert np.isfinite(g).all(), f"{what}: non-finite state"
    err = np.abs(g - w).max() / max(np.abs(w).max(), 1e-30)
    print(f"{what}: state max rel {err:.2e}, exact {float((g == w).mean()):.3f}", flush=True)
    assert err <= tol, f"{what}: state error {err:.3e} > {tol}"


def _conv_close(got, want, what):
    g, w = _f(got), _f(want)
    exact = float((got == want).mean())
    # one bf16 unit, or 1e-5 of the largest entry for a projection whose fp32
    # sum is so near zero that the summation order decides its sign
    bound = np.maximum(2.0 ** -7 * np.maximum(np.abs(g), np.abs(w)), 1e-5 * np.abs(w).max())
    worst = float((np.abs(g - w) - bound).max())
    print(f"{what}: conv exact {exact:.4f}", flush=True)
    assert worst <= 0, f"{what}: conv state off by more than one bf16 unit"
    assert exact >= 0.99, f"{what}: only {exact:.4f} of the conv state is bit-identical"


# ---- the delta rule (delta_decode._run convention) --------------------------

RULE_CASES = [  # (D, E, H, T)
    (128, 128, 32, 16),
    (128, 128, 32, 1),
    (64, 64, 4, 5),
    (256, 32, 3, 2),
    (128, 48, 6, 3),
]


@pytest.mark.parametrize("record", [False, True])
@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("bf16_state", [False, True])
@pytest.mark.parametrize("D,E,H,T", RULE_CASES)
def test_delta_rule_against_oracle(oracle, device, D, E, H, T, bf16_state, normalize, record):
    from lightreason_amd.delta import delta_rule

    what = f"delta_rule D={D} E={E} H={H} T={T} bf16_state={bf16_state} normalize={normalize} record={record}"
    print(f"[case] {what}", flush=True)
    rng = np.random.default_rng(D * 7 + E + H * 13 + T * 31 + 2 * bf16_state + normalize)
    s = 1.0 if normalize else 1.0 / np.sqrt(D)   # unnormalised keys of about unit norm keep it contractive
    q = _bf(rng.normal(size=(T, H, D)) * s)
    k = _bf(rng.normal(size=(T, H, D)) * s)
    v = _bf(rng.normal(size=(T, H, E)))
    g = (-rng.random((T, H)) * 0.5).astype(np.float32)
    beta = _bf(rng.random((T, H)))
    s0 = (rng.normal(size=(H, D, E)) * 0.05).astype(np.float32)
    init = _bf(s0) if bf16_state else s0
    G = torch.from_numpy(g).to(device).exp().cpu().numpy()   # exp as the GPU path takes it (torch)
    want_out, want_states = oracle.delta_rule(q, k, v, G, beta, init, normalize=normalize, record=record)

    tq, tk, tv, tb = (_dev_bf16(a, device)[None] for a in (q, k, v, beta))
    tg = torch.from_numpy(g).to(device)[None]
    tinit = (_dev_bf16(init, device) if bf16_state else torch.from_numpy(init).to(device))[None]
    out, states = delta_rule(tq, tk, tv, tg, tb, tinit, record=record, normalize=normalize)
    torch.cuda.synchronize()
    assert out.shape == (1, T, H, E) and out.dtype == torch.bfloat16
    assert states.shape == (T if record else 1, H, D, E) and states.dtype == tinit.dtype
    assert_close_bf16(_bits(out[0]).reshape(T * H, E), want_out.reshape(T * H, E), what=what)
    got_states = _bits(states) if bf16_state else states.cpu().numpy()
    tol = 1e-4 if not (bf16_state or normalize) else 1e-2
    _state_close(got_states, want_states, tol, what)
    # the initial state is not modified
    assert torch.equal(tinit.view(torch.int16) if bf16_state else tinit,
                       (_dev_bf16(init, device).view(torch.int16) if bf16_state else torch.from_numpy(init).to(device))[None])


def test_delta_rule_zero_tokens_copies_the_state(device):
    from lightreason_amd.delta import delta_rule

    init = torch.randn(1, 2, 64, 32, device=device)
    empty = torch.empty(1, 0, 2, 64, dtype=torch.bfloat16, device=device)
    out, states = delta_rule(empty, empty, torch.empty(1, 0, 2, 32, dtype=torch.bfloat16, device=device),
                             torch.empty(1, 0, 2, device=device), torch.empty(1, 0, 2, dtype=torch.bfloat16, device=device),
                             init, record=False, normalize=True)
    torch.cuda.synchronize()
    assert out.shape == (1, 0, 2, 32)
    assert torch.equal(states, init[0][None])


def test_delta_rule_rejects_unsupported_layouts(device):
    from lightreason_amd.delta import delta_rule

    q = torch.zeros(1, 2, 4, 96, dtype=torch.bfloat16, device=device)
    v = torch.zeros(1, 2, 4, 32, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="Unsupported recurrent layout"):
        delta_rule(q, q, v, torch.zeros(1, 2, 4, device=device), torch.zeros(1, 2, 4, dtype=torch.bfloat16, device=device),
                   torch.zeros(1, 4, 96, 32, device=device), record=False, normalize=False)
    q = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16, device=device)
    v = torch.zeros(1, 2, 4, 40, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="Unsupported recurrent layout"):
        delta_rule(q, q, v, torch.zeros(1, 2, 4, device=device), torch.zeros(1, 2, 4, dtype=torch.bfloat16, device=device),
                   torch.zeros(1, 4, 64, 40, device=device), record=False, normalize=False)


# ---- the whole mixer step -------------------------------------------------------

def mixer_weights_bits(seed: int) -> dict:
    """Random bf16 weights of one 35B Gated DeltaNet mixer (the scales of a
    trained layer: projections ~N(0, 0.02), conv ~N(0, 0.3), norm ~N(1, 0.1),
    A_log = log U(1, 16), dt_bias ~N(0, 0.5))."""
    rng = np.random.default_rng(seed)
    return dict(in_proj_qkv=_bf(rng.normal(0, 0.02, (8192, 2048))), in_proj_z=_bf(rng.normal(0, 0.02, (4096, 2048))),
                in_proj_b=_bf(rng.normal(0, 0.02, (32, 2048))), in_proj_a=_bf(rng.normal(0, 0.02, (32, 2048))),
                conv1d=_bf(rng.normal(0, 0.3, (8192, 4))), A_log=_bf(np.log(rng.uniform(1, 16, 32))),
                dt_bias=_bf(rng.normal(0, 0.5, 32)), norm=_bf(rng.normal(1, 0.1, 128)),
                out_proj=_bf(rng.normal(0, 0.02, (2048, 4096))))


@pytest.fixture(scope="module")
def mixer_case(device):
    from lightreason_amd.delta import DeltaMixer

    w = mixer_weights_bits(4242)
    mixer = DeltaMixer(**{name: _dev_bf16(bits, device) for name, bits in w.items()}, eps=1e-6)
    rng = np.random.default_rng(99)
    conv0 = _bf(rng.normal(0, 1.0, (8192, 4)))
    state0 = (rng.normal(size=(32, 128, 128)) * 0.05).astype(np.float32)
    return w, mixer, conv0, state0


def _oracle_chain(oracle, w, x, conv, state):
    """The oracle token by token: per-token conv states, states and outputs
    (equal to one call over the block, whose tokens are processed in order)."""
    outs, convs, states = [], [], []
    for t in range(x.shape[0]):
        out, conv, state, _ = oracle.delta_mixer(x[t:t + 1], w, conv, state)
        outs.append(out[0])
        convs.append(conv)
        states.append(state)
    return np.stack(outs), np.stack(convs), np.stack(states)


@pytest.mark.parametrize("bf16_state", [False, True])
@pytest.mark.parametrize("T", [1, 3, 16])
def test_delta_mixer_against_oracle(oracle, device, mixer_case, T, bf16_state):
    from lightreason_amd.delta import mixer_status

    w, mixer, conv0, s0 = mixer_case
    what = f"delta_mixer T={T} bf16_state={bf16_state}"
    print(f"[case] {what}", flush=True)
    rng = np.random.default_rng(1000 + T + bf16_state)
    x = _bf(rng.normal(0, 1.0, (T, 2048)))
    state0 = _bf(s0) if bf16_state else s0
    want_out, want_convs, want_states = _oracle_chain(oracle, w, x, conv0, state0)
    # the block at once agrees with the chain
    block_out, block_conv, block_state, block_rec = oracle.delta_mixer(x, w, conv0, state0, record=True)
    np.testing.assert_array_equal(block_out, want_out)
    np.testing.assert_array_equal(block_rec, want_states)

    conv = _dev_bf16(conv0, device)
    state = _dev_bf16(state0, device) if bf16_state else torch.from_numpy(state0).to(device)
    conv_rec = torch.empty((T, 8192, 4), dtype=torch.bfloat16, device=device)
    state_rec = torch.empty((T, 32, 128, 128), dtype=state.dtype, device=device)
    out = mixer.step(_dev_bf16(x, device), conv, state, conv_record=conv_rec, state_record=state_rec)
    torch.cuda.synchronize()
    assert mixer_status(device) == 0
    assert_close_bf16(_bits(out), want_out, what=what)
    _conv_close(_bits(conv), want_convs[-1], what)
    _conv_close(_bits(conv_rec), want_convs, what + " record")
    got_state = _bits(state) if bf16_state else state.cpu().numpy()
    _state_close(got_state, want_states[-1], 1e-2, what)
    got_rec = _bits(state_rec) if bf16_state else state_rec.cpu().numpy()
    _state_close(got_rec, want_states, 1e-2, what + " record")
    # the last recorded states are the final ones
    assert torch.equal(conv_rec[-1].view(torch.int16), conv.view(torch.int16))
    assert torch.equal(state_rec[-1].view(torch.int16) if bf16_state else state_rec[-1],
                       state.view(torch.int16) if bf16_state else state)


def test_delta_mixer_steps_chain_in_place(oracle, device, mixer_case):
    """Three single-token steps on one cache (no records) equal the oracle
    run over the three tokens; and a block of three gives the same state."""
    w, mixer, conv0, s0 = mixer_case
    rng = np.random.default_rng(77)
    x = _bf(rng.normal(0, 1.0, (3, 2048)))
    want_out, want_convs, want_states = _oracle_chain(oracle, w, x, conv0, s0)
    conv = _dev_bf16(conv0, device)
    state = torch.from_numpy(s0).to(device)
    outs = [mixer.step(_dev_bf16(x[t:t + 1], device), conv, state).clone() for t in range(3)]
    torch.cuda.synchronize()
    assert_close_bf16(np.concatenate([_bits(o) for o in outs]), want_out, what="three steps")
    _conv_close(_bits(conv), want_convs[-1], "three steps")
    _state_close(state.cpu().numpy(), want_states[-1], 1e-2, "three steps")
    conv_b = _dev_bf16(conv0, device)
    state_b = torch.from_numpy(s0).to(device)
    out_b = mixer.step(_dev_bf16(x, device), conv_b, state_b)
    torch.cuda.synchronize()
    # one block and three single steps run the same arithmetic per token
    assert torch.equal(torch.cat(outs).view(torch.int16), out_b.view(torch.int16))
    assert torch.equal(conv_b.view(torch.int16), conv.view(torch.int16))
    assert torch.equal(state_b, state)


def test_delta_mixer_rejects_bad_arguments(device, mixer_case):
    _, mixer, conv0, s0 = mixer_case
    conv = _dev_bf16(conv0, device)
    state = torch.from_numpy(s0).to(device)
    with pytest.raises(ValueError):
        mixer.step(torch.zeros(17, 2048, dtype=torch.bfloat16, device=device), conv, state)
    with pytest.raises(ValueError):
        mixer.step(torch.zeros(1, 2048, dtype=torch.bfloat16, device=device), conv, state.half())
    with pytest.raises(ValueError):
        mixer.step(torch.zeros(2, 2048, dtype=torch.bfloat16, device=device), conv, state,
                   state_record=torch.zeros(3, 32, 128, 128, device=device))
