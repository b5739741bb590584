"""The Gated DeltaNet decode oracle (oracle/lro.c lro_delta_rule,
lro_delta_mixer) pinned without the GPU: closed forms of the recurrence, an
independent float64 restatement, and the installed Transformers
implementation it restates (torch_recurrent_gated_delta_rule and the
Qwen3_5MoeGatedDeltaNet module itself, run on the CPU)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

D = E = 128


def _bf(x):
    from oracle import oracle as O

    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def _f(bits):
    from oracle import oracle as O

    return O.bf16_to_f32(bits)


def _inputs(T, H, seed, unit=False):
    """Random q, k, v, G, beta; with unit=True, q and k of about unit norm
    (as after l2norm), which keeps the recurrence contractive."""
    rng = np.random.default_rng(seed)
    s = 1.0 / np.sqrt(D) if unit else 1.0
    q = _bf(rng.normal(size=(T, H, D)) * s)
    k = _bf(rng.normal(size=(T, H, D)) * s)
    v = _bf(rng.normal(size=(T, H, E)))
    G = np.exp(-rng.random((T, H)) * 0.5).astype(np.float32)
    beta = _bf(rng.random((T, H)))
    return q, k, v, G, beta


def test_delta_rule_closed_form_first_token(oracle):
    """From a zero state, one token: state = k (x) beta v, out = beta (q.k / sqrt(D)) v."""
    q, k, v, G, beta = _inputs(1, 3, 1)
    out, states = oracle.delta_rule(q, k, v, G, beta, np.zeros((3, D, E), np.float32), normalize=False, record=True)
    qf, kf, vf, bf = (_f(a).astype(np.float64) for a in (q, k, v, beta))
    for h in range(3):
        want_state = np.outer(kf[0, h], bf[0, h] * vf[0, h])
        assert np.allclose(states[0, h], want_state, rtol=1e-6, atol=1e-7)
        want = bf[0, h] * (qf[0, h] @ kf[0, h]) / np.sqrt(D) * vf[0, h]
        got = _f(out[0, h]).astype(np.float64)
        assert np.all(np.abs(got - want) <= np.abs(want) * 2 ** -8 + 1e-6)
    # the decay applies to the carried state before the update: G = 0 forgets it
    big = np.full((3, D, E), 5.0, np.float32)
    out0, _ = oracle.delta_rule(q, k, v, np.zeros_like(G), beta, big, normalize=False, record=False)
    np.testing.assert_array_equal(out0, out)


def _float64_rule(q, k, v, G, beta, state, normalize, bf16_state):
    """An independent restatement in float64 (numpy), vectorised over heads."""
    T = q.shape[0]
    qf, kf, vf, bf = (_f(a).astype(np.float64) for a in (q, k, v, beta))
    if normalize:
        def l2(x):   # HF l2norm on bf16 values: every step rounded to bf16
            sq = _f(_bf(x * x)).astype(np.float64)
            s = _f(_bf(_f(_bf(sq.sum(-1, keepdims=True))) + 1e-6)).astype(np.float64)
            inv = _f(_bf(1.0 / np.sqrt(s))).astype(np.float64)
            return _f(_bf(x * inv)).astype(np.float64)
        qf, kf = l2(qf), l2(kf)
    S = (_f(state) if bf16_state else state).astype(np.float64).copy()
    outs, states = [], []
    for t in range(T):
        S = S * G[t][:, None, None]
        mem = np.einsum("hde,hd->he", S, kf[t])
        delta = (vf[t] - mem) * bf[t][:, None]
        S = S + kf[t][:, :, None] * delta[:, None, :]
        outs.append(np.einsum("hde,hd->he", S, qf[t] / np.sqrt(D)))
        if bf16_state:
            S = _f(_bf(S)).astype(np.float64)
        states.append(S.copy())
    return np.stack(outs), np.stack(states)


@pytest.mark.parametrize("bf16_state", [False, True])
@pytest.mark.parametrize("normalize", [False, True])
def test_delta_rule_against_float64(oracle, bf16_state, normalize):
    T, H = 6, 4
    q, k, v, G, beta = _inputs(T, H, 7 + bf16_state + 2 * normalize, unit=not normalize)
    rng = np.random.default_rng(3)
    s0 = (rng.normal(size=(H, D, E)) * 0.05).astype(np.float32)
    state = _bf(s0) if bf16_state else s0
    out, states = oracle.delta_rule(q, k, v, G, beta, state, normalize=normalize, record=True)
    want_out, want_states = _float64_rule(q, k, v, G, beta, state, normalize, bf16_state)
    got = _f(out).astype(np.float64)
    scale = np.abs(want_out).max(axis=-1, keepdims=True)
    assert np.all(np.abs(got - want_out) <= 1e-2 * scale), np.abs(got - want_out).max()
    got_states = (_f(states) if bf16_state else states).astype(np.float64)
    s_scale = np.abs(want_states).max()
    assert np.abs(got_states - want_states).max() <= (2 ** -7 if bf16_state else 1e-5) * s_scale
    # record=False returns the final state only, equal to the last recorded one
    _, final = oracle.delta_rule(q, k, v, G, beta, state, normalize=normalize, record=False)
    np.testing.assert_array_equal(final[0], states[-1])


def test_delta_rule_against_transformers(oracle):
    """[HF] torch_recurrent_gated_delta_rule (fp32 state, q/k l2norm in the
    kernel) on the CPU: same outputs within bf16 output rounding, same final
    state within fp32 summation order."""
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import torch_recurrent_gated_delta_rule

    T, H = 4, 6
    q, k, v, G, beta = _inputs(T, H, 11)
    g = np.log(G).astype(np.float32)
    G2 = np.exp(g.astype(np.float64)).astype(np.float32)   # exp(log G) as torch will compute it
    rng = np.random.default_rng(5)
    s0 = (rng.normal(size=(H, D, E)) * 0.05).astype(np.float32)
    out, states = oracle.delta_rule(q, k, v, G2, beta, s0, normalize=True, record=False)

    def tb(bits):
        return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)[None]
    ref_out, ref_state = torch_recurrent_gated_delta_rule(
        tb(q), tb(k), tb(v), g=torch.from_numpy(g)[None], beta=tb(beta), initial_state=torch.from_numpy(s0)[None],
        output_final_state=True, use_qk_l2norm_in_kernel=True)
    ref = ref_out[0].float().numpy().astype(np.float64)
    got = _f(out).astype(np.float64)
    # torch's CPU bf16 rsqrt rounds through a bf16 square root (1/sqrt(143)
    # gives 0x3DAC, not the nearest 0x3DAB that the oracle and a GPU take),
    # so l2norm'd keys can differ by one bf16 ulp: rows agree in L2 within
    # 1e-2, elements within 2e-2 of the row's magnitude.
    rows = np.linalg.norm(got - ref, axis=-1) / np.linalg.norm(ref, axis=-1)
    assert rows.max() <= 1e-2, rows.max()
    assert np.all(np.abs(got - ref) <= 2e-2 * np.abs(ref).max(axis=-1, keepdims=True))
    ref_s = ref_state[0].numpy()
    assert np.abs(states[0] - ref_s).max() <= 1e-2 * np.abs(ref_s).max()


def _hf_mixer(seed=21):
    from transformers import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeGatedDeltaNet

    torch.manual_seed(seed)
    cfg = Qwen3_5MoeTextConfig()
    m = Qwen3_5MoeGatedDeltaNet(cfg, 0)
    with torch.no_grad():
        for p in (m.in_proj_qkv.weight, m.in_proj_z.weight, m.in_proj_b.weight, m.in_proj_a.weight,
                  m.out_proj.weight):
            p.normal_(0.0, 0.02)
        m.conv1d.weight.normal_(0.0, 0.3)
        m.norm.weight.normal_(1.0, 0.1)
        m.dt_bias.normal_(0.0, 0.5)
    return cfg, m.to(torch.bfloat16).eval()


def _bits(t):
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16)


def mixer_weights(m):
    return dict(in_proj_qkv=_bits(m.in_proj_qkv.weight), in_proj_z=_bits(m.in_proj_z.weight),
                in_proj_b=_bits(m.in_proj_b.weight), in_proj_a=_bits(m.in_proj_a.weight),
                conv1d=_bits(m.conv1d.weight[:, 0, :]), A_log=_bits(m.A_log), dt_bias=_bits(m.dt_bias),
                norm=_bits(m.norm.weight), out_proj=_bits(m.out_proj.weight))


def test_delta_mixer_against_transformers_module(oracle):
    """One cached decode step of Qwen3_5MoeGatedDeltaNet (35B dims, random
    weights) on the CPU in bf16 against lro_delta_mixer on the same cache:
    output within 1e-2 of its magnitude, conv state bit-exact, recurrent
    state (fp32) within summation order."""
    from transformers.cache_utils import DynamicCache

    cfg, m = _hf_mixer()
    cache = DynamicCache(config=cfg)
    with torch.no_grad():
        m(torch.randn(1, 6, 2048).to(torch.bfloat16), cache_params=cache)   # prefill: fills the cache
    layer = cache.layers[0]
    conv0 = _bits(layer.conv_states[0][0]).copy()   # the forward updates the cache in place
    state0 = layer.recurrent_states[0][0].numpy().copy()
    x = torch.randn(1, 1, 2048).to(torch.bfloat16)
    with torch.no_grad():
        ref = m(x, cache_params=cache)
    out, conv1, state1, _ = oracle.delta_mixer(_bits(x[0]), mixer_weights(m), conv0, state0, eps=cfg.rms_norm_eps)
    np.testing.assert_array_equal(conv1, _bits(layer.conv_states[0][0]))
    ref_state = layer.recurrent_states[0][0].numpy()
    assert np.abs(state1 - ref_state).max() <= 1e-3 * np.abs(ref_state).max()
    got, want = _f(out[0]).astype(np.float64), ref[0, 0].float().numpy().astype(np.float64)
    err = np.abs(got - want).max() / np.abs(want).max()
    print(f"mixer vs transformers: max rel {err:.2e}, exact {(got == want).mean():.3f}")
    assert err <= 1e-2
    assert np.linalg.norm(got - want) <= 1e-2 * np.linalg.norm(want)
