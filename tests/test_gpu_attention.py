"""lrmoe_attn_decode -- the full-attention decode step of the 35B model
([HF] Qwen3_5MoeAttention with a key/value cache) -- on the GPU against the
oracle's lro_attn_decode (pinned against the Transformers module itself in
test_attn_oracle.py), through the C ABI.

Cases cover one chunk of positions and many (up to 128 per key/value head),
a first token with an empty cache, blocks of 3, 5, 8 and 16 tokens (causal
within the block), chunk and 32-position sub-block boundaries, and a cache
filled to its capacity.  Bars: the appended key and value rows equal the
oracle's but for a few elements (projection and norm summation order; see
_close_rows); every other cache row unchanged; the output within 1e-2
of its magnitude (max and L2; the kernel's softmax runs per chunk with
probabilities relative to the chunk maximum, the oracle's over all
positions with bf16 probabilities, as the Transformers eager forward)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

KV, D, ROT = 2, 256, 64
SENTINEL = 0x1234


def _bf(x):
    from oracle import oracle as O

    return O.f32_to_bf16(np.asarray(x, dtype=np.float32))


def _f(bits):
    from oracle import oracle as O

    return O.bf16_to_f32(bits)


def _dev(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def _host(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def attn_case(device):
    from lightreason_amd.attention import AttentionDecode

    rng = np.random.default_rng(77)
    w = dict(q_proj=_bf(rng.normal(0, 0.02, (8192, 2048))), k_proj=_bf(rng.normal(0, 0.02, (512, 2048))),
             v_proj=_bf(rng.normal(0, 0.02, (512, 2048))), o_proj=_bf(rng.normal(0, 0.02, (2048, 4096))),
             q_norm=_bf(rng.normal(0, 0.1, 256)), k_norm=_bf(rng.normal(0, 0.1, 256)))
    bound = AttentionDecode(**{k: _dev(v, device) for k, v in w.items()}, eps=1e-6)
    return w, bound


def _rope(T, start):
    from transformers import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeTextRotaryEmbedding

    rotary = Qwen3_5MoeTextRotaryEmbedding(Qwen3_5MoeTextConfig())
    cos, sin = rotary(torch.zeros(1, dtype=torch.bfloat16), torch.arange(start, start + T)[None])
    return _host(cos[0]), _host(sin[0])


def _close_rows(got, want, what):
    """Identical but for a few elements, each within one bf16 ulp of its
    value or, for a projection whose terms cancel, 2^-10 of its row's
    largest (the fp32 summation order moves a small sum by more than its own
    ulp)."""
    same = float((got == want).mean())
    g, w = _f(got).astype(np.float64), _f(want).astype(np.float64)
    bound = np.maximum(2.0 ** -7 * np.abs(w), 2.0 ** -10 * np.abs(w).max(axis=-1, keepdims=True))
    excess = float(np.max(np.abs(g - w) / bound)) if got.size else 0.0
    print(f"{what}: identical {same:.4f}, worst difference {excess:.2f} of its bound", flush=True)
    assert same >= 0.98 and excess <= 1.0, what


# Blocks of more than 4 tokens run the 64-row attention variants (above 8
# tokens a chunk's rows in two workgroups, split at the token half: 9 as
# 5 + 4, 13 as 7 + 6); past the chunk cap the chunks hold more than two
# 32-position sub-blocks and the last one the remainder (up to 128 chunks
# to merge): (9000, 8), (16383, 5) and (20000, 16).
CASES = [(0, 1), (1, 1), (37, 1), (63, 1), (300, 1), (2000, 1), (5000, 1), (20000, 1),
         (40, 3), (31, 5), (3000, 8), (130, 16), (600, 16), (4100, 16),
         (450, 9), (1000, 10), (3333, 13),
         (9000, 8), (16383, 5), (20000, 16)]


@pytest.mark.parametrize("L,T", CASES)
def test_attn_decode_against_oracle(oracle, device, attn_case, L, T):
    w, bound = attn_case
    what = f"attn_decode L={L} T={T}"
    print(f"[case] {what}", flush=True)
    rng = np.random.default_rng(1000 * T + L)
    cap = L + T + 7
    kc = np.full((KV, cap, D), SENTINEL, dtype=np.uint16)
    vc = np.full((KV, cap, D), SENTINEL, dtype=np.uint16)
    kc[:, :L] = _bf(rng.normal(0, 1.0, (KV, L, D)))
    vc[:, :L] = _bf(rng.normal(0, 1.0, (KV, L, D)))
    x = _bf(rng.normal(0, 1.0, (T, 2048)))
    cos, sin = _rope(T, L)
    want, want_k, want_v = oracle.attn_decode(x, w, cos, sin, kc, vc, L)

    k_dev, v_dev = _dev(kc, device), _dev(vc, device)
    out = bound.step(_dev(x, device), _dev(cos, device), _dev(sin, device), k_dev, v_dev, L)
    torch.cuda.synchronize()
    got_k, got_v, got = _host(k_dev), _host(v_dev), _host(out)
    np.testing.assert_array_equal(got_k[:, :L], kc[:, :L])
    np.testing.assert_array_equal(got_v[:, :L], vc[:, :L])
    assert np.all(got_k[:, L + T:] == SENTINEL) and np.all(got_v[:, L + T:] == SENTINEL)
    _close_rows(got_k[:, L:L + T], want_k[:, L:L + T], f"{what} keys")
    _close_rows(got_v[:, L:L + T], want_v[:, L:L + T], f"{what} values")
    g, wv = _f(got).astype(np.float64), _f(want).astype(np.float64)
    err = np.abs(g - wv).max() / np.abs(wv).max()
    l2 = np.linalg.norm(g - wv) / np.linalg.norm(wv)
    print(f"{what}: output max rel {err:.2e}, L2 rel {l2:.2e}", flush=True)
    assert err <= 1e-2 and l2 <= 1e-2


def test_attn_decode_fills_the_cache_to_capacity(oracle, device, attn_case):
    """length + tokens == capacity: the last rows of both caches are written
    and nothing past them is touched (the cache is a view of a longer
    buffer whose tail keeps its sentinel)."""
    w, bound = attn_case
    L, T = 90, 6
    rng = np.random.default_rng(5)
    kc = np.full((KV, L + T, D), SENTINEL, dtype=np.uint16)
    vc = kc.copy()
    kc[:, :L] = _bf(rng.normal(0, 1.0, (KV, L, D)))
    vc[:, :L] = _bf(rng.normal(0, 1.0, (KV, L, D)))
    x = _bf(rng.normal(0, 1.0, (T, 2048)))
    cos, sin = _rope(T, L)
    want, want_k, want_v = oracle.attn_decode(x, w, cos, sin, kc, vc, L)
    big_k = torch.full((KV * (L + T) * D + 4096,), SENTINEL, dtype=torch.int16).view(torch.bfloat16).to(device)
    big_v = big_k.clone()
    k_dev = big_k[:KV * (L + T) * D].view(KV, L + T, D)
    v_dev = big_v[:KV * (L + T) * D].view(KV, L + T, D)
    k_dev.copy_(_dev(kc, device))
    v_dev.copy_(_dev(vc, device))
    out = bound.step(_dev(x, device), _dev(cos, device), _dev(sin, device), k_dev, v_dev, L)
    torch.cuda.synchronize()
    assert np.all(_host(big_k)[KV * (L + T) * D:] == SENTINEL)
    assert np.all(_host(big_v)[KV * (L + T) * D:] == SENTINEL)
    _close_rows(_host(k_dev)[:, L:], want_k[:, L:], "full cache keys")
    _close_rows(_host(v_dev)[:, L:], want_v[:, L:], "full cache values")
    g, wv = _f(_host(out)).astype(np.float64), _f(want).astype(np.float64)
    assert np.linalg.norm(g - wv) <= 1e-2 * np.linalg.norm(wv)
    with pytest.raises(ValueError, match="capacity"):
        bound.step(_dev(x, device), _dev(cos, device), _dev(sin, device), k_dev, v_dev, L + 1)


@pytest.mark.parametrize("L,T", [(0, 1), (37, 3), (700, 8), (2050, 16), (5993, 1), (5984, 16)])
def test_attn_decode_at_reads_the_length_on_the_device(oracle, device, attn_case, L, T):
    """lrmoe_attn_decode_at (the length in device memory, chunks sized for
    the capacity, 6000 positions): the oracle's bars at lengths from an
    empty cache to a full one, rows past length + T untouched."""
    w, bound = attn_case
    what = f"attn_decode_at L={L} T={T}"
    print(f"[case] {what}", flush=True)
    cap = 6000
    rng = np.random.default_rng(3000 * T + L)
    kc = np.full((KV, cap, D), SENTINEL, dtype=np.uint16)
    vc = np.full((KV, cap, D), SENTINEL, dtype=np.uint16)
    kc[:, :L] = _bf(rng.normal(0, 1.0, (KV, L, D)))
    vc[:, :L] = _bf(rng.normal(0, 1.0, (KV, L, D)))
    x = _bf(rng.normal(0, 1.0, (T, 2048)))
    cos, sin = _rope(T, L)
    want, want_k, want_v = oracle.attn_decode(x, w, cos, sin, kc, vc, L)
    k_dev, v_dev = _dev(kc, device), _dev(vc, device)
    length = torch.tensor([L], dtype=torch.int32, device=device)
    out = bound.step(_dev(x, device), _dev(cos, device), _dev(sin, device), k_dev, v_dev, length)
    torch.cuda.synchronize()
    got_k, got_v, got = _host(k_dev), _host(v_dev), _host(out)
    np.testing.assert_array_equal(got_k[:, :L], kc[:, :L])
    np.testing.assert_array_equal(got_v[:, :L], vc[:, :L])
    assert np.all(got_k[:, L + T:] == SENTINEL) and np.all(got_v[:, L + T:] == SENTINEL)
    _close_rows(got_k[:, L:L + T], want_k[:, L:L + T], f"{what} keys")
    _close_rows(got_v[:, L:L + T], want_v[:, L:L + T], f"{what} values")
    g, wv = _f(got).astype(np.float64), _f(want).astype(np.float64)
    err = np.abs(g - wv).max() / np.abs(wv).max()
    l2 = np.linalg.norm(g - wv) / np.linalg.norm(wv)
    print(f"{what}: output max rel {err:.2e}, L2 rel {l2:.2e}", flush=True)
    assert err <= 1e-2 and l2 <= 1e-2


def test_attn_decode_at_bad_length_writes_nothing(device, attn_case):
    """A device length past capacity - tokens: the output rows are NaN and
    no cache row is written."""
    w, bound = attn_case
    cap, T = 300, 4
    rng = np.random.default_rng(11)
    kc = _bf(rng.normal(0, 1.0, (KV, cap, D)))
    vc = _bf(rng.normal(0, 1.0, (KV, cap, D)))
    x = _bf(rng.normal(0, 1.0, (T, 2048)))
    cos, sin = _rope(T, cap)
    k_dev, v_dev = _dev(kc, device), _dev(vc, device)
    for bad in (cap - T + 1, -5):
        length = torch.tensor([bad], dtype=torch.int32, device=device)
        out = bound.step(_dev(x, device), _dev(cos, device), _dev(sin, device), k_dev, v_dev, length)
        torch.cuda.synchronize()
        assert torch.isnan(out.float()).all(), bad
        np.testing.assert_array_equal(_host(k_dev), kc)
        np.testing.assert_array_equal(_host(v_dev), vc)


def test_attn_decode_one_block_equals_token_steps(device, attn_case):
    """A block of 8 tokens against the same tokens one at a time (causal
    masking inside the block): the caches agree exactly (same kernels, same
    inputs per row) and the outputs within the chunked softmax's rounding."""
    w, bound = attn_case
    L, T = 700, 8
    rng = np.random.default_rng(9)
    kc = _bf(rng.normal(0, 1.0, (KV, L + T, D)))
    vc = _bf(rng.normal(0, 1.0, (KV, L + T, D)))
    x = _bf(rng.normal(0, 1.0, (T, 2048)))
    cos, sin = _rope(T, L)
    kb, vb = _dev(kc, device), _dev(vc, device)
    block = bound.step(_dev(x, device), _dev(cos, device), _dev(sin, device), kb, vb, L)
    ks, vs = _dev(kc, device), _dev(vc, device)
    rows = [bound.step(_dev(x[t:t + 1], device), _dev(cos[t:t + 1], device), _dev(sin[t:t + 1], device), ks, vs, L + t)
            for t in range(T)]
    torch.cuda.synchronize()
    assert torch.equal(kb.view(torch.int16), ks.view(torch.int16))
    assert torch.equal(vb.view(torch.int16), vs.view(torch.int16))
    steps = torch.cat(rows).float()
    assert float((block.float() - steps).norm() / steps.norm()) <= 5e-3
