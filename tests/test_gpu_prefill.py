"""Prefill (T > 16: lrmoe_moe_layer's grouped MFMA path) against the oracle
at the sizes where every branch of the grouped kernels runs (needs an
MI355X).

The prefill plan cuts each expert's token list into work units of at most
128 tokens (the shared expert's units are tokens 128u .. 128u+127); the
expert launch gives each of 8 work lists a contiguous range of units.  A
unit of more than 64 tokens runs the 8-column-block gate/up MFMA loop and
stages more than 64 act rows per down item; an expert with more than 128
tokens is split over several units, which then share a list.  These tests
route so that all of this happens, assert that it did, and compare against
the oracle:

  - routes (indices and weights) bit-exact for every token;
  - outputs, for a token sample that covers every unit boundary of the
    hottest routed expert and of the shared expert (the last token of a
    unit, the first of the next, tokens 63, 64 and 65 of each unit) plus
    random tokens, within helpers.assert_layer_close (1e-2).

Each token's output depends only on its own row and routes, so the
oracle's result for the sample equals those rows of the whole batch's.
The T=2048 case is the prefill workload: hidden ~N(0, 1), logits = the
router's fp32 logits plus a per-expert bias ~N(0, 0.25) (max/mean load
about 4), shared expert.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_layer_close, from_u16, oracle_layer_rows, to_u16

pytestmark = pytest.mark.gpu

UNIT = 128


def _unit_sample(pair_tokens: np.ndarray) -> set:
    """Tokens at the unit-boundary and half-unit positions of one expert's
    ascending token list."""
    n = len(pair_tokens)
    pos = set()
    for start in range(0, n, UNIT):
        for off in (-1, 0, 63, 64, 65):
            if 0 <= start + off < n:
                pos.add(start + off)
    pos.add(n - 1)
    return {int(pair_tokens[p]) for p in pos}


def _run(model, x, logits, norm: bool):
    from lightreason_amd.moe import LayerWeights, Workspace, moe_layer

    base = model.layers[0]
    layer = LayerWeights(**{**base.__dict__, "norm_weight": base.norm_weight if norm else None})
    tokens = x.shape[0]
    ws = Workspace(x.device, tokens)
    idx = torch.empty((tokens, 8), dtype=torch.int64, device=x.device)
    wts = torch.empty((tokens, 8), dtype=torch.bfloat16, device=x.device)
    out = moe_layer(x, layer, indices=idx, weights=wts, logits_in=logits, workspace=ws)
    torch.cuda.synchronize()
    assert ws.status() == 0
    return layer, out, idx.cpu().numpy(), to_u16(wts)


def _check(model, oracle, host_experts, x, logits, norm: bool, what: str, random_tokens: int = 32):
    tokens = x.shape[0]
    print(f"[prefill] {what}: T={tokens} norm={norm} logits={'given' if logits is not None else 'router'}",
          flush=True)
    layer, out, idx, wts = _run(model, x, logits, norm)
    xb = to_u16(x)
    # routes of every token, bit-exact
    xin = oracle.rmsnorm(xb, to_u16(layer.norm_weight), layer.eps) if norm else xb
    if logits is None:
        _, o_idx, o_w = oracle.route(xin, to_u16(layer.router))
    else:
        o_idx, o_w = oracle.route_logits(to_u16(logits))
    np.testing.assert_array_equal(idx, o_idx)
    np.testing.assert_array_equal(wts, o_w)
    # the branches this size is meant to reach
    counts = np.bincount(idx.ravel(), minlength=256)
    hot = int(np.argmax(counts))
    assert counts[hot] > UNIT, f"hottest expert has {counts[hot]} tokens: no multi-unit expert"
    assert tokens > 64, "no unit of more than 64 tokens"
    # the token sample
    plan = oracle.bucket(idx)
    u = int(np.searchsorted(plan["expert"], hot))
    hot_tokens = plan["pair_token"][plan["offset"][u]:plan["offset"][u + 1]]
    sample = _unit_sample(hot_tokens) | _unit_sample(np.arange(tokens))
    rng = np.random.default_rng(tokens)
    sample |= set(rng.choice(tokens, size=min(random_tokens, tokens), replace=False).tolist())
    rows = np.array(sorted(sample))
    print(f"[prefill] {what}: hottest expert {hot} ({counts[hot]} tokens, {(counts[hot] + UNIT - 1) // UNIT} units), "
          f"{(counts > 0).sum()} experts hit, max/mean {counts.max() / counts.mean():.2f}, "
          f"{len(rows)} tokens checked", flush=True)
    want, _, _ = oracle_layer_rows(oracle, layer, xb, host_experts, rows=rows,
                                   logits_bits=None if logits is None else to_u16(logits))
    assert_layer_close(to_u16(out)[rows], want, xb[rows] if norm else None, what=what)


def test_prefill_t2048_bias_routing(model, oracle, host_experts):
    """The T=2048 prefill workload (bias sigma 0.25, shared expert)."""
    tokens = 2048
    x = model.hidden(tokens, step=4000)
    rng = np.random.default_rng(2030)
    base = (x.float() @ model.layers[0].router.float().T).cpu().numpy()
    bias = rng.normal(0.0, 0.25, size=(1, 256))
    logits = from_u16(_bf16_bits(base + bias), x.device)
    _check(model, oracle, host_experts, x, logits, norm=False, what="T=2048 bias 0.25")


def test_prefill_t512_zipf_with_norm(model, oracle, host_experts):
    """Zipf(1.1) popularity (hot experts of 100-300 tokens), RMSNorm and
    residual."""
    tokens = 512
    x = model.hidden(tokens, step=4001)
    rng = np.random.default_rng(512)
    ranks = rng.permutation(256) + 1
    logits = from_u16(_bf16_bits(-1.1 * np.log(ranks)[None, :] + rng.gumbel(size=(tokens, 256))), x.device)
    _check(model, oracle, host_experts, x, logits, norm=True, what="T=512 zipf norm")


def test_prefill_t300_router_with_norm(model, oracle, host_experts):
    """The router GEMV path (no caller logits) at T=300, every token checked."""
    tokens = 300
    x = model.hidden(tokens, step=4002)
    from lightreason_amd.moe import LayerWeights, Workspace, moe_layer

    # Skew the router so that one expert takes more than 128 tokens: add a
    # multiple of the mean hidden direction to one router row.
    base = model.layers[0]
    router = base.router.clone()
    direction = x.float().mean(dim=0)
    router[17] = (router[17].float() + 1.5 * direction / direction.norm()).to(torch.bfloat16)
    layer = LayerWeights(**{**base.__dict__, "router": router})
    ws = Workspace(x.device, tokens)
    idx = torch.empty((tokens, 8), dtype=torch.int64, device=x.device)
    wts = torch.empty((tokens, 8), dtype=torch.bfloat16, device=x.device)
    print("[prefill] T=300 router norm", flush=True)
    out = moe_layer(x, layer, indices=idx, weights=wts, workspace=ws)
    torch.cuda.synchronize()
    assert ws.status() == 0
    xb = to_u16(x)
    want, o_idx, o_w = oracle_layer_rows(oracle, layer, xb, host_experts)
    np.testing.assert_array_equal(idx.cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(wts), o_w)
    counts = np.bincount(o_idx.ravel(), minlength=256)
    assert counts.max() > UNIT, counts.max()
    assert_layer_close(to_u16(out), want, xb, what="T=300 router norm")


def _bf16_bits(values: np.ndarray) -> np.ndarray:
    f32 = np.ascontiguousarray(values, dtype=np.float32)
    bits = f32.view(np.uint32).astype(np.uint64)
    return (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)


@pytest.mark.parametrize("tokens", [20, 260])
def test_prefill_concentrated_routes(model, oracle, host_experts, tokens):
    """Every token routed to the same 8 experts (distinct weights per token):
    at T=260 each of them has 3 work units (128, 128, 4 tokens) and the
    shared expert 3, at T=20 one each -- 27 and 9 units over the 8 lists.
    Every token checked."""
    hot = np.array([3, 40, 77, 100, 150, 201, 230, 255])
    rng = np.random.default_rng(tokens + 11)
    base = rng.normal(0.0, 1.0, size=(tokens, 256))
    base[:, hot] += 12.0 + rng.normal(0.0, 1.0, size=(tokens, 8))
    x = model.hidden(tokens, step=4100 + tokens)
    logits = torch.from_numpy(base.astype(np.float32)).to(torch.bfloat16).to(x.device)
    print(f"[prefill] concentrated T={tokens}", flush=True)
    layer, out, idx, wts = _run(model, x, logits, norm=False)
    o_idx, o_w = oracle.route_logits(to_u16(logits))
    np.testing.assert_array_equal(idx, o_idx)
    np.testing.assert_array_equal(wts, o_w)
    assert set(np.unique(idx).tolist()) == set(hot.tolist())
    xb = to_u16(x)
    want, _, _ = oracle_layer_rows(oracle, layer, xb, host_experts, logits_bits=to_u16(logits))
    assert_layer_close(to_u16(out), want, None, what=f"concentrated T={tokens}")
