"""Helpers shared by the GPU parity tests (imported by test modules only)."""

from __future__ import annotations

import numpy as np
import torch


def to_u16(t: torch.Tensor) -> np.ndarray:
    """bf16 device/host tensor -> uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_u16(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def bf16_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_close_bf16(got_bits: np.ndarray, want_bits: np.ndarray, rel: float = 1e-2, what: str = "") -> dict:
    """Output tolerance for bf16 results with fp32 accumulation, rel = 1e-2:

    (a) max |got - want| <= rel * max |want| over the whole output, and
    (b) for every token row, ||got - want||_2 <= rel * ||want||_2.

    Elementwise relative bounds are not meaningful for bf16 outputs: one
    rounding flip of an intermediate bf16 value moves an output by ~2^-8 of
    the terms it sums, which can exceed 1e-2 of a small output element."""
    got = bf16_f32(got_bits).reshape(-1, got_bits.shape[-1]).astype(np.float64)
    want = bf16_f32(want_bits).reshape(-1, want_bits.shape[-1]).astype(np.float64)
    assert got.shape == want.shape
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    diff = np.abs(got - want)
    tensor_rel = float(diff.max() / max(np.abs(want).max(), 1e-30))
    row_rel = np.linalg.norm(got - want, axis=1) / np.maximum(np.linalg.norm(want, axis=1), 1e-30)
    worst_row = int(np.argmax(row_rel))
    stats = {"tensor_rel": tensor_rel, "worst_row_l2_rel": float(row_rel.max()), "worst_row": worst_row,
             "exact_fraction": float((got == want).mean()),
             "row_max_rel": float((diff.max(axis=1) / np.maximum(np.abs(want).max(axis=1), 1e-30)).max())}
    print(f"{what}: {stats}")
    assert tensor_rel <= rel, f"{what}: max error {tensor_rel:.3e} of max |ref| (limit {rel}); {stats}"
    assert row_rel.max() <= rel, f"{what}: row {worst_row} L2 error {row_rel.max():.3e} (limit {rel}); {stats}"
    return stats


def zipf_routes(tokens: int, seed: int, s: float = 1.1, experts: int = 256, topk: int = 8):
    """Gumbel-top-k over Zipf(s) log-popularity of a seeded rank permutation:
    exactly Zipf sampling without replacement per token.  Returns (indices
    int64 [T, 8] in rank order, weights bf16 bits [T, 8] renormalised)."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(experts) + 1
    logits = -s * np.log(ranks)[None, :] + rng.gumbel(size=(tokens, experts))
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :topk]
    top = np.take_along_axis(logits, idx, axis=1)
    w = np.exp(top - top.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    bits = w.view(np.uint32).astype(np.uint64)
    wb = (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)
    return idx.astype(np.int64), wb


def uniform_routes(tokens: int, seed: int, experts: int = 256, topk: int = 8):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(experts, topk, replace=False) for _ in range(tokens)]).astype(np.int64)
    w = rng.random((tokens, topk)).astype(np.float32) + 0.05
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    bits = w.view(np.uint32).astype(np.uint64)
    wb = (((bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFFFFFF) >> 16).astype(np.uint16)
    return idx, wb


class HostExperts:
    """Lazily copies experts of one bank layer to the host for the oracle."""

    def __init__(self, bank, layer: int):
        self.bank, self.layer, self.cache = bank, layer, {}

    def __call__(self, e: int):
        if e not in self.cache:
            gu, dn = self.bank.expert(self.layer, e)
            self.cache[e] = (to_u16(gu), to_u16(dn))
        return self.cache[e]


def _pool():
    import os
    from concurrent.futures import ThreadPoolExecutor

    global _POOL
    if _POOL is None:
        _POOL = ThreadPoolExecutor(max_workers=max(1, min(16, len(os.sched_getaffinity(0)))))
    return _POOL


_POOL = None


def oracle_experts(oracle, x_bits: np.ndarray, indices: np.ndarray, weights_bits: np.ndarray, host: HostExperts,
                   shared=None, sg_bits=None, residual_bits=None) -> np.ndarray:
    """Routed experts (+ shared, + residual) through the oracle.  Each token's
    result depends only on its own row, routes and weights, so any subset of
    a batch's tokens gives those tokens' rows of the whole batch's result.
    The per-pair expert products run on a thread pool (the oracle's ctypes
    calls release the GIL)."""
    plan = oracle.bucket(indices)
    tokens = x_bits.shape[0]
    y = np.zeros((8 * tokens, 2048), dtype=np.uint16)
    jobs = []
    for u, e in enumerate(plan["expert"].tolist()):
        gu, dn = host(e)
        for p in range(plan["offset"][u], plan["offset"][u + 1]):
            jobs.append((p, gu, dn, plan["pair_token"][p]))

    def pair(job):
        p, gu, dn, t = job
        y[p] = oracle.expert_pair(gu[:512], gu[512:], dn, x_bits[t])

    list(_pool().map(pair, jobs))
    y_shared = None
    if shared is not None:
        g, u_, d = shared
        y_shared = np.stack(list(_pool().map(lambda t: oracle.expert_pair(g, u_, d, x_bits[t]), range(tokens))))
    return oracle.combine(y, plan["route_pair"], plan["pair_slot"], np.ascontiguousarray(weights_bits),
                          y_shared, sg_bits, residual_bits)


def oracle_layer_rows(oracle, layer, x_bits: np.ndarray, host: HostExperts, rows=None, logits_bits=None):
    """The oracle's sparse MoE block for the tokens ``rows`` (all when None)
    of the batch ``x_bits`` [T, 2048]: RMSNorm when ``layer.norm_weight`` is
    set, the router (or top-8 of ``logits_bits`` [T, 256]), routed experts,
    shared expert and gate, ordered combine and residual.  Returns (out bits
    [R, 2048], indices [T, 8], weights bits [T, 8]) with the routes of every
    token, so that they can be compared in full."""
    norm = layer.norm_weight is not None
    xin = oracle.rmsnorm(x_bits, to_u16(layer.norm_weight), layer.eps) if norm else x_bits
    if logits_bits is None:
        _, idx, wts = oracle.route(xin, to_u16(layer.router))
    else:
        idx, wts = oracle.route_logits(logits_bits)
    sel = np.arange(x_bits.shape[0]) if rows is None else np.asarray(rows)
    shared = sg = None
    if layer.shared_down_proj is not None:
        shared = (to_u16(layer.shared_gate_proj), to_u16(layer.shared_up_proj), to_u16(layer.shared_down_proj))
        sg = oracle.shared_gate(np.ascontiguousarray(xin[sel]), to_u16(layer.shared_expert_gate))
    want = oracle_experts(oracle, np.ascontiguousarray(xin[sel]), np.ascontiguousarray(idx[sel]),
                          np.ascontiguousarray(wts[sel]), host, shared, sg,
                          np.ascontiguousarray(x_bits[sel]) if norm else None)
    return want, idx, wts


def assert_layer_close(got_bits: np.ndarray, want_bits: np.ndarray, x_bits: np.ndarray | None, what: str = "") -> None:
    """Output bar of a MoE block.  Without a residual (x_bits None):
    assert_close_bf16.  With one (out = bf16(h + moe)): every element within
    1e-2 of its row's MoE magnitude plus one bf16 ulp of the output for the
    final residual rounding."""
    if x_bits is None:
        assert_close_bf16(got_bits, want_bits, what=what)
        return
    got, exp_, h = bf16_f32(got_bits), bf16_f32(want_bits), bf16_f32(x_bits)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    moe_scale = np.abs(exp_ - h).max(axis=1, keepdims=True)
    excess = np.abs(got - exp_) - (1e-2 * moe_scale + 2.0 ** -7 * np.abs(exp_))
    worst = np.unravel_index(int(np.argmax(excess)), excess.shape)
    print(f"{what}: worst excess {excess.max():.3e} at {worst}, exact {float((got == exp_).mean()):.3f}")
    assert excess.max() <= 0, f"{what}: element {worst} off by {np.abs(got - exp_)[worst]:.3e}"


def resident_fixture_words():
    """The input of the reference's resident-row fixture
    (edge35b/test_gpu_resident_experts.py:14-20): 32 tiles of bf16 bits,
    every fourth with exponents 0..127 (does not fit the tile codec), the
    others within 8 exponents."""
    import numpy as np
    import torch

    gen = torch.Generator().manual_seed(7091)
    words = torch.randint(0, 128, (32, 256), generator=gen, dtype=torch.int32)
    words |= torch.randint(0, 2, words.shape, generator=gen, dtype=torch.int32) << 15
    exponents = 118 + torch.randint(0, 8, words.shape, generator=gen, dtype=torch.int32)
    exponents[1::4] = torch.arange(256) % 128
    words |= exponents << 7
    return words.to(torch.int16).numpy().view(np.uint16)
