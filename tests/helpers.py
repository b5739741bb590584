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


def oracle_experts(oracle, x_bits: np.ndarray, indices: np.ndarray, weights_bits: np.ndarray, host: HostExperts,
                   shared=None, sg_bits=None, residual_bits=None) -> np.ndarray:
    """Routed experts (+ shared, + residual) through the oracle."""
    plan = oracle.bucket(indices)
    tokens = x_bits.shape[0]
    y = np.zeros((8 * tokens, 2048), dtype=np.uint16)
    for u, e in enumerate(plan["expert"].tolist()):
        gu, dn = host(e)
        for p in range(plan["offset"][u], plan["offset"][u + 1]):
            t = plan["pair_token"][p]
            y[p] = oracle.expert_pair(gu[:512], gu[512:], dn, x_bits[t])
    y_shared = None
    if shared is not None:
        g, u_, d = shared
        y_shared = np.stack([oracle.expert_pair(g, u_, d, x_bits[t]) for t in range(tokens)])
    return oracle.combine(y, plan["route_pair"], plan["pair_slot"], np.ascontiguousarray(weights_bits),
                          y_shared, sg_bits, residual_bits)


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
