"""Pins the CPU oracle (oracle/lro.c) before anything is checked against it.

- Expert arithmetic: bit-exact against golden vectors produced by the
  reference's own edge35b/cpu_experts.c (tests/golden/make_golden.py), and
  live against oracle/_ref/libcpu_experts.so where it is built; planted
  mistakes (gate/up swapped, wrong token) must break the match.
- exp(): within 1 ulp of the correctly rounded exponential.
- Bucketing: brute force in the shape of edge35b/block_experts.py:102-121
  (a dict of per-expert lists, sorted), plus invariants.
- Combine: closed forms where the bf16 rounding order decides the answer.
- Router / shared gate / RMSNorm: against torch CPU (a library) on the
  Transformers formulas; indices exactly on tokens without a top-8 boundary
  near-tie, values within one bf16 ulp.
"""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

GOLDEN_SEED = 20261201


def _golden(oracle):
    from pathlib import Path

    return np.load(Path(__file__).resolve().parent / "golden" / "cpu_experts_golden.npz")


def _experts(oracle, count, stream0):
    gu = [oracle.normal_bf16((1024, 2048), GOLDEN_SEED, stream0 + 2 * e, 0.02) for e in range(count)]
    dn = [oracle.normal_bf16((2048, 512), GOLDEN_SEED, stream0 + 2 * e + 1, 0.02) for e in range(count)]
    return gu, dn


def _digest(arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


# ---- expert arithmetic ----------------------------------------------------------

def test_expert_rows_match_reference_golden(oracle):
    g = _golden(oracle)
    gu, dn = _experts(oracle, 8, 100)
    hidden = oracle.normal_bf16((2048,), GOLDEN_SEED, 1, 1.0)
    assert _digest([*gu, *dn, hidden]) == bytes(g["rows8_sha256"]).decode(), "generator drifted"
    np.testing.assert_array_equal(oracle.expert_rows(gu, dn, hidden), g["rows8_output"])
    np.testing.assert_array_equal(oracle.expert_rows(gu[2:5], dn[2:5], hidden), g["rows3_output"])


def test_expert_block_rows_match_reference_golden(oracle):
    g = _golden(oracle)
    gu, dn = _experts(oracle, 16, 300)
    tokens = oracle.normal_bf16((4, 2048), GOLDEN_SEED, 2, 1.0)
    assert _digest([*gu, *dn, tokens]) == bytes(g["block16_sha256"]).decode()
    out = oracle.expert_block_rows(gu, dn, tokens, g["block16_token_ids"])
    np.testing.assert_array_equal(out, g["block16_output"])


def test_expert_rows_special_values_golden(oracle):
    g = _golden(oracle)
    gu, dn = _experts(oracle, 2, 500)
    gu[0][:, :64] = 0
    gu[1][5] = 0x8000
    np.testing.assert_array_equal(oracle.expert_rows(gu, dn, g["special_hidden"]), g["special_output"])


def test_planted_mistakes_break_the_golden(oracle):
    g = _golden(oracle)
    gu, dn = _experts(oracle, 8, 100)
    hidden = oracle.normal_bf16((2048,), GOLDEN_SEED, 1, 1.0)
    # gate and up halves swapped
    swapped = [np.ascontiguousarray(np.concatenate([a[512:], a[:512]])) for a in gu]
    assert not np.array_equal(oracle.expert_rows(swapped, dn, hidden), g["rows8_output"])
    # down applied transposed-in-memory (rows of the wrong matrix)
    transposed = [np.ascontiguousarray(d.reshape(512, 2048).T.reshape(2048, 512)) for d in dn]
    assert not np.array_equal(oracle.expert_rows(gu, transposed, hidden), g["rows8_output"])
    # block rows fed the wrong token
    bgu, bdn = _experts(oracle, 16, 300)
    tokens = oracle.normal_bf16((4, 2048), GOLDEN_SEED, 2, 1.0)
    wrong = (g["block16_token_ids"] + 1) % 4
    assert not np.array_equal(oracle.expert_block_rows(bgu, bdn, tokens, wrong), g["block16_output"])


def test_expert_rows_match_reference_live(oracle):
    if oracle.reference() is None:
        pytest.skip("reference kernel not built (needs /root/reference)")
    for seed in (3, 4):
        gu = [oracle.normal_bf16((1024, 2048), seed, 10 + e, 0.02) for e in range(8)]
        dn = [oracle.normal_bf16((2048, 512), seed, 30 + e, 0.02) for e in range(8)]
        hidden = oracle.normal_bf16((2048,), seed, 7, 1.0)
        ref = oracle.reference_expert_rows(gu, dn, hidden, threads=2)
        np.testing.assert_array_equal(oracle.expert_rows(gu, dn, hidden), ref)
        tokens = oracle.normal_bf16((16, 2048), seed, 8, 1.0)
        ids = np.arange(8, dtype=np.int32) * 2 + 1
        ref = oracle.reference_expert_block_rows(gu, dn, tokens, ids, threads=2)
        np.testing.assert_array_equal(oracle.expert_block_rows(gu, dn, tokens, ids), ref)


def test_reference_workers_match_oracle_live(oracle):
    """The reference's persistent CPU workers (packed_workers.cpp) produce the
    oracle's expert rows bit for bit, and its packed_plan orders routes like
    the oracle's bucketing (ascending expert id, slot kept)."""
    import ctypes as C

    ref = oracle.reference_workers()
    if ref is None:
        pytest.skip("reference workers not built (needs /root/reference)")
    gu = [oracle.normal_bf16((1024, 2048), 5, 50 + e, 0.02) for e in range(8)]
    dn = [oracle.normal_bf16((2048, 512), 5, 70 + e, 0.02) for e in range(8)]
    hidden = oracle.normal_bf16((2048,), 5, 9, 1.0)
    workers = ref.packed_workers_create(3)
    try:
        for count in (8, 5):
            out = np.zeros((8, 2048), dtype=np.uint16)
            gates = (C.c_void_p * 8)(*[g.ctypes.data for g in gu])
            downs = (C.c_void_p * 8)(*[d.ctypes.data for d in dn])
            ref.packed_workers_submit(workers, gates, downs, hidden.ctypes.data, out.ctypes.data, count)
            ref.packed_workers_wait(workers)
            np.testing.assert_array_equal(out[:count], oracle.expert_rows(gu[:count], dn[:count], hidden))
    finally:
        ref.packed_workers_destroy(workers)
    ids = np.array([200, 3, 77, 150, 9, 31, 255, 0], dtype=np.int64)
    table = np.zeros(32, dtype=np.int64)
    last_seen = np.full(256, -4, dtype=np.int32)
    experts = np.zeros(8, dtype=np.int32)
    recent = np.zeros(8, dtype=np.uint8)
    ref.packed_plan(ids.ctypes.data, table.ctypes.data, last_seen.ctypes.data, 1, experts.ctypes.data,
                    recent.ctypes.data)
    plan = oracle.bucket(ids[None])
    np.testing.assert_array_equal(experts, plan["expert"][:8])
    np.testing.assert_array_equal(table.reshape(8, 4)[:, 2], plan["pair_slot"])


def test_expert_pair_against_float64_math(oracle):
    """The bf16-rounded SwiGLU stays within bf16 rounding of the exact math."""
    gu, dn = _experts(oracle, 1, 700)
    x = oracle.normal_bf16((2048,), GOLDEN_SEED, 9, 1.0)
    y = oracle.bf16_to_f32(oracle.expert_rows(gu, dn, x)[0]).astype(np.float64)
    w = oracle.bf16_to_f32(gu[0]).astype(np.float64)
    d = oracle.bf16_to_f32(dn[0]).astype(np.float64)
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    gate, up = w[:512] @ xf, w[512:] @ xf
    act = gate / (1.0 + np.exp(-gate)) * up
    exact = d @ act
    assert np.abs(y - exact).max() <= 2e-2 * np.abs(exact).max()
    assert np.corrcoef(y, exact)[0, 1] > 0.9999


def test_expert_pair_zero_gate_gives_zero(oracle):
    gu = np.zeros((1024, 2048), dtype=np.uint16)
    gu[512:] = oracle.normal_bf16((512, 2048), 1, 1, 0.02)
    dn = oracle.normal_bf16((2048, 512), 1, 2, 0.02)
    x = oracle.normal_bf16((2048,), 1, 3, 1.0)
    assert not oracle.expert_rows([gu], [dn], x).any() or np.all(
        oracle.bf16_to_f32(oracle.expert_rows([gu], [dn], x)) == 0)


# ---- exp ----------------------------------------------------------------------------

def test_exp_within_one_ulp(oracle):
    xs = np.concatenate([np.linspace(-87.0, 88.72, 40001), np.linspace(-1, 1, 20001)]).astype(np.float32)
    mine = np.array([oracle.exp(v) for v in xs], dtype=np.float32)
    exact = np.exp(xs.astype(np.float64)).astype(np.float32)
    ulps = np.abs(mine.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert oracle.exp(0.0) == 1.0
    assert oracle.exp(-87.5) == 0.0
    assert oracle.exp(89.0) == float("inf")
    assert np.isnan(oracle.exp(float("nan")))


# ---- generator ----------------------------------------------------------------------

def test_generator_statistics_and_known_values(oracle):
    v = oracle.bf16_to_f32(oracle.normal_bf16((1 << 20,), 5, 6, 0.5)).astype(np.float64)
    assert abs(v.mean()) < 2e-3
    assert abs(v.std() - 0.5) < 5e-3
    # index-addressable: a slice equals the same range of a longer draw
    long = oracle.normal_bf16((1000,), 5, 6, 0.5)
    np.testing.assert_array_equal(oracle.normal_bf16((100,), 5, 6, 0.5, first=900), long[900:])
    # splitmix64 of key + 0 for seed 0 stream 0: key = splitmix64(0)
    first = oracle.normal_bf16((4,), 0, 0, 1.0)
    assert first.tolist() == oracle.normal_bf16((4,), 0, 0, 1.0).tolist()


# ---- bucketing --------------------------------------------------------------------

def _brute_bucket(indices):
    """block_experts.py:102-121 shape: dict of per-expert (token, slot) lists."""
    routes = {}
    for token, top_k in enumerate(indices.tolist()):
        for slot, expert in enumerate(top_k):
            routes.setdefault(expert, []).append((token, slot))
    experts = sorted(routes)
    pairs, inverse = [], [[] for _ in range(len(indices))]
    for expert in experts:
        for token, slot in routes[expert]:
            inverse[token].append(len(pairs))
            pairs.append((token, slot))
    return experts, pairs, inverse


@pytest.mark.parametrize("tokens", [1, 3, 8, 16, 100])
def test_bucket_matches_brute_force(oracle, tokens):
    rng = np.random.default_rng(tokens)
    indices = np.stack([rng.choice(256, 8, replace=False) for _ in range(tokens)]).astype(np.int64)
    plan = oracle.bucket(indices)
    experts, pairs, inverse = _brute_bucket(indices)
    assert plan["unique"] == len(set(indices.ravel().tolist())) == len(experts)
    assert plan["expert"].tolist() == experts
    assert list(zip(plan["pair_token"].tolist(), plan["pair_slot"].tolist())) == pairs
    assert plan["route_pair"].tolist() == inverse
    # invariants: every (token, slot) exactly once; route order ascending by expert
    assert sorted(pairs) == [(t, s) for t in range(tokens) for s in range(8)]
    for t in range(tokens):
        chosen = [indices[t, pairs[p][1]] for p in inverse[t]]
        assert chosen == sorted(chosen)


def test_bucket_rejects_bad_routes(oracle):
    with pytest.raises(ValueError):
        oracle.bucket(np.array([[0, 1, 2, 3, 4, 5, 6, 256]], dtype=np.int64))
    with pytest.raises(ValueError):
        oracle.bucket(np.array([[0, 1, 2, 3, 4, 5, 6, 6]], dtype=np.int64))


# ---- combine --------------------------------------------------------------------------

def _bf(values):
    from oracle import oracle as O

    return O.f32_to_bf16(np.asarray(values, dtype=np.float32))


def test_combine_closed_forms(oracle):
    indices = np.array([[7, 3, 9, 1, 200, 5, 6, 4]], dtype=np.int64)
    plan = oracle.bucket(indices)
    ones = _bf(np.ones((1, 8)))
    # y rows in pair (ascending expert) order: 256, 1, -256, then zeros
    y = np.zeros((8, 2048), dtype=np.uint16)
    y[0], y[1], y[2] = _bf(256.0), _bf(1.0), _bf(-256.0)
    out = oracle.bf16_to_f32(oracle.combine(y, plan["route_pair"], plan["pair_slot"], ones))
    # ascending order: bf16(256 + 1) = 256, then 256 - 256 = 0
    assert np.all(out == 0.0)
    # any other order would keep the 1: e.g. (256 - 256) + 1
    y2 = y.copy()
    y2[1], y2[2] = y[2], y[1]
    assert np.all(oracle.bf16_to_f32(oracle.combine(y2, plan["route_pair"], plan["pair_slot"], ones)) == 1.0)
    # a single non-zero weight returns bf16(y * w)
    rng = np.random.default_rng(0)
    y3 = _bf(rng.normal(size=(8, 2048)))
    w = np.zeros((1, 8), dtype=np.float32)
    w[0, 4] = 0.3125  # slot 4 routes expert 200, the last in ascending order
    out = oracle.combine(y3, plan["route_pair"], plan["pair_slot"], _bf(w))
    np.testing.assert_array_equal(out[0], _bf(oracle.bf16_to_f32(y3[7]) * np.float32(0.3125)))
    # shared expert and residual are added after the routed sum
    sg = _bf([0.5])
    ysh = _bf(np.full((1, 2048), 2.0))
    res = _bf(np.full((1, 2048), 10.0))
    out = oracle.combine(np.zeros_like(y3), plan["route_pair"], plan["pair_slot"], _bf(w), ysh, sg, res)
    assert np.all(oracle.bf16_to_f32(out) == 11.0)


# ---- router, shared gate, RMSNorm against torch CPU ------------------------------------

def _torch_bf16(bits):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def test_router_against_torch(oracle):
    tokens = 96
    x = oracle.normal_bf16((tokens, 2048), 11, 1, 1.0)
    router = oracle.normal_bf16((256, 2048), 11, 2, 0.02)
    logits, indices, weights = oracle.route(x, router)
    xt, wt = _torch_bf16(x), _torch_bf16(router)
    t_logits = torch.nn.functional.linear(xt, wt)
    probs = torch.softmax(t_logits, dtype=torch.float, dim=-1)
    top, t_idx = torch.topk(probs, 8, dim=-1)
    top = (top / top.sum(dim=-1, keepdim=True)).to(torch.bfloat16)
    ours = oracle.bf16_to_f32(logits)
    theirs = t_logits.float().numpy()
    ulp = np.abs(ours - theirs) / np.maximum(np.abs(theirs), 1e-3)
    assert (ours == theirs).mean() > 0.99 and ulp.max() <= 2 ** -7
    checked = 0
    for t in range(tokens):
        row = np.sort(ours[t])[::-1]
        if row[7] - row[8] <= 2 * np.abs(row[7]) * 2 ** -8:
            continue  # boundary within two bf16 ulps: torch's order is not pinned there
        checked += 1
        assert sorted(indices[t].tolist()) == sorted(t_idx[t].tolist())
        mine = dict(zip(indices[t].tolist(), oracle.bf16_to_f32(weights[t]).tolist()))
        ref = dict(zip(t_idx[t].tolist(), top[t].float().tolist()))
        for e in mine:
            assert abs(mine[e] - ref[e]) <= abs(ref[e]) * 2 ** -7
    assert checked > tokens // 2
    assert np.allclose(oracle.bf16_to_f32(weights).sum(axis=1), 1.0, atol=2e-2)
    # ties break toward the lower expert id and indices come out in rank order
    flat = np.zeros((1, 2048), dtype=np.uint16)
    _, idx, w = oracle.route(flat, router)
    assert idx[0].tolist() == list(range(8))
    assert np.all(oracle.bf16_to_f32(w) == np.float32(0.125))


def test_route_logits_against_torch(oracle):
    """Top-8 on given logits (the decode layer's logits_in path) against
    torch CPU softmax + topk + renormalisation on bf16 Zipf(1.1) Gumbel
    logits, the headline workload's routing input."""
    tokens = 256
    rng = np.random.default_rng(77)
    ranks = rng.permutation(256) + 1
    raw = (-1.1 * np.log(ranks)[None, :] + rng.gumbel(size=(tokens, 256))).astype(np.float32)
    logits = oracle.f32_to_bf16(raw)
    indices, weights = oracle.route_logits(logits)
    lt = _torch_bf16(logits)
    probs = torch.softmax(lt.float(), dim=-1)
    top, t_idx = torch.topk(probs, 8, dim=-1)
    top = (top / top.sum(dim=-1, keepdim=True)).to(torch.bfloat16).float().numpy()
    values = oracle.bf16_to_f32(logits)
    checked = 0
    for t in range(tokens):
        row = np.sort(values[t])[::-1]
        if len(set(row[:9].tolist())) < 9:
            continue  # equal logits among the top 9: torch's order is not pinned there
        checked += 1
        assert indices[t].tolist() == t_idx[t].tolist()   # rank order, not just the set
        got = oracle.bf16_to_f32(weights[t])
        assert np.all(np.abs(got - top[t]) <= np.abs(top[t]) * 2 ** -8), (t, got, top[t])
    assert checked > tokens // 2
    # equal logits: the lower expert id first, uniform weights
    idx, w = oracle.route_logits(np.full((1, 256), 0x3F80, dtype=np.uint16))
    assert idx[0].tolist() == list(range(8)) and np.all(oracle.bf16_to_f32(w) == np.float32(0.125))
    # -0 ranks with +0; a larger logit wins over a lower id
    row = np.zeros((1, 256), dtype=np.uint16)
    row[0, 3] = 0x8000
    row[0, 200] = 0x3F80
    idx, _ = oracle.route_logits(row)
    assert idx[0].tolist() == [200, 0, 1, 2, 3, 4, 5, 6]


def test_shared_gate_and_rmsnorm_against_torch(oracle):
    x = oracle.normal_bf16((32, 2048), 12, 1, 1.0)
    gate_w = oracle.normal_bf16((2048,), 12, 2, 0.02)
    sg = oracle.bf16_to_f32(oracle.shared_gate(x, gate_w))
    xt = _torch_bf16(x)
    ref = torch.sigmoid(torch.nn.functional.linear(xt, _torch_bf16(gate_w)[None])).float().numpy()[:, 0]
    assert np.abs(sg - ref).max() <= 2 ** -8
    norm_w = oracle.normal_bf16((2048,), 12, 3, 0.02)
    ours = oracle.bf16_to_f32(oracle.rmsnorm(x, norm_w, 1e-6))
    xf = xt.float()
    theirs = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)) * (1.0 + _torch_bf16(norm_w).float())
    theirs = theirs.to(torch.bfloat16).float().numpy()
    assert (ours == theirs).mean() > 0.99
    assert np.abs(ours - theirs).max() <= np.abs(theirs).max() * 2 ** -7


def test_moe_layer_against_float32_torch(oracle):
    """Whole block (router + experts + shared + combine + norm + residual)
    against an fp32 torch evaluation of the Transformers formulas."""
    tokens = 4
    rng = np.random.default_rng(5)
    gu = [None] * 256
    dn = [None] * 256
    x = oracle.normal_bf16((tokens, 2048), 13, 1, 1.0)
    router = oracle.normal_bf16((256, 2048), 13, 2, 0.02)
    norm_w = oracle.normal_bf16((2048,), 13, 3, 0.02)
    shared = tuple(oracle.normal_bf16(s, 13, 4 + i, 0.02) for i, s in
                   enumerate([(512, 2048), (512, 2048), (2048, 512), (2048,)]))
    _, idx, _ = oracle.route(oracle.rmsnorm(x, norm_w), router)
    filler = np.zeros(1, dtype=np.uint16)
    for e in range(256):
        if e in idx:
            gu[e] = oracle.normal_bf16((1024, 2048), 13, 100 + e, 0.02)
            dn[e] = oracle.normal_bf16((2048, 512), 13, 400 + e, 0.02)
        else:
            gu[e] = dn[e] = filler
    out, indices, weights = oracle.moe_layer(x, router, gu, dn, shared, norm_w)
    assert np.array_equal(indices, idx)
    f = lambda a: torch.from_numpy(oracle.bf16_to_f32(a).astype(np.float32))  # noqa: E731
    xf = f(x)
    n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * (1 + f(norm_w))
    probs = torch.softmax(n @ f(router).T, dim=-1)
    top, t_idx = torch.topk(probs, 8, dim=-1)
    top = top / top.sum(-1, keepdim=True)
    routed = torch.zeros_like(n)
    for t in range(tokens):
        for k in range(8):
            e = int(t_idx[t, k])
            w = f(gu[e])
            h = n[t] @ w.T
            act = torch.nn.functional.silu(h[:512]) * h[512:]
            routed[t] += top[t, k] * (f(dn[e]) @ act)
    g, u, d, sgw = (f(s) for s in shared)
    sh = (torch.nn.functional.silu(n @ g.T) * (n @ u.T)) @ d.T
    expected = xf + routed + torch.sigmoid(n @ sgw[:, None]) * sh
    got = torch.from_numpy(oracle.bf16_to_f32(out))
    moe_got, moe_exp = got - xf, expected - xf
    assert (moe_got - moe_exp).abs().max() <= 3e-2 * moe_exp.abs().max()


# ---- lossless BF16 tile codec ---------------------------------------------------

def _fitting_tiles(rng, count):
    """Tiles whose 7-bit exponent fields lie in an 8-value window."""
    base = rng.integers(0, 121, size=(count, 1))
    field = base + rng.integers(0, 8, size=(count, 256))
    sign = rng.integers(0, 2, size=(count, 256))
    low = rng.integers(0, 256, size=(count, 256))
    return ((sign << 15) | (field << 8) | low).astype(np.uint16)


def test_codec_round_trips_every_bf16_pattern(oracle):
    # 256 consecutive patterns share bits 15..8, so each of these tiles fits.
    values = np.arange(65536, dtype=np.uint16).reshape(256, 256)
    packed, bases, misfit = oracle.codec_pack(values)
    assert misfit == 0
    np.testing.assert_array_equal(bases[:, 0], (np.arange(256) & 127).astype(np.uint8))
    np.testing.assert_array_equal(oracle.codec_unpack(packed, bases), values)
    # Shuffled, most tiles span more than 8 fields: exactly those are marked.
    shuffled = np.random.default_rng(5).permutation(values.ravel()).reshape(64, 1024)
    packed, bases, misfit = oracle.codec_pack(shuffled)
    fields = ((shuffled.reshape(64, 4, 256) >> 8) & 127).astype(np.int32)
    wide = fields.max(axis=2) - fields.min(axis=2) > 7
    assert misfit == int(wide.sum()) > 0
    np.testing.assert_array_equal(bases == 255, wide)
    restored = oracle.codec_unpack(packed, bases).reshape(64, 4, 256)
    np.testing.assert_array_equal(restored[~wide], shuffled.reshape(64, 4, 256)[~wide])


def test_codec_matches_the_reference_packer(oracle):
    ref = oracle.reference_tile_codec()
    if ref is None:
        pytest.skip("the reference's cpu_bf16_reads.h is not present")
    rng = np.random.default_rng(11)
    tiles = np.concatenate([_fitting_tiles(rng, 48), rng.integers(0, 65536, (16, 256), dtype=np.uint16),
                            np.full((1, 256), 0x3F80, dtype=np.uint16),          # one field, no sign
                            np.full((1, 256), 0x8000, dtype=np.uint16),          # negative zeros
                            np.tile(np.array([0x7F80, 0x0001], dtype=np.uint16), (1, 128))])  # inf and a denormal: 127 fields apart
    n = tiles.shape[0]
    ref_packed = np.zeros((n, 384), dtype=np.uint8)
    ref_bases = np.zeros(n, dtype=np.uint8)
    encoded = ref.ref_pack_cpu_read_tiles(tiles.ctypes.data, ref_packed.ctypes.data, ref_bases.ctypes.data, n)
    packed, bases, misfit = oracle.codec_pack(tiles)
    assert encoded == n - misfit
    np.testing.assert_array_equal(bases[:, 0], ref_bases)
    # Value k of the reference tile: low byte at k, code in nibble k of bytes
    # 256..383 (index order).  Here, for k = 8g + 32s + j: low byte at
    # 64(s/2) + 16g + 8(s%2) + j, code in nibble j/4 of byte
    # 256 + 64(s/4) + 16g + 4(s%4) + j%4.
    k = np.arange(256)
    g, s, j = (k >> 3) & 3, k >> 5, k & 7
    low_at = 64 * (s >> 1) + 16 * g + 8 * (s & 1) + j
    code_at = 256 + 64 * (s >> 2) + 16 * g + 4 * (s & 3) + (j & 3)
    # Every byte of the tile is used once (low bytes) or twice (code nibbles).
    assert sorted(low_at.tolist()) == list(range(256))
    assert np.all(np.bincount(code_at - 256, minlength=128) == 2)
    for t in np.flatnonzero(ref_bases != 255):
        ref_low = ref_packed[t, :256]
        ref_code = (ref_packed[t, 256 + k // 2] >> (4 * (k & 1))) & 15
        ours = packed[t, 0]
        np.testing.assert_array_equal(ours[low_at], ref_low)
        np.testing.assert_array_equal((ours[code_at] >> (4 * (j >> 2))) & 15, ref_code)
    assert (ref_bases == 255).sum() >= 17   # the random tiles and the inf/denormal tile


def test_codec_reference_order_equals_the_reference_packer(oracle):
    """codec_pack_reference_order gives the reference packer's bytes for
    every tile that fits (the reference leaves the others unspecified)."""
    ref = oracle.reference_tile_codec()
    if ref is None:
        pytest.skip("the reference's cpu_bf16_reads.h is not present")
    rng = np.random.default_rng(12)
    tiles = np.concatenate([_fitting_tiles(rng, 40), rng.integers(0, 65536, (8, 256), dtype=np.uint16)])
    n = len(tiles)
    ref_packed = np.zeros((n, 384), dtype=np.uint8)
    ref_bases = np.zeros(n, dtype=np.uint8)
    ref.ref_pack_cpu_read_tiles(tiles.ctypes.data, ref_packed.ctypes.data, ref_bases.ctypes.data, n)
    packed, bases, misfit = oracle.codec_pack_reference_order(tiles)
    np.testing.assert_array_equal(bases[:, 0], ref_bases)
    fit = ref_bases != 255
    assert misfit == int((~fit).sum()) >= 8
    np.testing.assert_array_equal(packed[fit, 0], ref_packed[fit])


def test_compact_rows_reference_fixture(oracle):
    from helpers import resident_fixture_words

    bits = resident_fixture_words()
    data, headers, encoded, fallback = oracle.compact_rows(bits)
    # The reference fixture's own expectation (test_gpu_resident_experts.py:22).
    assert (encoded, fallback) == (24, 8)
    assert data.nbytes == 24 * 384 + 8 * 512 and headers.dtype == np.uint32
    # Raw tiles 1, 5, 9, ...: header base 255, later headers count them.
    assert [h & 255 for h in headers[1::4].tolist()] == [255] * 8
    assert [h >> 8 for h in headers.tolist()] == [(t + 2) // 4 for t in range(32)]
    np.testing.assert_array_equal(oracle.decode_compact_rows(data, headers), bits)
    # Nothing to gain: the raw bytes and no headers.
    data, headers, encoded, fallback = oracle.compact_rows(np.arange(512, dtype=np.uint16) * 127)
    assert headers is None and (encoded, fallback) == (0, 2) and data.nbytes == 1024


def test_escape_codec_reference_fixture(oracle):
    """edge35b/test_freetoken_packed_transfer.py:15-25: every bf16 pattern
    round-trips; a bank plan keeps the all-patterns row raw (it escapes far
    more than 1%) and packs the constant rows without escapes."""
    values = np.arange(65536, dtype=np.uint16)
    base, escapes = oracle.escape_window(values)
    packed = oracle.escape_pack(values, base, escapes)
    assert packed.size == oracle.escape_row_bytes(values.size, escapes)
    np.testing.assert_array_equal(oracle.escape_restore(packed, values.size, base, escapes), values)
    common = np.full(values.shape, 0x3F80, dtype=np.uint16)
    plans, size = oracle.escape_plan(np.stack([common, values, common]))
    assert plans[1] is None
    assert plans[0][2] == 0
    assert plans[2][0] == oracle.escape_row_bytes(common.size, 0)
    assert size == 2 * oracle.escape_row_bytes(common.size, 0)


def test_escape_codec_closed_forms(oracle):
    # 1.0 (exponent 127): the first window holding it starts at 112; delta 15.
    one = np.full(64, 0x3F80, dtype=np.uint16)
    assert oracle.escape_window(one) == (112, 0)
    packed = oracle.escape_pack(one, 112, 0)
    assert np.all(packed[:64] == 0) and np.all(packed[64:96] == 0xFF)
    # Every pattern: the 16 exponents 0..15 hold 16 x 128 x 2 values, tied
    # with every other window; the first one wins.
    assert oracle.escape_window(np.arange(65536, dtype=np.uint16)) == (0, 65536 - 16 * 256)
    # One value escapes below the window, one above: indices in order.
    row = np.full(32, 0x4000, dtype=np.uint16)     # 2.0, exponent 128
    row[5], row[20] = 0x0001, 0x7F80               # exponent 0, +inf (255)
    base, escapes = oracle.escape_window(row)
    assert (base, escapes) == (113, 2)
    packed = oracle.escape_pack(row, base, escapes)
    assert packed[48:56].view("<i4").tolist() == [5, 20]
    assert packed[56:60].view("<u2").tolist() == [0x0001, 0x7F80]
    np.testing.assert_array_equal(oracle.escape_restore(packed, 32, base, escapes), row)


def test_codec_closed_forms(oracle):
    # 1.0 everywhere: field 63, no sign, low byte 0x80; code 0 in every nibble.
    one = np.full((1, 256), 0x3F80, dtype=np.uint16)
    packed, bases, misfit = oracle.codec_pack(one)
    assert misfit == 0 and bases[0, 0] == 63
    assert np.all(packed[0, 0, :256] == 0x80) and np.all(packed[0, 0, 256:] == 0)
    # -2.0 (0xC000): field 64, sign set -> code 8 in every nibble.
    packed, bases, _ = oracle.codec_pack(np.full((1, 256), 0xC000, dtype=np.uint16))
    assert bases[0, 0] == 64 and np.all(packed[0, 0, 256:] == 0x88) and np.all(packed[0, 0, :256] == 0)
