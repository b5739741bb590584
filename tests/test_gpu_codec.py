"""Lossless BF16 tile codec on an MI355X: packing against the oracle, and
decode layers reading codec experts against the same layers reading raw
rows.

Bar: packed bytes, tile bases and misfit counts bit-identical to the oracle
(oracle/lro.c lro_codec_pack, itself checked against the reference's tile
packer in tests/test_oracle.py); unpacking restores the raw bits; a decode
layer or chain reading codec experts gives bit-identical outputs and routes
to the same call reading the raw rows (each MFMA sees the same operands in
the same order).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import resident_fixture_words, to_u16

pytestmark = pytest.mark.gpu


def _mixed_matrix(rows: int, cols: int, seed: int) -> np.ndarray:
    """bf16 bits whose tiles mostly fit the codec; every 5th tile spans the
    whole exponent range (does not fit)."""
    rng = np.random.default_rng(seed)
    tiles = rows * cols // 256
    base = rng.integers(0, 121, size=(tiles, 1))
    field = base + rng.integers(0, 8, size=(tiles, 256))
    bits = (rng.integers(0, 2, size=(tiles, 256)) << 15) | (field << 8) | rng.integers(0, 256, size=(tiles, 256))
    bits[::5] = rng.integers(0, 65536, size=bits[::5].shape)
    return bits.astype(np.uint16).reshape(rows, cols)


@pytest.mark.parametrize("rows,cols", [(64, 2048), (200, 512), (3, 256)])
def test_codec_pack_matches_oracle(device, oracle, rows, cols):
    from lightreason_amd.moe import codec_pack, codec_unpack

    bits = _mixed_matrix(rows, cols, seed=rows + cols)
    w = torch.from_numpy(bits.view(np.int16)).to(device).view(torch.bfloat16)
    tiles = rows * cols // 256
    packed = torch.full((tiles * 384,), 0x5A, dtype=torch.uint8, device=device)
    bases = torch.full((tiles,), 0x5A, dtype=torch.uint8, device=device)
    misfit = torch.zeros(1, dtype=torch.int64, device=device)
    codec_pack(w, packed, bases, misfit)
    back = codec_unpack(packed, bases, rows, cols)
    torch.cuda.synchronize()
    o_packed, o_bases, o_misfit = oracle.codec_pack(bits)
    assert int(misfit.item()) == o_misfit > 0
    np.testing.assert_array_equal(bases.cpu().numpy(), o_bases.ravel())
    np.testing.assert_array_equal(packed.cpu().numpy(), o_packed.ravel())
    np.testing.assert_array_equal(to_u16(back), oracle.codec_unpack(o_packed, o_bases))


@pytest.fixture(scope="module")
def codec_bank(model):
    from lightreason_amd.moe import CodecBank

    layer = model.layers[0]
    bank = CodecBank(model.bank, [(layer.shared_gate_proj, layer.shared_up_proj, layer.shared_down_proj)])
    torch.cuda.synchronize()
    return bank


def test_codec_bank_round_trips_experts(model, codec_bank):
    from lightreason_amd.moe import CODEC_DN_PACKED, CODEC_GU_BASES, CODEC_GU_PACKED, CODEC_MISFIT, codec_unpack

    # Gaussian weights: about 1% of tiles hold a value too small for their
    # tile's window; every expert has some, and most units still read packed.
    assert int((codec_bank.misfit[0] > 0).sum()) == 257
    assert 0.5 < codec_bank.packed_fraction < 1.0
    blob = codec_bank.blob[0]
    gu0 = CODEC_GU_PACKED + CODEC_DN_PACKED
    for e in (0, 77, 255, 256):
        if e == 256:
            layer = model.layers[0]
            gate_up = torch.cat([layer.shared_gate_proj, layer.shared_up_proj])
            down = layer.shared_down_proj
        else:
            gate_up, down = model.bank.expert(0, e)
        block = blob[e]
        gu = codec_unpack(block[:CODEC_GU_PACKED], block[gu0:gu0 + CODEC_GU_BASES], 1024, 2048)
        dn = codec_unpack(block[CODEC_GU_PACKED:gu0], block[gu0 + CODEC_GU_BASES:], 2048, 512)
        torch.cuda.synchronize()
        # Tiles that fit restore exactly; the others decode to 0xffff.
        misfit = 0
        for got, want, bases, cols in ((gu, gate_up, block[gu0:gu0 + CODEC_GU_BASES], 2048),
                                       (dn, down, block[gu0 + CODEC_GU_BASES:gu0 + CODEC_GU_BASES + 4096], 512)):
            fits = (bases != CODEC_MISFIT).view(-1, cols // 256, 1).expand(-1, -1, 256).reshape(-1, cols)
            g16, w16 = got.view(torch.int16), want.reshape(-1, cols).view(torch.int16)
            assert torch.equal(g16[fits], w16[fits]), e
            assert bool((g16[~fits] == -1).all()), e
            misfit += int((~fits[:, ::256]).sum())
        assert int(codec_bank.misfit[0, e]) == misfit, e


def _layer_pair(model, codec_bank, norm: bool):
    from lightreason_amd.moe import LayerWeights

    base = model.layers[0]
    raw = LayerWeights(**{**base.__dict__, "norm_weight": base.norm_weight if norm else None, "codec": None})
    packed = LayerWeights(**{**raw.__dict__, "codec": codec_bank.table(0)})
    return raw, packed


@pytest.mark.parametrize("tokens", [1, 8, 16])
@pytest.mark.parametrize("norm,logits", [(True, False), (False, True)])
def test_codec_layer_equals_raw_layer(model, codec_bank, tokens, norm, logits):
    from lightreason_amd.moe import Workspace, moe_layer

    raw, packed = _layer_pair(model, codec_bank, norm)
    x = model.hidden(tokens, step=700 + tokens)
    lg = None
    if logits:
        lg = (x.float() @ raw.router.float().T).to(torch.bfloat16)
    ws = Workspace(x.device, tokens)
    results = []
    for layer in (raw, packed, raw):
        idx = torch.empty((tokens, 8), dtype=torch.int64, device=x.device)
        out = moe_layer(x, layer, indices=idx, logits_in=lg, workspace=ws)
        results.append((out, idx))
    torch.cuda.synchronize()
    print(f"codec layer T={tokens} norm={norm} logits={logits}", flush=True)
    assert torch.equal(results[0][1], results[1][1])
    assert torch.equal(results[0][0].view(torch.int16), results[1][0].view(torch.int16))
    assert torch.equal(results[0][0].view(torch.int16), results[2][0].view(torch.int16))
    assert ws.status() == 0


def test_codec_mixed_raw_and_packed_experts(model, codec_bank):
    """Experts whose codec row is zero are read raw inside the same call."""
    from lightreason_amd.moe import LayerWeights, Workspace, moe_layer

    raw, packed = _layer_pair(model, codec_bank, True)
    table = codec_bank.table(0).clone()
    table[1::3] = 0          # every third routed expert raw
    table[256] = 0           # and the shared expert
    mixed = LayerWeights(**{**packed.__dict__, "codec": table})
    tokens = 8
    x = model.hidden(tokens, step=750)
    ws = Workspace(x.device, tokens)
    want = moe_layer(x, raw, workspace=ws)
    got = moe_layer(x, mixed, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("tokens,pattern", [(8, "ccc"), (16, "ccc"), (8, "crc"), (16, "rcr")])
def test_codec_chain_equals_raw_chain(model, codec_bank, tokens, pattern):
    """Chains of codec (c) and raw (r) layers: the codec kernel instance
    runs the raw layers too, whose codec rows are left from earlier layers."""
    from lightreason_amd.moe import Workspace, moe_chain

    raw, packed = _layer_pair(model, codec_bank, True)
    x = model.hidden(tokens, step=760 + tokens)
    ws = Workspace(x.device, tokens)
    idx_raw = torch.empty((3, tokens, 8), dtype=torch.int64, device=x.device)
    idx_pk = torch.empty_like(idx_raw)
    want = moe_chain(x, [raw] * 3, indices=idx_raw, workspace=ws)
    got = moe_chain(x, [packed if c == "c" else raw for c in pattern], indices=idx_pk, workspace=ws)
    print(f"codec chain T={tokens} {pattern}", flush=True)
    torch.cuda.synchronize()
    assert torch.equal(idx_raw, idx_pk)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert ws.status() == 0


@pytest.mark.parametrize("tokens", [8, 16])
@pytest.mark.parametrize("norm,logits", [(True, False), (False, True)])
def test_codec_layer_against_oracle(model, codec_bank, oracle, host_experts, tokens, norm, logits):
    """A decode layer reading codec experts (the codec instance runs from 8
    tokens up) against the oracle on the raw weights: routes bit-exact,
    output within the layer bar."""
    from helpers import assert_layer_close, oracle_layer_rows
    from lightreason_amd.moe import Workspace, moe_layer

    _, packed = _layer_pair(model, codec_bank, norm)
    x = model.hidden(tokens, step=780 + tokens)
    lg = (x.float() @ packed.router.float().T).to(torch.bfloat16) if logits else None
    ws = Workspace(x.device, tokens)
    idx = torch.empty((tokens, 8), dtype=torch.int64, device=x.device)
    wts = torch.empty((tokens, 8), dtype=torch.bfloat16, device=x.device)
    print(f"codec layer vs oracle T={tokens} norm={norm} logits={logits}", flush=True)
    out = moe_layer(x, packed, indices=idx, weights=wts, logits_in=lg, workspace=ws)
    torch.cuda.synchronize()
    assert ws.status() == 0
    xb = to_u16(x)
    want, o_idx, o_w = oracle_layer_rows(oracle, packed, xb, host_experts,
                                         logits_bits=None if lg is None else to_u16(lg))
    np.testing.assert_array_equal(idx.cpu().numpy(), o_idx)
    np.testing.assert_array_equal(to_u16(wts), o_w)
    assert_layer_close(to_u16(out), want, xb if norm else None, what=f"codec layer T={tokens}")


@pytest.mark.parametrize("tokens", [8, 16])
def test_codec_chain_against_oracle(model, codec_bank, oracle, host_experts, tokens):
    """Three chained codec layers (RMSNorm + residual): the chain equals
    successive codec layer calls bit for bit, and every layer matches the
    oracle applied to that layer's input."""
    from helpers import assert_layer_close, oracle_layer_rows
    from lightreason_amd.moe import Workspace, moe_chain, moe_layer

    _, packed = _layer_pair(model, codec_bank, True)
    x = model.hidden(tokens, step=790 + tokens)
    ws = Workspace(x.device, tokens)
    idx = torch.empty((3, tokens, 8), dtype=torch.int64, device=x.device)
    print(f"codec chain vs oracle T={tokens}", flush=True)
    out = moe_chain(x, [packed] * 3, indices=idx, workspace=ws)
    inputs = [x]
    for _ in range(3):
        inputs.append(moe_layer(inputs[-1], packed, workspace=ws))
    torch.cuda.synchronize()
    assert ws.status() == 0
    assert torch.equal(out.view(torch.int16), inputs[-1].view(torch.int16))
    for l in range(3):
        xb = to_u16(inputs[l])
        want, o_idx, _ = oracle_layer_rows(oracle, packed, xb, host_experts)
        np.testing.assert_array_equal(idx[l].cpu().numpy(), o_idx)
        assert_layer_close(to_u16(inputs[l + 1]), want, xb, what=f"codec chain T={tokens} layer {l}")


def test_gather_resident_rows_reference_fixture(device, oracle):
    """edge35b/test_gpu_resident_experts.py:12-57 on lrmoe_gather_tiles: a
    compact row (24 packed tiles, 8 raw ones inline) and a raw row, the
    descriptors swapped between graph replays, counts 2, 0, 1."""
    from lightreason_amd.edge35b.native_bf16_gather import NativeBf16Gather

    bits = resident_fixture_words()
    data, headers, encoded, fallback = oracle.compact_rows(bits)
    assert (encoded, fallback) == (24, 8)
    packed = torch.from_numpy(data).to(device)
    meta = torch.from_numpy(headers.view(np.uint8)).to(device)
    original = torch.from_numpy(bits.view(np.int16))
    other = original ^ 31
    raw = other.to(device)
    descriptors = torch.tensor([[[packed.data_ptr(), meta.data_ptr(), -1], [0, 0, raw.data_ptr()]]],
                               device=device, dtype=torch.int64)
    output = torch.full((4, 32, 256), -123, device=device, dtype=torch.int16)
    destinations = torch.tensor([output.data_ptr()], device=device, dtype=torch.int64)
    sizes = torch.tensor([original.numel() * 2], device=device, dtype=torch.int64)
    ids = torch.tensor([0, 1], device=device, dtype=torch.int32)
    slots = torch.tensor([1, 3], device=device, dtype=torch.int32)
    count = torch.tensor([2], device=device, dtype=torch.int64)
    native = NativeBf16Gather()

    def copy():
        native.copy(descriptors, destinations, sizes, ids, slots, count, max_copies=2, experts=2,
                    geometry=(4, 256, "resident"))

    copy()
    torch.cuda.synchronize()
    assert torch.equal(output[1].cpu(), original) and torch.equal(output[3].cpu(), other)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        copy()
    references = [original, other]
    for n in (2, 0, 1):
        descriptors.copy_(descriptors.flip(1))
        references.reverse()
        output.fill_(-123)
        count.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        expected = torch.full_like(output.cpu(), -123)
        for slot, reference in zip((1, 3)[:n], references[:n]):
            expected[slot] = reference
        print(f"resident fixture replay count={n}", flush=True)
        assert torch.equal(output.cpu(), expected)


@pytest.mark.parametrize("geometry", [(4, 256, "cpu-tiles"), (8, 128, "cpu-tiles"), (16, 128, "cpu-tiles"),
                                      (4, 256, "resident")])
def test_gather_codec_expert_rows(model, device, oracle, geometry):
    """Whole expert rows (gate_up 4 MiB, down 2 MiB) of Gaussian weights in
    the reference tile layout, each tile that does not fit read from the raw
    row; a descriptor with bases 0 copies its raw row."""
    from lightreason_amd.edge35b.native_bf16_gather import NativeBf16Gather

    experts = (3, 200, 77)
    keep = []
    desc = torch.zeros((2, len(experts), 3), dtype=torch.int64)
    misfit = 0
    for i, e in enumerate(experts):
        for bank, w in enumerate(model.bank.expert(0, e)):
            bits = w.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, 256)
            packed, bases, m = oracle.codec_pack_reference_order(bits)
            misfit += m
            pk = torch.from_numpy(packed.reshape(-1)).to(device)
            bs = torch.from_numpy(bases.reshape(-1)).to(device)
            keep += [pk, bs]
            desc[bank, i] = torch.tensor([pk.data_ptr(), bs.data_ptr() if e != 77 else 0, w.data_ptr()])
    assert misfit > 0
    desc = desc.to(device)
    gate_dst = torch.full((4, 1024, 2048), -123, dtype=torch.int16, device=device)
    down_dst = torch.full((4, 2048, 512), -123, dtype=torch.int16, device=device)
    destinations = torch.tensor([gate_dst.data_ptr(), down_dst.data_ptr()], dtype=torch.int64, device=device)
    sizes = torch.tensor([1024 * 2048 * 2, 2048 * 512 * 2], dtype=torch.int64, device=device)
    src = torch.tensor([0, 1, 2], dtype=torch.int32, device=device)
    dst = torch.tensor([2, 0, 3], dtype=torch.int32, device=device)
    count = torch.tensor([3], dtype=torch.int64, device=device)
    NativeBf16Gather().copy(desc, destinations, sizes, src, dst, count, max_copies=3, experts=len(experts),
                            geometry=geometry)
    torch.cuda.synchronize()
    print(f"codec expert rows {geometry}", flush=True)
    for i, e in enumerate(experts):
        gu, dn = model.bank.expert(0, e)
        slot = int(dst[i])
        assert torch.equal(gate_dst[slot], gu.view(torch.int16)), e
        assert torch.equal(down_dst[slot], dn.view(torch.int16)), e
    assert bool((gate_dst[1] == -123).all()) and bool((down_dst[1] == -123).all())


@pytest.mark.parametrize("geometry", [(4, 256, "default"), (16, 128, "default"), (8, 256, "l2"), (16, 128, "l2")])
def test_gather_escape_codec_rows(model, device, oracle, geometry):
    """Escape-codec rows (bf16_expert_codec.py pack_row, decoded by
    bf16_gather_ada.cu:36-100): Gaussian expert rows with their few escapes,
    a row of every bf16 pattern (mostly escapes), and raw rows beside them."""
    from lightreason_amd.edge35b.native_bf16_gather import NativeBf16Gather

    rng = np.random.default_rng(5)
    patterns = rng.permutation(np.arange(65536, dtype=np.uint16))
    rows = [model.bank.expert(0, 9)[0], model.bank.expert(0, 41)[0],
            torch.from_numpy(np.tile(patterns, 32).view(np.int16)).to(device).view(torch.bfloat16).view(1024, 2048)]
    keep = []
    desc = torch.zeros((1, 4, 3), dtype=torch.int64)
    escapes_seen = []
    for i, w in enumerate(rows):
        bits = w.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        base, escapes = oracle.escape_window(bits)
        escapes_seen.append(escapes)
        pk = torch.from_numpy(oracle.escape_pack(bits, base, escapes)).to(device)
        keep.append(pk)
        desc[0, i] = torch.tensor([pk.data_ptr(), base, escapes])
    desc[0, 3] = torch.tensor([model.bank.expert(0, 50)[0].data_ptr(), -1, 0])
    assert escapes_seen[0] > 0 and escapes_seen[2] > 1_000_000
    desc = desc.to(device)
    out = torch.full((5, 1024, 2048), -123, dtype=torch.int16, device=device)
    destinations = torch.tensor([out.data_ptr()], dtype=torch.int64, device=device)
    sizes = torch.tensor([1024 * 2048 * 2], dtype=torch.int64, device=device)
    src = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device=device)
    dst = torch.tensor([4, 0, 2, 1], dtype=torch.int32, device=device)
    count = torch.tensor([4], dtype=torch.int64, device=device)
    gather = NativeBf16Gather()
    gather.copy(desc, destinations, sizes, src, dst, count, max_copies=4, experts=4, geometry=geometry)
    torch.cuda.synchronize()
    print(f"escape codec rows {geometry}", flush=True)
    expected = [rows[0], rows[1], rows[2], model.bank.expert(0, 50)[0]]
    for i, w in enumerate(expected):
        assert torch.equal(out[int(dst[i])], w.view(torch.int16)), i
    assert bool((out[3] == -123).all())
    assert gather.codec_rows_seen()


def test_reference_order_tile_packer(model, device, oracle):
    """moe.pack_tiles_reference_order (lrmoe_codec_pack, bytes rearranged on
    the device) against the oracle's reference-order packing."""
    from lightreason_amd.moe import pack_tiles_reference_order

    gate_up, _ = model.bank.expert(0, 12)
    packed, bases, misfit = pack_tiles_reference_order(gate_up)
    torch.cuda.synchronize()
    bits = gate_up.view(torch.int16).cpu().numpy().view(np.uint16)
    o_packed, o_bases, o_misfit = oracle.codec_pack_reference_order(bits)
    assert misfit == o_misfit > 0
    np.testing.assert_array_equal(bases.cpu().numpy(), o_bases.reshape(-1))
    np.testing.assert_array_equal(packed.cpu().numpy(), o_packed.reshape(-1, 384))
