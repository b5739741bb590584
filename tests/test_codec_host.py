"""Host side of the tile codec: the raw flags that tell each (item, wave)
unit of the decode kernel whether it reads codec or raw rows.

The flags are checked against their definition, tile by tile: gate/up item
i, wave w reads tiles 2(w%4), 2(w%4)+1 of gate rows and up rows
16i + 8(w/4) .. +7; down item i, wave w reads both tiles of down rows
128i + 16w .. +15 (the decode kernel's item geometry).  A unit is raw when
any of its tiles has the misfit base 255, which the oracle's packer gives.
"""

from __future__ import annotations

import numpy as np
import torch

from lightreason_amd.moe import CODEC_MISFIT, codec_unit_flags


def _expert_bases(oracle, seed):
    rng = np.random.default_rng(seed)
    # N(0, 0.02) weights in bf16: a few tiles hold a value so small that the
    # tile's exponent fields span more than 8 values, and do not fit.
    def bf16(shape):
        f = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        return (f.view(np.uint32) >> 16).astype(np.uint16)
    _, gu, gu_mis = oracle.codec_pack(bf16((1024, 2048)))
    _, dn, dn_mis = oracle.codec_pack(bf16((2048, 512)))
    return gu.reshape(1024, 8), dn.reshape(2048, 2), gu_mis + dn_mis


def test_unit_flags_follow_the_item_geometry(oracle):
    gu, dn, misfit = _expert_bases(oracle, 11)
    assert misfit > 0
    flags = codec_unit_flags(torch.from_numpy(gu.ravel()), torch.from_numpy(dn.ravel())).numpy()
    assert flags.shape == (48,) and flags.dtype == np.uint8
    for i in range(32):
        for w in range(8):
            rows = [h * 512 + 16 * i + 8 * (w >> 2) + r for h in (0, 1) for r in range(8)]
            raw = bool((gu[rows][:, [2 * (w & 3), 2 * (w & 3) + 1]] == CODEC_MISFIT).any())
            assert bool((flags[i] >> w) & 1) == raw, (i, w)
    for i in range(16):
        for w in range(8):
            raw = bool((dn[128 * i + 16 * w:128 * i + 16 * w + 16] == CODEC_MISFIT).any())
            assert bool((flags[32 + i] >> w) & 1) == raw, (i, w)


def test_unit_flags_extremes():
    fit_gu = torch.zeros(8192, dtype=torch.uint8)
    fit_dn = torch.zeros(4096, dtype=torch.uint8)
    assert int(codec_unit_flags(fit_gu, fit_dn).sum()) == 0
    # One misfit tile raises exactly one unit's flag: gate row 16*5 + 8 + 3,
    # tile 6 -> gate/up item 5, wave 4 + 3.
    one = fit_gu.clone()
    one[(16 * 5 + 8 + 3) * 8 + 6] = CODEC_MISFIT
    f = codec_unit_flags(one, fit_dn)
    assert f.tolist() == [0] * 5 + [1 << 7] + [0] * 42
    # Down row 128*9 + 16*2 + 15, tile 1 -> down item 9, wave 2.
    one = fit_dn.clone()
    one[(128 * 9 + 32 + 15) * 2 + 1] = CODEC_MISFIT
    f = codec_unit_flags(fit_gu, one)
    assert f.tolist() == [0] * 41 + [1 << 2] + [0] * 6
    every = codec_unit_flags(torch.full((8192,), CODEC_MISFIT, dtype=torch.uint8),
                             torch.full((4096,), CODEC_MISFIT, dtype=torch.uint8))
    assert f.dtype == torch.uint8 and every.tolist() == [255] * 48


def test_escape_packer_matches_the_oracle(oracle):
    """moe.pack_escape_row (torch, here on the CPU) against the oracle's
    restatement of bf16_expert_codec.py: every bf16 pattern, Gaussian
    weights, and a constant row."""
    import numpy as np

    from lightreason_amd.moe import pack_escape_row

    rng = np.random.default_rng(3)
    gauss = (rng.standard_normal(8192).astype(np.float32) * 0.02).view(np.uint32) >> 16
    for bits in (np.arange(65536, dtype=np.uint16), gauss.astype(np.uint16), np.full(64, 0x3F80, np.uint16)):
        w = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
        packed, base, escapes = pack_escape_row(w)
        assert (base, escapes) == oracle.escape_window(bits)
        np.testing.assert_array_equal(packed.numpy(), oracle.escape_pack(bits, base, escapes))
