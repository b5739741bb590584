"""fused_delta on a Transformers Qwen3.5-MoE model (35B layer dims, 4 layers
-- three Gated DeltaNet, one full attention -- 4 experts, vocabulary 512,
random weights) on the GPU: cached decode and verify blocks through
lrmoe_delta_mixer against the stock forward, and PrefixStates.commit
rolling a verified block back to its accepted prefix
(edge35b/delta_decode.py:58-126).

Bars: logits of every step within 2e-2 in L2 of the stock model's (both run
bf16 on the GPU; the stock mixer's projections and recurrence round in a
different order); after commit, the rolled-back states bit-identical to a
run that verified only the accepted prefix in the first linear-attention
layer (same kernels, same inputs), within 1e-2 in the later ones (their
inputs pass through stock torch ops on blocks of different lengths)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

PREFIX = 8


@pytest.fixture(scope="module")
def model(device):
    from transformers import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeForCausalLM

    torch.manual_seed(5150)
    cfg = Qwen3_5MoeTextConfig(num_hidden_layers=4, num_experts=4, num_experts_per_tok=2, vocab_size=512)
    m = Qwen3_5MoeForCausalLM(cfg)
    with torch.no_grad():
        for layer in m.model.layers:
            mixer = getattr(layer, "linear_attn", None)
            if mixer is not None:
                mixer.conv1d.weight.normal_(0.0, 0.3)
                mixer.norm.weight.normal_(1.0, 0.1)
                mixer.dt_bias.normal_(0.0, 0.5)
    return cfg, m.to(device=device, dtype=torch.bfloat16).eval()


def _cache(cfg):
    from transformers.cache_utils import DynamicCache

    return DynamicCache(config=cfg)


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


def _linear_states(cache):
    from lightreason_amd.delta import _live

    return {i: (_live(layer.conv_states)[0].clone(), _live(layer.recurrent_states)[0].clone())
            for i, layer in enumerate(cache.layers) if hasattr(layer, "conv_states")}


@torch.no_grad()
def test_fused_delta_decode_and_verify_match_stock(model, device):
    from lightreason_amd.delta import fused_delta

    cfg, m = model
    ids = torch.randint(0, 512, (1, PREFIX + 8), generator=torch.Generator().manual_seed(3), dtype=torch.long).to(device)

    def run(native):
        cache = _cache(cfg)
        logits = []
        ctx = fused_delta(m) if native else None
        if ctx is not None:
            ctx.__enter__()
        try:
            m(ids[:, :PREFIX], past_key_values=cache, use_cache=True)         # prefill: stock in both
            for i in range(PREFIX, PREFIX + 4):                               # four single-token steps
                logits.append(m(ids[:, i:i + 1], past_key_values=cache, use_cache=True).logits[0, -1])
            logits.extend(m(ids[:, PREFIX + 4:PREFIX + 8], past_key_values=cache, use_cache=True).logits[0])  # a block of 4
        finally:
            if ctx is not None:
                ctx.__exit__(None, None, None)
        torch.cuda.synchronize()
        return torch.stack(logits), _linear_states(cache)

    stock, stock_states = run(False)
    native, native_states = run(True)
    for i in range(stock.shape[0]):
        r = _rel(native[i], stock[i])
        print(f"position {PREFIX + i}: logits L2 rel {r:.2e}", flush=True)
        assert r <= 2e-2
    for i, (conv, state) in native_states.items():
        assert _rel(conv, stock_states[i][0]) <= 2e-2
        assert _rel(state, stock_states[i][1]) <= 2e-2
    # the patch is removed on exit
    assert all("forward" not in layer.linear_attn.__dict__ for layer in m.model.layers if hasattr(layer, "linear_attn"))


@torch.no_grad()
def test_prefix_commit_rolls_back_to_the_accepted_prefix(model, device):
    from lightreason_amd.delta import fused_delta

    cfg, m = model
    ids = torch.randint(0, 512, (1, PREFIX + 6), generator=torch.Generator().manual_seed(4), dtype=torch.long).to(device)
    with fused_delta(m) as histories:
        # verify 4 positions, accept 2
        cache = _cache(cfg)
        m(ids[:, :PREFIX], past_key_values=cache, use_cache=True)
        with histories.record(cache):
            m(ids[:, PREFIX:PREFIX + 4], past_key_values=cache, use_cache=True)
        assert sorted(histories.conv) == [0, 1, 2] and histories.recurrent[0].shape[0] == 4
        histories.commit(cache, PREFIX, 2, 4)
        assert cache.get_seq_length(3) == PREFIX + 2
        committed = _linear_states(cache)
        after = m(ids[:, PREFIX + 2:PREFIX + 3], past_key_values=cache, use_cache=True).logits[0, -1]

        # the same prefix verified with width 2
        ref = _cache(cfg)
        m(ids[:, :PREFIX], past_key_values=ref, use_cache=True)
        m(ids[:, PREFIX:PREFIX + 2], past_key_values=ref, use_cache=True)
        want = _linear_states(ref)
        ref_after = m(ids[:, PREFIX + 2:PREFIX + 3], past_key_values=ref, use_cache=True).logits[0, -1]
        torch.cuda.synchronize()
        # layer 0 sees the same embeddings either way: bit-identical; later
        # layers' inputs pass through stock torch ops on 4 vs 2 rows
        assert torch.equal(committed[0][0].view(torch.int16), want[0][0].view(torch.int16))
        assert torch.equal(committed[0][1], want[0][1])
        for i in want:
            assert _rel(committed[i][0], want[i][0]) <= 1e-2, f"layer {i} conv"
            assert _rel(committed[i][1], want[i][1]) <= 1e-2, f"layer {i} state"
        assert _rel(after, ref_after) <= 2e-2

        # all accepted: nothing to do; a missing record is an error
        histories.commit(cache, PREFIX, 4, 4)
        empty = type(histories)()
        with pytest.raises(RuntimeError, match="Missing target state"):
            empty.commit(cache, PREFIX, 1, 4)
