"""fused_attention (with fused_delta) on a Transformers Qwen3.5-MoE model
(35B layer dims, 4 layers -- three Gated DeltaNet, one full attention -- 4
experts, vocabulary 512, random weights) on the GPU: cached decode steps and
a verify block through lrmoe_attn_decode and lrmoe_delta_mixer against the
stock forward, the cache layer's rows living in the native buffer, and a
speculative rollback (PrefixStates.commit crops the attention rows) followed
by a step that matches a run which verified only the accepted prefix.

Bars: logits within 2e-2 in L2 of the stock model's (both bf16 on the GPU;
the stock attention is SDPA, whose softmax and sums round differently);
the cached key and value rows within 1e-2."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

PREFIX = 40
ATTN = 3  # the full-attention layer of the 4


@pytest.fixture(scope="module")
def model(device):
    from transformers import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeForCausalLM

    torch.manual_seed(6160)
    cfg = Qwen3_5MoeTextConfig(num_hidden_layers=4, num_experts=4, num_experts_per_tok=2, vocab_size=512)
    assert cfg.layer_types[ATTN] == "full_attention"
    m = Qwen3_5MoeForCausalLM(cfg)
    with torch.no_grad():
        for layer in m.model.layers:
            mixer = getattr(layer, "linear_attn", None)
            if mixer is not None:
                mixer.conv1d.weight.normal_(0.0, 0.3)
                mixer.norm.weight.normal_(1.0, 0.1)
                mixer.dt_bias.normal_(0.0, 0.5)
            attn = getattr(layer, "self_attn", None)
            if attn is not None:
                attn.q_norm.weight.normal_(0.0, 0.1)
                attn.k_norm.weight.normal_(0.0, 0.1)
    return cfg, m.to(device=device, dtype=torch.bfloat16).eval()


def _cache(cfg):
    from transformers.cache_utils import DynamicCache

    return DynamicCache(config=cfg)


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


@torch.no_grad()
def test_fused_attention_decode_and_verify_match_stock(model, device):
    from contextlib import ExitStack

    from lightreason_amd.attention import fused_attention
    from lightreason_amd.delta import fused_delta

    cfg, m = model
    ids = torch.randint(0, 512, (1, PREFIX + 8), generator=torch.Generator().manual_seed(7), dtype=torch.long).to(device)

    def run(native):
        cache = _cache(cfg)
        logits = []
        with ExitStack() as stack:
            if native:
                stack.enter_context(fused_delta(m))
                stack.enter_context(fused_attention(m))
            m(ids[:, :PREFIX], past_key_values=cache, use_cache=True)       # prefill: stock in both
            for i in range(PREFIX, PREFIX + 4):                             # four single-token steps
                logits.append(m(ids[:, i:i + 1], past_key_values=cache, use_cache=True).logits[0, -1])
            logits.extend(m(ids[:, PREFIX + 4:PREFIX + 8], past_key_values=cache, use_cache=True).logits[0])
        torch.cuda.synchronize()
        layer = cache.layers[ATTN]
        return torch.stack(logits), layer.keys.clone(), layer.values.clone(), layer

    stock, sk, sv, _ = run(False)
    native, nk, nv, layer = run(True)
    assert nk.shape == sk.shape == (1, 2, PREFIX + 8, 256)
    # lrmoe_attn_decode ran: the native path keeps the layer's rows as views
    # of a buffer with room to grow
    row_bytes = (PREFIX + 8) * 2 * 256 * 2
    assert layer.keys.untyped_storage().nbytes() > row_bytes
    assert layer.values.untyped_storage().nbytes() > row_bytes
    assert layer.get_seq_length() == PREFIX + 8
    for i in range(stock.shape[0]):
        r = _rel(native[i], stock[i])
        print(f"position {PREFIX + i}: logits L2 rel {r:.2e}", flush=True)
        assert r <= 2e-2
    assert _rel(nk, sk) <= 1e-2 and _rel(nv, sv) <= 1e-2
    # the patch is removed on exit
    assert all("forward" not in l.self_attn.__dict__ for l in m.model.layers if hasattr(l, "self_attn"))


@torch.no_grad()
def test_rollback_crops_the_native_rows(model, device):
    from lightreason_amd.attention import fused_attention
    from lightreason_amd.delta import fused_delta

    cfg, m = model
    ids = torch.randint(0, 512, (1, PREFIX + 6), generator=torch.Generator().manual_seed(8), dtype=torch.long).to(device)
    with fused_delta(m) as histories, fused_attention(m):
        cache = _cache(cfg)
        m(ids[:, :PREFIX], past_key_values=cache, use_cache=True)
        m(ids[:, PREFIX:PREFIX + 1], past_key_values=cache, use_cache=True)  # rows move to the native buffer
        with histories.record(cache):
            m(ids[:, PREFIX + 1:PREFIX + 5], past_key_values=cache, use_cache=True)  # verify 4
        histories.commit(cache, PREFIX + 1, 2, 4)                            # accept 2
        assert cache.get_seq_length(ATTN) == PREFIX + 3
        after = m(ids[:, PREFIX + 3:PREFIX + 4], past_key_values=cache, use_cache=True).logits[0, -1]
        keys = cache.layers[ATTN].keys.clone()

        ref = _cache(cfg)
        m(ids[:, :PREFIX], past_key_values=ref, use_cache=True)
        m(ids[:, PREFIX:PREFIX + 1], past_key_values=ref, use_cache=True)
        m(ids[:, PREFIX + 1:PREFIX + 3], past_key_values=ref, use_cache=True)
        ref_after = m(ids[:, PREFIX + 3:PREFIX + 4], past_key_values=ref, use_cache=True).logits[0, -1]
        ref_keys = ref.layers[ATTN].keys.clone()
        torch.cuda.synchronize()
    assert keys.shape == ref_keys.shape == (1, 2, PREFIX + 4, 256)
    assert _rel(keys, ref_keys) <= 1e-2
    assert _rel(after, ref_after) <= 2e-2
