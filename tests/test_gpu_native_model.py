"""Every native path at once on a Transformers Qwen3.5-MoE model with the 35B
layer dims (4 layers -- three Gated DeltaNet, one full attention -- 256
experts of 512 with top-8 routing and the shared expert, vocabulary 512,
random weights, bf16) on the GPU: the experts through ``patch_experts``
(mode "fused"), the mixers through ``fused_delta``, the attention through
``fused_attention``; prefill, four single-token steps and a block of four.

Bar: the native model is as close to an fp32 copy of the same weights as
the stock bf16 model is (mean L2 error of the logits over the positions
within 1.2x the stock one's, every position within 1.5x + 0.02).  Native
and stock bf16 differ from each other by about as much as each differs from
fp32: both round in bf16, in different orders, and a routing choice near a
tie can go either way."""

from __future__ import annotations

import copy
from contextlib import ExitStack

import pytest
import torch

pytestmark = pytest.mark.gpu


@torch.no_grad()
def test_all_native_paths_match_the_stock_models_accuracy(device):
    from transformers import Qwen3_5MoeTextConfig
    from transformers.cache_utils import DynamicCache
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeForCausalLM

    from lightreason_amd.attention import fused_attention
    from lightreason_amd.delta import fused_delta
    from lightreason_amd.edge35b.expert_stream import ExpertPool, patch_experts

    torch.manual_seed(777)
    cfg = Qwen3_5MoeTextConfig(num_hidden_layers=4, vocab_size=512)
    assert (cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size, cfg.hidden_size) == (256, 8, 512, 2048)
    with torch.device(device):
        m32 = Qwen3_5MoeForCausalLM(cfg).float().eval()
    for layer in m32.model.layers:
        mixer = getattr(layer, "linear_attn", None)
        if mixer is not None:
            mixer.conv1d.weight.normal_(0.0, 0.3)
            mixer.norm.weight.normal_(1.0, 0.1)
            mixer.dt_bias.normal_(0.0, 0.5)
        attn = getattr(layer, "self_attn", None)
        if attn is not None:
            attn.q_norm.weight.normal_(0.0, 0.1)
            attn.k_norm.weight.normal_(0.0, 0.1)
        layer.mlp.experts.gate_up_proj.normal_(0.0, 0.02)
        layer.mlp.experts.down_proj.normal_(0.0, 0.02)
    m16 = copy.deepcopy(m32).to(torch.bfloat16).eval().requires_grad_(False)
    ids = torch.randint(0, 512, (1, 40), generator=torch.Generator().manual_seed(7), dtype=torch.long).to(device)

    def run(model, native):
        cache = DynamicCache(config=cfg)
        logits = []
        with ExitStack() as stack:
            if native:
                stack.enter_context(patch_experts(model, mode="fused", pool=ExpertPool(device)))
                stack.enter_context(fused_delta(model))
                stack.enter_context(fused_attention(model))
            model(ids[:, :32], past_key_values=cache, use_cache=True)
            for i in range(32, 36):
                logits.append(model(ids[:, i:i + 1], past_key_values=cache, use_cache=True).logits[0, -1])
            logits.extend(model(ids[:, 36:40], past_key_values=cache, use_cache=True).logits[0])
        torch.cuda.synchronize()
        return torch.stack(logits).float()

    want = run(m32, False)
    stock = run(m16, False)
    native = run(m16, True)
    err = lambda a: (a - want).norm(dim=-1) / want.norm(dim=-1)  # noqa: E731
    e_stock, e_native = err(stock), err(native)
    print(f"stock bf16 vs fp32 {[round(float(v), 4) for v in e_stock]}", flush=True)
    print(f"native vs fp32     {[round(float(v), 4) for v in e_native]}", flush=True)
    assert float(e_native.mean()) <= 1.2 * float(e_stock.mean())
    assert bool((e_native <= 1.5 * e_stock + 0.02).all())
