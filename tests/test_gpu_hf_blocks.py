"""The MoE block hook installed on transformers' own modules (transformers 5.x): GPT-OSS's
``GptOssMLP`` (router ``router`` returning (logits, scores, indices); experts with fused,
interleaved gate/up, biases and the clamped SwiGLU) over MXFP4 experts, and Qwen3-MoE's
``Qwen3MoeSparseMoeBlock`` (router ``gate``, softmax -> top-k -> renormalised; experts with
gate and up halves and SiLU) over GGUF Q5_K / Q6_K experts from a GGUF file. The modules hold
the dequantised weights of the same experts; the hooked forward (``router_native``: the
module's own router, then the decode or the grouped prefill kernels) is checked against the
module's own experts forward run in fp32 on the CPU with the routing the module's router
made (tinyserve/_model_hooks.py:424-476,479-568 — the reference hooks these modules)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.gguf_writer import write_gguf
from tests.helpers import assert_close_bf16, bf16_dev
from tests.test_gpu_pipeline import _mx_store
from tinyserve_amd import synth
from tinyserve_amd.expert_pipeline import ExpertPipeline, install_offloaded_forward
from tinyserve_amd.gguf_store import MmapExpertStore

pytestmark = pytest.mark.gpu
transformers = pytest.importorskip("transformers")


def _module_reference(block, experts_attr: str, x: torch.Tensor, router_out) -> np.ndarray:
    """The module's experts forward in fp32 on the CPU for the routing its router gave."""
    _, scores, idx = router_out
    experts = getattr(block, experts_attr)
    ref = experts.float().cpu()
    with torch.no_grad():
        y = ref(x.float().cpu(), idx.cpu(), scores.float().cpu())
    return y.numpy()


@pytest.mark.parametrize("T", [1, 3, 40])  # routed decode (T <= 4) and the grouped prefill
def test_gpt_oss_mlp(T):
    from transformers.models.gpt_oss.configuration_gpt_oss import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssMLP

    H, I, E, k = 256, 128, 8, 4
    rng, store, experts = _mx_store(H, I, E, 1, seed=31 + T, tiled=True)
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k,
                       num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2, head_dim=64)
    mlp = GptOssMLP(cfg)
    torch.manual_seed(T)
    with torch.no_grad():
        mlp.router.weight.copy_(torch.randn(E, H) / H ** 0.5)
        mlp.router.bias.copy_(torch.randn(E) * 0.1)
        for e, ex in enumerate(experts[0]):
            wgu, wdn = oex.mxfp4_expert_weights(ex)  # [2I, H] (gate / up rows interleaved), [H, I]
            mlp.experts.gate_up_proj[e].copy_(torch.from_numpy(wgu.T))
            mlp.experts.down_proj[e].copy_(torch.from_numpy(wdn.T))
            mlp.experts.gate_up_proj_bias[e].copy_(torch.from_numpy(ex["gate_up_bias"]))
            mlp.experts.down_proj_bias[e].copy_(torch.from_numpy(ex["down_bias"]))
    mlp = mlp.to(device="cuda", dtype=torch.bfloat16)
    x = bf16_dev(synth.bf16_normal(rng, (T, H))).view(1, T, H)
    with torch.no_grad():
        router_out = mlp.router(x.view(T, H))
    ref = _module_reference(mlp, "experts", x.view(T, H), router_out)
    p = ExpertPipeline(store, None, "cuda")
    install_offloaded_forward(mlp, p, 0, "router", k, returns_router_logits=True, softmax_order="router_native")
    with torch.no_grad():
        y, logits = mlp(x)
    torch.cuda.synchronize()
    assert y.shape == (1, T, H) and y.dtype == torch.bfloat16
    assert torch.equal(logits, router_out[0])
    assert_close_bf16(y.view(T, H), ref, f"GptOssMLP T={T}")


@pytest.mark.parametrize("T", [2, 40])
def test_qwen3_moe_sparse_block(T, tmp_path):
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    H, I, E, k = 512, 256, 8, 2
    types = (13, 13, 14)
    rng = np.random.default_rng(41 + T)
    ex = [synth.make_gguf_expert(rng, H, I, *types) for _ in range(E)]
    tensors = [(f"blk.0.ffn_{proj}_exps.weight", ne, types[pi], np.concatenate([e[proj] for e in ex]))
               for pi, (proj, ne) in enumerate((("gate", (H, I, E)), ("up", (H, I, E)), ("down", (I, H, E))))]
    write_gguf(tmp_path / "q.gguf", tensors)
    st = MmapExpertStore.from_fused(tmp_path / "q.gguf")
    cfg = Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_tok=k,
                         norm_topk_prob=True, num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=2,
                         head_dim=64)
    blk = Qwen3MoeSparseMoeBlock(cfg)
    torch.manual_seed(T)
    with torch.no_grad():
        blk.gate.weight.copy_(torch.randn(E, H) / H ** 0.5)
        for e in range(E):
            wg, wu, wd = oex.gguf_expert_weights(ex[e])  # [I, H], [I, H], [H, I]
            blk.experts.gate_up_proj[e].copy_(torch.from_numpy(np.concatenate([wg, wu])))
            blk.experts.down_proj[e].copy_(torch.from_numpy(wd))
    blk = blk.to(device="cuda", dtype=torch.bfloat16)
    x = bf16_dev(synth.bf16_normal(rng, (T, H))).view(1, T, H)
    with torch.no_grad():
        router_out = blk.gate(x.view(T, H))
    ref = _module_reference(blk, "experts", x.view(T, H), router_out)
    p = ExpertPipeline(st, None, "cuda")
    install_offloaded_forward(blk, p, 0, "gate", k, softmax_order="router_native")
    with torch.no_grad():
        y = blk(x)
    torch.cuda.synchronize()
    assert y.shape == (1, T, H) and y.dtype == torch.bfloat16
    assert_close_bf16(y.view(T, H), ref, f"Qwen3MoeSparseMoeBlock T={T}")
    st.close()
