"""Experts loaded from files run through the decode kernels: a fused-tensor GGUF file
(MmapExpertStore.from_fused, mixed quantisation) and a GPT-OSS-style safetensors
checkpoint (ExpertStore.from_safetensors, checkpoint order and tile order), each pool
checked against the oracle on the experts the files were written from."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.gguf_writer import write_gguf
from tests.helpers import assert_close_bf16, bf16_dev
from tests.test_loaders import _write_mxfp4_checkpoint
from tinyserve_amd import ops, synth
from tinyserve_amd.expert_store import ExpertStore
from tinyserve_amd.gguf_store import MmapExpertStore

pytestmark = pytest.mark.gpu


def test_gguf_fused_file_decode(tmp_path):
    rng = np.random.default_rng(11)
    H, I, E, k, T = 512, 256, 8, 4, 2
    types = [(13, 13, 14), (12, 12, 14)]
    ex = {(li, e): synth.make_gguf_expert(rng, H, I, *types[li]) for li in range(2) for e in range(E)}
    tensors = []
    for li in range(2):
        for pi, (proj, ne) in enumerate((("gate", (H, I, E)), ("up", (H, I, E)), ("down", (I, H, E)))):
            tensors.append((f"blk.{li}.ffn_{proj}_exps.weight", ne, types[li][pi],
                            np.concatenate([ex[(li, e)][proj] for e in range(E)])))
    write_gguf(tmp_path / "m.gguf", tensors)
    st = MmapExpertStore.from_fused(tmp_path / "m.gguf")
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = synth.zipf_logits(rng, T, E)
    for li in range(2):  # layer 1 is padded to layer 0's slot size
        pool = st.load_layer(li, "cuda")
        y, idx, w = ops.moe_decode_routed(st.expert_layout(li), pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                                          torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k, "softmax_then_topk",
                                          return_routing=True)
        ridx, rw = oex.route_softmax_then_topk(logits, k)
        assert np.array_equal(idx.cpu().numpy(), ridx)
        ref = oex.moe_combine(synth.bf16_to_f32(x_bits), ridx, rw,
                              lambda e, xx: oex.gguf_expert_forward(xx, ex[(li, e)]))
        assert_close_bf16(y, ref, f"GGUF file layer {li}")
    st.close()


@pytest.mark.parametrize("tiled", [False, True])
def test_safetensors_checkpoint_decode(tmp_path, tiled):
    rng = np.random.default_rng(12 + tiled)
    H, I, E, k, T = 512, 384, 6, 4, 3
    exs = {0: [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]}
    _write_mxfp4_checkpoint(tmp_path, exs)
    st, _ = ExpertStore.from_safetensors(str(tmp_path), tiled=tiled)
    pool = st.load_layer(0, "cuda")
    x_bits = synth.bf16_normal(rng, (T, H))
    logits = rng.normal(size=(T, E)).astype(np.float32)
    y = ops.moe_decode_routed(st.expert_layout(), pool, torch.arange(E, dtype=torch.int32, device="cuda"),
                              torch.from_numpy(logits).cuda(), bf16_dev(x_bits), k)
    ridx, rw = oex.route_topk_then_softmax(logits, k)
    ref = oex.moe_combine(synth.bf16_to_f32(x_bits), ridx, rw, lambda e, xx: oex.mxfp4_expert_forward(xx, exs[0][e]))
    assert_close_bf16(y, ref, f"safetensors checkpoint tiled={tiled}")


def test_gguf_linears_into_a_module(tmp_path):
    """Non-expert weights of a GGUF file run as GGMLLinear after replace_linear_with_ggml
    (tinyserve/gguf_loader.py:610-665 selection, ggml_linear.py:120-173 replacement)."""
    from oracle import gguf as og
    from tests.gguf_writer import write_gguf as _w
    from tinyserve_amd import gguf_reader as gr
    from tinyserve_amd.ggml_linear import GGMLLinear, replace_linear_with_ggml
    from tinyserve_amd.gguf_store import gguf_linear_weights

    rng = np.random.default_rng(13)
    K, N = 512, 768
    q = synth.make_gguf(rng, 13, N * K)
    _w(tmp_path / "l.gguf", [("blk.0.attn_q.weight", (K, N), 13, q)])
    model = torch.nn.Module()
    model.q_proj = torch.nn.Linear(K, N, bias=True)
    with gr.GGUFReader(tmp_path / "l.gguf") as r:
        lw = gguf_linear_weights(r, {"blk.0.attn_q.weight": "q_proj.weight"})
    assert replace_linear_with_ggml(model, lw, "cuda") == 1 and isinstance(model.q_proj, GGMLLinear)
    x = torch.randn(3, K).to(torch.bfloat16)
    with torch.no_grad():
        y = model.q_proj(x.cuda()).float().cpu().numpy()
    ref = x.float().numpy() @ og.dequant_tensor(q, 13, (N, K)).T + model.q_proj.bias.detach().float().cpu().numpy()
    assert_close_bf16(y, ref, "GGMLLinear from a GGUF file")
