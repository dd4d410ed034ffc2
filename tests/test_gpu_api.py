"""The reference-shaped Python API on the GPU: torch.ops.tinyserve_ggml.ggml_mul_mat_vec,
GGMLLinear, GGMLExpertForward, the mxfp4 functions and ExpertBatcher, against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from oracle import gguf as og
from oracle import mxfp4 as omx
from tests.helpers import assert_close_bf16, bf16_dev, to_f32
from tinyserve_amd import ggml_ops, mxfp4, synth
from tinyserve_amd.expert_batcher import BatchItem, ExpertBatcher
from tinyserve_amd.expert_pipeline import ExpertPipeline
from tinyserve_amd.expert_store import ExpertStore
from tinyserve_amd.ggml_forward import GGMLExpertForward
from tinyserve_amd.ggml_linear import GGMLLinear, replace_linear_with_ggml

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def op():
    ggml_ops.register()
    return torch.ops.tinyserve_ggml.ggml_mul_mat_vec


@pytest.mark.parametrize("t,N,K", [(8, 64, 2880), (12, 48, 2048), (13, 96, 2048), (14, 40, 768)])
def test_ggml_mul_mat_vec_op(op, t, N, K):
    rng = np.random.default_rng(t + N)
    data = synth.make_gguf(rng, t, N * K)
    padded = np.concatenate([data, np.zeros(100, np.uint8)])  # padded slot: extra bytes are ignored
    x_bits = synth.bf16_normal(rng, (1, K + 7))  # the op uses the first K elements
    y = op(bf16_dev(x_bits), torch.from_numpy(padded).cuda(), t, N, K)
    assert y.shape == (1, N) and y.dtype == torch.bfloat16
    ref = og.ref_matvec(data, synth.bf16_to_f32(x_bits)[0, :K], t, N, K)
    assert_close_bf16(y, ref.reshape(1, N), f"ggml_mul_mat_vec type {t}")


def test_ggml_mul_mat_vec_errors(op):
    w = torch.zeros(34 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros(1, 64, device="cuda")
    with pytest.raises(RuntimeError, match="Unsupported ggml_type"):
        op(x, w, 99, 2, 64)
    with pytest.raises(RuntimeError, match=r"in_features \(48\) must be divisible by block_elements \(32\)"):
        op(x, w, 8, 2, 48)
    with pytest.raises(RuntimeError, match="weight_data too small: got 136 bytes, expected 204"):
        op(x, w, 8, 3, 64)
    with pytest.raises(RuntimeError, match="weight_data must be uint8"):
        op(x, w.float(), 8, 2, 64)
    with pytest.raises(RuntimeError, match="activation too small"):
        op(x[:, :32], w, 8, 2, 64)
    # like the reference op, K-quant rows must be whole super-blocks here (tsa_gguf_matvec and
    # GGMLLinear accept the straddling K = 2880 stream)
    with pytest.raises(RuntimeError, match=r"in_features \(2880\) must be divisible by block_elements \(256\)"):
        op(torch.zeros(1, 2880, device="cuda"), torch.zeros(144 * 45, dtype=torch.uint8, device="cuda"), 12, 4, 2880)


def test_ggml_linear_batches_and_bias():
    rng = np.random.default_rng(1)
    N, K = 96, 512
    data = synth.make_gguf(rng, 12, N * K)
    bias = torch.randn(N, device="cuda", dtype=torch.bfloat16)
    lin = GGMLLinear(data.tobytes(), 12, N, K, bias=bias, device="cuda")
    w = og.dequant_tensor(data, 12, (N, K))
    for T in (1, 5):
        x_bits = synth.bf16_normal(rng, (T, K))
        y = lin(bf16_dev(x_bits))
        ref = synth.bf16_to_f32(x_bits) @ w.T + to_f32(bias)
        assert y.shape == (T, N)
        assert_close_bf16(y, ref, f"GGMLLinear T={T}")


def test_replace_linear_with_ggml():
    rng = np.random.default_rng(2)
    model = torch.nn.Sequential(torch.nn.Linear(256, 64), torch.nn.ReLU(), torch.nn.Linear(64, 32, bias=False))
    d0 = synth.make_gguf(rng, 8, 64 * 256)
    d2 = synth.make_gguf(rng, 8, 32 * 64)
    n = replace_linear_with_ggml(model, {"0": (d0.tobytes(), 8, (64, 256)), "2": (d2.tobytes(), 8, (32, 64)),
                                         "9.x": (b"", 8, (1, 32))}, device="cuda")
    assert n == 2 and isinstance(model[0], GGMLLinear) and isinstance(model[2], GGMLLinear)
    assert model[0].bias is not None and model[2].bias is None


@pytest.mark.parametrize("types,T", [((12, 12, 14), 1), ((13, 13, 14), 3), ((12, 13, 14), 2)])
def test_ggml_expert_forward(types, T):
    H, I = 512, 256
    rng = np.random.default_rng(sum(types) + T)
    lay = synth.gguf_layout(H, I, *types)
    e = synth.make_gguf_expert(rng, H, I, *types)
    packed = torch.from_numpy(synth.pack_gguf_expert(e, lay)).cuda()
    fwd = GGMLExpertForward(lay, dict(zip(("gate", "up", "down"), types)), torch.nn.SiLU(),
                            {"gate": (H, I), "up": (H, I), "down": (I, H)})
    x_bits = synth.bf16_normal(rng, (T, H))
    y = fwd.forward(packed, bf16_dev(x_bits))
    assert y.shape == (T, H)
    assert_close_bf16(y, oex.gguf_expert_forward(synth.bf16_to_f32(x_bits), e), f"GGMLExpertForward {types}")


def test_mxfp4_functions():
    rng = np.random.default_rng(4)
    b = rng.integers(0, 256, (64, 8, 16), dtype=np.uint8)
    s = rng.integers(119, 135, (64, 8), dtype=np.uint8)
    tb, ts = torch.from_numpy(b).cuda(), torch.from_numpy(s).cuda()
    w = mxfp4.dequant_mxfp4_no_transpose(tb, ts)
    assert w.dtype == torch.bfloat16 and w.shape == (64, 256)
    assert np.array_equal(w.view(torch.int16).cpu().numpy().view(np.uint16),
                          omx.bf16_bits(omx.dequant_mxfp4_no_transpose(b, s, "bf16")))
    wt = mxfp4.dequant_mxfp4(tb, ts, dtype=torch.float32)
    assert np.array_equal(wt.cpu().numpy().view(np.uint32), omx.dequant_mxfp4(b, s, "f32").view(np.uint32))
    x_bits = synth.bf16_normal(rng, (1, 256))
    bias = torch.randn(64, device="cuda", dtype=torch.bfloat16)
    y = mxfp4.mxfp4_linear(bf16_dev(x_bits), tb, ts, bias)
    ref = omx.ref_matvec(b, s, synth.bf16_to_f32(x_bits)[0], to_f32(bias))
    assert_close_bf16(y, ref.reshape(1, -1), "mxfp4_linear")


def test_expert_batcher():
    H, I, E, k = 256, 128, 6, 2
    rng = np.random.default_rng(9)
    lay = synth.mxfp4_layout(H, I)
    experts = [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]
    data = torch.from_numpy(np.stack([synth.pack_mxfp4_expert(e, lay) for e in experts])).reshape(1, E, -1)
    batcher = ExpertBatcher(ExpertPipeline(ExpertStore(data, lay, 1, E), None, "cuda"))
    items, refs = [], []
    for r in range(5):
        x_bits = synth.bf16_normal(rng, (1, H))
        idx, w = oex.route_topk_then_softmax(rng.normal(size=(1, E)).astype(np.float32), k)
        items.append(BatchItem(bf16_dev(x_bits), torch.from_numpy(idx[0]).cuda(), torch.from_numpy(w[0]).cuda(), r))
        refs.append(oex.moe_combine(synth.bf16_to_f32(x_bits), idx, w,
                                    lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e])))
    outs = batcher.batch_execute(items, layer_idx=0)
    assert len(outs) == 5 and batcher.batch_execute([], 0) == []
    for o, ref in zip(outs, refs):
        assert o.shape == (1, H) and o.dtype == torch.bfloat16
        assert_close_bf16(o, ref, "ExpertBatcher")
