"""The torch CPU restatement (bench.py's timed CPU baseline) is bit-for-bit the numpy
oracle: every dequantiser on random blocks, on the reference-derived golden vectors and at
the MXFP4 scale extremes, and the expert FFNs on the same weights."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import expert as oex
from oracle import gguf as og
from oracle import mxfp4 as omx
from oracle import torch_cpu as otc
from tinyserve_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dequant_golden.npz")


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.asarray(a, dtype=np.float32), np.asarray(b, dtype=np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32),
                                                                            b[~nb].view(np.uint32))


@pytest.mark.filterwarnings("ignore::RuntimeWarning")  # random bytes hold inf/NaN f16 scales
@pytest.mark.parametrize("t", [8, 12, 13, 14])
def test_gguf_dequant_bit_exact(t):
    rng = np.random.default_rng(t)
    n = 8 * 2880
    data = synth.make_gguf(rng, t, n)
    ref = og.dequant_tensor(data, t, (8, 2880))
    got = otc.gguf_dequant(otc.as_u8(data), t, (8, 2880)).numpy()
    assert _same_bits(got, ref)
    raw = rng.integers(0, 256, synth.gguf_nbytes(t, 4096), dtype=np.uint8)  # any bytes, incl. odd f16 scales
    assert _same_bits(otc.gguf_dequant(otc.as_u8(raw), t, (4096,)).numpy(), og.dequant_tensor(raw, t, (4096,)))


def test_gguf_dequant_on_golden_vectors():
    with np.load(GOLDEN, allow_pickle=False) as g:
        for name, t in (("q5_k", 13), ("q6_k", 14), ("q4_k_k2880", 12), ("q6_k_k2880", 14)):
            data, want = g[f"{name}_data"], g[f"{name}_out"]
            got = otc.gguf_dequant(otc.as_u8(data), t, want.shape).numpy()
            assert _same_bits(got, want), name


def test_mxfp4_dequant_bit_exact_incl_scale_extremes():
    rng = np.random.default_rng(3)
    blocks = rng.integers(0, 256, (64, 90, 16), dtype=np.uint8)
    scales = rng.integers(0, 256, (64, 90), dtype=np.uint8)
    scales[0, :4] = (0, 1, 254, 255)
    ref = omx.dequant_mxfp4_no_transpose(blocks, scales, "f32")
    got = otc.mxfp4_dequant(torch.from_numpy(blocks), torch.from_numpy(scales)).numpy()
    assert _same_bits(got, ref)


def test_expert_ffns_match_the_oracle():
    rng = np.random.default_rng(5)
    H, I = 256, 128
    e = synth.make_mxfp4_expert(rng, H, I)
    x = synth.bf16_to_f32(synth.bf16_normal(rng, (3, H)))
    te = otc.torch_expert(e)
    wgu, wdn = otc.mxfp4_expert_weights(te)
    y = otc.mxfp4_expert_ffn(torch.from_numpy(x), wgu, wdn, te["gate_up_bias"], te["down_bias"]).numpy()
    np.testing.assert_allclose(y, oex.mxfp4_expert_forward(x, e), rtol=1e-4, atol=1e-4)
    g = synth.make_gguf_expert(rng, H, I, 12, 12, 14)
    tg = otc.torch_expert(g)
    y = otc.gguf_expert_ffn(torch.from_numpy(x), *otc.gguf_expert_weights(tg)).numpy()
    np.testing.assert_allclose(y, oex.gguf_expert_forward(x, g), rtol=1e-4, atol=1e-4)
