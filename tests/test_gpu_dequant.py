"""GPU dequantisation parity: bit-exact against the oracle and the golden vectors."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import gguf as og
from oracle import mxfp4 as omx
from tests.helpers import bits_equal, dev_u8
from tinyserve_amd import ops, synth

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "dequant_golden.npz")


@pytest.mark.parametrize("name,gtype,shape", [
    ("q5_k", 13, (6144,)), ("q6_k", 14, (6144,)), ("q4_k_k2880", 12, (4, 2880)), ("q6_k_k2880", 14, (4, 2880)),
])
def test_gguf_dequant_golden(name, gtype, shape):
    g = np.load(GOLDEN)
    out = ops.gguf_dequant(dev_u8(g[name + "_data"]), gtype, shape)
    assert bits_equal(out.cpu().numpy(), g[name + "_out"]), name


@pytest.mark.parametrize("gtype", [8, 12, 13, 14])
@pytest.mark.parametrize("offset", [0, 1, 2])
def test_gguf_dequant_random_vs_oracle(gtype, offset):
    rng = np.random.default_rng(7 + gtype + 100 * offset)
    be, ts = synth.QTYPE_SIZES[gtype]
    n = 256 * 37
    data = synth.make_gguf(rng, gtype, n)
    blk = data.reshape(-1, ts)
    # subnormal fp16 scales in every 9th block
    if gtype in (12, 13):
        blk[::9, 0:2] = np.array([0x08, 0x00], np.uint8)  # fp16 subnormal 8 * 2^-24
    elif gtype == 14:
        blk[::9, 208:210] = np.array([0x11, 0x00], np.uint8)
    else:
        blk[::9, 0:2] = np.array([0x03, 0x00], np.uint8)
    ref = og.dequant_tensor(data, gtype, (n,))
    out = ops.gguf_dequant(dev_u8(data, offset), gtype, (n,))
    assert bits_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("gtype", [12, 14])
def test_gguf_dequant_half_outputs(gtype):
    rng = np.random.default_rng(3)
    n = 256 * 8
    data = synth.make_gguf(rng, gtype, n)
    ref = og.dequant_tensor(data, gtype, (n,))
    out_bf = ops.gguf_dequant(dev_u8(data), gtype, (n,), torch.bfloat16)
    assert np.array_equal(out_bf.float().cpu().numpy(), omx.bf16_round(ref))
    out_h = ops.gguf_dequant(dev_u8(data), gtype, (n,), torch.float16)
    assert np.array_equal(out_h.float().cpu().numpy(), ref.astype(np.float16).astype(np.float32))


def test_gguf_dequant_f32_f16_passthrough():
    v = np.random.default_rng(1).normal(size=96).astype(np.float32)
    out = ops.gguf_dequant(dev_u8(v), 0, (96,))
    assert bits_equal(out.cpu().numpy(), v)
    h = v.astype(np.float16)
    out = ops.gguf_dequant(dev_u8(h), 1, (96,))
    assert bits_equal(out.cpu().numpy(), h.astype(np.float32))


def test_mxfp4_dequant_golden():
    g = np.load(GOLDEN)
    b, s = torch.from_numpy(g["mxfp4_blocks"]).cuda(), torch.from_numpy(g["mxfp4_scales"]).cuda()
    out32 = ops.mxfp4_dequant(b, s, torch.float32)
    assert bits_equal(out32.cpu().numpy(), g["mxfp4_out_f32"])
    outT = ops.mxfp4_dequant(b, s, torch.float32, transpose=True)
    assert bits_equal(outT.cpu().numpy(), g["mxfp4_T_out_f32"])
    out16 = ops.mxfp4_dequant(b, s, torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    ref16 = g["mxfp4_out_bf16_bits"].view(np.uint16)
    nan_ref, nan_out = (ref16 & 0x7FFF) > 0x7F80, (out16 & 0x7FFF) > 0x7F80
    assert np.array_equal(nan_ref, nan_out)
    assert np.array_equal(out16[~nan_out], ref16[~nan_ref])


@pytest.mark.parametrize("N,G", [(5760, 90), (33, 3), (1, 1)])
def test_mxfp4_dequant_random_vs_oracle(N, G):
    rng = np.random.default_rng(N + G)
    blocks = rng.integers(0, 256, size=(N, G, 16), dtype=np.uint8)
    scales = rng.integers(100, 150, size=(N, G), dtype=np.uint8)
    ref = omx.dequant_mxfp4_no_transpose(blocks, scales, "f32")
    out = ops.mxfp4_dequant(torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda(), torch.float32)
    assert bits_equal(out.cpu().numpy(), ref)
    out_bf = ops.mxfp4_dequant(torch.from_numpy(blocks).cuda(), torch.from_numpy(scales).cuda(), torch.bfloat16)
    assert np.array_equal(out_bf.float().cpu().numpy(), omx.bf16_round(ref))
