"""Host-side logic without a GPU: the MXFP4 tile packer, workload sizes, slot layouts,
the device checks of the torch wrappers and bench.py's one-GPU guard."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from tinyserve_amd import _lib, mx_tiles, ops, synth
from tinyserve_amd.expert_forward import gguf_expert_layout, mxfp4_expert_layout
from tinyserve_amd.expert_store import TensorLayout

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("N,K", [(16, 32), (32, 160), (64, 2880), (5760, 2880), (48, 4096)])
def test_tile_offsets_are_a_dense_bijection(N, K):
    G = K // 32
    boff, soff = mx_tiles.tile_offsets(N, K)
    bb, sb = mx_tiles.tile_sizes(N, K)
    assert bb == N * K // 2
    assert np.array_equal(np.sort(boff.reshape(-1)), np.arange(0, bb, 16))
    assert len(np.unique(soff)) == N * G and soff.max() < sb
    # the 1 KB piece of block (n, b) is group b // 4 of row tile n // 16, lane 16 (b % 4) + n % 16
    n, b = N - 1, G - 1
    assert boff[n, b] == (n // 16) * 256 * G + 1024 * (b // 4) + 16 * (16 * (b % 4) + n % 16)


def test_tile_packer_round_trip():
    rng = np.random.default_rng(0)
    N, K = 48, 2880
    blocks = rng.integers(0, 256, (N, K // 32, 16), dtype=np.uint8)
    scales = rng.integers(0, 256, (N, K // 32), dtype=np.uint8)
    tb, ts = mx_tiles.tile_mxfp4(blocks, scales)
    boff, soff = mx_tiles.tile_offsets(N, K)
    back = tb.reshape(-1, 16)[boff // 16]
    assert np.array_equal(back, blocks)
    assert np.array_equal(ts[soff], scales)
    pad = np.ones(ts.size, bool)
    pad[soff.reshape(-1)] = False
    assert not ts[pad].any(), "scale padding must be zero"


def test_tile_sizes_reject_bad_shapes():
    with pytest.raises(ValueError):
        mx_tiles.tile_sizes(20, 64)
    with pytest.raises(ValueError):
        mx_tiles.tile_sizes(32, 48)


def test_workload3_sizes_match_the_contract():
    """GPT-OSS-20B expert: 13,236,480 bytes; a decode step moves 52,957,568 algorithmic bytes."""
    lay = synth.mxfp4_layout(2880, 2880)
    assert lay.total_bytes == 13_236_480
    assert 4 * lay.total_bytes + 2 * 5760 + 128 == 52_957_568
    tl = synth.mxfp4_tiled_layout(2880, 2880)
    assert tl.sizes["gate_up_proj"] == lay.sizes["gate_up_proj"] and tl.sizes["down_proj"] == lay.sizes["down_proj"]
    assert all(o % 16 == 0 for o in tl.offsets.values())


def test_workload4_sizes_match_the_contract():
    lay = synth.gguf_layout(2048, 768, 13, 13, 14)
    assert lay.total_bytes == 3_452_928


def test_tensor_layout_contract():
    lay = TensorLayout({"a": ((3, 4), torch.uint8), "b": ((5,), torch.bfloat16), "c": ((2,), torch.float32)})
    assert lay.offsets == {"a": 0, "b": 12, "c": 22} and lay.sizes == {"a": 12, "b": 10, "c": 8}
    assert lay.total_bytes == 30


def test_layout_builders():
    L = mxfp4_expert_layout(synth.mxfp4_layout(512, 256))
    assert (L.format, L.act, L.hidden, L.inter, L.mx_tiled) == (_lib.EXPERT_MXFP4, _lib.ACT_SWIGLU_OAI, 512, 256, 0)
    assert L.bias_dtype == _lib.BF16 and L.gate_bias_off > 0 and L.down_bias_off > 0
    assert abs(L.swiglu_limit - 7.0) < 1e-6 and abs(L.swiglu_alpha - 1.702) < 1e-6
    Lt = mxfp4_expert_layout(synth.mxfp4_tiled_layout(512, 256), tiled=True)
    assert Lt.mx_tiled == 1
    G = gguf_expert_layout(synth.gguf_layout(2048, 768, 13, 13, 14), {"gate": 13, "up": 13, "down": 14},
                           {"gate": (2048, 768), "up": (2048, 768), "down": (768, 2048)})
    assert (G.format, G.act, G.hidden, G.inter) == (_lib.EXPERT_GGUF, _lib.ACT_SILU, 2048, 768)
    assert (G.gate_type, G.up_type, G.down_type) == (13, 13, 14)
    with pytest.raises(ValueError):
        mxfp4_expert_layout(TensorLayout({"gate_up_proj": ((10, 2, 16), torch.uint8),
                                          "gate_up_proj_scales": ((10, 2), torch.uint8),
                                          "down_proj": ((64, 1, 16), torch.uint8),
                                          "down_proj_scales": ((64, 1), torch.uint8)}))


def test_wrappers_reject_host_tensors():
    x = torch.zeros(32, dtype=torch.bfloat16)
    with pytest.raises((RuntimeError, ValueError), match="CUDA"):
        ops.gguf_matvec(x, torch.zeros(34, dtype=torch.uint8), 8, 1, 32)
    with pytest.raises((RuntimeError, ValueError), match="CUDA"):
        ops.mxfp4_dequant(torch.zeros((1, 1, 16), dtype=torch.uint8), torch.zeros((1, 1), dtype=torch.uint8))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
