"""tsa_moe_decode_routed_noalloc (workspace in the library's per-GPU device array) against
tsa_moe_decode_routed with a caller workspace, through the C-ABI: the same kernels on the same
inputs give identical outputs and routing, on two calls in a row (the second with fewer
tokens, so it reuses the array a larger call left behind), for both MXFP4 layouts; sizes
beyond the array are rejected."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import bf16_dev
from tinyserve_amd import _lib, ops, synth
from tinyserve_amd.expert_forward import mxfp4_expert_layout

pytestmark = pytest.mark.gpu


def _noalloc(L, pool, es, logits, x, k, y, idx, w):
    T, E = logits.shape
    return _lib.load().tsa_moe_decode_routed_noalloc(
        ctypes.byref(L), pool.data_ptr(), pool.shape[0], es.data_ptr(), E, logits.data_ptr(), _lib.F32, 0, T, k,
        x.data_ptr(), _lib.BF16, y.data_ptr(), _lib.BF16, idx.data_ptr(), w.data_ptr(),
        torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("tiled", [True, False])
def test_noalloc_decode_matches_workspace_decode(tiled):
    H, I, E, k = 1024, 512, 8, 4
    rng = np.random.default_rng(11 + tiled)
    experts = [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]
    if tiled:
        lay = synth.mxfp4_tiled_layout(H, I)
        pool = np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])
    else:
        lay = synth.mxfp4_layout(H, I)
        pool = np.stack([synth.pack_mxfp4_expert(e, lay) for e in experts])
    L = mxfp4_expert_layout(lay, tiled=tiled)
    pool = torch.from_numpy(pool).cuda()
    es = torch.arange(E, dtype=torch.int32, device="cuda")
    for T in (6, 2):  # the second call is smaller
        logits = torch.from_numpy(rng.normal(size=(T, E)).astype(np.float32)).cuda()
        x = bf16_dev(synth.bf16_normal(rng, (T, H)))
        ref, ridx, rw = ops.moe_decode_routed(L, pool, es, logits, x, k, return_routing=True)
        y = torch.empty_like(ref)
        idx = torch.empty_like(ridx)
        w = torch.empty_like(rw)
        _lib.check(_noalloc(L, pool, es, logits, x, k, y, idx, w))
        torch.cuda.synchronize()
        assert torch.equal(idx, ridx), f"T {T}: routing differs"
        assert torch.equal(w, rw), f"T {T}: weights differ"
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"T {T}: outputs differ"


def test_noalloc_decode_rejects_sizes_beyond_its_array():
    H = I = 2880
    L = mxfp4_expert_layout(synth.mxfp4_tiled_layout(H, I), tiled=True)
    n = ctypes.c_int64()
    T = 512
    _lib.check(_lib.load().tsa_moe_decode_workspace_size(ctypes.byref(L), T, 4, ctypes.byref(n)))
    assert n.value > 8 << 20
    dummy = torch.zeros(16, dtype=torch.int32, device="cuda")
    rc = _lib.load().tsa_moe_decode_routed_noalloc(
        ctypes.byref(L), dummy.data_ptr(), 1, dummy.data_ptr(), 4, dummy.data_ptr(), _lib.F32, 0, T, 4,
        dummy.data_ptr(), _lib.BF16, dummy.data_ptr(), _lib.BF16, None, None, torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.ERR_WORKSPACE
    assert "scratch" in _lib.load().tsa_last_error().decode()
