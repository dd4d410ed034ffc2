"""Router linear on the GPU (tsa_router_logits) against a float64 reference, and
hidden states -> router -> routed fused decode with no host round trip
(tinyserve/_model_hooks.py:424-476: the router nn.Linear, GPT-OSS's with bias)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import expert as oex
from tests.helpers import assert_close_bf16
from tinyserve_amd import ops, synth
from tinyserve_amd.expert_forward import mxfp4_expert_layout

pytestmark = pytest.mark.gpu


def _bf16_bits(a: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bit patterns, rounding once (to nearest even) from the exact value."""
    f = np.asarray(a, np.float64)
    u = f.astype(np.float32).view(np.uint32).astype(np.uint64)
    # round-to-nearest-even on the float32 value is exact unless float32 rounding already
    # moved it; the tolerance below (one bf16 ulp) covers that double rounding
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("T,H,E,xdt,wdt,bias,odt", [
    (1, 2880, 32, torch.bfloat16, torch.bfloat16, True, torch.bfloat16),    # GPT-OSS router, decode
    (2, 2880, 32, torch.bfloat16, torch.bfloat16, True, torch.bfloat16),    # decode kernel, two tokens
    (3, 4104, 20, torch.float32, torch.float32, True, torch.float32),       # decode kernel, two passes over H
    (4, 72, 5, torch.float16, torch.bfloat16, False, torch.float32),        # decode kernel, H below one pass
    (5, 2048, 128, torch.bfloat16, torch.bfloat16, False, torch.float32),   # Qwen3-MoE router, fp32 logits
    (37, 64, 3, torch.float32, torch.float32, True, torch.float32),         # E not a multiple of 4, ragged T
    (9, 512, 16, torch.float16, torch.bfloat16, True, torch.float16),
    (2048, 2880, 32, torch.bfloat16, torch.bfloat16, True, torch.bfloat16), # prefill-sized batch
])
def test_router_logits_vs_float64(T, H, E, xdt, wdt, bias, odt):
    g = torch.Generator().manual_seed(T * 7 + H + E)
    x = torch.randn(T, H, generator=g).to(xdt)
    w = (torch.randn(E, H, generator=g) * 0.02).to(wdt)
    b = (torch.randn(E, generator=g) * 0.02).to(wdt) if bias else None
    out = ops.router_logits(x.cuda(), w.cuda(), b.cuda() if bias else None, out_dtype=odt).cpu()
    ref = x.double().numpy() @ w.double().numpy().T + (b.double().numpy() if bias else 0.0)
    if odt == torch.bfloat16:
        got = out.view(torch.int16).numpy().astype(np.int32) & 0xFFFF
        want = _bf16_bits(ref).astype(np.int32)
        assert np.abs(got - want).max() <= 1, "bf16 logits more than one ulp from the exact value"
    else:
        scale = np.abs(x.double().numpy()) @ np.abs(w.double().numpy()).T + 1e-30
        err = np.abs(out.double().numpy() - ref) / scale
        tol = 2e-6 if odt == torch.float32 else 1e-3
        assert err.max() < tol, err.max()


def test_router_rejects_bad_shapes():
    x = torch.zeros(2, 12, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(4, 12, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ops.router_logits(x, w)


def test_gated_decode_from_hidden_states():
    """x -> router (bf16, with bias) -> top-4 -> tiled MXFP4 experts, all on the GPU."""
    rng = np.random.default_rng(21)
    H, I, E, k, T = 1024, 512, 8, 4, 3
    lay = synth.mxfp4_tiled_layout(H, I)
    experts = [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)]
    pool = torch.from_numpy(np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in experts])).cuda()
    L = mxfp4_expert_layout(lay, tiled=True)
    x_bits = synth.bf16_normal(rng, (T, H))
    x = torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16).cuda()
    rw = torch.from_numpy(synth.bf16_normal(rng, (E, H), 0.05).view(np.int16)).view(torch.bfloat16).cuda()
    rb = torch.from_numpy(synth.bf16_normal(rng, (E,), 0.05).view(np.int16)).view(torch.bfloat16).cuda()
    y, idx, w = ops.moe_decode_gated(L, pool, torch.arange(E, dtype=torch.int32, device="cuda"), x, rw, rb, k,
                                     return_routing=True)
    logits = ops.router_logits(x, rw, rb).float().cpu().numpy()  # the logits the decode routed
    ridx, rwt = oex.route_topk_then_softmax(logits, k)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_allclose(w.cpu().numpy(), rwt, rtol=1e-5)
    ref = oex.moe_combine(synth.bf16_to_f32(x_bits), ridx, rwt, lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))
    assert_close_bf16(y, ref, "gated decode")
