"""Seeded synthetic weights and activations in the native formats.

Shapes and distributions of the benchmark workloads (numbered 1-5):

1. Q8_0 matvec 2880x2880: d = fp16(|N(0, 0.02)|), q uniform int8 in [-127, 127], x fp32 N(0, 1).
2. One expert (Q4_K_M mix), hidden = inter = 2880: gate/up Q4_K (d, dmin = fp16(|N(0, 0.01)|),
   12 scale bytes and 128 quant bytes uniform), down Q6_K (ql/qh uniform, int8 sub-scales
   uniform, d = fp16(|N(0, 0.01)|)), x bf16 N(0, 1).
3. GPT-OSS-20B-shaped MoE layer: hidden 2880, inter 2880, 32 MXFP4 experts (nibbles uniform,
   e8m0 scales uniform in 119..125 = 2^-8..2^-2, bf16 biases N(0, 0.02)), router logits
   N(0, 1) -> top-4 -> softmax over the 4, clamped SwiGLU (7.0, 1.702).
4. Qwen3-30B-A3B-shaped MoE layer: hidden 2048, inter 768, 128 experts, gate/up Q5_K,
   down Q6_K, logits N(0, 1) - 1.1 ln(rank) (Zipf(1.1) popularity over a seeded rank
   permutation), softmax -> top-8 -> renormalise, SiLU-gated.
5. Prefill of workload 3 shapes: 2048 tokens, Zipf(1.1)-skewed top-4 of 32.

Everything is derived from ``numpy.random.default_rng(1000 + workload)`` so the
inputs are identical on any host.
"""
from __future__ import annotations

import numpy as np
import torch

from .expert_store import TensorLayout

QTYPE_SIZES = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def rng_for(workload: int, salt: int = 0) -> np.random.Generator:
    return np.random.default_rng(1000 + workload + 7919 * salt)


def _f16_abs_normal(rng, n, sigma) -> np.ndarray:
    return np.abs(rng.normal(0.0, sigma, n)).astype(np.float16).view(np.uint8).reshape(n, 2)


def make_gguf(rng: np.random.Generator, ggml_type: int, n_elems: int, sigma: float | None = None) -> np.ndarray:
    """Uniform random blocks of ``ggml_type`` covering n_elems values; fp16 scales |N(0, sigma)|."""
    be, ts = QTYPE_SIZES[ggml_type]
    assert n_elems % be == 0
    nb = n_elems // be
    if ggml_type == 8:
        blk = np.empty((nb, 34), dtype=np.uint8)
        blk[:, 0:2] = _f16_abs_normal(rng, nb, sigma or 0.02)
        blk[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
        return blk.reshape(-1)
    blk = rng.integers(0, 256, size=(nb, ts), dtype=np.uint8)
    s = sigma or 0.01
    if ggml_type in (12, 13):
        blk[:, 0:2] = _f16_abs_normal(rng, nb, s)
        blk[:, 2:4] = _f16_abs_normal(rng, nb, s)
    else:
        blk[:, 208:210] = _f16_abs_normal(rng, nb, s)
    return blk.reshape(-1)


def gguf_nbytes(ggml_type: int, n_elems: int) -> int:
    be, ts = QTYPE_SIZES[ggml_type]
    return n_elems // be * ts


def bf16_normal(rng, shape, sigma=1.0) -> np.ndarray:
    """bf16 values (as uint16 bits) of N(0, sigma), rounded to nearest even."""
    f = (rng.normal(0.0, sigma, shape)).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- MXFP4 experts
def mxfp4_layout(hidden: int, inter: int, bias: bool = True) -> TensorLayout:
    """GPT-OSS per-expert tensor order (safetensors key order)."""
    specs = {
        "gate_up_proj": ((2 * inter, hidden // 32, 16), torch.uint8),
        "gate_up_proj_scales": ((2 * inter, hidden // 32), torch.uint8),
    }
    if bias:
        specs["gate_up_proj_bias"] = ((2 * inter,), torch.bfloat16)
    specs["down_proj"] = ((hidden, inter // 32, 16), torch.uint8)
    specs["down_proj_scales"] = ((hidden, inter // 32), torch.uint8)
    if bias:
        specs["down_proj_bias"] = ((hidden,), torch.bfloat16)
    return TensorLayout(specs)


def make_mxfp4_expert(rng, hidden: int, inter: int, bias: bool = True, scale_lo: int = 119,
                      scale_hi: int = 125) -> dict:
    e = {
        "gate_up_blocks": rng.integers(0, 256, size=(2 * inter, hidden // 32, 16), dtype=np.uint8),
        "gate_up_scales": rng.integers(scale_lo, scale_hi + 1, size=(2 * inter, hidden // 32), dtype=np.uint8),
        "down_blocks": rng.integers(0, 256, size=(hidden, inter // 32, 16), dtype=np.uint8),
        "down_scales": rng.integers(scale_lo, scale_hi + 1, size=(hidden, inter // 32), dtype=np.uint8),
    }
    if bias:
        e["gate_up_bias_bits"] = bf16_normal(rng, (2 * inter,), 0.02)
        e["down_bias_bits"] = bf16_normal(rng, (hidden,), 0.02)
        e["gate_up_bias"] = bf16_to_f32(e["gate_up_bias_bits"])
        e["down_bias"] = bf16_to_f32(e["down_bias_bits"])
    return e


def pack_mxfp4_expert(e: dict, layout: TensorLayout) -> np.ndarray:
    slot = np.zeros(layout.total_bytes, dtype=np.uint8)
    parts = {
        "gate_up_proj": e["gate_up_blocks"],
        "gate_up_proj_scales": e["gate_up_scales"],
        "gate_up_proj_bias": e.get("gate_up_bias_bits"),
        "down_proj": e["down_blocks"],
        "down_proj_scales": e["down_scales"],
        "down_proj_bias": e.get("down_bias_bits"),
    }
    for name, arr in parts.items():
        if name in layout.offsets and arr is not None:
            o, n = layout.offsets[name], layout.sizes[name]
            slot[o : o + n] = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
    return slot


def mxfp4_tiled_layout(hidden: int, inter: int, bias: bool = True) -> TensorLayout:
    """The same tensors with both matrices in the 16-row MFMA tile order
    (tinyserve_amd.mx_tiles): blocks keep their shape and size, scales become
    [rows/16, tile_scale_bytes] per-tile areas."""
    from .mx_tiles import tile_scale_bytes

    specs = {
        "gate_up_proj": ((2 * inter, hidden // 32, 16), torch.uint8),
        "gate_up_proj_scales": ((2 * inter // 16, tile_scale_bytes(hidden)), torch.uint8),
    }
    if bias:
        specs["gate_up_proj_bias"] = ((2 * inter,), torch.bfloat16)
    specs["down_proj"] = ((hidden, inter // 32, 16), torch.uint8)
    specs["down_proj_scales"] = ((hidden // 16, tile_scale_bytes(inter)), torch.uint8)
    if bias:
        specs["down_proj_bias"] = ((hidden,), torch.bfloat16)
    return TensorLayout(specs)


def pack_mxfp4_expert_tiled(e: dict, layout: TensorLayout) -> np.ndarray:
    """Pack an expert (make_mxfp4_expert dict) into a mxfp4_tiled_layout slot."""
    from .mx_tiles import tile_mxfp4

    gb, gs = tile_mxfp4(e["gate_up_blocks"], e["gate_up_scales"])
    db, ds = tile_mxfp4(e["down_blocks"], e["down_scales"])
    return pack_mxfp4_expert({**e, "gate_up_blocks": gb, "gate_up_scales": gs, "down_blocks": db, "down_scales": ds},
                             layout)


# ----------------------------------------------------------------------------- GGUF experts
def gguf_layout(hidden: int, inter: int, gate_type: int, up_type: int, down_type: int) -> TensorLayout:
    """gate || up || down raw bytes (tinyserve/mmap_store.py:86-91)."""
    n = hidden * inter
    return TensorLayout({
        "gate": ((gguf_nbytes(gate_type, n),), torch.uint8),
        "up": ((gguf_nbytes(up_type, n),), torch.uint8),
        "down": ((gguf_nbytes(down_type, n),), torch.uint8),
    })


def make_gguf_expert(rng, hidden: int, inter: int, gate_type: int, up_type: int, down_type: int) -> dict:
    n = hidden * inter
    return {
        "hidden": hidden, "inter": inter,
        "gate_type": gate_type, "up_type": up_type, "down_type": down_type,
        "gate": make_gguf(rng, gate_type, n),
        "up": make_gguf(rng, up_type, n),
        "down": make_gguf(rng, down_type, n),
    }


def pack_gguf_expert(e: dict, layout: TensorLayout) -> np.ndarray:
    slot = np.zeros(layout.total_bytes, dtype=np.uint8)
    for name in ("gate", "up", "down"):
        o = layout.offsets[name]
        slot[o : o + e[name].size] = e[name]
    return slot


def zipf_logits(rng, T: int, E: int, s: float = 1.1) -> np.ndarray:
    """N(0, 1) logits plus a Zipf(s) popularity bias -s*ln(rank) over a seeded rank permutation."""
    ranks = rng.permutation(E) + 1
    bias = -s * np.log(ranks.astype(np.float64))
    return (rng.normal(0.0, 1.0, (T, E)) + bias).astype(np.float32)


# ----------------------------------------------------------------------------- workloads
def workload(n: int, n_experts: int | None = None, tokens: int | None = None) -> dict:
    """Inputs of benchmark workload ``n`` (1-5) as numpy arrays (experts packed per slot)."""
    rng = rng_for(n)
    if n == 1:
        N = K = 2880
        return {"type": 8, "N": N, "K": K, "w": make_gguf(rng, 8, N * K),
                "x": rng.normal(0.0, 1.0, K).astype(np.float32)}
    if n == 2:
        H = I = 2880
        e = make_gguf_expert(rng, H, I, 12, 12, 14)
        lay = gguf_layout(H, I, 12, 12, 14)
        return {"hidden": H, "inter": I, "expert": e, "layout": lay, "slot": pack_gguf_expert(e, lay),
                "x_bits": bf16_normal(rng, (1, H))}
    if n in (3, 5):
        H = I = 2880
        E = n_experts or 32
        lay = mxfp4_layout(H, I, bias=True)
        experts = [make_mxfp4_expert(rng, H, I) for _ in range(E)]
        pool = np.stack([pack_mxfp4_expert(e, lay) for e in experts])
        if n == 3:
            logits = rng.normal(0.0, 1.0, (1, E)).astype(np.float32)
            T = 1
        else:
            T = tokens or 2048
            logits = zipf_logits(rng, T, E)
        return {"hidden": H, "inter": I, "E": E, "top_k": 4, "experts": experts, "layout": lay, "pool": pool,
                "logits": logits, "x_bits": bf16_normal(rng, (T, H)), "route": "topk_then_softmax"}
    if n == 4:
        H, I = 2048, 768
        E = n_experts or 128
        lay = gguf_layout(H, I, 13, 13, 14)
        experts = [make_gguf_expert(rng, H, I, 13, 13, 14) for _ in range(E)]
        pool = np.stack([pack_gguf_expert(e, lay) for e in experts])
        T = tokens or 1
        return {"hidden": H, "inter": I, "E": E, "top_k": 8, "experts": experts, "layout": lay, "pool": pool,
                "logits": zipf_logits(rng, T, E), "x_bits": bf16_normal(rng, (T, H)), "route": "softmax_then_topk"}
    raise ValueError(f"unknown workload {n}")
