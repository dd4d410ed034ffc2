"""Write golden vectors for the oracle functions no known-answer test pins.

Run once, in the development container where the reference is mounted:

    python tests/golden/make_golden.py /root/reference

It loads exactly two reference modules by file path (both import only torch):
``tinyserve/gguf_dequant_torch.py`` and ``tinyserve/mxfp4.py``, and records
inputs + outputs for the cases the reference's own tests leave open:

* Q5_K and Q6_K dequantisation (no known-answer test exists in the reference);
* the flat block stream at K = 2880 (rows straddle 256-value super-blocks) for
  Q4_K and Q6_K;
* MXFP4 dequantisation at the e8m0 extremes (0, 1, 254, 255) in bf16 and fp32.

The fixtures are plain ``.npz`` arrays (no pickles). Nothing on the GPU box runs this.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(ref_root: str, rel: str, name: str):
    spec = importlib.util.spec_from_file_location(name, os.path.join(ref_root, rel))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _kquant_bytes(rng, ggml_type: int, n_blocks: int) -> np.ndarray:
    """Uniform random blocks with finite fp16 scales; every 5th block gets subnormal d/dmin."""
    ts = {12: 144, 13: 176, 14: 210}[ggml_type]
    blk = rng.integers(0, 256, size=(n_blocks, ts), dtype=np.uint8)
    offs = [0, 2] if ggml_type in (12, 13) else [208]
    for o in offs:
        v = np.abs(rng.normal(0.0, 0.01, n_blocks)).astype(np.float16)
        v[::5] = np.float16(2.0 ** -20)  # fp16 subnormal
        blk[:, o : o + 2] = v.view(np.uint8).reshape(n_blocks, 2)
    return blk.reshape(-1)


def main(ref_root: str) -> None:
    gdt = _load(ref_root, "tinyserve/gguf_dequant_torch.py", "_ref_gguf_dequant_torch")
    mx = _load(ref_root, "tinyserve/mxfp4.py", "_ref_mxfp4")
    rng = np.random.default_rng(20261201)
    arrays = {}

    # Q5_K / Q6_K: 24 blocks each, shape (24*256,)
    for t, name in ((13, "q5_k"), (14, "q6_k")):
        data = _kquant_bytes(rng, t, 24)
        out = gdt.dequant_tensor(torch.from_numpy(data.copy()), t, (24 * 256,)).numpy()
        arrays[f"{name}_data"] = data
        arrays[f"{name}_out"] = out.astype(np.float32)

    # Row-straddling flat stream: N=4 rows of K=2880 (45 super-blocks)
    for t, name in ((12, "q4_k_k2880"), (14, "q6_k_k2880")):
        data = _kquant_bytes(rng, t, 45)
        out = gdt.dequant_tensor(torch.from_numpy(data.copy()), t, (4, 2880)).numpy()
        arrays[f"{name}_data"] = data
        arrays[f"{name}_out"] = out.astype(np.float32)

    # MXFP4 extremes: 6 rows x 4 groups; scales cover 0, 1, 126, 127, 128, 254, 255
    blocks = rng.integers(0, 256, size=(6, 4, 16), dtype=np.uint8)
    blocks[0, 0, :] = np.arange(16, dtype=np.uint8) * 17  # both nibbles = every code
    scales = rng.integers(119, 126, size=(6, 4), dtype=np.uint8)
    scales[0] = [0, 1, 254, 255]
    scales[1] = [126, 127, 128, 255]
    scales[2, 0] = 0
    tb, ts_ = torch.from_numpy(blocks.copy()), torch.from_numpy(scales.copy())
    arrays["mxfp4_blocks"] = blocks
    arrays["mxfp4_scales"] = scales
    arrays["mxfp4_out_bf16_bits"] = mx.dequant_mxfp4_no_transpose(tb, ts_, torch.bfloat16).view(torch.int16).numpy()
    arrays["mxfp4_out_f32"] = mx.dequant_mxfp4_no_transpose(tb, ts_, torch.float32).numpy()
    arrays["mxfp4_T_out_f32"] = mx.dequant_mxfp4(tb, ts_, torch.float32).numpy()

    path = os.path.join(HERE, "dequant_golden.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: " + ", ".join(f"{k}{tuple(v.shape)}" for k, v in arrays.items()))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
