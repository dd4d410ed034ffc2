"""Benchmark of the MoE expert dequant-matvec hot path on one MI355X.

Default workload (workload 3, the headline metric's): GPT-OSS-20B-shaped MXFP4 MoE layer decode,
hidden 2880, 32 experts, top-4 (topk -> softmax), batch 1. One step = one token
through one MoE layer: router top-k on the GPU + the fused expert FFN (gate_up ->
clamped SwiGLU -> down, biases, weighted top-k sum). Steps rotate over --layers
distinct layers of 32 resident experts (24 x 423.6 MB = 10.2 GB by default), each
step with its own router logits and activations, so the 256 MB Infinity Cache
cannot serve repeated weight reads. Inputs are resident in HBM before timing.

Timed region: a HIP graph holding the steps, replayed between two HIP events on the
capture stream, bracketed by torch.cuda.synchronize(). value = algorithmic bytes per
step / time per step (GB/s); algorithmic bytes = the 4 selected experts' weights,
scales and biases + activations in/out + logits.

--workload 5 measures batched prefill instead: 2048 tokens x hidden 2880 through the same
layer shape with Zipf-skewed top-4 routing, grouped by expert and run on the grouped
MXFP4 MFMA GEMMs (one step = one whole prefill of the layer: routing, grouping, gate_up +
SwiGLU, down, weighted combine); value = algorithmic FLOPs / time (TFLOP/s), against the
dense bf16 MFMA peak.

--workload 1 / 2 / 4 measure the GGUF paths (a Q8_0 matvec, one Q4_K/Q6_K expert, a
Qwen3-30B-A3B-shaped Q5_K/Q6_K MoE layer) the same way, in GB/s of algorithmic bytes.

--workload 6 measures the grouped GGUF prefill at workload 4's layer shape (1024 tokens,
128 Q5_K/Q6_K experts, zipf top-8): routing, grouping, both grouped GEMMs on bf16 MFMA
(blocks decoded to bf16 in LDS) and the combine, in TFLOP/s against the dense bf16 peak.

--workload 7 measures the standalone MXFP4 matvec (tsa_mxfp4_matvec, the reference's
dot_scaled_vecmat / _mxfp4_linear) at GPT-OSS-20B's gate_up shape: 5760 x 2880 checkpoint-order
blocks and scales, bf16 bias and x, batch 1, in GB/s of algorithmic bytes.

--workload 8 is workload 3 from the hidden states: each step runs the GPT-OSS router linear
(bf16 weight [32, 2880] and bias, tsa_router_logits) and then the routed decode on its logits,
so it measures the per-layer cost from hidden states to y (router, gate_up, down).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload {1,2,3,4,5,6,7,8}]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from tinyserve_amd import _lib, ops, synth  # noqa: E402
from tinyserve_amd.expert_forward import gguf_expert_layout, mxfp4_expert_layout  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 (the prefill GEMMs' bf16 form)
# The fp6 form runs v_mfma_scale_f32_32x32x64_f8f6f4 on fp4 weights x fp6 activation terms
# (MI355X dense fp6/fp4: 10.1 PFLOP/s), two products (hi and lo term) per multiply-add of
# the GEMM: an algorithmic ceiling of 5.05 PFLOP/s (the int8 / fp8 dense peak is 5.0).
MFMA_F6F4_ALGO_PEAK_TFLOPS = 10100.0 / 2
COPY_ELEMS = 64 << 20  # calibration copy: 64 Mi float32 read + written (256 MiB each way)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def copy_calibration(dev) -> None:
    """A plain elementwise copy of known size (reads and writes 4 * COPY_ELEMS bytes),
    launched three times so that a rocprofv3 --pmc pass can scale FETCH_SIZE/WRITE_SIZE."""
    a = torch.ones(COPY_ELEMS, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    del a, b


def _pmc_rows(d: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, counter value per dispatch) from a rocprofv3 --output-format csv run."""
    import csv
    import glob

    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name") == counter:
                    rows.append((r["Kernel_Name"], float(r["Counter_Value"])))
    return rows


# The kernels of one step of each decode workload (name substrings; "3c" = workload 3 with
# the experts in checkpoint order).
STEP_KERNELS = {"1": ("gs_matvec_kernel",), "2": ("gs_gate_up_kernel", "gs_down_kernel"),
                "3": ("mxt_gate_up_kernel", "mxt_down_kernel"), "3c": ("mxt_gate_up_kernel", "mxt_down_kernel"),
                "4": ("gq_phase_a", "gq_phase_b"), "7": ("mxfp4_mv_mfma_kernel",),
                "8": ("router_logits_decode_kernel", "mxt_gate_up_kernel", "mxt_down_kernel"),
                "5": ("pf_gemm_kernel",), "6": ("gf_step_kernel", "gf_gemm_kernel")}


def summarize_pmc(fetch_dir: str, write_dir: str, key: str, command: str) -> dict:
    """Calibrated HBM bytes per step: for every kernel of the step (each distinct kernel
    name matching STEP_KERNELS[key]) the mean counter value per dispatch, summed."""
    out = {"workload": key, "kernels": {}, "command": command}
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        rows = _pmc_rows(d, counter)
        copy = [v for k, v in rows if "MulFunctor" in k]  # torch.mul's elementwise kernel
        names = sorted({k for k, _ in rows if any(s in k for s in STEP_KERNELS[key])})
        if not copy or not names:
            raise SystemExit(f"{counter}: no calibration copy ({len(copy)}) or step kernels ({names}) in {d}")
        copy_kib = max(copy)  # the 256 MiB copy is the largest elementwise dispatch
        factor = copy_kib * 1024.0 / (4.0 * COPY_ELEMS)
        per = {}
        for n in names:
            vals = [v for k, v in rows if k == n]
            per[n] = {"kib_per_dispatch": float(np.mean(vals)), "dispatches": len(vals),
                      "bytes_per_dispatch": float(np.mean(vals)) * 1024.0 / factor}
            out["kernels"].setdefault(n, {})[counter] = per[n]
        out[counter] = {"copy_kib": copy_kib, "copy_factor": factor,
                        "bytes_per_step": sum(v["bytes_per_dispatch"] for v in per.values())}
    out["traffic_bytes_per_step"] = out["FETCH_SIZE"]["bytes_per_step"] + out["WRITE_SIZE"]["bytes_per_step"]
    return out


def _read_traffic() -> dict:
    try:
        with open(TRAFFIC_FILE) as fh:
            t = json.load(fh)
        return t if isinstance(t, dict) and "workloads" in t else {"workloads": {}}
    except (OSError, ValueError):
        return {"workloads": {}}


def load_traffic(key: str):
    return _read_traffic()["workloads"].get(key)


def _bf16(bits: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16).to(dev)


class MoEWorkload:
    """Resident layers of experts + per-step router logits and activations."""

    def __init__(self, wl: int, n_layers: int, n_steps: int, dev: torch.device, tiled: bool = True):
        self.wl = wl
        self.gated = wl == 8  # workload 8: workload 3 from hidden states, through the router linear
        wl = 3 if self.gated else wl
        base = synth.workload(wl)
        self.H, self.I, self.E, self.k = base["hidden"], base["inter"], base["E"], base["top_k"]
        self.route = base["route"]
        lay = base["layout"]
        self.slot_bytes = lay.total_bytes  # the checkpoint-order expert: the algorithmic bytes
        pool0 = base["pool"]
        self.tiled = tiled and wl == 3
        if wl == 3:
            if self.tiled:  # the resident pool in the 16-row MFMA tile order (same weights)
                lay = synth.mxfp4_tiled_layout(self.H, self.I)
                pool0 = np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in base["experts"]])
            self.L = mxfp4_expert_layout(lay, tiled=self.tiled)
        else:
            self.L = gguf_expert_layout(lay, {"gate": 13, "up": 13, "down": 14},
                                        {"gate": (self.H, self.I), "up": (self.H, self.I), "down": (self.I, self.H)})
        g = torch.Generator(device=dev)
        g.manual_seed(20261201 + wl)
        # layer 0 = the seeded numpy workload (parity-checked by the tests); others random on the GPU
        self.pools = [torch.from_numpy(pool0).to(dev)]
        for _ in range(1, n_layers):
            p = torch.randint(0, 256, pool0.shape, dtype=torch.uint8, device=dev, generator=g)
            self._fix_scales(p, lay, g)
            self.pools.append(p)
        self.logits = torch.randn((n_steps, self.E), device=dev, generator=g)
        if wl == 4:
            self.logits += torch.from_numpy(synth.zipf_logits(np.random.default_rng(7), 1, self.E)).to(dev)
        self.x = torch.randn((n_steps, self.H), device=dev, generator=g).to(torch.bfloat16)
        self.y = torch.empty((n_steps, self.H), device=dev, dtype=torch.bfloat16)
        self.idx = torch.empty((n_steps, self.k), device=dev, dtype=torch.int32)
        self.w = torch.empty((n_steps, self.k), device=dev, dtype=torch.float32)
        self.ws = ops.moe_decode_workspace(self.L, 1, self.k, dev)
        self.expert_slot = torch.arange(self.E, dtype=torch.int32, device=dev)
        self.n_layers = n_layers
        if self.gated:  # GPT-OSS router per layer: bf16 weight [E, H] and bias, N(0, 1/H) and N(0, 0.02)
            self.router_w = [(torch.randn((self.E, self.H), device=dev, generator=g) * self.H ** -0.5).to(
                torch.bfloat16) for _ in range(n_layers)]
            self.router_b = [(torch.randn(self.E, device=dev, generator=g) * 0.02).to(torch.bfloat16)
                             for _ in range(n_layers)]
            self.step_logits = torch.empty((n_steps, self.E), device=dev, dtype=torch.bfloat16)

    @staticmethod
    def _fix_scales(p: torch.Tensor, lay, g, gguf_types=(13, 13, 14)):
        """Random bytes are valid MXFP4 nibbles; scales and biases need the workload's ranges
        (GGUF: the ggml types of gate, up and down)."""
        if "gate_up_proj_scales" in lay.offsets:
            for name in ("gate_up_proj_scales", "down_proj_scales"):
                o, n = lay.offsets[name], lay.sizes[name]
                p[:, o : o + n] = torch.randint(119, 126, (p.shape[0], n), dtype=torch.uint8, device=p.device,
                                                generator=g)
            for name in ("gate_up_proj_bias", "down_proj_bias"):
                if name in lay.offsets:
                    o, n = lay.offsets[name], lay.sizes[name]
                    b = (torch.randn((p.shape[0], n // 2), device=p.device, generator=g) * 0.02).to(torch.bfloat16)
                    p[:, o : o + n] = b.view(torch.uint8)
        else:  # GGUF: keep the fp16 super-block scales small and finite (one strided write per field)
            for name, t in zip(("gate", "up", "down"), gguf_types):
                o, n = lay.offsets[name], lay.sizes[name]
                be, ts = synth.QTYPE_SIZES[t]
                blk = p[:, o : o + n].view(p.shape[0], -1, ts)  # [experts, super-blocks, bytes]
                for off in ([0, 2] if t in (12, 13) else [208]):
                    d = (torch.randn(blk.shape[:2], device=p.device, generator=g).abs() * 0.01).to(torch.float16)
                    blk[:, :, off : off + 2] = d.view(torch.uint8).view(*blk.shape[:2], 2)

    def bytes_per_step(self) -> int:
        """Algorithmic HBM bytes of one step: k experts' weights + activations + logits (fp32
        in; workload 8 reads the bf16 router weight and bias and writes and reads bf16 logits)."""
        if self.gated:
            return self.k * self.slot_bytes + 2 * self.H * 2 + self.E * self.H * 2 + self.E * 2 + 2 * self.E * 2
        return self.k * self.slot_bytes + 2 * self.H * 2 + self.E * 4

    def step(self, s: int) -> None:
        """One token through one layer on the current stream: the routed decode (routing inside
        its launches) from the step's logits, or (workload 8) from the hidden states through
        the router linear first (tsa_router_logits)."""
        lib = _lib.load()
        st = torch.cuda.current_stream().cuda_stream
        li = s % self.n_layers
        pool = self.pools[li]
        lg, lg_dtype = self.logits[s : s + 1], _lib.F32
        if self.gated:
            lg, lg_dtype = self.step_logits[s : s + 1], _lib.BF16
            _lib.check(lib.tsa_router_logits(self.x[s].data_ptr(), _lib.BF16, 1, self.H, self.router_w[li].data_ptr(),
                                             _lib.BF16, self.router_b[li].data_ptr(), _lib.BF16, self.E, lg.data_ptr(),
                                             _lib.BF16, st))
        _lib.check(lib.tsa_moe_decode_routed(
            ctypes.byref(self.L), pool.data_ptr(), pool.shape[0], self.expert_slot.data_ptr(), self.E, lg.data_ptr(),
            lg_dtype, ops.ROUTE_MODES[self.route], 1, self.k, self.x[s].data_ptr(), _lib.BF16, self.y[s].data_ptr(),
            _lib.BF16, self.idx[s].data_ptr(), self.w[s].data_ptr(), self.ws.data_ptr(), self.ws.numel(), st))


class GgufWorkload:
    """Workloads 1 and 2: one GGUF matrix (Q8_0 2880 x 2880, fp32 x; tsa_gguf_matvec) or one
    GGUF expert (Q4_K gate/up, Q6_K down, bf16 x; tsa_moe_decode with k = 1), over copies of
    the seeded weights rotated per step (about 0.5 GB) so the 256 MB Infinity Cache cannot
    serve them."""

    def __init__(self, wl: int, n_steps: int, dev: torch.device):
        self.wl = wl
        base = synth.workload(wl)
        self.tiled = False
        if wl == 1:
            self.N, self.K = base["N"], base["K"]
            self.w_bytes = base["w"].size
            self.copies = 64
            self.w = torch.from_numpy(np.tile(base["w"], self.copies)).to(dev)
            self.x = torch.from_numpy(base["x"]).to(dev).view(1, -1)
            self.y = torch.empty((1, self.N), device=dev)
        else:
            self.H, self.I = base["hidden"], base["inter"]
            self.L = gguf_expert_layout(base["layout"], {"gate": 12, "up": 12, "down": 14},
                                        {"gate": (self.H, self.I), "up": (self.H, self.I), "down": (self.I, self.H)})
            self.copies = 32
            self.pool = torch.from_numpy(np.tile(base["slot"], self.copies)).to(dev).view(self.copies, -1)
            self.x = _bf16(base["x_bits"], dev).view(1, -1)
            self.y = torch.empty((1, self.H), device=dev, dtype=torch.bfloat16)
            self.slots = (torch.arange(n_steps, dtype=torch.int32, device=dev) % self.copies).view(-1, 1)
            self.one = torch.ones((1, 1), device=dev)
            self.ws = ops.moe_decode_workspace(self.L, 1, 1, dev)
            self.slot_bytes = base["layout"].total_bytes
        self.logits = self.x  # the step count source for the warmup loop

    def bytes_per_step(self) -> int:
        """Algorithmic bytes: weights + activations in and out (fp32 for workload 1, bf16 for 2)."""
        if self.wl == 1:
            return self.w_bytes + 2 * 4 * self.K
        return self.slot_bytes + 2 * 2 * self.H

    def step(self, s: int) -> None:
        lib = _lib.load()
        st = torch.cuda.current_stream().cuda_stream
        if self.wl == 1:
            w = self.w[(s % self.copies) * self.w_bytes:]
            _lib.check(lib.tsa_gguf_matvec(8, w.data_ptr(), self.w_bytes, self.x.data_ptr(), _lib.F32, 1, self.K,
                                           self.y.data_ptr(), _lib.F32, self.N, st))
        else:
            _lib.check(lib.tsa_moe_decode(ctypes.byref(self.L), self.pool.data_ptr(), self.copies,
                                          self.slots[s].data_ptr(), self.one.data_ptr(), 1, 1, self.x.data_ptr(),
                                          _lib.BF16, self.y.data_ptr(), _lib.BF16, self.ws.data_ptr(), self.ws.numel(),
                                          st))


class MxMatvecWorkload:
    """Workload 7: one MXFP4 matrix in the checkpoint order ([N, K/32, 16] blocks, [N, K/32]
    e8m0 scales, bf16 bias), GPT-OSS-20B's gate_up shape, y = x W^T + b for one bf16 token
    (tsa_mxfp4_matvec), over copies rotated per step (about 0.56 GB) so the 256 MB
    Infinity Cache cannot serve them. Random codes, scales in 2^-8 .. 2^-2."""

    def __init__(self, n_steps: int, dev: torch.device):
        self.N, self.K = 5760, 2880
        G = self.K // 32
        self.copies = 64
        g = torch.Generator(device=dev)
        g.manual_seed(20261207)
        self.blocks = torch.randint(0, 256, (self.copies, self.N, G * 16), dtype=torch.uint8, device=dev, generator=g)
        self.scales = torch.randint(119, 126, (self.copies, self.N, G), dtype=torch.uint8, device=dev, generator=g)
        self.bias = (torch.randn(self.N, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        self.x = torch.randn((n_steps, self.K), device=dev, generator=g).to(torch.bfloat16)
        self.y = torch.empty((n_steps, self.N), device=dev, dtype=torch.bfloat16)
        self.logits = self.x  # the step count source for the warmup loop
        self.tiled = False

    def bytes_per_step(self) -> int:
        """Blocks (K/2 bytes per row) + scales (K/32) + bf16 bias, x and y."""
        return self.N * (self.K // 2 + self.K // 32) + 2 * self.N + 2 * self.K + 2 * self.N

    def step(self, s: int) -> None:
        lib = _lib.load()
        st = torch.cuda.current_stream().cuda_stream
        c = s % self.copies
        _lib.check(lib.tsa_mxfp4_matvec(self.blocks[c].data_ptr(), self.scales[c].data_ptr(), self.bias.data_ptr(),
                                        _lib.BF16, self.x[s].data_ptr(), _lib.BF16, 1, self.y[s].data_ptr(), _lib.BF16,
                                        self.N, self.K, st))


def _routed_experts(logits: torch.Tensor, k: int) -> int:
    """Distinct experts in the top-k of every token (the selection is by logit in every
    routing mode)."""
    return int(torch.unique(torch.topk(logits.float().cpu(), k, dim=-1).indices).numel())


class PrefillWorkload:
    """Workload 5: resident tiled MXFP4 layers, router logits and activations of a
    2048-token prefill; one step = one layer's whole batched MoE."""

    def __init__(self, n_layers: int, dev: torch.device, prefill_mfma: int = _lib.PREFILL_FP6):
        base = synth.workload(5)
        self.H, self.I, self.E, self.k = base["hidden"], base["inter"], base["E"], base["top_k"]
        lay = synth.mxfp4_tiled_layout(self.H, self.I)
        self.L = mxfp4_expert_layout(lay, tiled=True, prefill_mfma=prefill_mfma)
        self.slot_bytes = lay.total_bytes
        pool0 = np.stack([synth.pack_mxfp4_expert_tiled(e, lay) for e in base["experts"]])
        g = torch.Generator(device=dev)
        g.manual_seed(20261205)
        self.pools = [torch.from_numpy(pool0).to(dev)]
        for _ in range(1, n_layers):  # further layers: random nibbles, scales and biases in range
            p = torch.randint(0, 256, pool0.shape, dtype=torch.uint8, device=dev, generator=g)
            MoEWorkload._fix_scales(p, lay, g)
            self.pools.append(p)
        self.logits = torch.from_numpy(base["logits"]).to(dev)
        self.x = _bf16(base["x_bits"], dev)
        self.T = self.x.shape[0]
        self.y = torch.empty_like(self.x)
        self.idx = torch.empty((self.T, self.k), dtype=torch.int32, device=dev)
        self.w = torch.empty((self.T, self.k), dtype=torch.float32, device=dev)
        self.expert_slot = torch.arange(self.E, dtype=torch.int32, device=dev)
        self.ws = ops.moe_prefill_workspace(self.L, self.T, self.k, self.E, dev)
        self.n_layers = n_layers

    def flops_per_step(self) -> int:
        """2 x (gate_up 2I x H + down H x I) multiply-adds per (token, expert) assignment."""
        return 2 * self.T * self.k * (2 * self.I * self.H + self.H * self.I)

    def min_bytes_per_step(self) -> int:
        """HBM bytes the step cannot avoid: every routed expert's slot once, x in, y out."""
        return _routed_experts(self.logits, self.k) * self.slot_bytes + 2 * self.T * self.H * 2

    def step(self, s: int) -> None:
        lib = _lib.load()
        st = torch.cuda.current_stream().cuda_stream
        pool = self.pools[s % self.n_layers]
        _lib.check(lib.tsa_route_topk(self.logits.data_ptr(), _lib.F32, self.T, self.E, self.k,
                                      ops.ROUTE_MODES["topk_then_softmax"], self.idx.data_ptr(), self.w.data_ptr(), st))
        _lib.check(lib.tsa_moe_prefill(
            ctypes.byref(self.L), pool.data_ptr(), pool.shape[0], self.expert_slot.data_ptr(), self.E,
            self.idx.data_ptr(), self.w.data_ptr(), self.T, self.k, self.x.data_ptr(), _lib.BF16, self.y.data_ptr(),
            _lib.BF16, self.ws.data_ptr(), self.ws.numel(), st))


class GgufPrefillWorkload:
    """Workload 6: resident GGUF layers at workload 4's expert shapes (Q5_K gate/up
    2048 -> 768, Q6_K down, 128 experts), router logits and activations of a 1024-token
    prefill; one step = one layer's whole batched MoE (softmax -> top-8).
    ``shape="2880"``: workload 2's expert (Q4_K gate/up 2880 -> 2880, Q6_K down; every
    matrix's rows straddle super-blocks) in 32-expert layers, a 512-token prefill with
    Zipf-skewed top-4 (top-k -> softmax) routing."""

    def __init__(self, n_layers: int, dev: torch.device, shape: str = "qwen3"):
        g = torch.Generator(device=dev)
        g.manual_seed(20261206)
        if shape == "qwen3":
            base = synth.workload(4, tokens=1024)
            self.H, self.I, self.E, self.k = base["hidden"], base["inter"], base["E"], base["top_k"]
            self.types, self.route = (13, 13, 14), "softmax_then_topk"
            lay = base["layout"]
            self.pools = [torch.from_numpy(base["pool"]).to(dev)]
            logits, x_bits = base["logits"], base["x_bits"]
        else:  # every layer random codes with in-range super-block scales
            rng = synth.rng_for(6)
            self.H = self.I = 2880
            self.E, self.k, T = 32, 4, 512
            self.types, self.route = (12, 12, 14), "topk_then_softmax"
            lay = synth.gguf_layout(self.H, self.I, *self.types)
            self.pools = []
            logits, x_bits = synth.zipf_logits(rng, T, self.E), synth.bf16_normal(rng, (T, self.H))
        self.L = gguf_expert_layout(lay, dict(zip(("gate", "up", "down"), self.types)),
                                    {"gate": (self.H, self.I), "up": (self.H, self.I), "down": (self.I, self.H)})
        self.slot_bytes = lay.total_bytes
        while len(self.pools) < n_layers:  # further layers: random codes, super-block scales in range
            p = torch.randint(0, 256, (self.E, lay.total_bytes), dtype=torch.uint8, device=dev, generator=g)
            MoEWorkload._fix_scales(p, lay, g, self.types)
            self.pools.append(p)
        self.logits = torch.from_numpy(logits).to(dev)
        self.x = _bf16(x_bits, dev)
        self.T = self.x.shape[0]
        self.y = torch.empty_like(self.x)
        self.idx = torch.empty((self.T, self.k), dtype=torch.int32, device=dev)
        self.w = torch.empty((self.T, self.k), dtype=torch.float32, device=dev)
        self.expert_slot = torch.arange(self.E, dtype=torch.int32, device=dev)
        self.ws = ops.moe_prefill_workspace(self.L, self.T, self.k, self.E, dev)
        self.n_layers = n_layers

    def flops_per_step(self) -> int:
        return 2 * self.T * self.k * (2 * self.I * self.H + self.H * self.I)

    def min_bytes_per_step(self) -> int:
        return _routed_experts(self.logits, self.k) * self.slot_bytes + 2 * self.T * self.H * 2

    def step(self, s: int) -> None:
        lib = _lib.load()
        st = torch.cuda.current_stream().cuda_stream
        pool = self.pools[s % self.n_layers]
        _lib.check(lib.tsa_route_topk(self.logits.data_ptr(), _lib.F32, self.T, self.E, self.k,
                                      ops.ROUTE_MODES[self.route], self.idx.data_ptr(), self.w.data_ptr(), st))
        _lib.check(lib.tsa_moe_prefill(
            ctypes.byref(self.L), pool.data_ptr(), pool.shape[0], self.expert_slot.data_ptr(), self.E,
            self.idx.data_ptr(), self.w.data_ptr(), self.T, self.k, self.x.data_ptr(), _lib.BF16, self.y.data_ptr(),
            _lib.BF16, self.ws.data_ptr(), self.ws.numel(), st))


def run_prefill(args, dev) -> int:
    gguf = args.workload == 6
    fp6 = args.prefill_mfma == "fp6" and not gguf
    if gguf:
        wl = GgufPrefillWorkload(args.layers_prefill, dev, args.gguf_shape)
    else:
        wl = PrefillWorkload(args.layers_prefill, dev, _lib.PREFILL_FP6 if fp6 else _lib.PREFILL_BF16)
    peak = MFMA_F6F4_ALGO_PEAK_TFLOPS if fp6 else MFMA_BF16_PEAK_TFLOPS
    K, W = args.steps, args.warmup
    for s in range(W):
        wl.step(s)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        ev0.record(stream)
        for s in range(K):
            wl.step(s)
        ev1.record(stream)
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / K
    tflops = wl.flops_per_step() / (ms_step * 1e-3) / 1e12
    line = {
        "metric": "MoE batched-prefill grouped " + ("GGUF" if gguf else "MXFP4") + " expert GEMM TFLOP/s",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 4),
        "tokens_per_s": round(wl.T / (ms_step * 1e-3)),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": (f"gguf {'q5_k' if wl.types[0] == 13 else 'q4_k'}/q6_k blocks decoded and rounded to bf16 (as the "
                  "reference's .to(bf16)), bf16 activations, bf16 MFMA, fp32 accumulate" if gguf else
                  "mxfp4 weights x activations as two fp6 (e2m3) terms with per-32 e8m0 scales (from bf16), "
                  "scaled fp4 x fp6 MFMA, fp32 accumulate" if fp6 else
                  "mxfp4 weights expanded exactly to bf16, bf16 activations, bf16 MFMA, fp32 accumulate"),
        "data": (f"synthetic: {args.layers_prefill} random q4_k/q6_k layers rotated per step, seeded routing and "
                 "activations" if gguf and args.gguf_shape == "2880" else
                 f"synthetic: seeded workload-{4 if gguf else 5} layer + {args.layers_prefill - 1} random layers "
                 "rotated per step"),
        "config": {"workload": ("workload-2-expert gguf moe layer prefill (512 tokens, hidden 2880, 32 q4_k/q6_k "
                                "experts, zipf top-4; rows straddle super-blocks)" if gguf and args.gguf_shape == "2880"
                                else "qwen3-30b-a3b-shaped gguf moe layer prefill (1024 tokens, hidden 2048, 128 "
                                "experts, zipf top-8)" if gguf else
                                "gpt-oss-20b-shaped mxfp4 moe layer prefill (2048 tokens, hidden 2880, 32 experts, "
                                "zipf top-4)"), "flops_per_step": wl.flops_per_step(), "tokens": wl.T,
                   "prefill_mfma": "bf16" if gguf else args.prefill_mfma},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None,
                     "note": "whole step (routing, grouping, activation terms, both GEMMs, combine) per HIP-event "
                             "time; " + ("peak = the dense fp6/fp4 MFMA rate (10.1 PFLOP/s) / 2 products per "
                                         "multiply-add (hi and lo activation terms)" if fp6 else
                                         "peak = dense bf16 MFMA")},
    }
    tr = load_traffic(str(args.workload)) if not (gguf and args.gguf_shape == "2880") and (gguf or fp6) else None
    if tr:
        line["roofline"]["traffic"] = round(tr["traffic_bytes_per_step"])
        line["roofline"]["traffic_note"] = (
            f"HBM bytes per step of the two GEMM launches ({STEP_KERNELS[str(args.workload)][0]}) from rocprofv3 "
            f"FETCH_SIZE + WRITE_SIZE, each scaled by the counter's reading for a 256 MiB copy (factors "
            f"{tr['FETCH_SIZE']['copy_factor']:.3f}, {tr['WRITE_SIZE']['copy_factor']:.3f}); the step's "
            f"unavoidable bytes (every routed expert's slot once, x, y) are {wl.min_bytes_per_step()}")
    if not args.no_cpu_baseline:
        # the 2880-wide GGUF form has no CPU leg: its layers are random codes, not oracle experts
        line["cpu_baseline"] = None if gguf and args.gguf_shape == "2880" else cpu_baseline(args.workload)
    print(json.dumps(line))
    return 0


def _cpu_host() -> tuple[int, str]:
    """Threads for torch = the cores this process may run on; the CPU model name."""
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, model


def cpu_baseline(wl_id: int, min_runs: int = 20, warmup: int = 3, budget_s: float = 10.0) -> dict:
    """The reference's CPU path restated in torch (oracle.torch_cpu: whole-tensor vectorised
    dequant, then fp32 matmuls), timed on this host's cores: the median of >= min_runs runs
    after `warmup`, dequant and matmul timed separately. Workloads 1-4 time one decode step
    (router top-k, then the selected experts); workloads 5 and 6 a grouped prefill of a token
    sample; workload 7 one MXFP4 matvec. The routing itself (numpy top-k over the step's logits) is outside the timing."""
    from oracle import expert as oex
    from oracle import torch_cpu as otc

    cores, model = _cpu_host()
    wl = {6: lambda: synth.workload(4, tokens=1024), 7: dict,
          8: lambda: synth.workload(3)}.get(wl_id, lambda: synth.workload(wl_id))()
    if wl_id == 1:
        x = torch.from_numpy(wl["x"]).reshape(1, -1)
        w = otc.as_u8(wl["w"])
        dequant = lambda: otc.gguf_dequant(w, 8, (wl["N"], wl["K"]))  # noqa: E731
        matmul = lambda W: x @ W.T  # noqa: E731
        work, unit, what = wl["w"].size + 2 * 4 * wl["K"], "GB/s", "Q8_0 2880 x 2880 matvecs"
    elif wl_id == 2:
        x = torch.from_numpy(synth.bf16_to_f32(wl["x_bits"])).reshape(1, -1)
        e = otc.torch_expert(wl["expert"])
        dequant = lambda: otc.gguf_expert_weights(e)  # noqa: E731
        matmul = lambda W: otc.gguf_expert_ffn(x, *W)  # noqa: E731
        work, unit, what = wl["layout"].total_bytes + 2 * 2 * wl["hidden"], "GB/s", "single-expert FFNs"
    elif wl_id == 7:
        N, K = 5760, 2880
        rng = np.random.default_rng(7)
        blocks = torch.from_numpy(rng.integers(0, 256, (N, K // 32, 16), dtype=np.uint8))
        scales = torch.from_numpy(rng.integers(119, 126, (N, K // 32), dtype=np.uint8))
        bias = torch.from_numpy(rng.normal(0.0, 0.02, N).astype(np.float32))
        x = torch.from_numpy(rng.normal(0.0, 1.0, (1, K)).astype(np.float32))
        dequant = lambda: otc.mxfp4_dequant(blocks, scales)  # noqa: E731
        matmul = lambda W: x @ W.T + bias  # noqa: E731
        work, unit, what = N * (K // 2 + K // 32) + 2 * N + 2 * K + 2 * N, "GB/s", "MXFP4 5760 x 2880 matvecs"
    elif wl_id in (3, 4, 8):
        x = torch.from_numpy(synth.bf16_to_f32(wl["x_bits"][:1]))
        route = oex.route_softmax_then_topk if wl_id == 4 else oex.route_topk_then_softmax
        logits = wl["logits"][:1]
        if wl_id == 8:  # the router linear from the hidden states (timed with the matmuls)
            rr = np.random.default_rng(8)
            wr = torch.from_numpy(synth.bf16_to_f32(synth.bf16_normal(rr, (wl["E"], wl["hidden"]), wl["hidden"] ** -0.5)))
            br = torch.from_numpy(synth.bf16_to_f32(synth.bf16_normal(rr, (wl["E"],), 0.02)))
            logits = (x @ wr.T + br).numpy()
        idx, wts = route(logits, wl["top_k"])
        sel = [otc.torch_expert(wl["experts"][int(e)]) for e in idx[0]]
        if wl_id != 4:
            dequant = lambda: [otc.mxfp4_expert_weights(e) for e in sel]  # noqa: E731
            ffn = lambda W, e: otc.mxfp4_expert_ffn(x, *W, e["gate_up_bias"], e["down_bias"])  # noqa: E731
        else:
            dequant = lambda: [otc.gguf_expert_weights(e) for e in sel]  # noqa: E731
            ffn = lambda W, e: otc.gguf_expert_ffn(x, *W)  # noqa: E731
        matmul = lambda Ws: sum(float(c) * ffn(W, e) for c, W, e in zip(wts[0], Ws, sel))  # noqa: E731
        work = wl["top_k"] * wl["layout"].total_bytes + 2 * wl["hidden"] * 2 + wl["E"] * 4
        if wl_id == 8:
            experts_only = matmul
            matmul = lambda Ws: (x @ wr.T + br, experts_only(Ws))[1]  # noqa: E731
            work += wl["E"] * wl["hidden"] * 2 + wl["E"] * 2  # router weight and bias; logits bf16 out and in
        unit, what = "GB/s", f"single-token MoE-layer decodes (top-{wl['top_k']} of {wl['E']} experts)"
    else:
        n_tok = 64
        route = oex.route_topk_then_softmax if wl_id == 5 else oex.route_softmax_then_topk
        idx, wts = route(wl["logits"][:n_tok], wl["top_k"])
        x = torch.from_numpy(synth.bf16_to_f32(wl["x_bits"][:n_tok]))
        groups = oex.group_tokens_by_expert(idx)
        sel = {e: otc.torch_expert(wl["experts"][e]) for e in groups}
        if wl_id == 5:
            dequant = lambda: {e: otc.mxfp4_expert_weights(t) for e, t in sel.items()}  # noqa: E731
            ffn = lambda xs, W, e: otc.mxfp4_expert_ffn(xs, *W, sel[e]["gate_up_bias"], sel[e]["down_bias"])  # noqa: E731
        else:
            dequant = lambda: {e: otc.gguf_expert_weights(t) for e, t in sel.items()}  # noqa: E731
            ffn = lambda xs, W, e: otc.gguf_expert_ffn(xs, *W)  # noqa: E731

        def matmul(Ws):
            out = torch.zeros_like(x)
            for e, pairs in groups.items():
                toks = torch.tensor([p[0] for p in pairs])
                c = torch.tensor([float(wts[t, j]) for t, j in pairs]).unsqueeze(1)
                out.index_add_(0, toks, c * ffn(x[toks], Ws[e], e))
            return out

        work = 2 * n_tok * wl["top_k"] * 3 * wl["hidden"] * wl["inter"]
        unit, what = "TFLOP/s", f"grouped prefills of the first {n_tok} tokens ({len(groups)} routed experts)"
    for _ in range(warmup):
        matmul(dequant())
    td, tm, tt = [], [], []
    t_end = time.perf_counter() + budget_s
    while len(tt) < min_runs or time.perf_counter() < t_end and len(tt) < 200:
        t0 = time.perf_counter()
        W = dequant()
        t1 = time.perf_counter()
        matmul(W)
        t2 = time.perf_counter()
        td.append(t1 - t0)
        tm.append(t2 - t1)
        tt.append(t2 - t0)
        if len(tt) >= min_runs and time.perf_counter() >= t_end:
            break
    med = float(np.median(tt))
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"value": round(work / med / scale, 5), "unit": unit, "cores": cores, "kind": "port",
            "cpu_model": model, "total_ms": round(med * 1e3, 3), "dequant_ms": round(float(np.median(td)) * 1e3, 3),
            "matmul_ms": round(float(np.median(tm)) * 1e3, 3), "runs": len(tt),
            "sample": f"{len(tt)} {what} of workload {wl_id} after {warmup} warmups; torch on the CPU "
                      f"(torch.set_num_threads({cores})): whole-tensor dequant, then fp32 matmuls; medians"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=480)
    ap.add_argument("--warmup", type=int, default=48)
    ap.add_argument("--workload", type=int, default=3, choices=[1, 2, 3, 4, 5, 6, 7, 8])
    ap.add_argument("--layers-prefill", type=int, default=3, help="workloads 5, 6: distinct layers rotated per step")
    ap.add_argument("--prefill-mfma", choices=["fp6", "bf16"], default="fp6",
                    help="workload 5: the GEMMs' MFMA form (fp4 x fp6 terms, or weights expanded to bf16)")
    ap.add_argument("--layers", type=int, default=24)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--gguf-shape", choices=["qwen3", "2880"], default="qwen3",
                    help="workload 6: workload 4's layer shape (default), or workload 2's 2880-wide Q4_K/Q6_K "
                         "expert in 32-expert layers (512 tokens, top-4)")
    ap.add_argument("--decode-form", choices=["one", "two"], default="two",
                    help="workload 3: the tiled decode in one launch (down waits for gate_up in-kernel) or two")
    ap.add_argument("--checkpoint-order", action="store_true",
                    help="workload 3: keep the experts in the checkpoint order (the MFMA decode loading lane by lane)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="launch a 256 MiB copy first (for rocprofv3 --pmc traffic calibration)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write profiles/traffic.json from two rocprofv3 --pmc csv runs (no GPU work)")
    ap.add_argument("--pmc-command", default="", help="the profiled command, recorded with --summarize-pmc")
    args = ap.parse_args()
    traffic_key = "3c" if args.workload == 3 and args.checkpoint_order else str(args.workload)
    if args.summarize_pmc:
        t = summarize_pmc(*args.summarize_pmc, traffic_key, args.pmc_command)
        allt = _read_traffic()
        allt["workloads"][traffic_key] = t
        os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
        with open(TRAFFIC_FILE, "w") as fh:
            json.dump(allt, fh, indent=1)
        print(json.dumps(t))
        return 0
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (use --gpus 1)", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload in (5, 6):
        if "--steps" not in sys.argv:
            args.steps = 20
        if "--warmup" not in sys.argv:
            args.warmup = 3
        if args.copy_calibration:
            copy_calibration(dev)
        return run_prefill(args, dev)
    K, W = args.steps, args.warmup
    n_layers = args.layers
    ops.set_decode_options(0 if args.decode_form == "one" else 1)
    if args.copy_calibration:
        copy_calibration(dev)
    if args.workload in (1, 2):
        wl = GgufWorkload(args.workload, max(K, W), dev)
        n_layers = wl.copies
    elif args.workload == 7:
        wl = MxMatvecWorkload(max(K, W), dev)
        n_layers = wl.copies
    else:
        wl = MoEWorkload(args.workload, n_layers, max(K, W, n_layers), dev, tiled=not args.checkpoint_order)
    torch.cuda.synchronize()

    # warmup (eager), also validates every call
    for s in range(W):
        wl.step(s % max(len(wl.logits), 1) if args.workload in (3, 4, 8) else s)
    torch.cuda.synchronize()

    stream = torch.cuda.Stream()
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            torch.cuda.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                for s in range(K):
                    wl.step(s)
        torch.cuda.synchronize()
        graph.replay()  # one untimed replay
        torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        if args.no_graph:
            for s in range(K):
                wl.step(s)
        else:
            graph.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1)
    ms_step = ms / K
    nbytes = wl.bytes_per_step()
    gbs = nbytes / (ms_step * 1e-3) / 1e9

    line = {
        "metric": "MoE expert dequant-matvec HBM GB/s (% of 8 TB/s); MoE-layer decode us/token",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_step, 5),
        "us_per_layer_token": round(ms_step * 1e3, 2),
        "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {1: "gguf q8_0 weights, fp32 activations (int8 hi/lo terms per 32 values), int32 dots, fp32 accumulate",
                  2: "gguf q4_k/q6_k weights, bf16 activations, fp32 accumulate",
                  3: "mxfp4 weights (e2m1 x e8m0) x bf16 activations carried as two fp8 e4m3 terms per value "
                     "with a per-32-value e8m0 block scale (exact for values within 2^9 of their block's maximum) "
                     "on the scaled fp8 x fp4 MFMA, fp32 accumulate; h rounded to bf16 between the launches",
                  4: "gguf q5_k/q6_k weights, bf16 activations, fp32 accumulate",
                  8: "bf16 router linear (fp32 accumulate, bf16 logits), then as workload 3: mxfp4 weights x bf16 "
                     "activations as two fp8 e4m3 terms per value with per-32-value e8m0 block scales on the scaled "
                     "fp8 x fp4 MFMA, fp32 accumulate",
                  7: "mxfp4 weights (e2m1 x e8m0), bf16 activations and bias, fp32 accumulate"}[args.workload],
        "data": f"synthetic: seeded native-format weights, {n_layers} resident layers (or copies) rotated per step",
        "config": {
            "workload": {1: "gguf q8_0 matvec 2880 x 2880 (GGMLLinear, batch 1)",
                         2: "one gguf expert ffn, q4_k gate/up 2880 -> 2880, q6_k down (batch 1)",
                         3: "gpt-oss-20b-shaped mxfp4 moe layer decode (hidden 2880, 32 experts, top-4, batch 1)",
                         4: "qwen3-30b-a3b-shaped gguf moe layer decode (hidden 2048, 128 experts, top-8)",
                         7: "mxfp4 matvec 5760 x 2880 (gpt-oss-20b gate_up shape, dot_scaled_vecmat, batch 1)",
                         8: "gpt-oss-20b-shaped mxfp4 moe layer decode from hidden states: router linear (bias) + "
                            "top-4 of 32 + experts (hidden 2880, batch 1)"}[args.workload],
            "bytes_per_step": nbytes,
            "layers_rotated": n_layers,
            "pool_layout": "mxfp4 16-row mfma tiles" if wl.tiled else "checkpoint order",
            "decode_form": (args.decode_form + " launch" + ("" if args.decode_form == "one" else "es")) if wl.tiled
            else None,
            "graph": not args.no_graph,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "note": "achieved = algorithmic bytes per step / HIP-event time per step over the timed graph replay, "
                    "on the stream the kernels run on; a step is the launches of "
                    f"{' + '.join(STEP_KERNELS[traffic_key])} (gaps between them included)",
        },
    }
    tr = load_traffic(traffic_key)
    if tr:
        line["roofline"]["traffic"] = round(tr["traffic_bytes_per_step"])
        line["roofline"]["traffic_note"] = (
            f"HBM bytes per step ({' + '.join(STEP_KERNELS[traffic_key])}) from rocprofv3 FETCH_SIZE + WRITE_SIZE, "
            f"each scaled by the counter's reading for a {4 * COPY_ELEMS >> 20} MiB copy (factors "
            f"{tr['FETCH_SIZE']['copy_factor']:.3f}, {tr['WRITE_SIZE']['copy_factor']:.3f}); algorithmic bytes "
            f"{nbytes}")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(args.workload)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
