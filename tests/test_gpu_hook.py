"""The MoE block hook with the reference's routing modes (tinyserve/_model_hooks.py:424-476,
479-568), on the GPU against the oracle: HF-style routers that return (logits, scores,
indices) under ``router_native`` (GPT-OSS: top-k of the logits, softmax over the k; Qwen3-MoE:
softmax, top-k, renormalised or not), a router returning logits only (sigmoid top-k) and one
returning a pair, ``norm_topk_prob=False`` with an ``nn.Linear`` router, and the
reference-shaped prefetch calls on the next layers' pipelines."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import expert as oex
from tests.helpers import assert_close_bf16, bf16_dev, to_f32
from tests.test_gpu_pipeline import _mx_ref, _mx_store
from tinyserve_amd import synth
from tinyserve_amd.expert_pipeline import ExpertPipeline, install_offloaded_forward

pytestmark = pytest.mark.gpu


class _TripleRouter(nn.Module):
    """A router shaped like transformers' GPT-OSS / Qwen3-MoE routers: a linear layer, then
    (logits, scores [T, k], indices [T, k])."""

    def __init__(self, H, E, k, kind, renorm=True):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(E, H, dtype=torch.bfloat16) / H ** 0.5)
        self.bias = nn.Parameter(torch.randn(E, dtype=torch.bfloat16) * 0.1)
        self.k, self.kind, self.renorm = k, kind, renorm

    def forward(self, x):
        logits = F.linear(x, self.weight, self.bias)
        if self.kind == "gpt_oss":  # top-k of the logits, softmax over the k
            vals, idx = torch.topk(logits, self.k, dim=-1)
            return logits, F.softmax(vals.float(), dim=-1).to(logits.dtype), idx
        p = F.softmax(logits, dim=-1, dtype=torch.float)
        w, idx = torch.topk(p, self.k, dim=-1)
        if self.renorm:
            w = w / w.sum(dim=-1, keepdim=True)
        return logits, w.to(logits.dtype), idx


class _PairRouter(_TripleRouter):
    """Returns (full scores [T, E], indices [T, k]) (first of the reference's pair forms)."""

    def forward(self, x):
        logits = F.linear(x, self.weight, self.bias)
        p = F.softmax(logits, dim=-1, dtype=torch.float)
        _, idx = torch.topk(p, self.k, dim=-1)
        return p.to(logits.dtype), idx


class _LogitRouter(_TripleRouter):
    """Returns logits only: the reference's router_native then takes sigmoid top-k."""

    def forward(self, x):
        return F.linear(x, self.weight, self.bias)


class _Block(nn.Module):
    def __init__(self, router, norm_topk_prob=None):
        super().__init__()
        self.gate = router
        if norm_topk_prob is not None:
            self.norm_topk_prob = norm_topk_prob


def _bf16(t):
    return to_f32(t.to(torch.bfloat16))


def _native_ref(router, x, k):
    """(idx, weights) as the reference's router_native reads the router's result, weights
    rounded to the hidden dtype (bf16) as it passes them on."""
    with torch.no_grad():
        r = router(x)
    if isinstance(r, torch.Tensor):
        w, idx = torch.topk(torch.sigmoid(r), k, dim=-1)
    elif len(r) == 3:
        _, w, idx = r
    else:
        w_full, idx = r
        w = w_full.gather(-1, idx)
    return idx.cpu().numpy(), _bf16(w.to(x.dtype))


@pytest.mark.parametrize("T", [1, 3, 24])  # decode through the unrouted decode / prefill
@pytest.mark.parametrize("router_cls,kind,renorm", [
    (_TripleRouter, "gpt_oss", True), (_TripleRouter, "qwen3", True), (_TripleRouter, "qwen3", False),
    (_PairRouter, "qwen3", True), (_LogitRouter, "qwen3", True),
])
def test_router_native(T, router_cls, kind, renorm):
    H, I, E, k = 256, 128, 8, 4
    rng, store, experts = _mx_store(H, I, E, 1, seed=7 + T, tiled=True)
    torch.manual_seed(T)
    router = router_cls(H, E, k, kind, renorm).cuda()
    blk = _Block(router)
    p = ExpertPipeline(store, None, "cuda")
    install_offloaded_forward(blk, p, 0, "gate", k, returns_router_logits=True, softmax_order="router_native")
    x = bf16_dev(synth.bf16_normal(rng, (T, H)))
    with torch.no_grad():
        y, logits = blk.forward(x)
    torch.cuda.synchronize()
    idx, w = _native_ref(router, x, k)
    assert_close_bf16(y, _mx_ref(experts[0], to_f32(x), idx, w), f"{router_cls.__name__} {kind} renorm={renorm} T={T}")
    if router_cls is _TripleRouter:
        assert logits is not None and logits.shape == (T, E)
    else:
        assert logits is None  # as the reference: no logits from these router forms


@pytest.mark.parametrize("T", [2, 24])
def test_norm_topk_prob_false_with_linear_router(T):
    """softmax_then_topk without renormalisation (a block whose norm_topk_prob is False), on
    the router kernel and the routed decode (T = 2) or the device top-k and prefill (T = 24)."""
    H, I, E, k = 256, 128, 8, 2
    rng, store, experts = _mx_store(H, I, E, 1, seed=90 + T, tiled=True)
    torch.manual_seed(5)
    router = nn.Linear(H, E, bias=True, dtype=torch.bfloat16).cuda()
    blk = _Block(router, norm_topk_prob=False)
    p = ExpertPipeline(store, None, "cuda")
    install_offloaded_forward(blk, p, 0, "gate", k, returns_router_logits=True, softmax_order="softmax_then_topk")
    x = bf16_dev(synth.bf16_normal(rng, (T, H)))
    with torch.no_grad():
        y, logits = blk.forward(x)
    torch.cuda.synchronize()
    lg = to_f32(logits)
    xf = to_f32(x)
    wr, br = router.weight.detach().float().cpu().numpy(), router.bias.detach().float().cpu().numpy()
    assert_close_bf16(logits, xf @ wr.T + br, "router kernel logits")
    idx, w = oex.route_softmax_then_topk(lg, k, renormalize=False)
    assert w.sum(axis=-1).max() < 0.999, "the test needs weights that do not sum to 1"
    assert_close_bf16(y, _mx_ref(experts[0], xf, idx, w), f"no renormalisation T={T}")


class _Recorder:
    """Stands in for the next layers' pipelines: records schedule_prefetch calls."""

    def __init__(self):
        self.calls = []

    def schedule_prefetch(self, layer_idx, expert_ids=None):
        self.calls.append(layer_idx)


def test_reference_shaped_prefetch_calls():
    """With next_pipeline / all_pipelines given (the reference's FATE and multi-hop prefetch),
    a one-token decode calls schedule_prefetch on the next layers; a real ExpertPipeline
    accepts the call (all experts stay resident) and the output is unchanged."""
    H, I, E, k = 256, 128, 8, 2
    rng, store, experts = _mx_store(H, I, E, 4, seed=61, tiled=True)
    torch.manual_seed(2)
    p = ExpertPipeline(store, None, "cuda")
    rec = _Recorder()
    router = nn.Linear(H, E, bias=True, dtype=torch.bfloat16).cuda()
    blk = _Block(router)
    install_offloaded_forward(blk, p, 0, "gate", k, softmax_order="topk_then_softmax", next_pipeline=rec,
                              next_route=lambda h: None, all_pipelines=[p, p, rec, rec])
    x = bf16_dev(synth.bf16_normal(rng, (1, H)))
    with torch.no_grad():
        y = blk.forward(x)
        lg = router(x)
    torch.cuda.synchronize()
    assert rec.calls == [1, 2, 3]
    idx, w = oex.route_topk_then_softmax(to_f32(lg), k)
    assert_close_bf16(y, _mx_ref(experts[0], to_f32(x), idx, w), "decode with prefetch calls")
    p.schedule_prefetch(3, torch.tensor([0, 5], device="cuda"))  # a real pipeline: residency only
    assert p.cache.layer_resident(3, E)
    assert p.execute_batched_experts([], 0) == []
    # execute_batched_experts: several requests, one grouped call (ExpertBatcher)
    from tinyserve_amd.expert_batcher import BatchItem

    R = 3
    xb = synth.bf16_normal(rng, (R, H))
    idx, w = oex.route_topk_then_softmax(rng.normal(size=(R, E)).astype(np.float32), k)
    items = [BatchItem(bf16_dev(xb[r : r + 1]), torch.from_numpy(idx[r]).cuda(), torch.from_numpy(w[r]).cuda(), r)
             for r in range(R)]
    outs = p.execute_batched_experts(items, 2)
    assert_close_bf16(torch.cat(outs), _mx_ref(experts[2], synth.bf16_to_f32(xb), idx, w), "execute_batched_experts")
