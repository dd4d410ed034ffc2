"""The Python boundary on the GPU, against the oracle: ExpertBatcher and the template /
inline forwards behind a pipeline shaped like the reference's (cache, store,
staging_buffer_a, template, _param_refs, _inline_fwd), ExpertPipeline's entry points on
MXFP4 and GGUF stores, and a two-layer MoE whose blocks run through the offloaded forward
hook (router linear, routed decode or batched prefill, shared expert on a side stream)."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import expert as oex
from tests.gguf_writer import write_gguf
from tests.helpers import assert_close_bf16, bf16_dev, to_f32
from tinyserve_amd import ops, synth
from tinyserve_amd.expert_batcher import BatchItem, ExpertBatcher
from tinyserve_amd.expert_cache import ExpertCache
from tinyserve_amd.expert_forward import (MXFP4ExpertModule, _build_mxfp4_inline_forward, _precompute_param_refs,
                                          forward_from_packed, mxfp4_expert_layout, swap_weights_and_forward)
from tinyserve_amd.expert_pipeline import ExpertPipeline, install_offloaded_forward
from tinyserve_amd.expert_store import ExpertStore
from tinyserve_amd.gguf_store import MmapExpertStore

pytestmark = pytest.mark.gpu


def _mx_store(H, I, E, n_layers, seed, tiled):
    rng = np.random.default_rng(seed)
    lay = synth.mxfp4_tiled_layout(H, I) if tiled else synth.mxfp4_layout(H, I)
    pack = synth.pack_mxfp4_expert_tiled if tiled else synth.pack_mxfp4_expert
    experts = [[synth.make_mxfp4_expert(rng, H, I) for _ in range(E)] for _ in range(n_layers)]
    data = np.stack([np.stack([pack(e, lay) for e in row]) for row in experts])
    return rng, ExpertStore(torch.from_numpy(data), lay, n_layers, E, tiled=tiled), experts


def _stub_pipeline(store):
    """The attributes the reference's ExpertBatcher reads from its ExpertPipeline."""
    t = None if store.tiled else MXFP4ExpertModule(store.layout, "cuda")
    cache = ExpertCache(store.num_layers * store.num_experts, store.expert_bytes, "cuda",
                        num_layers=store.num_layers, num_experts=store.num_experts)
    return SimpleNamespace(cache=cache, store=store, staging_buffer_a=store.allocate_buffer("cuda"), template=t,
                           _param_refs=_precompute_param_refs(t, store.layout) if t is not None else None,
                           _inline_fwd=_build_mxfp4_inline_forward(store.layout, None))


def _mx_ref(experts, xf, idx, w):
    return oex.moe_combine(xf, idx, w, lambda e, xx: oex.mxfp4_expert_forward(xx, experts[e]))


@pytest.mark.parametrize("H,I,E,k,R,tiled", [
    (256, 128, 8, 4, 6, False),
    (512, 512, 6, 2, 5, False),    # hidden == inter
    (256, 128, 8, 4, 6, True),
    (2880, 2880, 4, 2, 3, True),   # the GPT-OSS expert shape
])
def test_batcher_over_reference_shaped_pipeline(H, I, E, k, R, tiled):
    rng, store, experts = _mx_store(H, I, E, 2, seed=H + I + R, tiled=tiled)
    pipe = _stub_pipeline(store)
    layer = 1
    xs = synth.bf16_normal(rng, (R, H))
    logits = synth.zipf_logits(rng, R, E)
    idx, w = oex.route_topk_then_softmax(logits, k)
    items = [BatchItem(bf16_dev(xs[r : r + 1]), torch.from_numpy(idx[r]).cuda(), torch.from_numpy(w[r]).cuda(), r)
             for r in range(R)]
    b = ExpertBatcher(pipe)
    ref = _mx_ref(experts[layer], synth.bf16_to_f32(xs), idx, w)
    for rnd in range(2):  # the first call makes the layer resident, the second finds it so
        outs = b.batch_execute(items, layer)
        assert len(outs) == R and all(o.shape == (1, H) and o.dtype == torch.bfloat16 for o in outs)
        assert_close_bf16(torch.cat(outs), ref, f"batcher round {rnd} H={H} I={I} tiled={tiled}")
    assert pipe.cache.layer_resident(layer, E) and not pipe.cache.layer_resident(0, E)
    assert b.batch_execute([], layer) == []


def test_template_and_inline_forwards_on_mxfp4_slots():
    H, I, E = 512, 256, 3
    rng, store, experts = _mx_store(H, I, E, 1, seed=5, tiled=False)
    pipe = _stub_pipeline(store)
    slot = pipe.cache.allocate(0, 2)
    store.copy_to_buffer_slot(pipe.cache, slot, 0, 2)
    for T in (1, 5, 24):  # 24 rows: the inline forward takes the prefill kernels
        xb = synth.bf16_normal(rng, (T, H))
        ref = oex.mxfp4_expert_forward(synth.bf16_to_f32(xb), experts[0][2])
        y = forward_from_packed(pipe.template, pipe.cache.get_packed(slot), pipe._param_refs, bf16_dev(xb))
        assert_close_bf16(y, ref, f"forward_from_packed T={T}")
        y = pipe._inline_fwd(pipe.cache.get_packed(slot), bf16_dev(xb))
        assert_close_bf16(y, ref, f"inline forward T={T}")
    store.copy_to_buffer(pipe.staging_buffer_a, 0, 1)
    xb = synth.bf16_normal(rng, (4, H))
    y = swap_weights_and_forward(pipe.template, pipe.staging_buffer_a, bf16_dev(xb))
    assert_close_bf16(y, oex.mxfp4_expert_forward(synth.bf16_to_f32(xb), experts[0][1]), "swap_weights_and_forward")
    # the swap wrote into the template's own storage, not into the cache slot it viewed before
    assert torch.equal(pipe.cache.get_packed(slot).cpu(), store.get_expert_data(0, 2))


def test_prefill_checkpoint_layout_ignores_workspace_contents():
    """Prefill over checkpoint-order MXFP4 slots with hidden == inter and a workspace filled
    with 0xFF, twice (the second call with fewer tokens): nothing is read before written."""
    H = I = 512
    E, k = 6, 2
    rng, store, experts = _mx_store(H, I, E, 1, seed=17, tiled=False)
    L = mxfp4_expert_layout(store.layout)
    pool = store.load_layer(0, "cuda")
    es = torch.arange(E, dtype=torch.int32, device="cuda")
    ws = ops.moe_prefill_workspace(L, 3, k, E, "cuda").fill_(0xFF)
    for T in (3, 2):
        xb = synth.bf16_normal(rng, (T, H))
        idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
        y = ops.moe_prefill(L, pool, es, torch.from_numpy(idx.astype(np.int32)).cuda(), torch.from_numpy(w).cuda(),
                            bf16_dev(xb), workspace=ws)
        assert_close_bf16(y, _mx_ref(experts[0], synth.bf16_to_f32(xb), idx, w), f"prefill T={T}")
        ws.fill_(0xFF)


@pytest.mark.parametrize("H,I,E,k,tiled,tile_on_copy", [
    (256, 128, 8, 4, False, False),  # checkpoint-order slots, kernels on checkpoint order
    (256, 128, 8, 4, False, True),   # checkpoint-order store, tiled on the copy into the cache
    (256, 128, 8, 4, True, True),    # a tiled store, copied as it is
    (2880, 2880, 4, 2, False, True),  # the GPT-OSS expert shape, tiled on the copy
])
def test_pipeline_entry_points_mxfp4(H, I, E, k, tiled, tile_on_copy):
    rng, store, experts = _mx_store(H, I, E, 2, seed=23 + H, tiled=tiled)
    p = ExpertPipeline(store, None, "cuda", tile_mxfp4=tile_on_copy)
    want_tiled = tiled or tile_on_copy
    assert p._inline_fwd is not None and p._cpp_layout_args["layout"].mx_tiled == int(want_tiled)
    assert p.kernel_layout(0).mx_tiled == int(want_tiled)
    if tile_on_copy and not tiled:
        p.ensure_resident(1)
        # the cache slot holds exactly the bytes the host tiler gives for the same expert
        tl = synth.mxfp4_tiled_layout(H, I)
        want = synth.pack_mxfp4_expert_tiled(experts[1][E - 1], tl)
        assert p.cache.expert_bytes == tl.total_bytes and p.cache_layout.offsets == tl.offsets
        got = p.cache.get_packed(p.cache.lookup(1, E - 1)).cpu().numpy()
        assert np.array_equal(got, want)
    for layer in (1, 0):
        for T in (1, 3):
            xb = synth.bf16_normal(rng, (T, H))
            idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
            y = p.execute_layer_experts(bf16_dev(xb), layer, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda())
            assert_close_bf16(y, _mx_ref(experts[layer], synth.bf16_to_f32(xb), idx, w), f"decode L{layer} T={T}")
        T = 40
        xb = synth.bf16_normal(rng, (T, H))
        idx, w = oex.route_topk_then_softmax(synth.zipf_logits(rng, T, E), k)
        y = p.execute_layer_experts_batched(bf16_dev(xb), layer, torch.from_numpy(idx).cuda(),
                                            torch.from_numpy(w).cuda())
        assert_close_bf16(y, _mx_ref(experts[layer], synth.bf16_to_f32(xb), idx, w), f"prefill L{layer}")
        T = 2
        xb = synth.bf16_normal(rng, (T, H))
        logits = synth.zipf_logits(rng, T, E)
        y, ridx, rw = p.execute_layer_logits(bf16_dev(xb), layer, torch.from_numpy(logits).cuda(), k,
                                             return_routing=True)
        idx, w = oex.route_topk_then_softmax(logits, k)
        assert np.array_equal(ridx.cpu().numpy(), idx)
        assert_close_bf16(y, _mx_ref(experts[layer], synth.bf16_to_f32(xb), idx, w), f"routed L{layer}")
    assert p.cache.layer_resident(0, E) and p.cache.layer_resident(1, E)


def test_pipeline_and_batcher_gguf_store(tmp_path):
    """A GGUF file with two layers of different ggml types: decode, batched prefill (64
    tokens, tsa_moe_prefill on GGUF slots) and the batcher through ExpertPipeline."""
    rng = np.random.default_rng(29)
    H, I, E, k = 512, 256, 8, 4
    types = [(12, 12, 14), (13, 13, 14)]
    ex = {(li, e): synth.make_gguf_expert(rng, H, I, *types[li]) for li in range(2) for e in range(E)}
    tensors = []
    for li in range(2):
        for pi, (proj, ne) in enumerate((("gate", (H, I, E)), ("up", (H, I, E)), ("down", (I, H, E)))):
            tensors.append((f"blk.{li}.ffn_{proj}_exps.weight", ne, types[li][pi],
                            np.concatenate([ex[(li, e)][proj] for e in range(E)])))
    write_gguf(tmp_path / "m.gguf", tensors)
    st = MmapExpertStore.from_fused(tmp_path / "m.gguf")
    p = ExpertPipeline(st, None, "cuda")

    def ref(li, xf, idx, w):
        return oex.moe_combine(xf, idx, w, lambda e, xx: oex.gguf_expert_forward(xx, ex[(li, e)]))

    for li in (0, 1):
        for T in (2, 64):
            xb = synth.bf16_normal(rng, (T, H))
            idx, w = oex.route_softmax_then_topk(synth.zipf_logits(rng, T, E), k)
            args = (bf16_dev(xb), li, torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda())
            y = p.execute_layer_experts(*args) if T == 2 else p.execute_layer_experts_batched(*args)
            assert_close_bf16(y, ref(li, synth.bf16_to_f32(xb), idx, w), f"GGUF layer {li} T={T}")
        R = 3
        xb = synth.bf16_normal(rng, (R, H))
        idx, w = oex.route_softmax_then_topk(synth.zipf_logits(rng, R, E), k)
        items = [BatchItem(bf16_dev(xb[r : r + 1]), torch.from_numpy(idx[r]).cuda(), torch.from_numpy(w[r]).cuda(), r)
                 for r in range(R)]
        outs = ExpertBatcher(p).batch_execute(items, li)
        assert_close_bf16(torch.cat(outs), ref(li, synth.bf16_to_f32(xb), idx, w), f"GGUF batcher layer {li}")
    st.close()


# ----------------------------------------------------------------------------- two-layer MoE through the hook
class _SharedMLP(nn.Module):
    def __init__(self, H, S):
        super().__init__()
        self.gate_up = nn.Linear(H, 2 * S, bias=False, dtype=torch.bfloat16)
        self.down = nn.Linear(S, H, bias=False, dtype=torch.bfloat16)

    def forward(self, x):
        g, u = self.gate_up(x).chunk(2, dim=-1)
        return self.down(torch.nn.functional.silu(g) * u)


class _MoEBlock(nn.Module):
    def __init__(self, H, E, shared):
        super().__init__()
        self.router = nn.Linear(H, E, bias=True, dtype=torch.bfloat16)
        if shared:
            self.shared_expert = _SharedMLP(H, 64)


class _TinyMoE(nn.Module):
    """x -> x + block0(x) -> ... per layer; each block returns (out, router_logits)."""

    def __init__(self, blocks):
        super().__init__()
        self.blocks = nn.ModuleList(blocks)

    def forward(self, x):
        trace = []
        for blk in self.blocks:
            y, logits = blk(x)
            trace.append((x, logits, y))
            x = x + y
        return x, trace


def _shared_ref(mlp: _SharedMLP, xf: np.ndarray) -> np.ndarray:
    wgu = mlp.gate_up.weight.detach().float().cpu().numpy()
    wd = mlp.down.weight.detach().float().cpu().numpy()
    gu = xf @ wgu.T
    S = wgu.shape[0] // 2
    return oex.silu_gate(gu[:, :S], gu[:, S:]) @ wd.T


@pytest.mark.parametrize("T", [2, 24])  # routed decode / router + batched prefill
def test_two_layer_moe_through_the_hook(T):
    H, I, E, k = 256, 128, 8, 2
    rng, store, experts = _mx_store(H, I, E, 2, seed=31 + T, tiled=True)
    torch.manual_seed(T)
    blocks = [_MoEBlock(H, E, shared=False), _MoEBlock(H, E, shared=True)]
    model = _TinyMoE(blocks).cuda()
    p = ExpertPipeline(store, None, "cuda")
    orders = ("topk_then_softmax", "softmax_then_topk")
    for li, blk in enumerate(blocks):
        install_offloaded_forward(blk, p, li, "router", k, returns_router_logits=True, softmax_order=orders[li])
    x = bf16_dev(synth.bf16_normal(rng, (T, H)))
    with torch.no_grad():
        out, trace = model(x)
    torch.cuda.synchronize()
    for li, (xin, logits, y) in enumerate(trace):
        xf, lg = to_f32(xin), to_f32(logits)
        wr = blocks[li].router.weight.detach().float().cpu().numpy()
        br = blocks[li].router.bias.detach().float().cpu().numpy()
        assert_close_bf16(logits, xf @ wr.T + br, f"router logits layer {li}")
        if li == 0:
            idx, w = oex.route_topk_then_softmax(lg, k)
        else:
            idx, w = oex.route_softmax_then_topk(lg, k)
        ref = _mx_ref(experts[li], xf, idx, w)
        if li == 1:
            ref = ref + _shared_ref(blocks[1].shared_expert, xf)
        assert_close_bf16(y, ref, f"layer {li} T={T}")
    assert out.shape == (T, H) and out.dtype == torch.bfloat16
