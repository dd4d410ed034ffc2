"""The Python boundary's host logic on the CPU: the all-resident ExpertCache, the MXFP4
lookup table names, the template-binding forwards and the batcher's loop over
unquantised experts (torch on the CPU; no library call)."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn as nn

from tinyserve_amd import mxfp4
from tinyserve_amd.expert_batcher import BatchItem, ExpertBatcher
from tinyserve_amd.expert_cache import ExpertCache
from tinyserve_amd.expert_forward import (_build_cpp_layout_args, _build_inline_forward, _build_mxfp4_inline_forward,
                                          _precompute_param_refs, forward_from_packed, swap_weights_and_forward)
from tinyserve_amd.expert_store import ExpertStore, TensorLayout, pack_tensors
from tinyserve_amd import synth


# ----------------------------------------------------------------------------- ExpertCache
def test_cache_allocate_lookup_and_stats():
    c = ExpertCache(4, 64, "cpu", num_layers=2, num_experts=3)
    assert c._packed.shape == (4, 64) and c._packed.dtype == torch.uint8
    assert c.lookup(0, 1) is None and c.misses == 1
    s = c.allocate(0, 1)
    assert c.allocate(0, 1) == s, "a second allocate returns the same slot"
    assert c.lookup(0, 1) == s and c.hits == 1
    assert c.hit_rate == 0.5
    assert c.get_layer_stats() == {0: {"hits": 1, "misses": 1, "hit_rate": 0.5}}
    c.reset_stats()
    assert c.hits == c.misses == 0


def test_cache_never_evicts_and_reuses_released_slots():
    c = ExpertCache(2, 8, "cpu")
    a, b = c.allocate(0, 0), c.allocate(0, 1)
    assert sorted((a, b)) == [0, 1]
    with pytest.raises(RuntimeError, match="full"):
        c.allocate(0, 2)
    assert c.contains(0, 0) and c.contains(0, 1), "a failed allocate evicts nothing"
    c.release(0, 0)
    assert c.allocate(1, 5) == a, "a released slot is reused"
    assert not c.contains(0, 0)


def test_cache_device_slot_tables():
    c = ExpertCache(6, 8, "cpu", num_layers=1, num_experts=2)
    c.allocate(0, 1)
    c.allocate(2, 4)  # grows the table past its initial shape
    c.allocate(2, 0)
    es = c.expert_slot(2)
    assert es.dtype == torch.int32 and es.tolist() == [2, -1, -1, -1, 1]
    ids = torch.tensor([[4, 0], [3, 9], [-1, 1]])
    assert c.lookup_slots(2, ids).tolist() == [[1, 2], [-1, -1], [-1, -1]]
    assert c.lookup_slots(7, ids).tolist() == [[-1, -1]] * 3, "unknown layer: all -1"
    assert not c.layer_resident(2, 5) and c.layer_resident(0, 0)
    c.allocate(0, 0)
    assert c.layer_resident(0, 2)
    c.clear()
    assert c.expert_slot(2).tolist() == [-1] * 5 and not c.contains(2, 4)


def test_cache_slot_contents_round_trip():
    lay = TensorLayout({"a": ((4,), torch.float32), "b": ((3,), torch.uint8)})
    c = ExpertCache(2, lay.total_bytes, "cpu")
    buf = SimpleNamespace(packed=torch.arange(lay.total_bytes, dtype=torch.uint8))
    c.store_from_buffer(1, buf)
    assert torch.equal(c.get_packed(1), buf.packed)
    out = SimpleNamespace(packed=torch.zeros(lay.total_bytes, dtype=torch.uint8))
    c.load_to_buffer(1, out)
    assert torch.equal(out.packed, buf.packed)


# ----------------------------------------------------------------------------- mxfp4 names
def test_fp4_lut_and_get_lut():
    assert mxfp4.FP4_LUT.dtype == torch.bfloat16 and mxfp4.FP4_LUT.shape == (16,)
    # e2m1: code c and c | 8 are negatives of each other; magnitudes 0, 0.5 .. 6
    assert torch.equal(mxfp4.FP4_LUT[8:], -mxfp4.FP4_LUT[:8])
    assert mxfp4.FP4_LUT[:8].tolist() == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    lut = mxfp4.get_lut(torch.float32, "cpu")
    assert lut.dtype == torch.float32 and lut is mxfp4.get_lut(torch.float32, "cpu")
    assert mxfp4.FP4_VALUES == mxfp4.FP4_LUT.tolist()


# ----------------------------------------------------------------------------- template forwards
class _BF16Expert(nn.Module):
    """The layout of an unquantised fused expert: gate_up [2I, H], down [H, I], SiLU gating."""

    def __init__(self, H, I):
        super().__init__()
        self.gate_up_proj = nn.Parameter(torch.zeros(2 * I, H), requires_grad=False)
        self.down_proj = nn.Parameter(torch.zeros(H, I), requires_grad=False)
        self._act_fn = nn.SiLU()

    def forward(self, h):
        g, u = torch.nn.functional.linear(h, self.gate_up_proj).chunk(2, dim=-1)
        return torch.nn.functional.linear(self._act_fn(g) * u, self.down_proj)


def _bf16_store(H, I, E, seed=0):
    torch.manual_seed(seed)
    lay = TensorLayout({"gate_up_proj": ((2 * I, H), torch.float32), "down_proj": ((H, I), torch.float32)})
    data = torch.empty(1, E, lay.total_bytes, dtype=torch.uint8)
    weights = []
    for e in range(E):
        w = {"gate_up_proj": torch.randn(2 * I, H) / H ** 0.5, "down_proj": torch.randn(H, I) / I ** 0.5}
        pack_tensors(data[0, e], lay, w)
        weights.append(w)
    return ExpertStore(data, lay, 1, E), weights


def _direct(w, h):
    g, u = (h @ w["gate_up_proj"].T).chunk(2, dim=-1)
    return (torch.nn.functional.silu(g) * u) @ w["down_proj"].T


def test_template_forwards_bind_packed_slots():
    H, I, E = 32, 48, 3
    store, weights = _bf16_store(H, I, E)
    t = _BF16Expert(H, I)
    h = torch.randn(5, H)
    refs = _precompute_param_refs(t, store.layout)
    packed = store.get_expert_data(0, 1)
    torch.testing.assert_close(forward_from_packed(t, packed, refs, h), _direct(weights[1], h))
    buf = store.allocate_buffer("cpu")
    store.copy_to_buffer(buf, 0, 2)
    torch.testing.assert_close(swap_weights_and_forward(t, buf, h), _direct(weights[2], h))
    # the swap copied into storage the template owns: the packed slot 1 was not overwritten
    assert torch.equal(packed, store.get_expert_data(0, 1))
    inline = _build_inline_forward(store.layout, nn.SiLU())
    torch.testing.assert_close(inline(packed, h), _direct(weights[1], h))


def test_builders_on_quantised_layouts():
    mx = synth.mxfp4_layout(256, 128)
    assert _build_inline_forward(mx, None) is None
    args = _build_cpp_layout_args(mx, None)
    assert args["layout"].hidden == 256 and args["layout"].inter == 128
    f = _build_mxfp4_inline_forward(mx, None)
    assert f.expert_layout.slot_bytes == mx.total_bytes
    gg = synth.gguf_layout(256, 512, 12, 12, 14)
    assert _build_cpp_layout_args(gg, None) is None and _build_mxfp4_inline_forward(gg, None) is None


def test_batcher_loop_for_unquantised_experts():
    """The reference's per-expert loop (hits through _inline_fwd, misses through the staging
    buffer, then cached) against a direct per-request sum."""
    H, I, E, k = 32, 48, 4, 2
    store, weights = _bf16_store(H, I, E, seed=1)
    t = _BF16Expert(H, I)
    cache = ExpertCache(E, store.expert_bytes, "cpu")
    pipe = SimpleNamespace(cache=cache, store=store, staging_buffer_a=store.allocate_buffer("cpu"), template=t,
                           _param_refs=_precompute_param_refs(t, store.layout),
                           _inline_fwd=_build_inline_forward(store.layout, nn.SiLU()))
    rng = np.random.default_rng(0)
    items = []
    for r in range(5):
        ids = torch.from_numpy(rng.choice(E, k, replace=False))
        items.append(BatchItem(torch.randn(1, H), ids, torch.softmax(torch.randn(k), 0), r))
    b = ExpertBatcher(pipe)
    for rnd in range(2):  # first round: misses; second: cache hits
        outs = b.batch_execute(items, 0)
        for it, y in zip(items, outs):
            ref = sum(float(wt) * _direct(weights[int(e)], it.hidden_states)
                      for e, wt in zip(it.expert_indices, it.routing_weights))
            torch.testing.assert_close(y, ref, rtol=1e-5, atol=1e-5)
    assert cache.hits > 0 and cache.misses > 0
    assert b.batch_execute([], 0) == []


@pytest.mark.parametrize("in_out", [True, False])
def test_inline_forward_square_down(in_out):
    """hidden == inter (GPT-OSS: 2880 both): the down matrix is square, so its orientation
    comes from gate_up's. [in, out] storage (HF GPT-OSS: gate_up [H, 2I], down [I, H]) and
    [out, in] storage (F.linear's) both give x @ W against a direct matmul."""
    H = I = 16
    torch.manual_seed(3)
    wgu = torch.randn(2 * I, H) / H ** 0.5  # [out, in]
    wdn = torch.randn(H, I) / I ** 0.5
    shapes = {"gate_up_proj": (H, 2 * I) if in_out else (2 * I, H), "down_proj": (I, H) if in_out else (H, I)}
    lay = TensorLayout({n: (s, torch.float32) for n, s in shapes.items()})
    packed = torch.empty(lay.total_bytes, dtype=torch.uint8)
    pack_tensors(packed, lay, {"gate_up_proj": wgu.T.contiguous() if in_out else wgu,
                               "down_proj": wdn.T.contiguous() if in_out else wdn})
    h = torch.randn(3, H)
    g, u = (h @ wgu.T).chunk(2, dim=-1)
    ref = (torch.nn.functional.silu(g) * u) @ wdn.T
    inline = _build_inline_forward(lay, nn.SiLU())
    torch.testing.assert_close(inline(packed, h), ref)
