"""GGUF reader, the GGUF slot store and the safetensors expert store on the CPU
(tinyserve/gguf_reader.py:15-225, tinyserve/mmap_store.py:31-274,
tinyserve/expert_store.py:290-400)."""
from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from tests.gguf_writer import write_gguf
from tinyserve_amd import gguf_reader as gr
from tinyserve_amd import mx_tiles, synth
from tinyserve_amd.expert_store import ExpertStore
from tinyserve_amd.gguf_store import MmapExpertStore


def test_gguf_header_by_hand(tmp_path):
    """A file assembled field by field from the format description (not by the test writer)."""
    name = b"w"
    meta_key = b"general.architecture"
    arch = b"qwen3moe"
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 1)
    head += struct.pack("<Q", len(meta_key)) + meta_key + struct.pack("<I", 8) + struct.pack("<Q", len(arch)) + arch
    head += struct.pack("<Q", len(name)) + name + struct.pack("<I", 1) + struct.pack("<Q", 4)
    head += struct.pack("<IQ", 0, 0)  # F32 at data offset 0
    pad = (-len(head)) % 32
    data = np.arange(4, dtype=np.float32).tobytes()
    p = tmp_path / "hand.gguf"
    p.write_bytes(head + b"\0" * pad + data)
    with gr.GGUFReader(p) as r:
        assert r.version == 3
        assert r.metadata == {"general.architecture": "qwen3moe"}
        (t,) = r.tensors
        assert (t.name, t.shape, t.ggml_type, t.ggml_type_name, t.offset, t.nbytes, t.block_size) == \
            ("w", (4,), 0, "F32", 0, 16, 1)
        assert r.data_offset == len(head) + pad
        assert np.array_equal(np.frombuffer(r.get_tensor_data(t), np.float32), np.arange(4, dtype=np.float32))
        assert np.array_equal(r.tensor_view(t, 4, 8).view(np.float32), [1.0, 2.0])


def test_gguf_metadata_value_types(tmp_path):
    meta = {
        "u8": (gr.VT_UINT8, 200), "i8": (gr.VT_INT8, -5), "u16": (gr.VT_UINT16, 60000), "i16": (gr.VT_INT16, -300),
        "u32": (gr.VT_UINT32, 4_000_000_000), "i32": (gr.VT_INT32, -70000), "f32": (gr.VT_FLOAT32, 1.5),
        "b": (gr.VT_BOOL, True), "s": (gr.VT_STRING, "héllo"), "u64": (gr.VT_UINT64, 2**40),
        "i64": (gr.VT_INT64, -(2**40)), "f64": (gr.VT_FLOAT64, 0.1),
        "arr_i32": (gr.VT_ARRAY, (gr.VT_INT32, [1, -2, 3])), "arr_s": (gr.VT_ARRAY, (gr.VT_STRING, ["a", "bc"])),
        "arr_empty": (gr.VT_ARRAY, (gr.VT_FLOAT32, [])),
    }
    p = tmp_path / "meta.gguf"
    write_gguf(p, [("t", (32,), 8, synth.make_gguf(np.random.default_rng(0), 8, 32))], meta)
    with gr.GGUFReader(p) as r:
        got = r.metadata
        for k, (vt, v) in meta.items():
            want = list(v[1]) if vt == gr.VT_ARRAY else v
            assert got[k] == pytest.approx(want) if vt in (gr.VT_FLOAT32, gr.VT_FLOAT64) else got[k] == want, k
        (t,) = r.tensors
        assert (t.ggml_type_name, t.nbytes, t.block_size) == ("Q8_0", 34, 32)


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_gguf_alignment(tmp_path, alignment):
    rng = np.random.default_rng(1)
    blobs = [synth.make_gguf(rng, 12, 256 * n) for n in (1, 3)]
    p = tmp_path / "align.gguf"
    write_gguf(p, [("a", (256,), 12, blobs[0]), ("b", (256, 3), 12, blobs[1])], alignment=alignment)
    with gr.GGUFReader(p) as r:
        assert r.data_offset % (alignment or 32) == 0
        for t, blob in zip(r.tensors, blobs):
            assert t.offset % (alignment or 32) == 0
            assert r.get_tensor_data(t) == blob.tobytes()


def test_gguf_rejects_bad_files(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(ValueError, match="Not a GGUF file"):
        gr.GGUFReader(bad)
    p = tmp_path / "ok.gguf"
    write_gguf(p, [("t", (256,), 14, synth.make_gguf(np.random.default_rng(2), 14, 256))])
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(p.read_bytes()[:-10])
    with pytest.raises(ValueError, match="past the end|truncated"):
        gr.GGUFReader(cut)
    v9 = tmp_path / "v9.gguf"
    v9.write_bytes(struct.pack("<IIQQ", 0x46554747, 9, 0, 0))
    with pytest.raises(ValueError, match="version 9"):
        gr.GGUFReader(v9)


def _experts(rng, n_layers, n_experts, H, I, types_per_layer):
    return {(li, e): synth.make_gguf_expert(rng, H, I, *types_per_layer[li])
            for li in range(n_layers) for e in range(n_experts)}


def test_mmap_store_per_expert_tensors(tmp_path):
    rng = np.random.default_rng(3)
    H, I, L, E = 256, 512, 2, 3
    ex = _experts(rng, L, E, H, I, [(12, 12, 14)] * L)
    tensors = []
    for (li, e), d in ex.items():
        tensors += [(f"blk.{li}.ffn_gate.{e}.weight", (H, I), 12, d["gate"]),
                    (f"blk.{li}.ffn_up.{e}.weight", (H, I), 12, d["up"]),
                    (f"blk.{li}.ffn_down.{e}.weight", (I, H), 14, d["down"])]
    tensors.append(("token_embd.weight", (H, 8), 0, np.zeros(H * 8, np.float32)))
    p = tmp_path / "experts.gguf"
    write_gguf(p, tensors)
    st = MmapExpertStore(p)
    assert (st.num_layers, st.num_experts) == (L, E)
    assert st.ggml_types == {"gate": 12, "up": 12, "down": 14}
    assert st.proj_shapes == {"gate": (H, I), "up": (H, I), "down": (I, H)}
    lay = synth.gguf_layout(H, I, 12, 12, 14)
    assert st.layout.sizes == lay.sizes and st.layout.offsets == lay.offsets
    for (li, e), d in ex.items():
        assert np.array_equal(st.get_expert_data(li, e).numpy(), synth.pack_gguf_expert(d, lay))
    pool = torch.zeros((E + 1, st.expert_bytes), dtype=torch.uint8)
    st.copy_to_buffer_slot(pool, 2, 1, 0)
    assert np.array_equal(pool[2].numpy(), synth.pack_gguf_expert(ex[(1, 0)], lay))
    assert np.array_equal(st.load_layer(0, "cpu").numpy(),
                          np.stack([synth.pack_gguf_expert(ex[(0, e)], lay) for e in range(E)]))
    st.close()


def test_mmap_store_fused_mixed_quant(tmp_path):
    """Fused [in, out, experts] tensors; layer 1 uses Q4_K gate/up where layer 0 has Q5_K,
    so its slots are padded to layer 0's sizes and keep their own ggml types."""
    rng = np.random.default_rng(4)
    H, I, E = 256, 256, 4
    types = [(13, 13, 14), (12, 12, 14)]
    ex = _experts(rng, 2, E, H, I, types)
    tensors = []
    for li in range(2):
        for proj, ne in (("gate", (H, I, E)), ("up", (H, I, E)), ("down", (I, H, E))):
            t = types[li][("gate", "up", "down").index(proj)]
            tensors.append((f"blk.{li}.ffn_{proj}_exps.weight", ne, t,
                            np.concatenate([ex[(li, e)][proj] for e in range(E)])))
    p = tmp_path / "fused.gguf"
    write_gguf(p, tensors, {"general.architecture": (gr.VT_STRING, "qwen3moe")}, alignment=64)
    st = MmapExpertStore.from_fused(p)
    assert (st.num_layers, st.num_experts) == (2, E)
    assert st.layer_ggml_types == {0: {"gate": 13, "up": 13, "down": 14}, 1: {"gate": 12, "up": 12, "down": 14}}
    lay = synth.gguf_layout(H, I, 13, 13, 14)  # the larger layer sets the slot
    assert st.layout.sizes == lay.sizes
    for (li, e), d in ex.items():
        assert np.array_equal(st.get_expert_data(li, e).numpy(), synth.pack_gguf_expert(d, lay))
    L1 = st.expert_layout(1)
    assert (L1.gate_type, L1.down_type, L1.slot_bytes, L1.up_off) == (12, 14, lay.total_bytes, lay.offsets["up"])
    st.close()


def test_mmap_store_rejects_incomplete(tmp_path):
    rng = np.random.default_rng(5)
    d = synth.make_gguf_expert(rng, 256, 256, 12, 12, 14)
    p = tmp_path / "half.gguf"
    write_gguf(p, [("blk.0.ffn_gate.0.weight", (256, 256), 12, d["gate"]),
                   ("blk.0.ffn_down.0.weight", (256, 256), 14, d["down"])])
    with pytest.raises(ValueError, match="lacks"):
        MmapExpertStore(p)
    with pytest.raises(ValueError, match="No fused expert tensors"):
        MmapExpertStore.from_fused(p)


def _write_mxfp4_checkpoint(path, experts_by_layer, extra_layer_key=True):
    """GPT-OSS key names: model.layers.<i>.mlp.experts.{gate_up,down}_proj_{blocks,scales,bias}."""
    from safetensors.torch import save_file

    out = {}
    for li, exs in experts_by_layer.items():
        pre = f"model.layers.{li}.mlp.experts."
        out[pre + "gate_up_proj_blocks"] = torch.from_numpy(np.stack([e["gate_up_blocks"] for e in exs]))
        out[pre + "gate_up_proj_scales"] = torch.from_numpy(np.stack([e["gate_up_scales"] for e in exs]))
        out[pre + "gate_up_proj_bias"] = torch.from_numpy(np.stack([e["gate_up_bias_bits"] for e in exs])).view(torch.bfloat16)
        out[pre + "down_proj_blocks"] = torch.from_numpy(np.stack([e["down_blocks"] for e in exs]))
        out[pre + "down_proj_scales"] = torch.from_numpy(np.stack([e["down_scales"] for e in exs]))
        out[pre + "down_proj_bias"] = torch.from_numpy(np.stack([e["down_bias_bits"] for e in exs])).view(torch.bfloat16)
        if extra_layer_key:
            out[f"model.layers.{li}.self_attn.q_proj.weight"] = torch.zeros(8, 8, dtype=torch.bfloat16)
    save_file(out, str(path / "model.safetensors"))


_SLOT_PARTS = {"gate_up_proj": "gate_up_blocks", "gate_up_proj_scales": "gate_up_scales",
               "gate_up_proj_bias": "gate_up_bias_bits", "down_proj": "down_blocks",
               "down_proj_scales": "down_scales", "down_proj_bias": "down_bias_bits"}


@pytest.mark.parametrize("tiled", [False, True])
def test_safetensors_expert_store(tmp_path, tiled):
    rng = np.random.default_rng(6)
    H, I, E = 64, 96, 3
    exs = {li: [synth.make_mxfp4_expert(rng, H, I) for _ in range(E)] for li in (1, 3)}
    _write_mxfp4_checkpoint(tmp_path, exs)
    st, n = ExpertStore.from_safetensors(str(tmp_path), "mlp", "experts", tiled=tiled)
    assert (n, st.num_layers, st.layer_indices) == (E, 2, [1, 3])
    assert set(st.layout.specs) == set(_SLOT_PARTS)
    for si, li in enumerate((1, 3)):
        for e, ex in enumerate(exs[li]):
            slot = st.get_expert_data(si, e).numpy()
            want = {k: np.ascontiguousarray(ex[v]).view(np.uint8).reshape(-1) for k, v in _SLOT_PARTS.items()}
            if tiled:
                want["gate_up_proj"], want["gate_up_proj_scales"] = mx_tiles.tile_mxfp4(ex["gate_up_blocks"], ex["gate_up_scales"])
                want["down_proj"], want["down_proj_scales"] = mx_tiles.tile_mxfp4(ex["down_blocks"], ex["down_scales"])
            for name, w in want.items():
                o, nb = st.layout.offsets[name], st.layout.sizes[name]
                assert nb == w.size and np.array_equal(slot[o : o + nb], w), (li, e, name)
    L = st.expert_layout()
    assert (L.hidden, L.inter, L.mx_tiled) == (H, I, int(tiled))
    st1, _ = ExpertStore.from_safetensors(str(tmp_path), layer_indices=[3])
    assert st1.layer_indices == [3] and torch.equal(st1.get_expert_data(0, 2), ExpertStore.from_safetensors(
        str(tmp_path))[0].get_expert_data(1, 2))


def test_safetensors_store_without_experts(tmp_path):
    from safetensors.torch import save_file

    save_file({"model.layers.0.self_attn.q_proj.weight": torch.zeros(4, 4)}, str(tmp_path / "model.safetensors"))
    with pytest.raises(ValueError, match="No expert tensors"):
        ExpertStore.from_safetensors(str(tmp_path))


def test_gguf_hf_name_convention():
    """GGUF <-> Hugging Face names as the reference's loader maps them
    (gguf_loader.py:121-229): per-expert FFN tensors, model-level and per-layer tensors,
    both directions, and unknown names passed through unchanged."""
    from tinyserve_amd.gguf_store import gguf_to_hf_name, hf_to_gguf_name

    known = {
        "token_embd.weight": ("model.embed_tokens.weight", False, None, None),
        "output_norm.weight": ("model.norm.weight", False, None, None),
        "output.weight": ("lm_head.weight", False, None, None),
        "blk.0.attn_q.weight": ("model.layers.0.self_attn.q_proj.weight", False, 0, None),
        "blk.11.attn_output.bias": ("model.layers.11.self_attn.o_proj.bias", False, 11, None),
        "blk.3.attn_k_norm.weight": ("model.layers.3.self_attn.k_norm.weight", False, 3, None),
        "blk.5.ffn_norm.weight": ("model.layers.5.post_attention_layernorm.weight", False, 5, None),
        "blk.5.ffn_gate_inp.weight": ("model.layers.5.mlp.gate.weight", False, 5, None),
        "blk.2.ffn_up_exps.weight": ("model.layers.2.mlp.shared_expert.up_proj.weight", False, 2, None),
        "blk.2.ffn_gate_up_exps.weight": ("model.layers.2.mlp.shared_expert.gate_up_proj.weight", False, 2, None),
        "blk.7.ffn_down.127.weight": ("model.layers.7.mlp.experts.127.down_proj.weight", True, 7, 127),
        "blk.0.ffn_gate.0.weight": ("model.layers.0.mlp.experts.0.gate_proj.weight", True, 0, 0),
    }
    for g, want in known.items():
        assert gguf_to_hf_name(g) == want, g
        assert hf_to_gguf_name(want[0]) == g, g
    for odd in ("blk.x.attn_q.weight", "blk.1.attn_qkv.weight", "blk.1.ffn_gate.x.weight", "rope_freqs.weight",
                "blk.1.ffn_gate.3.bias"):
        assert gguf_to_hf_name(odd) == (odd, False, None, None), odd
    for odd in ("model.layers.1.unknown.weight", "model.layers.x.self_attn.q_proj.weight", "something"):
        assert hf_to_gguf_name(odd) == odd


def test_gguf_linear_weights_default_names(tmp_path):
    """Without a name map, gguf_linear_weights names the quantised non-expert linears by the
    GGUF -> Hugging Face convention and leaves per-expert tensors, norms and F32 tensors out."""
    from tinyserve_amd.gguf_store import gguf_linear_weights

    rng = np.random.default_rng(9)
    q = synth.make_gguf(rng, 13, 256 * 64)
    tensors = [("blk.1.attn_v.weight", (256, 64), 13, q),
               ("blk.1.ffn_up.0.weight", (256, 64), 13, q),
               ("blk.1.attn_norm.weight", (256,), 0, np.ones(256, np.float32)),
               ("output.weight", (256, 64), 13, q),
               ("blk.1.mystery.weight", (256, 64), 13, q)]
    p = tmp_path / "names.gguf"
    write_gguf(p, tensors)
    with gr.GGUFReader(p) as r:
        lw = gguf_linear_weights(r)
    assert sorted(lw) == ["lm_head", "model.layers.1.self_attn.v_proj"]
    assert lw["lm_head"][1:] == (13, (64, 256))


def test_gguf_linear_weights_selection(tmp_path):
    """Quantised 2-D .weight tensors named by the map become replace_linear_with_ggml input
    ((out, in) from ne = [in, out]); norms, embeddings' F32 and unmapped names are left out."""
    from tinyserve_amd.gguf_store import gguf_linear_weights

    rng = np.random.default_rng(8)
    q = synth.make_gguf(rng, 12, 256 * 512)
    tensors = [("blk.0.attn_q.weight", (256, 512), 12, q),
               ("blk.0.attn_norm.weight", (256,), 0, np.ones(256, np.float32)),
               ("blk.0.ffn_gate_inp.weight", (256, 8), 0, np.zeros(256 * 8, np.float32)),
               ("output.weight", (256, 512), 12, q)]
    p = tmp_path / "lin.gguf"
    write_gguf(p, tensors)
    names = {"blk.0.attn_q.weight": "model.layers.0.self_attn.q_proj.weight",
             "blk.0.attn_norm.weight": "model.layers.0.input_layernorm.weight",
             "blk.0.ffn_gate_inp.weight": "model.layers.0.mlp.gate.weight"}
    with gr.GGUFReader(p) as r:
        lw = gguf_linear_weights(r, names)
        assert list(lw) == ["model.layers.0.self_attn.q_proj"]
        raw, t, shape = lw["model.layers.0.self_attn.q_proj"]
        assert (t, shape) == (12, (512, 256)) and np.array_equal(raw.numpy(), q)
        assert list(gguf_linear_weights(r, lambda n: "lm_head.weight" if n == "output.weight" else None)) == ["lm_head"]
