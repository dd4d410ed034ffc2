"""GGUF experts as packed slots (gate || up || down raw bytes), read from a memory-mapped file.

Mirrors the reference's ``MmapExpertStore`` (tinyserve/mmap_store.py:31-274): the same
attributes (``num_layers``, ``num_experts``, ``layout``, ``expert_bytes``,
``buffer_expert_bytes``, ``ggml_types``, ``proj_shapes``) and methods
(``get_expert_data``, ``allocate_buffer``, ``copy_to_buffer``, ``copy_to_buffer_slot``,
``from_fused``, ``close``). A slot is the expert's gate, up and down tensors in their
native GGUF block streams, each padded to the largest size that projection has in any
layer (mixed quantisation, e.g. Q4_K_M: some layers' tensors are smaller), which is the
layout the decode kernels read (``expert_forward.gguf_expert_layout``; the per-layer
ggml types are in ``layer_ggml_types``).

What this build adds: ``load_layer`` copies a whole layer's experts into one device pool
(all experts resident, as the 288 GB of one GPU allows) and ``expert_layout`` gives the
matching ``tsa_expert_layout`` for that layer.

Non-expert weights: ``gguf_linear_weights`` selects the native-quantised linears for
``replace_linear_with_ggml``, named by ``gguf_to_hf_name`` / ``hf_to_gguf_name`` (the
GGUF <-> Hugging Face convention of tinyserve/gguf_loader.py:121-229) unless the caller
gives its own map.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from .expert_store import ExpertBuffer, TensorLayout
from .gguf_reader import GGUFReader, GGUFTensorInfo, tensor_nbytes

_PROJS = ("gate", "up", "down")


class MmapExpertStore:
    """Per-expert GGUF tensors (``blk.<L>.ffn_<proj>.<E>.weight``) as packed slots."""

    def __init__(self, path: str | Path):
        reader = GGUFReader(path)
        groups = reader.list_expert_tensors()
        if not groups:
            reader.close()
            raise ValueError(f"No per-expert tensors found in {path}")
        for key, projs in groups.items():
            missing = set(_PROJS) - set(projs)
            if missing:
                reader.close()
                raise ValueError(f"{path}: layer {key[0]} expert {key[1]} lacks {sorted(missing)}")
        self._init(reader, groups, sorted({k[0] for k in groups}), sorted({k[1] for k in groups}))

    @classmethod
    def from_fused(cls, path: str | Path) -> "MmapExpertStore":
        """Fused tensors ``blk.<L>.ffn_<proj>_exps.weight`` with ne = [in, out, experts]:
        expert i of a projection is the byte range offset + i * bytes_per_expert
        (tinyserve/mmap_store.py:166-274); nothing is converted."""
        reader = GGUFReader(path)
        fused = reader.list_fused_expert_tensors()
        if not fused:
            reader.close()
            raise ValueError(f"No fused expert tensors in {path}")
        layers = sorted(fused)
        groups: dict[tuple[int, int], dict[str, GGUFTensorInfo]] = {}
        n_experts = None
        for li in layers:
            if set(_PROJS) - set(fused[li]):
                reader.close()
                raise ValueError(f"{path}: layer {li} lacks fused {sorted(set(_PROJS) - set(fused[li]))}")
            for proj in _PROJS:
                info = fused[li][proj]
                if len(info.shape) != 3:
                    reader.close()
                    raise ValueError(f"{path}: {info.name} has {len(info.shape)} dims, fused experts have 3")
                if n_experts is None:
                    n_experts = int(info.shape[2])
                elif int(info.shape[2]) != n_experts:
                    reader.close()
                    raise ValueError(f"{path}: {info.name} holds {info.shape[2]} experts, expected {n_experts}")
                per = tensor_nbytes(info.ggml_type, info.shape[:2])
                for e in range(n_experts):
                    groups.setdefault((li, e), {})[proj] = GGUFTensorInfo(
                        name=f"blk.{li}.ffn_{proj}.{e}.weight", shape=tuple(int(d) for d in info.shape[:2]),
                        ggml_type=info.ggml_type, ggml_type_name=info.ggml_type_name,
                        offset=info.offset + e * per, nbytes=per, block_size=info.block_size)
        store = cls.__new__(cls)
        store._init(reader, groups, layers, list(range(n_experts)))
        return store

    def _init(self, reader: GGUFReader, groups, layers: list[int], experts: list[int]) -> None:
        self._reader = reader
        self._groups = groups
        self.num_layers = len(layers)
        self.num_experts = len(experts)
        self._layers = layers
        self._experts = experts
        self._layer_map = {li: i for i, li in enumerate(layers)}
        self._expert_map = {e: i for i, e in enumerate(experts)}
        first = groups[(layers[0], experts[0])]
        self.ggml_types = {p: first[p].ggml_type for p in _PROJS}
        self.proj_shapes = {p: tuple(first[p].shape[:2]) for p in _PROJS}
        self.layer_ggml_types: dict[int, dict[str, int]] = {}
        nbytes = {p: 0 for p in _PROJS}
        for (li, _e), projs in groups.items():
            types = {p: projs[p].ggml_type for p in _PROJS}
            if self.layer_ggml_types.setdefault(li, types) != types:
                raise ValueError(f"layer {li}: experts with different ggml types {types}")
            for p in _PROJS:
                if tuple(projs[p].shape[:2]) != self.proj_shapes[p]:
                    raise ValueError(f"{projs[p].name}: shape {projs[p].shape} differs from {self.proj_shapes[p]}")
                nbytes[p] = max(nbytes[p], projs[p].nbytes)
        self.layout = TensorLayout({p: ((nbytes[p],), torch.uint8) for p in _PROJS})
        self._bf16_layout = self.layout
        self.expert_bytes = self.layout.total_bytes
        self.buffer_expert_bytes = self.expert_bytes
        self._staging: torch.Tensor | None = None

    # ---- one expert
    def _fill(self, dest: np.ndarray, layer_idx: int, expert_idx: int) -> None:
        projs = self._groups[(layer_idx, expert_idx)]
        for p in _PROJS:
            info, off, size = projs[p], self.layout.offsets[p], self.layout.sizes[p]
            dest[off : off + info.nbytes] = self._reader.tensor_view(info)
            dest[off + info.nbytes : off + size] = 0  # padding of a smaller (mixed-quant) tensor

    def get_expert_data(self, layer_idx: int, expert_idx: int) -> torch.Tensor:
        """The packed expert (gate || up || down, padded) as a CPU uint8 tensor."""
        out = np.empty(self.expert_bytes, dtype=np.uint8)
        self._fill(out, layer_idx, expert_idx)
        return torch.from_numpy(out)

    def _staged(self, layer_idx: int, expert_idx: int) -> torch.Tensor:
        if self._staging is None:
            self._staging = torch.empty(self.expert_bytes, dtype=torch.uint8,
                                        pin_memory=torch.cuda.is_available())
        self._fill(self._staging.numpy(), layer_idx, expert_idx)
        return self._staging

    def allocate_buffer(self, device: torch.device | str) -> ExpertBuffer:
        return ExpertBuffer(self.layout, device)

    def copy_to_buffer(self, buf: ExpertBuffer, layer_idx: int, expert_idx: int, non_blocking: bool = False) -> None:
        buf.packed.copy_(self._staged(layer_idx, expert_idx), non_blocking=non_blocking)
        if non_blocking and buf.packed.is_cuda:
            torch.cuda.current_stream(buf.packed.device).synchronize()  # the staging buffer is reused

    def copy_to_buffer_slot(self, cache, slot: int, layer_idx: int, expert_idx: int) -> None:
        """Copy into row ``slot`` of a slot pool (an object with ``_packed`` [slots, bytes], or the tensor)."""
        packed = getattr(cache, "_packed", cache)
        packed[slot].copy_(self._staged(layer_idx, expert_idx))

    # ---- whole layers
    def load_layer(self, layer_idx: int, device: torch.device | str = "cuda") -> torch.Tensor:
        """All experts of a layer as a [num_experts, expert_bytes] uint8 pool on ``device``
        (expert e in slot e)."""
        host = np.empty((self.num_experts, self.expert_bytes), dtype=np.uint8)
        for i, e in enumerate(self._experts):
            self._fill(host[i], layer_idx, e)
        return torch.from_numpy(host).to(device)

    def expert_layout(self, layer_idx: int):
        """The kernels' tsa_expert_layout for this layer's slots (its own ggml types)."""
        from .expert_forward import gguf_expert_layout

        return gguf_expert_layout(self.layout, self.layer_ggml_types[layer_idx], self.proj_shapes, self.expert_bytes)

    @property
    def layers(self) -> list[int]:
        return list(self._layers)

    def close(self) -> None:
        self._reader.close()


# GGUF <-> Hugging Face parameter names (the naming convention the reference's loader
# applies, tinyserve/gguf_loader.py:121-229): three model-level tensors, per-layer suffixes
# under blk.<L>. <-> model.layers.<L>., and per-expert FFN tensors blk.<L>.ffn_<p>.<E>.weight
# <-> model.layers.<L>.mlp.experts.<E>.<p>_proj.weight. The pairs are the convention itself,
# so they are listed as the reference lists them.
_GLOBAL_NAMES = (
    ("token_embd.weight", "model.embed_tokens.weight"),
    ("output_norm.weight", "model.norm.weight"),
    ("output.weight", "lm_head.weight"),
)
_LAYER_NAMES = (
    ("attn_q.weight", "self_attn.q_proj.weight"),
    ("attn_k.weight", "self_attn.k_proj.weight"),
    ("attn_v.weight", "self_attn.v_proj.weight"),
    ("attn_output.weight", "self_attn.o_proj.weight"),
    ("attn_norm.weight", "input_layernorm.weight"),
    ("attn_q_norm.weight", "self_attn.q_norm.weight"),
    ("attn_k_norm.weight", "self_attn.k_norm.weight"),
    ("ffn_norm.weight", "post_attention_layernorm.weight"),
    ("ffn_gate_inp.weight", "mlp.gate.weight"),
    ("ffn_gate_exps.weight", "mlp.shared_expert.gate_proj.weight"),
    ("ffn_up_exps.weight", "mlp.shared_expert.up_proj.weight"),
    ("ffn_down_exps.weight", "mlp.shared_expert.down_proj.weight"),
    ("ffn_gate_up_exps.weight", "mlp.shared_expert.gate_up_proj.weight"),
    ("attn_q.bias", "self_attn.q_proj.bias"),
    ("attn_k.bias", "self_attn.k_proj.bias"),
    ("attn_v.bias", "self_attn.v_proj.bias"),
    ("attn_output.bias", "self_attn.o_proj.bias"),
)
_G2H_GLOBAL, _H2G_GLOBAL = dict(_GLOBAL_NAMES), {h: g for g, h in _GLOBAL_NAMES}
_G2H_LAYER, _H2G_LAYER = dict(_LAYER_NAMES), {h: g for g, h in _LAYER_NAMES}


def _split_layer(name: str, prefix: str) -> tuple[int, str] | None:
    """``<prefix><L>.<rest>`` -> (L, rest), else None."""
    if not name.startswith(prefix):
        return None
    head, dot, rest = name[len(prefix):].partition(".")
    return (int(head), rest) if dot and head.isascii() and head.isdigit() else None


def gguf_to_hf_name(gguf_name: str) -> tuple[str, bool, int | None, int | None]:
    """(hf_name, is_expert, layer, expert) for a GGUF tensor name, as the reference's
    ``gguf_to_hf_name`` (tinyserve/gguf_loader.py:163-195): a per-expert FFN tensor maps
    to ``model.layers.<L>.mlp.experts.<E>.<p>_proj.weight`` with is_expert True; a
    model-level or known per-layer tensor to its Hugging Face name; anything else comes
    back unchanged (layer None)."""
    parsed = _split_layer(gguf_name, "blk.")
    if parsed is not None:
        layer, rest = parsed
        parts = rest.split(".")
        if (len(parts) == 3 and parts[2] == "weight" and parts[1].isdigit()
                and parts[0] in ("ffn_gate", "ffn_up", "ffn_down")):
            proj, expert = parts[0][4:], int(parts[1])
            return f"model.layers.{layer}.mlp.experts.{expert}.{proj}_proj.weight", True, layer, expert
    if gguf_name in _G2H_GLOBAL:
        return _G2H_GLOBAL[gguf_name], False, None, None
    if parsed is not None and parsed[1] in _G2H_LAYER:
        return f"model.layers.{parsed[0]}.{_G2H_LAYER[parsed[1]]}", False, parsed[0], None
    return gguf_name, False, None, None


def hf_to_gguf_name(hf_name: str) -> str:
    """The inverse (tinyserve/gguf_loader.py:198-229); unknown names come back unchanged."""
    if hf_name in _H2G_GLOBAL:
        return _H2G_GLOBAL[hf_name]
    parsed = _split_layer(hf_name, "model.layers.")
    if parsed is None:
        return hf_name
    layer, rest = parsed
    parts = rest.split(".")
    if (len(parts) == 5 and parts[:2] == ["mlp", "experts"] and parts[2].isdigit() and parts[4] == "weight"
            and parts[3] in ("gate_proj", "up_proj", "down_proj")):
        return f"blk.{layer}.ffn_{parts[3][:-5]}.{parts[2]}.weight"
    if rest in _H2G_LAYER:
        return f"blk.{layer}.{_H2G_LAYER[rest]}"
    return hf_name


def _default_linear_name(gguf_name: str) -> str | None:
    """A non-expert tensor's Hugging Face name, or None for expert and unknown tensors."""
    hf, is_expert, _, _ = gguf_to_hf_name(gguf_name)
    return None if is_expert or hf == gguf_name else hf


_QUANT_TYPES = (2, 3, 6, 7, 8, 10, 11, 12, 13, 14, 15)


def gguf_linear_weights(reader: GGUFReader, name_map=None) -> dict[str, tuple[torch.Tensor, int, tuple[int, int]]]:
    """Native-quantised 2-D ``.weight`` tensors of a GGUF file as ``replace_linear_with_ggml``
    input: module path -> (raw bytes, ggml type, (out_features, in_features)), the selection
    the reference's loader makes for non-expert linears (tinyserve/gguf_loader.py:610-623:
    GGUF ne = [in, out]). ``name_map`` maps GGUF tensor names to model parameter names (a
    dict, or a callable returning None to skip; by default the generic convention of
    ``gguf_to_hf_name`` without the expert tensors); only types ``GGMLLinear`` can run are
    kept (the row kernels serve Q8_0 / Q4_K / Q5_K / Q6_K)."""
    if name_map is None:
        name_map = _default_linear_name
    from .ops import gguf_block_info

    out: dict[str, tuple[torch.Tensor, int, tuple[int, int]]] = {}
    for info in reader.tensors:
        hf = name_map(info.name) if callable(name_map) else name_map.get(info.name)
        if hf is None or not hf.endswith(".weight") or len(info.shape) != 2 or info.ggml_type not in _QUANT_TYPES:
            continue
        try:
            gguf_block_info(info.ggml_type)
        except Exception:
            continue  # a quantisation the kernels do not implement: left to the caller
        out[hf.rsplit(".weight", 1)[0]] = (torch.from_numpy(reader.tensor_view(info).copy()), info.ggml_type,
                                           (int(info.shape[1]), int(info.shape[0])))
    return out
