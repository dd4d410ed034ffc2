"""The C ABI without a GPU: the library loads, exports every symbol the header declares,
and its host-side validation (sizes, layouts, error texts) behaves; no kernel launches."""
from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from tinyserve_amd import _lib, synth
from tinyserve_amd.expert_forward import gguf_expert_layout, mxfp4_expert_layout

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "tinyserve_amd.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    return _lib.load()


def _declared() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:int|const char\*)\s+(tsa_\w+)\s*\(", text, flags=re.M))


def test_header_and_binding_list_agree():
    assert _declared() == set(_lib.SIGNATURES), "include/tinyserve_amd.h and _lib.SIGNATURES differ"


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in sorted(_declared()) if not hasattr(raw, s)]
    assert not missing, f"not exported: {missing}"


def test_version_and_status_strings(lib):
    assert lib.tsa_version() >= 1
    assert lib.tsa_status_string(0) == b"ok" or lib.tsa_status_string(0)
    for code in range(-7, 1):
        assert lib.tsa_status_string(code)


@pytest.mark.parametrize("t,be,ts", [(8, 32, 34), (12, 256, 144), (13, 256, 176), (14, 256, 210)])
def test_gguf_block_info(lib, t, be, ts):
    a, b = ctypes.c_int64(), ctypes.c_int64()
    assert lib.tsa_gguf_block_info(t, ctypes.byref(a), ctypes.byref(b)) == 0
    assert (a.value, b.value) == (be, ts)


def test_unsupported_type_message(lib):
    a, b = ctypes.c_int64(), ctypes.c_int64()
    rc = lib.tsa_gguf_block_info(99, ctypes.byref(a), ctypes.byref(b))
    assert rc == _lib.ERR_UNSUPPORTED_TYPE
    assert b"Unsupported ggml_type: 99. Supported: Q8_0(8), Q4_K(12), Q5_K(13), Q6_K(14)" in lib.tsa_last_error()
    rc = lib.tsa_gguf_matvec(99, None, 0, None, 0, 1, 32, None, 0, 1, None)
    assert rc == _lib.ERR_UNSUPPORTED_TYPE and b"Unsupported ggml_type: 99" in lib.tsa_last_error()


def test_matvec_shape_errors(lib):
    rc = lib.tsa_gguf_matvec(8, None, 34, None, 0, 1, 33, None, 0, 1, None)
    assert rc == _lib.ERR_SHAPE and b"must be divisible by block_elements (32)" in lib.tsa_last_error()
    rc = lib.tsa_gguf_matvec(8, ctypes.c_void_p(16), 33, ctypes.c_void_p(16), 0, 1, 32, ctypes.c_void_p(16), 0, 1, None)
    assert rc == _lib.ERR_WEIGHT_TOO_SMALL and b"weight_data too small" in lib.tsa_last_error()


def test_tile_sizes(lib):
    bb, sb = ctypes.c_int64(), ctypes.c_int64()
    assert lib.tsa_mxfp4_tile_sizes(5760, 2880, ctypes.byref(bb), ctypes.byref(sb)) == 0
    assert (bb.value, sb.value) == (5760 * 1440, 360 * 256 * 6)
    assert lib.tsa_mxfp4_tile_sizes(20, 64, ctypes.byref(bb), ctypes.byref(sb)) == _lib.ERR_SHAPE


def _ws(lib, L, T=1, k=4):
    n = ctypes.c_int64()
    rc = lib.tsa_moe_decode_workspace_size(ctypes.byref(L), T, k, ctypes.byref(n))
    return rc, n.value


def test_decode_layout_validation(lib):
    lay = synth.mxfp4_layout(2880, 2880)
    L = mxfp4_expert_layout(lay)
    rc, n = _ws(lib, L)
    assert rc == 0 and n >= 4 * 2880 * 4  # float h of 4 pairs
    L.slot_bytes = lay.total_bytes - 2  # the down bias no longer fits
    assert _ws(lib, L)[0] == _lib.ERR_WEIGHT_TOO_SMALL
    L = mxfp4_expert_layout(lay)
    L.format = 7
    assert _ws(lib, L)[0] == _lib.ERR_INVALID_ARG
    L = mxfp4_expert_layout(lay)
    L.hidden = 2880 + 16
    assert _ws(lib, L)[0] in (_lib.ERR_SHAPE, _lib.ERR_WEIGHT_TOO_SMALL)


def test_tiled_layout_validation(lib):
    lay = synth.mxfp4_tiled_layout(2880, 2880)
    L = mxfp4_expert_layout(lay, tiled=True)
    assert _ws(lib, L)[0] == 0
    L.gate_off += 8
    rc, _ = _ws(lib, L)
    assert rc == _lib.ERR_SHAPE and b"16-byte aligned" in lib.tsa_last_error()
    G = gguf_expert_layout(synth.gguf_layout(2048, 768, 13, 13, 14), {"gate": 13, "up": 13, "down": 14},
                           {"gate": (2048, 768), "up": (2048, 768), "down": (768, 2048)})
    assert _ws(lib, G, 1, 8)[0] == 0
    G.mx_tiled = 1
    assert _ws(lib, G, 1, 8)[0] == _lib.ERR_INVALID_ARG


def test_gguf_layout_needs_one_gate_up_type(lib):
    G = gguf_expert_layout(synth.gguf_layout(256, 256, 12, 13, 14), {"gate": 12, "up": 13, "down": 14},
                           {"gate": (256, 256), "up": (256, 256), "down": (256, 256)})
    rc, _ = _ws(lib, G, 1, 2)
    assert rc == _lib.ERR_UNSUPPORTED_TYPE


def test_null_and_bad_routing_args(lib):
    L = mxfp4_expert_layout(synth.mxfp4_layout(256, 128))
    rc = lib.tsa_moe_decode_routed(ctypes.byref(L), None, 1, None, 2000, None, 0, 0, 1, 4, None, 2, None, 2, None, None,
                                   None, 0, None)
    assert rc == _lib.ERR_SHAPE and b"E 2000" in lib.tsa_last_error()
    rc = lib.tsa_route_topk(None, 0, 1, 8, 4, 9, None, None, None)
    assert rc == _lib.ERR_INVALID_ARG


def test_router_logits_argument_checks(lib):
    """Shapes, dtypes and pointers are checked before anything is launched; T = 0 is a no-op."""
    rc = lib.tsa_router_logits(None, 2, 1, 12, None, 2, None, 2, 4, None, 2, None)
    assert rc == _lib.ERR_SHAPE and b"multiple of 8" in lib.tsa_last_error()
    rc = lib.tsa_router_logits(None, 7, 1, 16, None, 2, None, 2, 4, None, 2, None)
    assert rc == _lib.ERR_INVALID_ARG and b"bad dtype" in lib.tsa_last_error()
    rc = lib.tsa_router_logits(None, 2, 1, 16, None, 2, None, 2, 4, None, 2, None)
    assert rc == _lib.ERR_INVALID_ARG and b"null pointer" in lib.tsa_last_error()
    assert lib.tsa_router_logits(None, 2, 0, 16, None, 2, None, 2, 4, None, 2, None) == 0


def test_pipeline_tiles_checkpoint_mxfp4_on_copy(lib):
    """The cache layout a device pipeline picks for an MXFP4 store: the tile order for
    checkpoint-order slots whose shapes the tiled kernels take, nothing for tiled stores,
    shapes past the tiled limits or a given cache too small for the tiled bytes."""
    from types import SimpleNamespace

    from tinyserve_amd.expert_pipeline import ExpertPipeline

    pick = ExpertPipeline._mxfp4_tiled_cache_layout
    for H, I in ((256, 128), (2880, 2880)):
        ck, tl = synth.mxfp4_layout(H, I), synth.mxfp4_tiled_layout(H, I)
        got = pick(SimpleNamespace(layout=ck, tiled=False), None, None)
        assert got is not None and got.specs == tl.specs and got.offsets == tl.offsets
        assert list(got.specs) == list(ck.specs)
        assert pick(SimpleNamespace(layout=tl, tiled=True), None, None) is None
        assert pick(SimpleNamespace(layout=ck, tiled=False), SimpleNamespace(expert_bytes=tl.total_bytes - 1),
                    None) is None
        assert pick(SimpleNamespace(layout=ck, tiled=False), SimpleNamespace(expert_bytes=tl.total_bytes),
                    None) is not None
    assert pick(SimpleNamespace(layout=synth.mxfp4_layout(4096, 256), tiled=False), None, None) is None
    assert pick(SimpleNamespace(layout=synth.mxfp4_layout(256, 128), tiled=False), None, torch.nn.SiLU()) is None
