"""ctypes binding of ``libtinyserve_amd.so`` (the C ABI declared in include/tinyserve_amd.h).

The library is built in-tree by ``tinyserve_amd.build`` (or ``__graft_entry__.build()``).
Loading fails loudly: there is no fallback implementation behind these calls.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtinyserve_amd.so")

# tsa_status
OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED_TYPE = -2
ERR_SHAPE = -3
ERR_WEIGHT_TOO_SMALL = -4
ERR_ACT_TOO_SMALL = -5
ERR_WORKSPACE = -6
ERR_HIP = -7

# tsa_dtype
F32, F16, BF16 = 0, 1, 2
_TORCH_TO_TSA = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# routing modes / activations / expert formats
ROUTE_TOPK_SOFTMAX, ROUTE_SOFTMAX_TOPK, ROUTE_SOFTMAX_TOPK_RENORM = 0, 1, 2
ACT_SILU, ACT_SWIGLU_OAI = 0, 1
EXPERT_MXFP4, EXPERT_GGUF = 1, 2
PREFILL_FP6, PREFILL_BF16 = 0, 1


class ExpertLayout(ctypes.Structure):
    """Mirror of ``tsa_expert_layout``."""

    _fields_ = [
        ("format", ctypes.c_int32),
        ("act", ctypes.c_int32),
        ("hidden", ctypes.c_int64),
        ("inter", ctypes.c_int64),
        ("slot_bytes", ctypes.c_int64),
        ("gate_type", ctypes.c_int32),
        ("up_type", ctypes.c_int32),
        ("down_type", ctypes.c_int32),
        ("bias_dtype", ctypes.c_int32),
        ("gate_off", ctypes.c_int64),
        ("up_off", ctypes.c_int64),
        ("down_off", ctypes.c_int64),
        ("gate_scales_off", ctypes.c_int64),
        ("down_scales_off", ctypes.c_int64),
        ("gate_bias_off", ctypes.c_int64),
        ("down_bias_off", ctypes.c_int64),
        ("swiglu_limit", ctypes.c_float),
        ("swiglu_alpha", ctypes.c_float),
        ("mx_tiled", ctypes.c_int32),
        ("prefill_mfma", ctypes.c_int32),
    ]


# name -> (restype, argtypes); every symbol include/tinyserve_amd.h declares.
_P, _I64, _I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
_LP = ctypes.POINTER(ExpertLayout)
SIGNATURES = {
    "tsa_version": (_I32, []),
    "tsa_status_string": (ctypes.c_char_p, [_I32]),
    "tsa_last_error": (ctypes.c_char_p, []),
    "tsa_gguf_block_info": (_I32, [_I32, ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "tsa_gguf_dequant": (_I32, [_I32, _P, _I64, _I64, _P, _I32, _P]),
    "tsa_gguf_matvec": (_I32, [_I32, _P, _I64, _P, _I32, _I64, _I64, _P, _I32, _I64, _P]),
    "tsa_mxfp4_dequant": (_I32, [_P, _P, _I64, _I64, _P, _I32, _I32, _P]),
    "tsa_mxfp4_tile_sizes": (_I32, [_I64, _I64, _P, _P]),
    "tsa_mxfp4_tile": (_I32, [_P, _P, _I64, _I64, _P, _P, _P]),
    "tsa_mxfp4_matvec": (_I32, [_P, _P, _P, _I32, _P, _I32, _I64, _P, _I32, _I64, _I64, _P]),
    "tsa_route_topk": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _P, _P, _P]),
    "tsa_router_logits": (_I32, [_P, _I32, _I64, _I64, _P, _I32, _P, _I32, _I64, _P, _I32, _P]),
    "tsa_moe_decode_workspace_size": (_I32, [_LP, _I64, _I32, ctypes.POINTER(_I64)]),
    "tsa_moe_decode": (_I32, [_LP, _P, _I64, _P, _P, _I64, _I32, _P, _I32, _P, _I32, _P, _I64, _P]),
    "tsa_moe_decode_routed": (_I32, [_LP, _P, _I64, _P, _I64, _P, _I32, _I32, _I64, _I32, _P, _I32, _P, _I32, _P, _P,
                                     _P, _I64, _P]),
    "tsa_moe_decode_routed_noalloc": (_I32, [_LP, _P, _I64, _P, _I64, _P, _I32, _I32, _I64, _I32, _P, _I32, _P, _I32,
                                             _P, _P, _P]),
    "tsa_set_decode_options": (_I32, [_I32, ctypes.c_uint32]),
    "tsa_moe_decode_workspace_status": (_I32, [_P, _I64, ctypes.POINTER(_I32), _P]),
    "tsa_group_by_expert": (_I32, [_P, _I64, _I32, _I64, _P, _P, _P, _P]),
    "tsa_moe_prefill_workspace_size": (_I32, [_LP, _I64, _I32, _I64, ctypes.POINTER(_I64)]),
    "tsa_moe_prefill": (_I32, [_LP, _P, _I64, _P, _I64, _P, _P, _I64, _I32, _P, _I32, _P, _I32, _P, _I64, _P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library (raises RuntimeError if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"tinyserve_amd HIP library not found at {LIB_PATH}; build it with "
                "`python -m tinyserve_amd.build` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        lib = load()
        msg = lib.tsa_last_error().decode() or lib.tsa_status_string(rc).decode()
        raise RuntimeError(msg)


def tsa_dtype(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_TSA[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def stream_handle(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors: torch.Tensor, what: str = "tensor") -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"{what} must be on CUDA")
