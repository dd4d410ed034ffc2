"""MI355X-native (gfx950) expert-FFN hot path: fused dequant + matvec over native GGUF
(Q8_0, Q4_K, Q5_K, Q6_K) and MXFP4 expert weights, fused top-k MoE decode, and the
grouped-by-expert prefill, behind the C ABI in include/tinyserve_amd.h."""

__version__ = "0.1.0"
