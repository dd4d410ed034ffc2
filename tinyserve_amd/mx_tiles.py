"""Host-side packing of MXFP4 matrices into the 16-row MFMA tile order.

The fast decode kernels read each expert matrix as 16-row tiles in which every 1 KB
piece is one wave-wide MFMA operand (see tinyserve_amd/csrc/mx_tile.hip for the
layout). ``tile_mxfp4`` is the numpy version used when building host-side expert
stores; ``ops.mxfp4_tile`` does the same on the GPU. Both produce identical bytes.
"""
from __future__ import annotations

import numpy as np


def tile_groups(K: int) -> int:
    """MFMA groups (1 KB pieces) per 16-row tile of a K-column matrix."""
    return (K // 32 + 3) // 4


def tile_scale_words(K: int) -> int:
    """32-bit scale words per lane of a 16-row tile (byte m % 4 of word m // 4 = group m)."""
    return (tile_groups(K) + 3) // 4


def tile_scale_bytes(K: int) -> int:
    """Scale bytes per 16-row tile (64 lanes' words, zero-padded)."""
    return 256 * tile_scale_words(K)


def tile_sizes(N: int, K: int) -> tuple[int, int]:
    if N <= 0 or K <= 0 or N % 16 or K % 32:
        raise ValueError(f"tiled MXFP4 needs N % 16 == 0 and K % 32 == 0 (N {N}, K {K})")
    return N * K // 2, N // 16 * tile_scale_bytes(K)


def tile_offsets(N: int, K: int) -> tuple[np.ndarray, np.ndarray]:
    """Byte offset of block (n, b) in the tiled blocks and of its scale in the tiled
    scales, as [N, G] int64 arrays."""
    G = K // 32
    n = np.arange(N, dtype=np.int64)[:, None]
    b = np.arange(G, dtype=np.int64)[None, :]
    r, i = n // 16, n % 16
    lane = 16 * (b % 4) + i
    boff = r * 256 * G + 1024 * (b // 4) + 16 * lane
    W = tile_scale_words(K)
    w = b // 16  # the lane's word holding group m = b // 4 (byte m % 4); words go in chunks of 4
    ch = w // 4
    width = np.minimum(4, W - 4 * ch)
    soff = r * 256 * W + 1024 * ch + 4 * width * lane + 4 * (w % 4) + (b // 4) % 4
    return boff, soff


def tile_mxfp4(blocks: np.ndarray, scales: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """blocks [N, G, 16] uint8 + scales [N, G] uint8 -> (tiled blocks, tiled scales) as
    flat uint8 arrays of ``tile_sizes(N, 32 G)`` bytes."""
    N, G = scales.shape
    K = 32 * G
    bb, sb = tile_sizes(N, K)
    boff, soff = tile_offsets(N, K)
    tb = np.empty(bb // 16, dtype=np.dtype((np.uint8, 16)))
    tb[(boff // 16).reshape(-1)] = np.ascontiguousarray(blocks).reshape(N * G, 16)
    ts = np.zeros(sb, dtype=np.uint8)
    ts[soff.reshape(-1)] = np.ascontiguousarray(scales).reshape(-1)
    return tb.view(np.uint8).reshape(-1), ts
