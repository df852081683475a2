"""numpy model of the gfx950 tile layouts that the repack kernels write (test infrastructure).

The layouts are this build's own (the reference's Marlin tile order is vLLM
internal and deliberately not reproduced).  This model is the byte-level
definition the HIP repack is compared against; it is pinned by

* ``unpack(repack(x)) == x`` bit-exactly on random pack-quantized tensors, and
* ``dequant(repack(x)) == qdq.decode_weight(x)`` bit-exactly,

so a wrong index or nibble order fails one of those checks.

W4 layout (G a multiple of 128, K a multiple of G, N a multiple of 8)
--------------------------------------------------------------------
``tiles``: uint32 ``[N16/16, K/128, 64, 4]``.  One 1 KiB block holds 16 rows x
128 k.  Lane ``l`` of a wavefront owns row ``16*t + l%16`` and k range
``128*blk + 32*(l//16) + [0, 32)``; its word ``w`` covers
``k0 = 128*blk + 32*(l//16) + 8*w`` .. ``k0+7`` with nibble ``p`` holding
element ``NIBBLE_ORDER[p]``.  That order puts elements (0,1), (2,3), (4,5),
(6,7) in the two 16-bit halves of ``w & 0x000F000F``, ``w & 0x00F000F0``,
``(w>>8) & 0x000F000F`` and ``(w>>8) & 0x00F000F0`` so the GPU builds fp16
pairs with one AND-OR each.  Rows past N are zero.

``meta``: 40 bytes per (16-row tile, group): 16 fp16 scales (rows in order)
then the two zero-point words of those rows, copied from
``weight_zero_point[2t, g]`` and ``[2t+1, g]`` (``0x88888888`` = z 8 for the
symmetric uint4b8 format).

INT8 layout (K a multiple of 128)
---------------------------------
``tiles``: int8 ``[ceil(N/16), K/128, 2, 64, 16]``: per (16-row tile ``t``,
128-k block ``b``) two 1 KiB pieces; lane ``l`` of piece ``p`` holds
``q[16t + l%16, 128b + 64p + 16*(l//16) + j]`` for ``j`` in 0..15, the 16 bytes
the INT8 kernels feed to lane ``l`` (pieces 0 and 1 = the first and second
64 k of the block).  Rows past N are zero.  The row-major ``[N, K]`` weight
stays the public form; this one is pinned by ``w8_unpack(w8_repack(q)) == q``
and by the GPU linears returning the same bits from either form.
"""
from __future__ import annotations

import numpy as np

NIBBLE_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)   # nibble p holds element NIBBLE_ORDER[p]
W4_BLOCK_K = 128
W4_META_BYTES = 40
SYMMETRIC_ZERO_WORD = 0x88888888


def _ceil16(n: int) -> int:
    return -(-n // 16) * 16


def permute_nibbles(words: np.ndarray) -> np.ndarray:
    """Source word (element e at nibble e) -> tile word (NIBBLE_ORDER)."""
    src = np.asarray(words).view(np.uint32).astype(np.uint64)
    out = np.zeros_like(src)
    for p, e in enumerate(NIBBLE_ORDER):
        out |= ((src >> np.uint64(4 * e)) & np.uint64(0xF)) << np.uint64(4 * p)
    return out.astype(np.uint32)


def unpermute_nibbles(words: np.ndarray) -> np.ndarray:
    src = np.asarray(words).view(np.uint32).astype(np.uint64)
    out = np.zeros_like(src)
    for p, e in enumerate(NIBBLE_ORDER):
        out |= ((src >> np.uint64(4 * p)) & np.uint64(0xF)) << np.uint64(4 * e)
    return out.astype(np.uint32)


def w4_check(n: int, k: int, group_size: int) -> None:
    if n <= 0 or k <= 0 or n % 8 or k % W4_BLOCK_K or group_size % W4_BLOCK_K or k % group_size:
        raise ValueError('W4 tile layout needs N % 8 == 0, G % 128 == 0 and K % G == 0')


def w4_repack(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray | None,
              n: int, k: int, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    w4_check(n, k, group_size)
    n16, nblk, ngrp = _ceil16(n), k // W4_BLOCK_K, k // group_size
    src = np.zeros((n16, k // 8), dtype=np.uint32)
    src[:n] = np.asarray(packed).view(np.uint32)
    # src word index for (tile t, blk, lane l, word w) = 16*blk + 4*(l//16) + w
    lanes = np.arange(64)
    rows = (np.arange(n16 // 16)[:, None, None, None] * 16 + (lanes % 16)[None, None, :, None])
    cols = (np.arange(nblk)[None, :, None, None] * 16 + 4 * (lanes // 16)[None, None, :, None]
            + np.arange(4)[None, None, None, :])
    tiles = permute_nibbles(src[rows, cols])
    meta = np.zeros((n16 // 16, ngrp, W4_META_BYTES), dtype=np.uint8)
    s = np.zeros((n16, ngrp), dtype=np.float16)
    s[:n] = np.asarray(scale).astype(np.float16).reshape(n, ngrp)
    meta[:, :, :32] = s.reshape(n16 // 16, 16, ngrp).transpose(0, 2, 1).copy().view(np.uint8).reshape(n16 // 16, ngrp, 32)
    z = np.zeros((n16 // 8, ngrp), dtype=np.uint32)
    if zero is None:
        z[:n // 8] = SYMMETRIC_ZERO_WORD
    else:
        z[:n // 8] = np.asarray(zero).view(np.uint32).reshape(n // 8, ngrp)
    meta[:, :, 32:] = z.reshape(n16 // 16, 2, ngrp).transpose(0, 2, 1).copy().view(np.uint8).reshape(n16 // 16, ngrp, 8)
    return tiles, meta


def w4_unpack(tiles: np.ndarray, meta: np.ndarray, n: int, k: int,
              group_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Inverse of :func:`w4_repack`: ``(packed [N,K/8] int32, scale [N,K/G] fp16, zero [N/8,K/G] int32)``."""
    w4_check(n, k, group_size)
    n16, nblk, ngrp = _ceil16(n), k // W4_BLOCK_K, k // group_size
    t = np.asarray(tiles).view(np.uint32).reshape(n16 // 16, nblk, 4, 16, 4)   # [t, blk, b, i, w]
    words = unpermute_nibbles(t).transpose(0, 3, 1, 2, 4).reshape(n16, k // 8)
    m = np.asarray(meta).view(np.uint8).reshape(n16 // 16, ngrp, W4_META_BYTES)
    s = m[:, :, :32].copy().view(np.float16).reshape(n16 // 16, ngrp, 16).transpose(0, 2, 1).reshape(n16, ngrp)
    z = m[:, :, 32:].copy().view(np.uint32).reshape(n16 // 16, ngrp, 2).transpose(0, 2, 1).reshape(n16 // 8, ngrp)
    return (words[:n].view(np.int32).copy(), s[:n].copy(), z[:n // 8].view(np.int32).copy())


def w4_dequant(tiles: np.ndarray, meta: np.ndarray, n: int, k: int, group_size: int) -> np.ndarray:
    """fp16 ``(q - z) * s`` read back from the tile layout (model of the GPU dequant)."""
    packed, scale, zero = w4_unpack(tiles, meta, n, k, group_size)
    from .qdq import unpack_unsigned
    q = unpack_unsigned(packed, 4, 1, k).astype(np.float32)
    z = unpack_unsigned(zero, 4, 0, n).astype(np.float32)
    groups = np.arange(k) // group_size
    return ((q - z[:, groups]) * scale.astype(np.float32)[:, groups]).astype(np.float16)


def w8_repack(q: np.ndarray) -> np.ndarray:
    """Row-major INT8 ``[N, K]`` -> tiles ``[ceil(N/16), K/128, 2, 64, 16]`` int8."""
    q = np.asarray(q, dtype=np.int8)
    n, k = q.shape
    if k % W4_BLOCK_K:
        raise ValueError(f'INT8 tiles need k % 128 == 0, got k={k}')
    qp = np.zeros((_ceil16(n), k), dtype=np.int8)
    qp[:n] = q
    # [t, i, b, p, kb, j] -> [t, b, p, kb, i, j]: lane l = 16*kb + i
    v = qp.reshape(-1, 16, k // 128, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5)
    return np.ascontiguousarray(v).reshape(-1, k // 128, 2, 64, 16)


def w8_unpack(tiles: np.ndarray, n: int, k: int) -> np.ndarray:
    t = np.asarray(tiles, dtype=np.int8).reshape(-1, k // 128, 2, 4, 16, 16)
    q = t.transpose(0, 4, 1, 2, 3, 5).reshape(-1, k)
    return np.ascontiguousarray(q[:n])

