"""Seeded synthetic inputs for the parity tests and the benchmark (test infrastructure).

There is no checkpoint or network here, so weights are random and quantized by
the rules below.  The rules only have to produce valid pack-quantized tensors;
parity is always measured against ``qdq.decode_weight`` of whatever they emit.

* W4 (configs 2-4): ``W = fp16(N(0,1) * 0.02)``; per (row, 128-group along K)
  asymmetric min-max round-to-nearest with the range widened to include 0
  (the compressed-tensors min-max observer convention): ``s = fp16((max-min)/15)``,
  ``z = clip(rint(-min/s), 0, 15)``, ``q = clip(rint(w/s) + z, 0, 15)``;
  codes packed 8 per int32 along K and zero points 8 per int32 along N,
  exactly the layout ``backend.py:109-118`` validates.
* INT8 (config 1): ``W = fp16(N(0,1) * 0.02)`` through
  ``qdq.quantize_linear_weight``.
* Activations: ``fp16(N(0,1))``.

All draws come from ``numpy.random.default_rng(seed)`` in a fixed order
(weights first, then activations).
"""
from __future__ import annotations

import numpy as np

from . import qdq


def awq_quantize(w: np.ndarray, group_size: int = 128, *, symmetric: bool = False) -> dict:
    """Quantize fp16 ``w [N, K]`` to pack-quantized uint4 tensors (unprefixed keys)."""
    w32 = np.asarray(w).astype(np.float32)
    n, k = w32.shape
    if k % group_size or k % 8 or n % 8:
        raise ValueError('need K % group_size == 0, K % 8 == 0 and N % 8 == 0')
    g = w32.reshape(n, k // group_size, group_size)
    if symmetric:
        absmax = np.abs(g).max(axis=-1)
        s16 = (absmax / np.float32(7.5)).astype(np.float16)
        s16 = np.where(s16 == 0, np.float16(1), s16).astype(np.float16)
        s = s16.astype(np.float32)[..., None]
        q = np.clip(np.rint(g / s) + 8, 0, 15).astype(np.int32).reshape(n, k)
        return {'weight_packed': qdq.pack_unsigned(q, 4, 1),
                'weight_scale': s16,
                'weight_shape': np.array([n, k], dtype=np.int64)}
    mn = np.minimum(g.min(axis=-1), 0)
    mx = np.maximum(g.max(axis=-1), 0)
    s16 = ((mx - mn) / np.float32(15)).astype(np.float16)
    s16 = np.where(s16 == 0, np.float16(1), s16).astype(np.float16)
    s = s16.astype(np.float32)
    z = np.clip(np.rint(-mn / s), 0, 15).astype(np.int32)
    q = np.clip(np.rint(g / s[..., None]) + z[..., None], 0, 15).astype(np.int32).reshape(n, k)
    return {'weight_packed': qdq.pack_unsigned(q, 4, 1),
            'weight_scale': s16,
            'weight_zero_point': qdq.pack_unsigned(z, 4, 0),
            'weight_shape': np.array([n, k], dtype=np.int64)}


def prefixed(tensors: dict, name: str) -> dict:
    """Attach the layer prefix of ``name`` (e.g. ``mlp.up_proj.weight``) to the keys."""
    prefix = name.removesuffix('.weight')
    return {f'{prefix}.{key}': value for key, value in tensors.items()}


def w4_case(n: int, k: int, m: int, *, seed: int = 0, group_size: int = 128,
            symmetric: bool = False, name: str = 'mlp.up_proj.weight') -> tuple[dict, np.ndarray]:
    """One W4A16 case: ``(weights dict with prefixed keys, x fp16 [m, k])``."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    return prefixed(awq_quantize(w, group_size, symmetric=symmetric), name), x


def int8_case(n: int, k: int, m: int, *, seed: int = 0) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """One INT8 case (config 1): ``(w fp16, qweight int8, scale fp16, x fp16)``."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float16)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    q, s = qdq.quantize_linear_weight(w)
    return w, q, s, x
