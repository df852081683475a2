"""Resident fp16 KV cache for the quantized Qwen3 decoder.

The callers' interface is the reference's (``ondeviceinfer/cache.py:11-92``):
the ``KVCache`` protocol (``get_seq_length`` / ``update`` / ``reset``),
``CacheStats`` and ``ResidentKVCache(num_layers=, batch_size=,
num_key_value_heads=, max_seq_len=, head_dim=, device=, dtype=)`` with
per-layer ``key_cache`` / ``value_cache`` tensors ``[batch, kv_heads,
max_seq_len, head_dim]`` and per-layer ``lengths``.

Storage here is one block per cache, ``[2, layers, batch, kv_heads,
max_seq_len, head_dim]`` (K then V), and the per-layer tensors are views of
it.  A cache can also be laid over storage someone else owns
(``ResidentKVCache.over``): the model keeps a pool of such blocks so that a
captured decode graph, which holds their addresses, is reused by every cache
of the same shape.  The batch-1 decode and prefill kernels write rows of the
views in place; ``update`` is the path of every other caller.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol

import torch
from torch import Tensor


class KVCache(Protocol):
    def get_seq_length(self, layer_idx: int = 0) -> int: ...

    def update(self, layer_idx: int, key_states: Tensor, value_states: Tensor) -> tuple[Tensor, Tensor]: ...

    def reset(self) -> None: ...


@dataclass
class CacheStats:
    """Host <-> device traffic of a cache; a resident cache moves none."""

    cpu_to_gpu_bytes: int = 0
    gpu_to_cpu_bytes: int = 0


def kv_block(num_layers: int, batch_size: int, num_key_value_heads: int, max_seq_len: int, head_dim: int, *,
             device: torch.device | str, dtype: torch.dtype, zero: bool = False) -> Tensor:
    """One allocation for the K and V rows of every layer:
    ``[2, layers, batch, kv_heads, max_seq_len, head_dim]``."""
    shape = (2, num_layers, batch_size, num_key_value_heads, max_seq_len, head_dim)
    return (torch.zeros if zero else torch.empty)(shape, device=device, dtype=dtype)


class ResidentKVCache:
    """All layers' K/V rows resident on one device, with one logical length
    per layer (layers advance one after another inside a forward)."""

    def __init__(self, *, num_layers: int, batch_size: int, num_key_value_heads: int, max_seq_len: int,
                 head_dim: int, device: torch.device | str, dtype: torch.dtype) -> None:
        if max_seq_len <= 0:
            raise ValueError(f'max_seq_len must be positive, got {max_seq_len}')
        self._bind(kv_block(num_layers, batch_size, num_key_value_heads, max_seq_len, head_dim,
                            device=device, dtype=dtype))

    @classmethod
    def over(cls, block: Tensor) -> 'ResidentKVCache':
        """A cache (lengths 0) over an existing ``kv_block``-shaped tensor."""
        if block.dim() != 6 or block.shape[0] != 2:
            raise ValueError(f'expected a [2, layers, batch, heads, seq, dim] block, got {tuple(block.shape)}')
        if block.shape[4] <= 0:
            raise ValueError('max_seq_len must be positive')
        cache = cls.__new__(cls)
        cache._bind(block)
        return cache

    def _bind(self, block: Tensor) -> None:
        self._block = block
        _, layers, self.batch_size, _, self.max_seq_len, _ = block.shape
        self.key_cache = list(block[0].unbind(0))
        self.value_cache = list(block[1].unbind(0))
        self.lengths = [0] * layers
        self.stats = CacheStats()

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.lengths[layer_idx]

    def _span(self, layer_idx: int, key_states: Tensor, value_states: Tensor) -> tuple[int, int]:
        if key_states.shape != value_states.shape:
            raise ValueError(f'key/value shapes differ: {tuple(key_states.shape)} vs {tuple(value_states.shape)}')
        if key_states.shape[0] != self.batch_size:
            raise ValueError(f'cache holds batch {self.batch_size}, got {key_states.shape[0]} (the batch size '
                             'is fixed at allocation)')
        begin = self.lengths[layer_idx]
        stop = begin + key_states.shape[-2]
        if stop > self.max_seq_len:
            raise ValueError(f'KV cache capacity exceeded: requested {stop}, capacity {self.max_seq_len}')
        return begin, stop

    def update(self, layer_idx: int, key_states: Tensor, value_states: Tensor) -> tuple[Tensor, Tensor]:
        """Append ``[batch, kv_heads, tokens, head_dim]`` rows to layer
        ``layer_idx``; returns the layer's K and V rows up to the new length."""
        begin, stop = self._span(layer_idx, key_states, value_states)
        count = stop - begin
        keys, values = self.key_cache[layer_idx], self.value_cache[layer_idx]
        keys.narrow(2, begin, count).copy_(key_states)
        values.narrow(2, begin, count).copy_(value_states)
        self.lengths[layer_idx] = stop
        return keys.narrow(2, 0, stop), values.narrow(2, 0, stop)

    def reset(self) -> None:
        """Forget every row (the storage stays allocated)."""
        self.lengths = [0] * len(self.lengths)
        self.stats = CacheStats()

    @property
    def storage_bytes(self) -> int:
        return self._block.numel() * self._block.element_size()
