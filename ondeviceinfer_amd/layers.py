"""Rotary embedding for the Qwen3 forward.

Mirrors ``ondeviceinfer/layers.py:36-80``: ``RotaryEmbedding`` builds fp16
``cos``/``sin`` from fp32 angles ``position * inv_freq`` with
``inv_freq = 1 / theta ** (arange(0, d, 2) / d)`` and duplicated halves;
``apply_rotary_pos_emb`` is ``x * cos + rotate_half(x) * sin``.  The decode
kernel reads the same tables (``RotaryEmbedding.table``) row by row.
"""
from __future__ import annotations

import torch
from torch import Tensor, nn


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, theta: float = 1_000_000.0) -> None:
        super().__init__()
        if head_dim % 2 != 0:
            raise ValueError('RoPE requires an even head dimension')
        exponent = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
        inv_freq = 1.0 / (theta ** exponent)
        self.register_buffer('inv_freq', inv_freq, persistent=False)

    @torch.no_grad()
    def forward(self, x: Tensor, position_ids: Tensor) -> tuple[Tensor, Tensor]:
        """``cos, sin`` shaped ``[batch, seq_len, head_dim]`` in ``x``'s dtype."""
        if position_ids.ndim != 2:
            raise ValueError('position_ids must have shape [batch, seq_len]')
        positions = position_ids.to(device=x.device, dtype=torch.float32)
        inv_freq = self.inv_freq.to(device=x.device)
        frequencies = positions.unsqueeze(-1) * inv_freq
        angles = torch.cat((frequencies, frequencies), dim=-1)
        return angles.cos().to(x.dtype), angles.sin().to(x.dtype)

    @torch.no_grad()
    def table(self, max_positions: int, device, dtype=torch.float16) -> tuple[Tensor, Tensor]:
        """Contiguous ``[max_positions, head_dim]`` tables, row p = position p."""
        probe = torch.empty(0, device=device, dtype=dtype)
        cos, sin = self.forward(probe, torch.arange(max_positions, device=device).unsqueeze(0))
        return cos[0].contiguous(), sin[0].contiguous()


def rotate_half(x: Tensor) -> Tensor:
    """``[x1, x2] -> [-x2, x1]`` along the head dimension."""
    first, second = x.chunk(2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def apply_rotary_pos_emb(query: Tensor, key: Tensor, cos: Tensor, sin: Tensor) -> tuple[Tensor, Tensor]:
    """RoPE on ``[batch, heads, seq, dim]`` tensors."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return query * cos + rotate_half(query) * sin, key * cos + rotate_half(key) * sin
