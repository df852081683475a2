"""Decoder-layer tensor names, mirroring ``ondeviceinfer/runtime/quantized.py:27-54``.

These names are the keys of the per-layer weight dicts that the linear
backends read (``prefix.qweight`` / ``prefix.scale`` for the INT8 v1 format,
``prefix.weight_packed`` ... for compressed-tensors pack-quantized).
"""
from __future__ import annotations

LINEAR_WEIGHT_NAMES = (
    'self_attn.q_proj.weight',
    'self_attn.k_proj.weight',
    'self_attn.v_proj.weight',
    'self_attn.o_proj.weight',
    'mlp.gate_proj.weight',
    'mlp.up_proj.weight',
    'mlp.down_proj.weight',
)

NORM_WEIGHT_NAMES = (
    'input_layernorm.weight',
    'post_attention_layernorm.weight',
    'self_attn.q_norm.weight',
    'self_attn.k_norm.weight',
)


def qweight_name(weight_name: str) -> str:
    """``x.weight`` -> ``x.qweight`` (``runtime/quantized.py:45-48``)."""
    if not weight_name.endswith('.weight'):
        raise ValueError(f'Expected a .weight suffix, got {weight_name!r}')
    return weight_name.removesuffix('.weight') + '.qweight'


def scale_name(weight_name: str) -> str:
    """``x.weight`` -> ``x.scale`` (``runtime/quantized.py:51-54``)."""
    if not weight_name.endswith('.weight'):
        raise ValueError(f'Expected a .weight suffix, got {weight_name!r}')
    return weight_name.removesuffix('.weight') + '.scale'
