"""Cached grouped-query attention for the prefill path (mirrors
``ondeviceinfer/attention.py:14-85``); single-token decode goes to the HIP
``wq_decode_attention`` kernel instead (see ``quantized_model``)."""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

from .cache import KVCache


def build_causal_mask(query_length: int, key_length: int, *, device: torch.device) -> Tensor:
    """Absolute-position boolean mask; True participates in attention."""
    if query_length > key_length:
        raise ValueError('query_length cannot exceed key_length')
    past_length = key_length - query_length
    query_positions = torch.arange(past_length, key_length, device=device).unsqueeze(-1)
    key_positions = torch.arange(key_length, device=device).unsqueeze(0)
    return key_positions <= query_positions


def cached_scaled_dot_product_attention(query: Tensor, key: Tensor, value: Tensor, *, layer_idx: int,
                                        cache: KVCache | None, attention_mask: Tensor | None = None,
                                        dropout_p: float = 0.0) -> Tensor:
    query_length = query.shape[-2]
    if cache is not None:
        key, value = cache.update(layer_idx, key, value)
    key_length = key.shape[-2]
    is_causal = False
    if attention_mask is None and query_length > 1:
        if key_length == query_length:
            is_causal = True
        else:
            attention_mask = build_causal_mask(query_length, key_length, device=query.device)
    return F.scaled_dot_product_attention(query.contiguous(), key.contiguous(), value.contiguous(),
                                          attn_mask=attention_mask, dropout_p=dropout_p, is_causal=is_causal,
                                          enable_gqa=True)


def strided_prefill_attention(query: Tensor, key: Tensor, value: Tensor) -> Tensor:
    """The causal attention of ``cached_scaled_dot_product_attention`` for a
    resident cache, without its ``.contiguous()`` copies: ``query`` is a
    ``[batch, q_heads, tokens, d]`` view of token-major memory and ``key`` /
    ``value`` the attended cache rows ``[batch, kv_heads, end, d]`` read in
    place.  torch's fused SDPA then returns token-major output, so the
    decoder's ``transpose(1, 2).contiguous()`` copies nothing; same values as
    the contiguous form."""
    query_length, key_length = query.shape[-2], key.shape[-2]
    attention_mask, is_causal = None, False
    if query_length > 1:
        if key_length == query_length:
            is_causal = True
        else:
            attention_mask = build_causal_mask(query_length, key_length, device=query.device)
    return F.scaled_dot_product_attention(query, key, value, attn_mask=attention_mask, dropout_p=0.0,
                                          is_causal=is_causal, enable_gqa=True)
