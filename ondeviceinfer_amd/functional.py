"""Stateless Qwen3 decoder math used by the prefill path.

Mirrors ``ondeviceinfer/functional.py:17-22``.  ``rms_norm`` on GPU tensors of
the shape the decoder uses runs the HIP ``wq_add_rmsnorm`` kernel (same
operation order: fp32 normalize, cast to fp16, scale in fp16); other shapes
(per-head q/k norms) use the same formula in torch.
"""
from __future__ import annotations

import torch
from torch import Tensor

from . import _native


def _native_norm_ok(hidden_states: Tensor, weight: Tensor) -> bool:
    return (hidden_states.is_cuda and hidden_states.dtype == torch.float16 and weight.dtype == torch.float16
            and hidden_states.is_contiguous() and hidden_states.shape[-1] % 8 == 0
            and hidden_states.shape[-1] >= 256)


def add_rms_norm(residual: Tensor, delta: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """``(residual + delta, rms_norm(residual + delta))``: the decoder's residual
    add followed by the next RMSNorm (``quantized_model.py:208-215``), one HIP
    launch on GPU tensors of the decoder's shape.  The kernel adds in fp16 like
    torch's ``+``, so both outputs equal the two-step form bit for bit."""
    if (_native_norm_ok(residual, weight) and delta.is_contiguous() and delta.dtype == residual.dtype
            and delta.shape == residual.shape):
        summed = torch.empty_like(residual)
        normed = _native.add_rmsnorm(residual, weight.contiguous(), eps, delta=delta, out_sum=summed)
        return summed, normed
    summed = residual + delta
    return summed, rms_norm(summed, weight, eps)


def rms_norm(hidden_states: Tensor, weight: Tensor, eps: float) -> Tensor:
    """``weight * fp16(x32 * rsqrt(mean(x32^2) + eps))`` over the last dimension."""
    if _native_norm_ok(hidden_states, weight):
        return _native.add_rmsnorm(hidden_states, weight.contiguous(), eps)
    input_dtype = hidden_states.dtype
    states_fp32 = hidden_states.float()
    variance = states_fp32.square().mean(dim=-1, keepdim=True)
    normalized = states_fp32 * torch.rsqrt(variance + eps)
    return weight * normalized.to(input_dtype)
