"""Symmetric per-output-channel INT8 linear weights on MI355X.

Mirrors ``ondeviceinfer/quantization.py``: the same format constants, the
same validated ``QuantizedLinearWeight`` container and manifest, the same
``FP16DequantScratch``, and the same functions.  The arithmetic runs in HIP:

* ``quantize_linear_weight`` -> ``wq_w8_quantize`` (bit-identical to the
  reference quantizer, ``quantization.py:226-285``);
* ``dequantize_linear_weight`` -> ``wq_w8_decode`` into the caller's scratch
  (``quantization.py:320-330``);
* ``quantized_linear`` -> ``wq_w8a16_linear``, a fused INT8 x fp16 MFMA
  linear that reads the INT8 weight directly (1 byte per element instead of
  the reference's 5, ``quantization.py:333-353``).  ``scratch`` is validated
  and left untouched.

All tensors must be on the GPU; there is no CPU path.
"""
from __future__ import annotations

from collections.abc import Iterable, Mapping
from dataclasses import dataclass
from math import prod
from typing import Any

import torch
from torch import Tensor

from . import _native

QUANTIZATION_FORMAT = 'int8_per_output_channel_symmetric'
QUANTIZATION_VERSION = 1
QMIN = -127
QMAX = 127


def _state_key(prefix: str, suffix: str) -> str:
    prefix = prefix.rstrip('.')
    return f'{prefix}.{suffix}' if prefix else suffix


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix('torch.')


@dataclass(frozen=True)
class QuantizedLinearWeight:
    """``qweight`` int8 ``[out, in]`` and positive finite ``scale`` ``[out]``;
    a row is ``qweight[row] * scale[row]`` (``quantization.py:37-158``)."""

    qweight: Tensor
    scale: Tensor

    def __post_init__(self) -> None:
        if self.qweight.ndim != 2:
            raise ValueError('qweight must have shape [out_features, in_features]')
        if self.qweight.dtype != torch.int8:
            raise TypeError('qweight must have dtype torch.int8')
        if self.scale.ndim != 1 or self.scale.shape[0] != self.qweight.shape[0]:
            raise ValueError('scale must have shape [out_features]')
        if not self.scale.is_floating_point():
            raise TypeError('scale must use a floating-point dtype')
        if self.qweight.device != self.scale.device:
            raise ValueError('qweight and scale must be on the same device')
        if not bool(torch.isfinite(self.scale).all()):
            raise ValueError('scale must contain only finite values')
        if not bool((self.scale > 0).all()):
            raise ValueError('scale values must be strictly positive')

    @property
    def shape(self) -> torch.Size:
        return self.qweight.shape

    @property
    def out_features(self) -> int:
        return self.qweight.shape[0]

    @property
    def in_features(self) -> int:
        return self.qweight.shape[1]

    @property
    def device(self) -> torch.device:
        return self.qweight.device

    @property
    def storage_nbytes(self) -> int:
        return self.qweight.nbytes + self.scale.nbytes

    def to(self, device, *, non_blocking: bool = False) -> 'QuantizedLinearWeight':
        return type(self)(qweight=self.qweight.to(device=device, non_blocking=non_blocking),
                          scale=self.scale.to(device=device, non_blocking=non_blocking))

    def pin_memory(self) -> 'QuantizedLinearWeight':
        if self.device.type != 'cpu':
            raise ValueError('only CPU quantized weights can be pinned')
        return type(self)(qweight=self.qweight.pin_memory(), scale=self.scale.pin_memory())

    def tensor_dict(self, prefix: str = '') -> dict[str, Tensor]:
        return {_state_key(prefix, 'qweight'): self.qweight, _state_key(prefix, 'scale'): self.scale}

    @classmethod
    def from_tensor_dict(cls, tensors: Mapping[str, Tensor], prefix: str = '') -> 'QuantizedLinearWeight':
        return cls(qweight=tensors[_state_key(prefix, 'qweight')], scale=tensors[_state_key(prefix, 'scale')])

    def manifest_entry(self, prefix: str = '') -> dict[str, Any]:
        return {
            'format': QUANTIZATION_FORMAT,
            'version': QUANTIZATION_VERSION,
            'axis': 0,
            'zero_point': 0,
            'quant_min': QMIN,
            'quant_max': QMAX,
            'shape': list(self.shape),
            'qweight_key': _state_key(prefix, 'qweight'),
            'scale_key': _state_key(prefix, 'scale'),
            'qweight_dtype': _dtype_name(self.qweight.dtype),
            'scale_dtype': _dtype_name(self.scale.dtype),
        }

    def dequantize(self, scratch: 'FP16DequantScratch | Tensor') -> Tensor:
        return dequantize_linear_weight(self, scratch)

    def linear(self, input: Tensor, scratch: 'FP16DequantScratch | Tensor', bias: Tensor | None = None) -> Tensor:
        return quantized_linear(input, self, scratch, bias=bias)


@dataclass
class FP16DequantScratch:
    """Reusable flat fp16 storage for one dequantized weight at a time
    (``quantization.py:161-223``)."""

    buffer: Tensor

    def __post_init__(self) -> None:
        if self.buffer.dtype != torch.float16:
            raise TypeError('dequantization scratch must have dtype torch.float16')
        if self.buffer.ndim != 1:
            raise ValueError('dequantization scratch must be a flat tensor')
        if not self.buffer.is_contiguous():
            raise ValueError('dequantization scratch must be contiguous')

    @classmethod
    def allocate(cls, capacity: int, *, device) -> 'FP16DequantScratch':
        if capacity <= 0:
            raise ValueError('scratch capacity must be positive')
        return cls(torch.empty(capacity, dtype=torch.float16, device=device))

    @classmethod
    def for_weights(cls, weights: Iterable[QuantizedLinearWeight], *, device=None) -> 'FP16DequantScratch':
        weights = tuple(weights)
        if not weights:
            raise ValueError('at least one weight is required')
        target = torch.device(device) if device is not None else weights[0].device
        return cls.allocate(max(w.qweight.numel() for w in weights), device=target)

    @property
    def capacity(self) -> int:
        return self.buffer.numel()

    @property
    def device(self) -> torch.device:
        return self.buffer.device

    def view_for(self, shape: Iterable[int]) -> Tensor:
        shape = tuple(shape)
        required = prod(shape)
        if required > self.capacity:
            raise ValueError(f'scratch capacity {self.capacity} is smaller than required {required}')
        return self.buffer[:required].view(shape)


@torch.no_grad()
def quantize_linear_weight(weight: Tensor, *, row_block_size: int = 256,
                           scale_dtype: torch.dtype = torch.float16) -> QuantizedLinearWeight:
    """Quantize ``[out, in]`` rows on the GPU (``quantization.py:226-285``).

    fp32 arithmetic, ``absmax/127`` stored as fp16 (zero rows: 1; underflow:
    smallest positive fp16), the stored scale divides, round-half-even, clamp
    +-127.  ``row_block_size`` is validated; the kernel processes one row per
    workgroup, which gives the same result for every block size.
    """
    if weight.ndim != 2:
        raise ValueError('linear weight must have shape [out_features, in_features]')
    if not weight.is_floating_point():
        raise TypeError('linear weight must use a floating-point dtype')
    if weight.shape[0] == 0 or weight.shape[1] == 0:
        raise ValueError('linear weight dimensions must be nonzero')
    if row_block_size <= 0:
        raise ValueError('row_block_size must be positive')
    if not torch.empty((), dtype=scale_dtype).is_floating_point():
        raise TypeError('scale_dtype must be floating point')
    if scale_dtype != torch.float16:
        raise ValueError(f'scale_dtype {scale_dtype} is not supported by the GPU quantizer (float16 only)')
    q, s = _native.w8_quantize(weight)
    return QuantizedLinearWeight(qweight=q, scale=s)


def quantize_per_output_channel_int8(weight: Tensor, *, row_block_size: int = 256,
                                     scale_dtype: torch.dtype = torch.float16) -> QuantizedLinearWeight:
    """Explicitly named alias for :func:`quantize_linear_weight`."""
    return quantize_linear_weight(weight, row_block_size=row_block_size, scale_dtype=scale_dtype)


def _scratch_view(scratch: 'FP16DequantScratch | Tensor', shape: torch.Size) -> Tensor:
    if isinstance(scratch, FP16DequantScratch):
        return scratch.view_for(shape)
    if scratch.dtype != torch.float16:
        raise TypeError('dequantization scratch must have dtype torch.float16')
    if not scratch.is_contiguous():
        raise ValueError('dequantization scratch must be contiguous')
    required = prod(shape)
    if scratch.numel() < required:
        raise ValueError(f'scratch capacity {scratch.numel()} is smaller than required {required}')
    return scratch.view(-1)[:required].view(shape)


@torch.no_grad()
def dequantize_linear_weight(weight: QuantizedLinearWeight, scratch: 'FP16DequantScratch | Tensor') -> Tensor:
    """Reconstruct ``weight`` into the reusable fp16 ``scratch``."""
    output = _scratch_view(scratch, weight.shape)
    if output.device != weight.device:
        raise ValueError('scratch and quantized weight must be on the same device')
    output.copy_(_native.w8_decode(weight.qweight, weight.scale))
    return output


@torch.no_grad()
def quantized_linear(input: Tensor, weight: QuantizedLinearWeight, scratch: 'FP16DequantScratch | Tensor', *,
                     bias: Tensor | None = None) -> Tensor:
    """``F.linear(input, dequant(weight), bias)`` computed by the fused W8A16 kernel."""
    if input.dtype != torch.float16:
        raise TypeError('quantized_linear expects FP16 input activations')
    if input.device != weight.device:
        raise ValueError('input and quantized weight must be on the same device')
    if input.shape[-1] != weight.in_features:
        raise ValueError(f'input has {input.shape[-1]} features, expected {weight.in_features}')
    if bias is not None and (bias.dtype != torch.float16 or bias.device != input.device):
        raise ValueError('bias must be FP16 and on the input device')
    _scratch_view(scratch, weight.shape)   # same capacity contract as the reference
    scale = weight.scale if weight.scale.dtype == torch.float16 else weight.scale.half()
    x = input.reshape(-1, weight.in_features)
    y = _native.w8a16_linear(x, weight.qweight, scale, bias=bias)
    return y.reshape(*input.shape[:-1], weight.out_features)


__all__ = [
    'FP16DequantScratch', 'QMAX', 'QMIN', 'QUANTIZATION_FORMAT', 'QUANTIZATION_VERSION',
    'QuantizedLinearWeight', 'dequantize_linear_weight', 'quantize_linear_weight',
    'quantize_per_output_channel_int8', 'quantized_linear',
]
