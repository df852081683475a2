"""Symmetric per-output-channel INT8 linear weights on MI355X.

Keeps the callers' interface of ``ondeviceinfer/quantization.py``: the INT8
v1 format constants and manifest entry, the validated
``QuantizedLinearWeight`` container, ``FP16DequantScratch`` and the same
functions and exceptions.  The arithmetic runs in HIP:

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


def _join_key(prefix: str, leaf: str) -> str:
    """``prefix.leaf`` (a trailing dot on the prefix is ignored; no prefix: ``leaf``)."""
    return '.'.join(part for part in (prefix.rstrip('.'), leaf) if part)


def _check_all(rules) -> None:
    """Raise the exception of the first rule ``(ok, exc_type, message)`` whose
    condition is false; conditions may be callables, evaluated in order (the
    value checks read device memory, so they run only after the cheap ones)."""
    for ok, exc_type, message in rules:
        if not (ok() if callable(ok) else ok):
            raise exc_type(message)


@dataclass(frozen=True)
class QuantizedLinearWeight:
    """One linear weight in the INT8 v1 format: ``qweight`` int8 ``[out, in]``
    and a strictly positive, finite floating-point ``scale [out]``; row ``r``
    stands for ``qweight[r] * scale[r]`` (symmetric, zero point 0).  Same
    fields, methods and errors as ``quantization.py:37-158``."""

    qweight: Tensor
    scale: Tensor

    def __post_init__(self) -> None:
        q, s = self.qweight, self.scale
        _check_all((
            (q.dim() == 2, ValueError, 'qweight must have shape [out_features, in_features]'),
            (q.dtype == torch.int8, TypeError, 'qweight must have dtype torch.int8'),
            (s.dim() == 1 and s.shape[0] == q.shape[0], ValueError, 'scale must have shape [out_features]'),
            (s.is_floating_point(), TypeError, 'scale must use a floating-point dtype'),
            (q.device == s.device, ValueError, 'qweight and scale must be on the same device'),
            (lambda: bool(torch.isfinite(s).all()), ValueError, 'scale must contain only finite values'),
            (lambda: bool((s > 0).all()), ValueError, 'scale values must be strictly positive'),
        ))

    shape = property(lambda self: self.qweight.shape)
    out_features = property(lambda self: int(self.qweight.shape[0]))
    in_features = property(lambda self: int(self.qweight.shape[1]))
    device = property(lambda self: self.qweight.device)

    @property
    def storage_nbytes(self) -> int:
        """Bytes of the INT8 codes plus the scales."""
        return sum(t.numel() * t.element_size() for t in (self.qweight, self.scale))

    def _map(self, fn) -> 'QuantizedLinearWeight':
        return type(self)(qweight=fn(self.qweight), scale=fn(self.scale))

    def to(self, device, *, non_blocking: bool = False) -> 'QuantizedLinearWeight':
        """Both tensors on ``device``, dtypes unchanged."""
        return self._map(lambda t: t.to(device=device, non_blocking=non_blocking))

    def pin_memory(self) -> 'QuantizedLinearWeight':
        """Page-locked host copies (for asynchronous uploads); host weights only."""
        if self.device.type != 'cpu':
            raise ValueError('only CPU quantized weights can be pinned')
        return self._map(Tensor.pin_memory)

    def tensor_dict(self, prefix: str = '') -> dict[str, Tensor]:
        """``{prefix.qweight, prefix.scale}``: the checkpoint keys."""
        return {_join_key(prefix, leaf): getattr(self, leaf) for leaf in ('qweight', 'scale')}

    @classmethod
    def from_tensor_dict(cls, tensors: Mapping[str, Tensor], prefix: str = '') -> 'QuantizedLinearWeight':
        """Inverse of :meth:`tensor_dict`."""
        return cls(**{leaf: tensors[_join_key(prefix, leaf)] for leaf in ('qweight', 'scale')})

    def manifest_entry(self, prefix: str = '') -> dict[str, Any]:
        """The JSON record of this tensor in an INT8 v1 manifest."""
        entry: dict[str, Any] = dict(_MANIFEST_CONSTANTS)
        entry['shape'] = [int(d) for d in self.shape]
        for leaf in ('qweight', 'scale'):
            entry[f'{leaf}_key'] = _join_key(prefix, leaf)
        for leaf in ('qweight', 'scale'):
            entry[f'{leaf}_dtype'] = str(getattr(self, leaf).dtype).split('.')[-1]
        return entry

    def dequantize(self, scratch: 'FP16DequantScratch | Tensor') -> Tensor:
        return dequantize_linear_weight(self, scratch)

    def linear(self, input: Tensor, scratch: 'FP16DequantScratch | Tensor', bias: Tensor | None = None) -> Tensor:
        return quantized_linear(input, self, scratch, bias=bias)


# Fields every INT8 v1 manifest entry carries, in the format's key order.
_MANIFEST_CONSTANTS = (('format', QUANTIZATION_FORMAT), ('version', QUANTIZATION_VERSION), ('axis', 0),
                       ('zero_point', 0), ('quant_min', QMIN), ('quant_max', QMAX))


@dataclass
class FP16DequantScratch:
    """A flat, contiguous fp16 buffer that holds one dequantized weight at a
    time; any shape up to its capacity is a view of its head.  Same API as
    ``quantization.py:161-223`` (reuse is ordered by the stream it is used on)."""

    buffer: Tensor

    def __post_init__(self) -> None:
        b = self.buffer
        _check_all((
            (b.dtype == torch.float16, TypeError, 'dequantization scratch must have dtype torch.float16'),
            (b.dim() == 1, ValueError, 'dequantization scratch must be a flat tensor'),
            (b.is_contiguous(), ValueError, 'dequantization scratch must be contiguous'),
        ))

    @classmethod
    def allocate(cls, capacity: int, *, device) -> 'FP16DequantScratch':
        if capacity <= 0:
            raise ValueError(f'scratch capacity must be positive, got {capacity}')
        return cls(torch.empty(capacity, dtype=torch.float16, device=device))

    @classmethod
    def for_weights(cls, weights: Iterable[QuantizedLinearWeight], *, device=None) -> 'FP16DequantScratch':
        """Sized for the largest of ``weights``, on ``device`` (default: the first weight's)."""
        sizes, first_device = [], None
        for w in weights:
            sizes.append(w.qweight.numel())
            first_device = first_device or w.device
        if not sizes:
            raise ValueError('at least one weight is required')
        return cls.allocate(max(sizes), device=torch.device(device) if device is not None else first_device)

    capacity = property(lambda self: self.buffer.numel())
    device = property(lambda self: self.buffer.device)

    def view_for(self, shape: Iterable[int]) -> Tensor:
        return _head_view(self.buffer, tuple(shape))


def _head_view(flat: Tensor, shape: tuple) -> Tensor:
    need = prod(shape)
    if need > flat.numel():
        raise ValueError(f'scratch capacity {flat.numel()} is smaller than required {need}')
    return flat.narrow(0, 0, need).view(shape)


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
    """``shape``-view of the head of a scratch object or of a raw fp16 tensor
    (held to the same rules as ``FP16DequantScratch``)."""
    if not isinstance(scratch, FP16DequantScratch):
        scratch = FP16DequantScratch(scratch.view(-1) if scratch.is_contiguous() else scratch)
    return scratch.view_for(shape)


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
