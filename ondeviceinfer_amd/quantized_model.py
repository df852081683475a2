"""Runtime INT8 weight-only linear for the INT8 v1 checkpoint format.

Mirrors ``int8_weight_only_linear`` and ``QuantizedComputeStats`` of
``ondeviceinfer/quantized_model.py:27-121``.  The reference dequantizes each
matrix into a shared fp16 scratch (``copy_`` + ``mul_``) and then runs an fp16
GEMM; here one fused HIP kernel (``wq_w8a16_linear``) reads the INT8 weight
once, so ``scratch`` is only validated and the dequant timing list stays
empty.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Mapping

import torch
from torch import Tensor

from . import _native
from .profiling import nvtx_range
from .runtime.quantized import LINEAR_WEIGHT_NAMES, qweight_name, scale_name


@dataclass
class QuantizedComputeStats:
    """Optional event timing of the linear kernels (``quantized_model.py:27-60``)."""

    enabled: bool = False
    dequant_events: list = field(default_factory=list)
    gemm_events: list = field(default_factory=list)
    dequantized_weight_bytes: int = 0
    linear_calls: int = 0

    def reset(self) -> None:
        self.dequant_events.clear()
        self.gemm_events.clear()
        self.dequantized_weight_bytes = 0
        self.linear_calls = 0

    @staticmethod
    def _seconds(events) -> float:
        if not events:
            return 0.0
        torch.cuda.synchronize()
        return sum(start.elapsed_time(end) for start, end in events) / 1000.0

    def dequant_seconds(self) -> float:
        return self._seconds(self.dequant_events)

    def gemm_seconds(self) -> float:
        return self._seconds(self.gemm_events)


def int8_weight_only_linear(inputs: Tensor, weights: Mapping[str, Tensor], weight_name: str, scratch: Tensor, *,
                            stats: QuantizedComputeStats | None = None) -> Tensor:
    """``inputs . (qweight * scale)^T`` for one decoder linear, fused on the GPU.

    Same keys (``prefix.qweight`` int8 ``[N, K]``, ``prefix.scale`` fp16 ``[N]``),
    same validation and errors as ``quantized_model.py:76-101``; work is queued
    on the current stream.
    """
    if weight_name not in LINEAR_WEIGHT_NAMES:
        raise KeyError(f'Unsupported quantized linear tensor {weight_name!r}')
    qweight = weights[qweight_name(weight_name)]
    scale = weights[scale_name(weight_name)]
    if qweight.device != inputs.device or scale.device != inputs.device:
        raise ValueError('INT8 weights, scales, and activations must share a device')
    if qweight.numel() > scratch.numel():
        raise ValueError(f'Scratch has {scratch.numel()} elements, but {weight_name} needs {qweight.numel()}')
    if stats is not None:
        stats.linear_calls += 1
    n, k = qweight.shape
    x = inputs.reshape(-1, k)
    scale16 = scale if scale.dtype == torch.float16 else scale.half()
    with nvtx_range(f'w8a16_linear::{weight_name}'):
        if stats is not None and stats.enabled and inputs.device.type == 'cuda':
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            y = _native.w8a16_linear(x, qweight, scale16)
            end.record()
            stats.gemm_events.append((start, end))
        else:
            y = _native.w8a16_linear(x, qweight, scale16)
    return y.reshape(*inputs.shape[:-1], n)
