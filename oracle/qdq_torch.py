"""torch-on-CPU restatement of the reference's explicit QDQ path (test and
baseline infrastructure only).

Used by ``bench.py``'s ``cpu_baseline`` leg (multi-threaded CPU timing of the
path the HIP kernels replace) and by ``tests/``; the product never imports it.

* ``decode_weight`` restates ``ondeviceinfer/weight_quantization/backend.py:35-54``
  (W4 pack-quantized: ``fp16((q - z) * s)`` in fp32, ``z = 8`` without a zero
  point; INT8 channel: ``fp16(q * s[n])``), with the nibble extraction of
  ``unpack_unsigned`` (``backend.py:26-32``);
* ``qdq_linear`` is that decode followed by ``F.linear`` accumulated in fp32
  and rounded to fp16 (``backend.py:257-263``; the parity contract fixes the
  accumulation type);
* ``int8_qdq_linear`` restates ``int8_weight_only_linear``
  (``quantized_model.py:101-121``): ``fp16(q * s)`` then the same linear.

Pinned by ``tests/test_oracle.py``: ``decode_weight`` is bit-identical to
``oracle.qdq.decode_weight`` (itself pinned by the reference's KATs) on W4
with and without zero points and on INT8; the linears agree with
``oracle.qdq.linear_fp32`` within fp32 summation-order rounding.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def unpack_unsigned(packed: torch.Tensor, bits: int, axis: int, length: int) -> torch.Tensor:
    """b-bit fields of int32 words, lowest field first; ``axis=1`` along
    columns, ``axis=0`` along rows (``backend.py:26-32``).  Returns int32."""
    words = packed.to(torch.int32)
    if axis == 0:
        words = words.t()
    shifts = torch.arange(0, 32, bits, dtype=torch.int32)
    fields = torch.bitwise_and(torch.bitwise_right_shift(words.unsqueeze(-1), shifts), (1 << bits) - 1)
    out = fields.reshape(words.shape[0], -1)[:, :length]
    return out.t().contiguous() if axis == 0 else out.contiguous()


def decode_weight(weights: dict, name: str, *, group_size: int = 128) -> torch.Tensor:
    prefix = name.removesuffix('.weight')
    if prefix + '.weight_packed' not in weights:
        q = weights[name].to(torch.float32)
        return (q * weights[prefix + '.weight_scale'].to(torch.float32).reshape(-1, 1)).half()
    n, k = (int(v) for v in weights[prefix + '.weight_shape'].tolist())
    q = unpack_unsigned(weights[prefix + '.weight_packed'], 4, 1, k).to(torch.float32)
    scale = weights[prefix + '.weight_scale'].to(torch.float32)
    zero = weights.get(prefix + '.weight_zero_point')
    z = torch.full_like(scale, 8.0) if zero is None else unpack_unsigned(zero, 4, 0, n).to(torch.float32)
    groups = torch.arange(k) // group_size
    return ((q - z[:, groups]) * scale[:, groups]).half()


def qdq_linear(x: torch.Tensor, weights: dict, name: str, *, group_size: int = 128) -> torch.Tensor:
    w = decode_weight(weights, name, group_size=group_size)
    return F.linear(x.float(), w.float()).half()


def int8_qdq_linear(x: torch.Tensor, qweight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    w = (qweight.to(torch.float32) * scale.to(torch.float32).reshape(-1, 1)).half()
    return F.linear(x.float(), w.float()).half()
