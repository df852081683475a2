"""numpy restatement of the reference's explicit QDQ path (test oracle only).

Test infrastructure: imported only by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, always as the checker.

Every function cites the reference lines it restates.  Pinning (what checks
this oracle independently of its own formulas):

=========================  ====================================================
function                   pinned by
=========================  ====================================================
unpack_unsigned            reference KAT ``tests/test_weight_quant_backend.py:7-11``
                           (fixture ``kat_unpack``), closed form on random words
pack_unsigned              inverse round trip with ``unpack_unsigned`` on random
                           codes; reproduces the KAT words ``0x76543210``
decode_weight (W4)         reference KATs ``test_weight_quant_backend.py:14-25``,
                           ``:28-32`` (fixtures ``kat_group_decode``,
                           ``kat_symmetric``); brute-force per-element loop
decode_weight (INT8)       reference KAT ``test_weight_quant_backend.py:33-35``
                           (fixture ``kat_int8_channel``)
decode_rows                reference KAT ``test_weight_quant_backend.py:38-45``
                           (fixture ``kat_sampled_rows``)
quantize_linear_weight     reference invariants ``tests/test_quantization.py:21-62``
                           (row-block invariance, error <= 0.6*scale, zero and
                           tiny rows); hand-derived vectors for round-half-even,
                           stored-scale use and the fp16 underflow rule
dequantize_linear_weight   reference KAT ``test_weight_quant_backend.py:33-35``
linear_fp32                float64 brute-force loop on small non-square shapes
quantize_activations_      hand-derived vectors (round-half-even ties at scale
  per_token                1, the fp32 scale bits, the 1e-12 floor of a zero
                           row); the reference's torch expression
                           (``backend.py:258-260``) evaluated on the CPU
reference_w8a8_linear      the reference's torch lines (``backend.py:257-263``)
                           evaluated on the CPU (amax/div/round/clamp, F.linear
                           in fp32)
w8a8_linear_int            Python-integer brute force + float32 scaling on
                           small shapes
parity_metrics             closed-form values on hand-made vectors
=========================  ====================================================
"""
from __future__ import annotations

import numpy as np

QMIN = -127
QMAX = 127


def unpack_unsigned(packed: np.ndarray, bits: int, axis: int, length: int) -> np.ndarray:
    """b-bit unsigned fields of int32 words, least-significant field first.

    Restates ``backend.py:26-32``: ``axis=1`` unpacks along columns
    (``[R, C/8] -> [R, C]``); ``axis=0`` unpacks along rows by unpacking the
    transpose, so ``[R/8, C] -> [R, C]``.  Returns int32.
    """
    value = np.asarray(packed, dtype=np.int32)
    if axis == 0:
        value = value.T
    shifts = np.arange(0, 32, bits, dtype=np.int32)
    fields = (value[..., None] >> shifts) & ((1 << bits) - 1)
    unpacked = fields.reshape(value.shape[0], -1)[:, :length].astype(np.int32)
    return unpacked.T.copy() if axis == 0 else unpacked


def pack_unsigned(values: np.ndarray, bits: int, axis: int) -> np.ndarray:
    """Inverse of :func:`unpack_unsigned` (compressed-tensors ``pack-quantized``).

    ``axis=1`` packs ``32/bits`` consecutive columns into one int32 word,
    first column in the lowest bits (weights ``[N, K] -> [N, K/8]``);
    ``axis=0`` packs consecutive rows (zero points ``[N, G] -> [N/8, G]``).
    Trailing fields of a partial last word are zero.
    """
    v = np.asarray(values, dtype=np.int64)
    if axis == 0:
        v = v.T
    per = 32 // bits
    rows, cols = v.shape
    padded = -(-cols // per) * per
    if padded != cols:
        v = np.concatenate([v, np.zeros((rows, padded - cols), dtype=np.int64)], axis=1)
    if v.min(initial=0) < 0 or v.max(initial=0) >= (1 << bits):
        raise ValueError('values out of range for the field width')
    shifts = np.arange(0, 32, bits, dtype=np.int64)
    words = (v.reshape(rows, -1, per) << shifts).sum(axis=-1)
    words = words.astype(np.uint32).view(np.int32)
    return words.T.copy() if axis == 0 else words


def decode_weight(weights: dict, name: str, *, group_size: int = 128) -> np.ndarray:
    """Explicit dequantization to fp16, restating ``backend.py:35-54``.

    * INT8 channel format (``prefix.weight`` int8 + ``prefix.weight_scale``
      ``[N, 1]``): ``fp16(q * s[n])`` computed in fp32 (``:37-40``).
    * W4 pack-quantized: ``fp16((q - z) * s)`` in fp32 with ``z = 8`` when
      there is no zero point (uint4b8, ``:45-46``); per-column groups come
      from ``weight_g_idx`` when present, else ``k // group_size``
      (``:49-53``).
    """
    prefix = name.removesuffix('.weight')
    if prefix + '.weight_packed' not in weights:
        q = np.asarray(weights[name])
        scale = np.asarray(weights[prefix + '.weight_scale'])
        return (q.astype(np.float32) * scale.astype(np.float32).reshape(-1, 1)).astype(np.float16)
    n, k = (int(x) for x in np.asarray(weights[prefix + '.weight_shape']).tolist())
    packed = np.asarray(weights[prefix + '.weight_packed'])
    scale = np.asarray(weights[prefix + '.weight_scale']).astype(np.float32)
    zero = weights.get(prefix + '.weight_zero_point')
    if zero is None:
        zero = np.full(scale.shape, 8, dtype=np.int32)
    else:
        zero = unpack_unsigned(zero, 4, 0, n)
    g_idx = weights.get(prefix + '.weight_g_idx')
    if g_idx is not None and np.asarray(g_idx).size:
        groups = np.asarray(g_idx).astype(np.int64)
    else:
        groups = np.arange(k) // group_size
    out = np.empty((n, k), dtype=np.float16)

    def rows(r0: int, r1: int) -> None:
        # Every row decodes independently; blocks of rows keep the
        # temporaries small, and numpy runs the blocks on several threads.
        q = unpack_unsigned(packed[r0:r1], 4, 1, k).astype(np.float32)
        out[r0:r1] = (q - zero[r0:r1][:, groups].astype(np.float32)) * scale[r0:r1][:, groups]

    _row_blocks(n, k, rows)
    return out


def _row_blocks(n: int, k: int, fn) -> None:
    """Run ``fn(r0, r1)`` over row blocks of about 2M elements, on a thread
    pool when there is more than one block."""
    step = max(8, (1 << 21) // max(k, 1) // 8 * 8)
    blocks = [(r0, min(n, r0 + step)) for r0 in range(0, n, step)]
    if len(blocks) == 1:
        fn(*blocks[0])
        return
    import os
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=min(len(blocks), os.cpu_count() or 1, 16)) as pool:
        list(pool.map(lambda b: fn(*b), blocks))


def decode_rows(weights: dict, name: str, rows: np.ndarray) -> np.ndarray:
    """Row-sampled decode, restating ``benchmarks/validate_weight_reconstruction.py:20-31``.

    Like the reference it hard-codes groups of 128 along K.
    """
    rows = np.asarray(rows, dtype=np.int64)
    prefix = name.removesuffix('.weight')
    if prefix + '.weight_packed' not in weights:
        q = np.asarray(weights[name])[rows].astype(np.float32)
        s = np.asarray(weights[prefix + '.weight_scale'])[rows].astype(np.float32).reshape(-1, 1)
        return (q * s).astype(np.float16)
    n, k = (int(x) for x in np.asarray(weights[prefix + '.weight_shape']).tolist())
    q = unpack_unsigned(np.asarray(weights[prefix + '.weight_packed'])[rows], 4, 1, k).astype(np.float32)
    zero = weights.get(prefix + '.weight_zero_point')
    scale = np.asarray(weights[prefix + '.weight_scale'])[rows].astype(np.float32)
    groups = np.arange(k) // 128
    if zero is not None:
        z = unpack_unsigned(zero, 4, 0, n)[rows].astype(np.float32)[:, groups]
    else:
        z = np.float32(8)
    return ((q - z) * scale[:, groups]).astype(np.float16)


def quantize_linear_weight(weight: np.ndarray, *, row_block_size: int = 256,
                           scale_dtype=np.float16) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-channel INT8 quantizer, restating ``quantization.py:226-285``.

    Per row, in fp32: ``absmax / 127`` (zero rows get scale 1), stored in
    ``scale_dtype``; a nonzero scale that underflows becomes the smallest
    positive value of that dtype; the *stored* scale (back in fp32) divides
    the row, then round-half-even and clamp to [-127, 127].  Rows are
    processed in blocks of ``row_block_size`` (the result does not depend on
    it).  Returns ``(qweight int8 [N, K], scale [N])``.
    """
    weight = np.asarray(weight)
    if weight.ndim != 2:
        raise ValueError('linear weight must have shape [out_features, in_features]')
    if not np.issubdtype(weight.dtype, np.floating):
        raise TypeError('linear weight must use a floating-point dtype')
    if weight.shape[0] == 0 or weight.shape[1] == 0:
        raise ValueError('linear weight dimensions must be nonzero')
    if row_block_size <= 0:
        raise ValueError('row_block_size must be positive')
    if not np.issubdtype(np.dtype(scale_dtype), np.floating):
        raise TypeError('scale_dtype must be floating point')
    out_features = weight.shape[0]
    qweight = np.empty(weight.shape, dtype=np.int8)
    scales = np.empty(out_features, dtype=scale_dtype)
    smallest = np.nextafter(np.zeros((), dtype=scale_dtype), np.ones((), dtype=scale_dtype))
    for start in range(0, out_features, row_block_size):
        end = min(start + row_block_size, out_features)
        block = weight[start:end].astype(np.float32)
        if not np.isfinite(block).all():
            raise ValueError('linear weight contains NaN or infinity')
        absmax = np.abs(block).max(axis=1)
        raw = absmax / np.float32(QMAX)
        raw = np.where(absmax == 0, np.float32(1), raw).astype(np.float32)
        with np.errstate(over='ignore'):
            stored = raw.astype(scale_dtype)
        underflow = (absmax != 0) & (stored == 0)
        stored = np.where(underflow, smallest, stored).astype(scale_dtype)
        if not np.isfinite(stored).all():
            raise OverflowError('row scale is not representable in scale_dtype')
        q = np.rint(block / stored.astype(np.float32)[:, None])
        np.clip(q, QMIN, QMAX, out=q)
        qweight[start:end] = q.astype(np.int8)
        scales[start:end] = stored
    return qweight, scales


def dequantize_linear_weight(qweight: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """``fp16(q * s[row])``: restates ``quantization.py:320-330`` and the
    copy+mul of ``quantized_model.py:103-106`` (exact product, one rounding)."""
    return (np.asarray(qweight).astype(np.float32)
            * np.asarray(scale).astype(np.float32).reshape(-1, 1)).astype(np.float16)


def linear_fp32(x: np.ndarray, weight_fp16: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """``F.linear(x, W)`` with fp32 accumulation, rounded to fp16.

    The reference's ``F.linear`` on fp16 operands (``backend.py:263``,
    ``quantization.py:353``, ``quantized_model.py:121``); the accumulation type
    is fixed to fp32 as the parity contract states.  ``x [..., K]``, ``W [N, K]``.
    """
    return _linear_w32(x, np.asarray(weight_fp16).astype(np.float32), bias)


def _linear_w32(x: np.ndarray, w32: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    x32 = np.asarray(x).astype(np.float32)
    lead = x32.shape[:-1]
    y = x32.reshape(-1, x32.shape[-1]) @ w32.T
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32)
    return y.astype(np.float16).reshape(*lead, w32.shape[0])


class DecodedLinear:
    """``qdq_linear`` (or ``linear_fp32`` of an fp16 weight) with the decode
    and the fp32 widening of the weight done once, for repeated calls at
    model scale: every call returns exactly what ``qdq_linear`` would."""

    def __init__(self, weights: dict | None, name: str | None = None, *, group_size: int = 128,
                 weight_fp16: np.ndarray | None = None):
        w16 = weight_fp16 if weights is None else decode_weight(weights, name, group_size=group_size)
        self.w32 = np.asarray(w16).astype(np.float32)

    def __call__(self, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
        return _linear_w32(x, self.w32, bias)


def qdq_linear(x: np.ndarray, weights: dict, name: str, *, group_size: int = 128) -> np.ndarray:
    """The ``reference_int4`` backend: ``decode_weight`` then ``F.linear``
    (``backend.py:257-263``)."""
    return linear_fp32(x, decode_weight(weights, name, group_size=group_size))


def int8_weight_only_linear(x: np.ndarray, qweight: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """INT8 explicit path, restating ``quantized_model.py:76-121``: dequantize
    into fp16 then ``F.linear``."""
    return linear_fp32(x, dequantize_linear_weight(qweight, scale))


def quantize_activations_per_token(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token symmetric INT8 of the ``reference_w8a8`` backend
    (``backend.py:258-260``): in fp32, ``scale = max(absmax_row, 1e-12) / 127``,
    ``q = clamp(round(x / scale), -127, 127)`` with round-half-even.  Returns
    ``(q int8 [M, K], scale fp32 [M])``; the reference multiplies them back
    (``* scale``) before its fp16 linear."""
    x32 = np.asarray(x).astype(np.float32)
    absmax = np.abs(x32).max(axis=-1, keepdims=True)
    scale = (np.maximum(absmax, np.float32(1e-12)) / np.float32(127)).astype(np.float32)
    q = np.clip(np.rint(x32 / scale), QMIN, QMAX).astype(np.int8)
    return q, scale[..., 0]


def reference_w8a8_linear(x: np.ndarray, qweight: np.ndarray, w_scale: np.ndarray) -> np.ndarray:
    """The ``reference_w8a8`` backend (``backend.py:257-263``): the channel-INT8
    weight decoded to fp16 (``decode_weight``, ``:37-40``), the activations
    fake-quantized per token (``q * scale`` rounded to fp16), then ``F.linear``."""
    q, s = quantize_activations_per_token(x)
    xq = (q.astype(np.float32) * s[:, None]).astype(np.float16)
    return linear_fp32(xq, dequantize_linear_weight(qweight, w_scale))


def w8a8_linear_int(qx: np.ndarray, x_scale: np.ndarray, qweight: np.ndarray, w_scale: np.ndarray,
                    bias: np.ndarray | None = None) -> np.ndarray:
    """The ``int8_gemm`` backend's scaled INT8 GEMM (vLLM ``cutlass_scaled_mm``,
    called at ``backend.py:254``): the int8 x int8 products summed exactly, then
    ``fp16(float(acc) * x_scale[m] * w_scale[n] (+ bias[n]))`` in fp32, left to
    right.  vLLM (``vllm==0.12.0``) is absent here; this restates the published
    semantics of a scaled int8 matmul (exact integer accumulation, one fp32
    rescale) and is pinned by brute force on small shapes."""
    acc = np.asarray(qx).astype(np.int64) @ np.asarray(qweight).astype(np.int64).T
    y = acc.astype(np.float32) * np.asarray(x_scale).astype(np.float32)[:, None]
    y = y * np.asarray(w_scale).astype(np.float32).reshape(1, -1)
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float32).reshape(1, -1)
    return y.astype(np.float16)


def parity_metrics(actual: np.ndarray, expected: np.ndarray) -> dict:
    """Error statistics of ``actual`` against ``expected`` (both any float dtype).

    ``max_abs`` and ``ref_inf`` give the max-abs criterion
    (``max_abs <= 1e-2 * ref_inf``); ``mean_rel`` is ``mean|d| / mean|y_ref|``;
    ``cosine`` and ``relative_l2`` follow
    ``benchmarks/validate_weight_quant_kernels.py:57-59``.
    """
    a = np.asarray(actual).astype(np.float64).ravel()
    e = np.asarray(expected).astype(np.float64).ravel()
    d = a - e
    ref_inf = float(np.abs(e).max(initial=0.0))
    mean_abs_ref = float(np.abs(e).mean()) if e.size else 0.0
    na, ne = float(np.linalg.norm(a)), float(np.linalg.norm(e))
    cosine = float(a @ e / (na * ne)) if na > 0 and ne > 0 else (1.0 if na == ne else 0.0)
    return {
        'max_abs': float(np.abs(d).max(initial=0.0)),
        'ref_inf': ref_inf,
        'mean_rel': float(np.abs(d).mean() / max(mean_abs_ref, 1e-30)) if d.size else 0.0,
        'relative_l2': float(np.linalg.norm(d) / max(ne, 1e-12)),
        'cosine': cosine,
        'finite': bool(np.isfinite(a).all()),
    }


def parity_ok(metrics: dict) -> bool:
    """The parity bar: max|d| <= 1e-2*||y_ref||_inf, mean rel <= 2e-3, finite,
    plus the reference harness's cosine >= 0.9999 and rel-L2 <= 0.02
    (``validate_weight_quant_kernels.py:76``)."""
    return (metrics['finite']
            and metrics['max_abs'] <= 1e-2 * metrics['ref_inf']
            and metrics['mean_rel'] <= 2e-3
            and metrics['cosine'] >= 0.9999
            and metrics['relative_l2'] <= 0.02)
