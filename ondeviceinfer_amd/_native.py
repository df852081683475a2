"""ctypes binding of ``libondeviceinfer_wq.so`` (the C ABI in ``include/ondeviceinfer_wq.h``
and ``include/ondeviceinfer_decode.h``).

torch is imported first so its bundled HIP runtime (``libamdhip64.so.7``) is
the one the library binds to: the kernels then run in torch's context and on
torch's streams.  The library is built in-tree by
``python -m ondeviceinfer_amd.build``; if it is missing, every entry point
raises instead of computing anything another way.

The tensor-level helpers below validate dtype/shape/device/contiguity in
Python (raising ``TypeError``/``ValueError`` like the reference), pass raw
device pointers plus ``torch.cuda.current_stream()``, and map a nonzero status
to an exception carrying ``wq_last_error()``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import NamedTuple

import torch

LIB_PATH = Path(__file__).resolve().parent / 'libondeviceinfer_wq.so'

WQ_OK = 0
WQ_ERR_INVALID_ARGUMENT = 1
WQ_ERR_UNSUPPORTED = 2
WQ_ERR_HIP = 3
WQ_ERR_WORKSPACE = 4
ABI_VERSION = 2

W4_BLOCK_K = 128
DECODE_ATTENTION_MAX_SEQ = 16384   # wq_decode_attention: the largest cache (max_seq) it takes
W4_META_BYTES = 40
W8_BLOCK_K = 128

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SIZE_P = ctypes.POINTER(ctypes.c_size_t)

# name -> argtypes (restype is int for all but wq_last_error)
_SIGNATURES = {
    'wq_abi_version': [],
    'wq_w4_repack_size': [_I64, _I64, _I64, _SIZE_P, _SIZE_P],
    'wq_w4_repack': [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P],
    'wq_w4_unpack': [_P, _P, _I64, _I64, _I64, _P, _P, _P, _P],
    'wq_w4_dequant': [_P, _P, _I64, _I64, _I64, _P, _P],
    'wq_w4_decode': [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P],
    'wq_w4_decode_rows': [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P],
    'wq_w4a16_workspace_size': [_I64, _I64, _I64, _I64, _SIZE_P],
    'wq_w4a16_linear': [_P, _I64, _I64, _P, _P, _I64, _I64, _P, _P, ctypes.c_size_t, _P],
    'wq_w4a16_linear_noalloc': [_P, _I64, _I64, _P, _P, _I64, _I64, _P, _P],
    'wq_w4a16_epilogue_supported': [_I64, _I64, _I64, _I64, ctypes.c_int32],
    'wq_w4a16_linear_epilogue': [_P, _I64, _I64, _P, _P, _I64, _I64, ctypes.c_int32, _P, _P, _P],
    'wq_w8a16_epilogue_supported': [_I64, _I64, _I64, ctypes.c_int32],
    'wq_w8a16_linear_epilogue': [_P, _I64, _I64, _P, _P, _I64, ctypes.c_int32, _P, _P, _P],
    'wq_w4a16_decode_fused': [_P, _I64, _P, _P, _I64, _I64, ctypes.c_int32, _P, _P, _I64, ctypes.c_float, _P, _P,
                              _P, _P, ctypes.c_size_t, _P],
    'wq_w8a16_decode_fused': [_P, _I64, _P, _P, _I64, ctypes.c_int32, _P, _P, _I64, ctypes.c_float, _P, _P, _P, _P,
                              ctypes.c_size_t, _P],
    'wq_w8a16_decode_fused_tiled': [_P, _I64, _P, _P, _I64, ctypes.c_int32, _P, _P, _I64, ctypes.c_float, _P, _P, _P, _P,
                              ctypes.c_size_t, _P],
    'wq_w8_decode': [_P, _P, _I64, _I64, _P, _P],
    'wq_w8_tiles_size': [_I64, _I64, _SIZE_P],
    'wq_w8_repack': [_P, _I64, _I64, _P, _P],
    'wq_w8_unpack': [_P, _I64, _I64, _P, _P],
    'wq_w8a16_linear_tiled': [_P, _I64, _I64, _P, _P, _I64, _P, _P, _P, ctypes.c_size_t, _P],
    'wq_w8a8_linear_tiled': [_P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P],
    'wq_w8a16_workspace_size': [_I64, _I64, _I64, _SIZE_P],
    'wq_w8a16_linear': [_P, _I64, _I64, _P, _P, _I64, _P, _P, _P, ctypes.c_size_t, _P],
    'wq_w8a8_quantize': [_P, _I64, _I64, _P, _P, _P],
    'wq_w8a8_linear': [_P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P],
    'wq_w8_quantize': [_P, _I64, _I64, _P, _P, _P, _P],
    # include/ondeviceinfer_decode.h
    'wq_add_rmsnorm': [_P, _P, _P, _I64, _I64, ctypes.c_float, _P, _P, _P],
    'wq_silu_mul': [_P, _I64, _I64, _P, _P],
    'wq_decode_attention_workspace_size': [_I64, _I64, _I64, _I64, _SIZE_P],
    'wq_decode_attention': [_P, _I64, _I64, _I64, _P, _P, ctypes.c_float, _P, _P, _P, _P, _P, _I64,
                            ctypes.c_float, _P, _P, ctypes.c_size_t, _P],
    'wq_prefill_qk_rope': [_P, _I64, _I64, _I64, _I64, _P, _P, ctypes.c_float, _P, _P, _I64, _P, _P, _I64, _P, _P],
    'wq_prefill_attention': [_P, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64, ctypes.c_float, _P, _P],
    'wq_lm_head_workspace_size': [_I64, _I64, _SIZE_P],
    'wq_argmax_f16_workspace_size': [_I64, _SIZE_P],
    'wq_argmax_f16': [_P, _I64, _P, _P, ctypes.c_size_t, _P],
    'wq_lm_head': [_P, _I64, _P, _I64, _P, _P, _P, ctypes.c_size_t, _P],
    'wq_host_device_pointer': [_P, ctypes.POINTER(ctypes.c_void_p)],
    'wq_embed_rows': [_P, _I64, _I64, _P, _I64, _P, _P, _P],
    'wq_lm_head_rmsnorm': [_P, _I64, _P, _P, _I64, ctypes.c_float, _P, _I64, _P, _P, _P, ctypes.c_size_t, _P],
}
EXPORTED_SYMBOLS = ('wq_last_error', *_SIGNATURES)

_lib = None
_lock = threading.Lock()


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or unusable; there is no other code path."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argtypes/restypes set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f'{LIB_PATH.name} is not built; run `python -m ondeviceinfer_amd.build` '
                '(needs hipcc with gfx950 support)')
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.wq_last_error.restype = ctypes.c_char_p
        lib.wq_last_error.argtypes = []
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = ctypes.c_int
            fn.argtypes = args
        version = lib.wq_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f'ABI version {version} != expected {ABI_VERSION}; rebuild the library')
        _lib = lib
        return lib


def _raise_for(status: int, what: str) -> None:
    if status == WQ_OK:
        return
    msg = f'{what}: {load().wq_last_error().decode(errors="replace")}'
    if status in (WQ_ERR_INVALID_ARGUMENT, WQ_ERR_UNSUPPORTED, WQ_ERR_WORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def _call(name: str, *args) -> None:
    _raise_for(getattr(load(), name)(*args), name)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != 'cuda':
            raise ValueError(f'expected a GPU tensor, got one on {t.device}; this build has no CPU path')
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f'tensors on different devices: {device} and {t.device}')
    if device is None:
        raise ValueError('no tensor given')
    return device


def _check(t: torch.Tensor, dtype: torch.dtype, shape: tuple, name: str) -> None:
    if t.dtype != dtype:
        raise TypeError(f'{name}: expected {dtype}, got {t.dtype}')
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f'{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}')
    if not t.is_contiguous():
        raise ValueError(f'{name}: must be contiguous')


def _aligned(t: torch.Tensor) -> torch.Tensor:
    return t if t.data_ptr() % 16 == 0 else t.clone()


# ----------------------------------------------------------------------------- W4

def w4_repack_size(n: int, k: int, group_size: int) -> tuple[int, int]:
    tb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    _call('wq_w4_repack_size', n, k, group_size, ctypes.byref(tb), ctypes.byref(mb))
    return tb.value, mb.value


def w4_repack(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor | None,
              n: int, k: int, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """compressed-tensors tensors -> (tiles uint8, meta uint8) in the gfx950 layout."""
    device = _require_gpu(packed, scale, zero)
    _check(packed, torch.int32, (n, k // 8), 'weight_packed')
    _check(scale, torch.float16, (n, k // group_size), 'weight_scale')
    if zero is not None:
        _check(zero, torch.int32, (n // 8, k // group_size), 'weight_zero_point')
    tiles_bytes, meta_bytes = w4_repack_size(n, k, group_size)
    tiles = torch.empty(tiles_bytes, dtype=torch.uint8, device=device)
    meta = torch.empty(meta_bytes, dtype=torch.uint8, device=device)
    _call('wq_w4_repack', _ptr(packed), _ptr(scale), _ptr(zero), n, k, group_size,
          _ptr(tiles), _ptr(meta), _stream(device))
    return tiles, meta


def w4_unpack(tiles: torch.Tensor, meta: torch.Tensor, n: int, k: int,
              group_size: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    device = _require_gpu(tiles, meta)
    tb, mb = w4_repack_size(n, k, group_size)
    _check(tiles, torch.uint8, (tb,), 'tiles')
    _check(meta, torch.uint8, (mb,), 'meta')
    packed = torch.empty((n, k // 8), dtype=torch.int32, device=device)
    scale = torch.empty((n, k // group_size), dtype=torch.float16, device=device)
    zero = torch.empty((n // 8, k // group_size), dtype=torch.int32, device=device)
    _call('wq_w4_unpack', _ptr(tiles), _ptr(meta), n, k, group_size, _ptr(packed), _ptr(scale), _ptr(zero),
          _stream(device))
    return packed, scale, zero


def w4_dequant(tiles: torch.Tensor, meta: torch.Tensor, n: int, k: int, group_size: int) -> torch.Tensor:
    device = _require_gpu(tiles, meta)
    tb, mb = w4_repack_size(n, k, group_size)
    _check(tiles, torch.uint8, (tb,), 'tiles')
    _check(meta, torch.uint8, (mb,), 'meta')
    out = torch.empty((n, k), dtype=torch.float16, device=device)
    _call('wq_w4_dequant', _ptr(tiles), _ptr(meta), n, k, group_size, _ptr(out), _stream(device))
    return out


def w4_decode(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor | None,
              g_idx: torch.Tensor | None, n: int, k: int, group_size: int) -> torch.Tensor:
    """Explicit QDQ decode from compressed-tensors tensors (any group size, g_idx)."""
    device = _require_gpu(packed, scale, zero, g_idx)
    if packed.dtype != torch.int32 or packed.dim() != 2 or packed.shape[0] != n or packed.shape[1] * 8 < k:
        raise ValueError(f'weight_packed must be int32 [{n}, {k // 8}], got {packed.dtype} {tuple(packed.shape)}')
    if k % 8:
        raise ValueError('decode needs k % 8 == 0')
    packed = packed[:, :k // 8].contiguous()
    scale32 = scale.float().contiguous()
    if scale32.dim() != 2 or scale32.shape[0] != n:
        raise ValueError(f'weight_scale must be [{n}, groups], got {tuple(scale.shape)}')
    if zero is not None:
        if zero.dtype != torch.int32 or tuple(zero.shape) != ((n + 7) // 8, scale32.shape[1]):
            raise ValueError(f'weight_zero_point must be int32 [{(n + 7) // 8}, {scale32.shape[1]}]')
        zero = zero.contiguous()
    gi = None
    if g_idx is not None and g_idx.numel():
        gi = g_idx.to(torch.int32).contiguous()
        if gi.numel() != k:
            raise ValueError('weight_g_idx must have k entries')
        if int(gi.min()) < 0 or int(gi.max()) >= scale32.shape[1]:
            raise ValueError('weight_g_idx entries out of range')
    out = torch.empty((n, k), dtype=torch.float16, device=device)
    _call('wq_w4_decode', _ptr(packed), _ptr(scale32), _ptr(zero), _ptr(gi), n, k, scale32.shape[1], group_size,
          _ptr(out), _stream(device))
    return out


def w4_decode_rows(packed: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor | None, rows: torch.Tensor,
                   n: int, k: int, group_size: int = 128) -> torch.Tensor:
    """fp16 ``[len(rows), k]``: the explicit decode of the given rows only."""
    device = _require_gpu(packed, scale, zero, rows)
    if packed.dtype != torch.int32 or tuple(packed.shape) != (n, k // 8) or k % 8:
        raise ValueError(f'weight_packed must be int32 [{n}, {k // 8}], got {packed.dtype} {tuple(packed.shape)}')
    scale32 = scale.float().contiguous()
    if scale32.dim() != 2 or scale32.shape[0] != n:
        raise ValueError(f'weight_scale must be [{n}, groups], got {tuple(scale.shape)}')
    if zero is not None:
        if zero.dtype != torch.int32 or tuple(zero.shape) != ((n + 7) // 8, scale32.shape[1]):
            raise ValueError(f'weight_zero_point must be int32 [{(n + 7) // 8}, {scale32.shape[1]}]')
        zero = zero.contiguous()
    idx = rows.reshape(-1).to(device=device, dtype=torch.int64).contiguous()
    if idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= n):
        raise IndexError(f'row indices must lie in [0, {n})')
    out = torch.empty((idx.numel(), k), dtype=torch.float16, device=device)
    _call('wq_w4_decode_rows', _ptr(packed.contiguous()), _ptr(scale32), _ptr(zero), _ptr(idx), idx.numel(), n, k,
          scale32.shape[1], group_size, _ptr(out), _stream(device))
    return out


def w4a16_workspace_size(m: int, n: int, k: int, group_size: int) -> int:
    b = ctypes.c_size_t()
    _call('wq_w4a16_workspace_size', m, n, k, group_size, ctypes.byref(b))
    return b.value


def w8a16_workspace_size(m: int, n: int, k: int) -> int:
    b = ctypes.c_size_t()
    _call('wq_w8a16_workspace_size', m, n, k, ctypes.byref(b))
    return b.value


_workspaces: dict = {}


def shared_workspace(device: torch.device, nbytes: int, layout: tuple) -> torch.Tensor | None:
    """Zero-filled workspace for callers that do not bring their own.

    One buffer per (device, layout), never freed (a graph may have captured
    its address).  ``layout`` names the operation and the shape that fix where
    its counters and partials lie (e.g. ``('w4a16', n, k, group)``): the
    kernels return the counters to zero after every call but leave partials
    behind, so buffers are shared only between calls with the same layout,
    and only when those calls are ordered on one stream (concurrent streams
    need their own workspace: pass ``workspace=``).
    """
    if nbytes <= 0:
        return None
    key = (device.type, device.index) + tuple(layout)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _workspaces.setdefault(('retired',) + key, []).append(_workspaces.get(key))
        _workspaces[key] = buf
    return buf


def w4a16_linear(x: torch.Tensor, tiles: torch.Tensor, meta: torch.Tensor, n: int, group_size: int,
                 out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``y[m, n] = x[m, k] . dequant(W)^T`` on the repacked weight."""
    device = _require_gpu(x, tiles, meta, out)
    if x.dtype != torch.float16 or x.dim() != 2:
        raise TypeError(f'x must be a 2-D float16 tensor, got {x.dtype} {tuple(x.shape)}')
    m, k = x.shape
    x = _aligned(x.contiguous())
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, (m, n), 'out')
        if out.data_ptr() % 16:
            raise ValueError('out must be 16-byte aligned')
    if workspace is None and m <= 4:
        workspace = shared_workspace(device, w4a16_workspace_size(m, n, k, group_size), ('w4a16', m, n, k, group_size))
    elif workspace is None:
        # The small-batch kernel's and the deep-ring GEMM's split partials:
        # their counters sit in a fixed region at the front and are zero
        # after every call, so all such shapes share one buffer.
        nbytes = w4a16_workspace_size(m, n, k, group_size)
        if nbytes:
            workspace = shared_workspace(device, nbytes, ('w4a16-split',))
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _call('wq_w4a16_linear', _ptr(x), m, k, _ptr(tiles), _ptr(meta), n, group_size, _ptr(out), ws_ptr, ws_bytes,
          _stream(device))
    return out


EPI_SILU_MUL, EPI_RESIDUAL = 1, 2


def w4a16_epilogue_supported(m: int, n: int, k: int, group_size: int, mode: int) -> bool:
    """Whether ``w4a16_linear_epilogue`` runs this shape (the prefill GEMM
    grids that carry a fused epilogue; m > 64)."""
    return bool(load().wq_w4a16_epilogue_supported(m, n, k, group_size, mode))


def w4a16_linear_epilogue(x: torch.Tensor, tiles: torch.Tensor, meta: torch.Tensor, n: int, group_size: int,
                          mode: int, residual: torch.Tensor | None = None,
                          out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill W4A16 linear with the MLP's next elementwise op fused in, bit-
    identical to ``w4a16_linear`` followed by it.  ``EPI_SILU_MUL``: ``W`` is
    a fused ``[gate | up]`` of ``n`` rows and the result is
    ``silu(gate) * up`` as ``[m, n // 2]`` (``silu_mul``'s arithmetic).
    ``EPI_RESIDUAL``: ``residual + x . W^T`` as ``[m, n]`` (``out`` may be
    ``residual``).  Raises ``ValueError`` for shapes that
    ``w4a16_epilogue_supported`` rejects."""
    device = _require_gpu(x, tiles, meta, residual, out)
    if x.dtype != torch.float16 or x.dim() != 2:
        raise TypeError(f'x must be a 2-D float16 tensor, got {x.dtype} {tuple(x.shape)}')
    if mode not in (EPI_SILU_MUL, EPI_RESIDUAL):
        raise ValueError(f'mode must be EPI_SILU_MUL or EPI_RESIDUAL, got {mode}')
    m, k = x.shape
    n_out = n // 2 if mode == EPI_SILU_MUL else n
    x = _aligned(x.contiguous())
    res_ptr = None
    if mode == EPI_RESIDUAL:
        if residual is None:
            raise ValueError('EPI_RESIDUAL needs a residual tensor')
        _check(residual, torch.float16, (m, n), 'residual')
        if not residual.is_contiguous() or residual.data_ptr() % 8:
            raise ValueError('residual must be contiguous and 8-byte aligned')
        res_ptr = residual.data_ptr()
    if out is None:
        out = torch.empty((m, n_out), dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, (m, n_out), 'out')
        if not out.is_contiguous() or out.data_ptr() % 16:
            raise ValueError('out must be contiguous and 16-byte aligned')
    _call('wq_w4a16_linear_epilogue', _ptr(x), m, k, _ptr(tiles), _ptr(meta), n, group_size, mode, res_ptr,
          _ptr(out), _stream(device))
    return out


def w8a16_epilogue_supported(m: int, n: int, k: int, mode: int) -> bool:
    """Whether ``w8a16_linear_epilogue`` runs this shape (INT8 tiles, m > 64,
    the prefill GEMM grids that carry a fused epilogue)."""
    return bool(load().wq_w8a16_epilogue_supported(m, n, k, mode))


def w8a16_linear_epilogue(x: torch.Tensor, qweight: 'W8Tiles', scale: torch.Tensor, mode: int,
                          residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``w4a16_linear_epilogue`` for an INT8 weight as ``W8Tiles`` with fp16
    per-row ``scale``: bit-identical to ``w8a16_linear`` followed by
    ``silu_mul`` (``EPI_SILU_MUL``, fused ``[gate | up]`` weight) or the fp16
    residual add (``EPI_RESIDUAL``)."""
    n, k, q, tiled = _w8_weight(qweight)
    if not tiled:
        raise ValueError('the INT8 GEMM epilogue streams W8Tiles (wq_w8_repack)')
    device = _require_gpu(x, q, scale, residual, out)
    if x.dtype != torch.float16 or x.dim() != 2 or x.shape[1] != k:
        raise TypeError(f'x must be a 2-D float16 tensor with {k} features, got {x.dtype} {tuple(x.shape)}')
    if scale.dtype != torch.float16 or scale.numel() != n:
        raise ValueError(f'scale must be float16 with {n} entries')
    if mode not in (EPI_SILU_MUL, EPI_RESIDUAL):
        raise ValueError(f'mode must be EPI_SILU_MUL or EPI_RESIDUAL, got {mode}')
    m = x.shape[0]
    n_out = n // 2 if mode == EPI_SILU_MUL else n
    x = _aligned(x.contiguous())
    res_ptr = None
    if mode == EPI_RESIDUAL:
        if residual is None:
            raise ValueError('EPI_RESIDUAL needs a residual tensor')
        _check(residual, torch.float16, (m, n), 'residual')
        if residual.data_ptr() % 8:
            raise ValueError('residual must be 8-byte aligned')
        res_ptr = residual.data_ptr()
    if out is None:
        out = torch.empty((m, n_out), dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, (m, n_out), 'out')
        if out.data_ptr() % 16:
            raise ValueError('out must be 16-byte aligned')
    _call('wq_w8a16_linear_epilogue', _ptr(x), m, k, _ptr(q), _ptr(scale.contiguous()), n, mode, res_ptr,
          _ptr(out), _stream(device))
    return out


X_PLAIN, X_RMSNORM, X_SILU_MUL = 0, 1, 2


def _decode_fused_args(x, n, x_mode, norm_weight, sumsq_in, residual, sumsq_out, out, device):
    """Checks shared by the fused decode linears; returns (k, out)."""
    if x.dtype != torch.float16 or not x.is_contiguous():
        raise TypeError('x must be a contiguous float16 tensor')
    k = x.numel() // 2 if x_mode == X_SILU_MUL else x.numel()
    if norm_weight is not None:
        _check(norm_weight, torch.float16, (k,), 'norm_weight')
    if sumsq_in is not None and (sumsq_in.dtype != torch.float32 or not sumsq_in.is_contiguous()):
        raise TypeError('sumsq_in must be contiguous float32')
    if sumsq_out is not None:
        _check(sumsq_out, torch.float32, ((n + 15) // 16,), 'sumsq_out')
    if residual is not None:
        if residual.dtype != torch.float16 or residual.numel() != n or not residual.is_contiguous():
            raise ValueError(f'residual must be contiguous float16 with {n} elements')
    if out is None:
        out = torch.empty((1, n), dtype=torch.float16, device=device)
    elif out.dtype != torch.float16 or out.numel() != n or not out.is_contiguous():
        raise ValueError(f'out must be contiguous float16 with {n} elements')
    return k, out


def _ws_args(workspace):
    if workspace is None:
        return None, 0
    return workspace.data_ptr(), workspace.numel() * workspace.element_size()


def w4a16_decode_fused(x: torch.Tensor, tiles: torch.Tensor, meta: torch.Tensor, n: int, group_size: int, *,
                       x_mode: int = X_PLAIN, norm_weight: torch.Tensor | None = None,
                       sumsq_in: torch.Tensor | None = None, eps: float = 1e-6,
                       residual: torch.Tensor | None = None, sumsq_out: torch.Tensor | None = None,
                       out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One decode-token W4A16 linear with the fused prologue/epilogue of
    ``wq_w4a16_decode_fused`` (x_mode ``X_PLAIN`` / ``X_RMSNORM`` /
    ``X_SILU_MUL``; ``residual`` added in fp16; per-tile ``sumsq_out``)."""
    device = _require_gpu(x, tiles, meta, norm_weight, sumsq_in, residual, sumsq_out, out, workspace)
    k, out = _decode_fused_args(x, n, x_mode, norm_weight, sumsq_in, residual, sumsq_out, out, device)
    if workspace is None:
        workspace = shared_workspace(device, w4a16_workspace_size(1, n, k, group_size), ('w4a16', 1, n, k, group_size))
    ws_ptr, ws_bytes = _ws_args(workspace)
    _call('wq_w4a16_decode_fused', _ptr(x), k, _ptr(tiles), _ptr(meta), n, group_size, x_mode, _ptr(norm_weight),
          _ptr(sumsq_in), 0 if sumsq_in is None else sumsq_in.numel(), float(eps), _ptr(residual), _ptr(sumsq_out),
          _ptr(out), ws_ptr, ws_bytes, _stream(device))
    return out


def w8a16_decode_fused(x: torch.Tensor, qweight, scale: torch.Tensor, *,
                       x_mode: int = X_PLAIN, norm_weight: torch.Tensor | None = None,
                       sumsq_in: torch.Tensor | None = None, eps: float = 1e-6,
                       residual: torch.Tensor | None = None, sumsq_out: torch.Tensor | None = None,
                       out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """The INT8 (row-major [n, k] weight or ``W8Tiles``, fp16 row scale)
    counterpart of ``w4a16_decode_fused`` (``wq_w8a16_decode_fused`` /
    ``wq_w8a16_decode_fused_tiled``)."""
    if not isinstance(qweight, W8Tiles) and (qweight.dtype != torch.int8 or qweight.dim() != 2 or
                                             not qweight.is_contiguous()):
        raise TypeError('qweight must be a contiguous 2-D INT8 tensor or W8Tiles')
    n, kq, q, tiled = _w8_weight(qweight)
    device = _require_gpu(x, q, scale, norm_weight, sumsq_in, residual, sumsq_out, out, workspace)
    if scale.dtype != torch.float16 or scale.numel() != n or not scale.is_contiguous():
        raise ValueError(f'scale must be contiguous float16 with {n} entries')
    k, out = _decode_fused_args(x, n, x_mode, norm_weight, sumsq_in, residual, sumsq_out, out, device)
    if k != kq:
        raise ValueError(f'input has {k} features, expected {kq}')
    if workspace is None:
        workspace = shared_workspace(device, w8a16_workspace_size(1, n, k), ('w8a16', 1, n, k))
    ws_ptr, ws_bytes = _ws_args(workspace)
    _call('wq_w8a16_decode_fused_tiled' if tiled else 'wq_w8a16_decode_fused', _ptr(x), k, _ptr(q), _ptr(scale), n,
          x_mode, _ptr(norm_weight),
          _ptr(sumsq_in), 0 if sumsq_in is None else sumsq_in.numel(), float(eps), _ptr(residual), _ptr(sumsq_out),
          _ptr(out), ws_ptr, ws_bytes, _stream(device))
    return out


# ----------------------------------------------------------------------------- W8

class W8Tiles(NamedTuple):
    """An INT8 weight [n, k] in the tile layout the INT8 kernels stream
    (``wq_w8_repack``): 2 KiB per (16-row tile, 128-k block), each half one
    contiguous 1 KiB wave load; rows past n are zero.  Same values as the
    row-major weight, so every linear gives the same bits."""
    tiles: torch.Tensor   # uint8 [ceil(n/16) * (k/128) * 2048]
    n: int
    k: int

    @property
    def shape(self) -> tuple[int, int]:
        return self.n, self.k

    @property
    def device(self) -> torch.device:
        return self.tiles.device


def w8_tiles_size(n: int, k: int) -> int:
    b = ctypes.c_size_t()
    _call('wq_w8_tiles_size', n, k, ctypes.byref(b))
    return b.value


def w8_repack(qweight: torch.Tensor, out: torch.Tensor | None = None) -> W8Tiles:
    """Row-major INT8 [n, k] (k % 128 == 0) -> ``W8Tiles``."""
    device = _require_gpu(qweight, out)
    if qweight.dtype != torch.int8 or qweight.dim() != 2:
        raise TypeError(f'expected a 2-D INT8 weight, got {qweight.dtype} {tuple(qweight.shape)}')
    n, k = qweight.shape
    size = w8_tiles_size(n, k)
    if out is None:
        out = torch.empty(size, dtype=torch.uint8, device=device)
    else:
        _check(out, torch.uint8, (size,), 'out')
    _call('wq_w8_repack', _ptr(_aligned(qweight.contiguous())), n, k, _ptr(out), _stream(device))
    return W8Tiles(out, n, k)


def w8_unpack(w: W8Tiles) -> torch.Tensor:
    """``W8Tiles`` -> row-major INT8 [n, k] (the inverse of ``w8_repack``)."""
    device = _require_gpu(w.tiles)
    _check(w.tiles, torch.uint8, (w8_tiles_size(w.n, w.k),), 'tiles')
    q = torch.empty((w.n, w.k), dtype=torch.int8, device=device)
    _call('wq_w8_unpack', _ptr(w.tiles), w.n, w.k, _ptr(q), _stream(device))
    return q


def _w8_weight(qweight) -> tuple[int, int, torch.Tensor, bool]:
    """(n, k, device buffer, tiled) of a row-major INT8 tensor or ``W8Tiles``."""
    if isinstance(qweight, W8Tiles):
        _check(qweight.tiles, torch.uint8, (w8_tiles_size(qweight.n, qweight.k),), 'tiles')
        return qweight.n, qweight.k, qweight.tiles, True
    if qweight.dtype != torch.int8 or qweight.dim() != 2:
        raise TypeError(f'qweight must be a 2-D INT8 tensor or W8Tiles, got {qweight.dtype}')
    return qweight.shape[0], qweight.shape[1], _aligned(qweight.contiguous()), False


def w8_decode(qweight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    device = _require_gpu(qweight, scale)
    if qweight.dtype != torch.int8 or qweight.dim() != 2:
        raise TypeError(f'expected a 2-D INT8 weight, got {qweight.dtype} {tuple(qweight.shape)}')
    n, k = qweight.shape
    s = scale.float().reshape(-1).contiguous()
    if s.numel() != n:
        raise ValueError(f'scale must have {n} entries, got {s.numel()}')
    out = torch.empty((n, k), dtype=torch.float16, device=device)
    _call('wq_w8_decode', _ptr(qweight.contiguous()), _ptr(s), n, k, _ptr(out), _stream(device))
    return out


def w8a16_linear(x: torch.Tensor, qweight, scale: torch.Tensor, bias: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``y = x . (q * scale)^T (+ bias)`` straight from the INT8 weight:
    row-major [n, k] (``wq_w8a16_linear``) or ``W8Tiles`` (``wq_w8a16_linear_tiled``)."""
    n, k, q, tiled = _w8_weight(qweight)
    device = _require_gpu(x, q, scale, bias, out)
    if x.dtype != torch.float16 or x.dim() != 2:
        raise TypeError(f'x must be a 2-D float16 tensor, got {x.dtype} {tuple(x.shape)}')
    if x.shape[1] != k:
        raise ValueError(f'input has {x.shape[1]} features, expected {k}')
    if scale.dtype != torch.float16 or scale.numel() != n:
        raise ValueError(f'scale must be float16 with {n} entries')
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != n):
        raise ValueError('bias must be FP16 with one entry per output feature')
    m = x.shape[0]
    x = _aligned(x.contiguous())
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, (m, n), 'out')
    if workspace is None and m <= 4:
        workspace = shared_workspace(device, w8a16_workspace_size(m, n, k), ('w8a16', m, n, k))
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    _call('wq_w8a16_linear_tiled' if tiled else 'wq_w8a16_linear', _ptr(x), m, k, _ptr(q), _ptr(scale.contiguous()), n,
          _ptr(None if bias is None else bias.contiguous()), _ptr(out), ws_ptr, ws_bytes, _stream(device))
    return out


def w8a8_quantize(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Dynamic per-token symmetric INT8: ``(qx int8 [m, k], x_scale fp32 [m])``
    with ``x_scale = max(absmax, 1e-12) / 127`` (``wq_w8a8_quantize``)."""
    device = _require_gpu(x)
    if x.dtype != torch.float16 or x.dim() != 2:
        raise TypeError(f'x must be a 2-D float16 tensor, got {x.dtype} {tuple(x.shape)}')
    m, k = x.shape
    x = _aligned(x.contiguous())
    qx = torch.empty((m, k), dtype=torch.int8, device=device)
    scale = torch.empty(m, dtype=torch.float32, device=device)
    _call('wq_w8a8_quantize', _ptr(x), m, k, _ptr(qx), _ptr(scale), _stream(device))
    return qx, scale


def w8a8_linear(qx: torch.Tensor, x_scale: torch.Tensor, qweight, w_scale: torch.Tensor,
                bias: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``y = fp16(float(qx . qweight^T) * x_scale[m] * w_scale[n] (+ bias))``,
    int32 accumulation on the int8 matrix cores; ``qweight`` row-major INT8
    (``wq_w8a8_linear``) or ``W8Tiles`` (``wq_w8a8_linear_tiled``)."""
    n, kw, q, tiled = _w8_weight(qweight)
    device = _require_gpu(qx, x_scale, q, w_scale, bias, out)
    if qx.dtype != torch.int8 or qx.dim() != 2:
        raise TypeError('qx must be a 2-D INT8 tensor')
    m, k = qx.shape
    if kw != k:
        raise ValueError(f'input has {k} features, expected {kw}')
    _check(x_scale, torch.float32, (m,), 'x_scale')
    if w_scale.dtype != torch.float32 or w_scale.numel() != n:
        raise ValueError(f'w_scale must be float32 with {n} entries')
    if bias is not None and (bias.dtype != torch.float16 or bias.numel() != n):
        raise ValueError('bias must be FP16 with one entry per output feature')
    qx = _aligned(qx.contiguous())
    if out is None:
        out = torch.empty((m, n), dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, (m, n), 'out')
    _call('wq_w8a8_linear_tiled' if tiled else 'wq_w8a8_linear', _ptr(qx), _ptr(x_scale.contiguous()), m, k, _ptr(q), _ptr(w_scale.contiguous()), n,
          _ptr(None if bias is None else bias.contiguous()), _ptr(out), _stream(device))
    return out


def w8_quantize(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric INT8 quantization on the GPU -> (qweight int8, scale fp16)."""
    device = _require_gpu(weight)
    n, k = weight.shape
    w32 = weight.to(torch.float32).contiguous()
    q = torch.empty((n, k), dtype=torch.int8, device=device)
    s = torch.empty(n, dtype=torch.float16, device=device)
    flags = torch.zeros(1, dtype=torch.int32, device=device)
    _call('wq_w8_quantize', _ptr(w32), n, k, _ptr(q), _ptr(s), _ptr(flags), _stream(device))
    f = int(flags.item())
    if f & 1:
        raise ValueError('linear weight contains NaN or infinity')
    if f & 2:
        raise OverflowError('row scale is not representable in scale_dtype')
    return q, s


# ----------------------------------------------------------------------------- decode-step operators

def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, delta: torch.Tensor | None = None,
                out: torch.Tensor | None = None, out_sum: torch.Tensor | None = None) -> torch.Tensor:
    """``rms_norm(x + delta)`` over the last dimension; ``out_sum`` (may be
    ``x`` itself) receives ``x + delta``."""
    device = _require_gpu(x, weight, delta, out, out_sum)
    n = x.shape[-1]
    rows = x.numel() // n if n else 0
    for t, name in ((x, 'x'), (delta, 'delta'), (out_sum, 'out_sum')):
        if t is not None:
            _check(t, torch.float16, tuple(x.shape), name)
    _check(weight, torch.float16, (n,), 'weight')
    if out is None:
        out = torch.empty_like(x)
    else:
        _check(out, torch.float16, tuple(x.shape), 'out')
    _call('wq_add_rmsnorm', _ptr(x), _ptr(delta), _ptr(weight), rows, n, float(eps), _ptr(out), _ptr(out_sum),
          _stream(device))
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate) * up`` of a fused ``[..., 2n]`` = ``[gate | up]`` tensor -> ``[..., n]``."""
    device = _require_gpu(gate_up, out)
    if gate_up.dtype != torch.float16 or not gate_up.is_contiguous() or gate_up.shape[-1] % 2:
        raise ValueError('gate_up must be a contiguous float16 tensor with an even last dimension')
    n = gate_up.shape[-1] // 2
    rows = gate_up.numel() // (2 * n) if n else 0
    shape = tuple(gate_up.shape[:-1]) + (n,)
    if out is None:
        out = torch.empty(shape, dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, shape, 'out')
    _call('wq_silu_mul', _ptr(gate_up), rows, n, _ptr(out), _stream(device))
    return out


def decode_attention_workspace_size(q_heads: int, kv_heads: int, head_dim: int, max_seq: int) -> int:
    b = ctypes.c_size_t()
    _call('wq_decode_attention_workspace_size', q_heads, kv_heads, head_dim, max_seq, ctypes.byref(b))
    return b.value


def decode_attention(qkv: torch.Tensor, q_heads: int, kv_heads: int, q_norm: torch.Tensor | None,
                     k_norm: torch.Tensor | None, eps: float, cos_table: torch.Tensor, sin_table: torch.Tensor,
                     position: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor, scale: float,
                     out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One decode token of GQA attention (batch 1); appends row ``position``
    of the caches (``[kv_heads, max_seq, head_dim]`` fp16)."""
    device = _require_gpu(qkv, q_norm, k_norm, cos_table, sin_table, position, key_cache, value_cache, out, workspace)
    if key_cache.dim() != 3 or key_cache.shape != value_cache.shape or key_cache.shape[0] != kv_heads:
        raise ValueError(f'caches must be [kv_heads={kv_heads}, max_seq, head_dim], got {tuple(key_cache.shape)}')
    _, max_seq, head_dim = key_cache.shape
    for t, name in ((key_cache, 'key_cache'), (value_cache, 'value_cache')):
        _check(t, torch.float16, (kv_heads, max_seq, head_dim), name)
    _check(qkv, torch.float16, ((q_heads + 2 * kv_heads) * head_dim,), 'qkv')
    for t, name in ((q_norm, 'q_norm'), (k_norm, 'k_norm')):
        if t is not None:
            _check(t, torch.float16, (head_dim,), name)
    if cos_table.dtype != torch.float16 or sin_table.dtype != torch.float16 or cos_table.shape != sin_table.shape \
            or cos_table.dim() != 2 or cos_table.shape[1] != head_dim or cos_table.shape[0] < max_seq \
            or not cos_table.is_contiguous() or not sin_table.is_contiguous():
        raise ValueError(f'cos/sin tables must be contiguous float16 [>= {max_seq}, {head_dim}]')
    _check(position, torch.int32, (1,), 'position')
    if out is None:
        out = torch.empty(q_heads * head_dim, dtype=torch.float16, device=device)
    else:
        _check(out, torch.float16, (q_heads * head_dim,), 'out')
    need = decode_attention_workspace_size(q_heads, kv_heads, head_dim, max_seq)
    if workspace is None and need:
        workspace = shared_workspace(device, need, ('attention', q_heads, kv_heads, max_seq))
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(),
                                                             workspace.numel() * workspace.element_size())
    _call('wq_decode_attention', _ptr(qkv), q_heads, kv_heads, head_dim, _ptr(q_norm), _ptr(k_norm), float(eps),
          _ptr(cos_table), _ptr(sin_table), _ptr(position), _ptr(key_cache), _ptr(value_cache), max_seq,
          float(scale), _ptr(out), ws_ptr, ws_bytes, _stream(device))
    return out


def prefill_attention(query: torch.Tensor, q_heads: int, kv_heads: int, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, start: int, scale: float,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA attention of ``tokens`` queries at positions ``start ..``
    (batch 1) over cache rows ``0 .. start + tokens - 1``, which must already
    hold these tokens' keys and values: ``query`` and the result are
    token-major ``[tokens, q_heads, head_dim]`` fp16 (``wq_prefill_qk_rope``'s
    q layout), the caches ``[kv_heads, max_seq, head_dim]``."""
    device = _require_gpu(query, key_cache, value_cache, out)
    if key_cache.dim() != 3 or key_cache.shape != value_cache.shape or key_cache.shape[0] != kv_heads:
        raise ValueError(f'caches must be [kv_heads={kv_heads}, max_seq, head_dim], got {tuple(key_cache.shape)}')
    _, max_seq, head_dim = key_cache.shape
    for t, name in ((key_cache, 'key_cache'), (value_cache, 'value_cache')):
        _check(t, torch.float16, (kv_heads, max_seq, head_dim), name)
    if query.dim() != 3 or query.shape[1:] != (q_heads, head_dim):
        raise ValueError(f'query must be [tokens, {q_heads}, {head_dim}], got {tuple(query.shape)}')
    _check(query, torch.float16, tuple(query.shape), 'query')
    if out is None:
        out = torch.empty_like(query)
    else:
        _check(out, torch.float16, tuple(query.shape), 'out')
    _call('wq_prefill_attention', _ptr(query), query.shape[0], q_heads, kv_heads, head_dim, _ptr(key_cache),
          _ptr(value_cache), max_seq, start, float(scale), _ptr(out), _stream(device))
    return out


def prefill_qk_rope(qkv: torch.Tensor, q_heads: int, kv_heads: int, q_norm: torch.Tensor | None,
                    k_norm: torch.Tensor | None, eps: float, cos_rows: torch.Tensor, sin_rows: torch.Tensor,
                    start: int, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    q_out: torch.Tensor | None = None) -> torch.Tensor:
    """q/k RMSNorm + RoPE of ``tokens`` rows of a fused QKV projection (batch 1)
    at positions ``start ..``; k and v land in rows ``start ..`` of the caches
    (``[kv_heads, max_seq, head_dim]`` fp16); returns q as
    ``[tokens, q_heads, head_dim]`` (token-major)."""
    device = _require_gpu(qkv, q_norm, k_norm, cos_rows, sin_rows, key_cache, value_cache, q_out)
    if key_cache.dim() != 3 or key_cache.shape != value_cache.shape or key_cache.shape[0] != kv_heads:
        raise ValueError(f'caches must be [kv_heads={kv_heads}, max_seq, head_dim], got {tuple(key_cache.shape)}')
    _, max_seq, head_dim = key_cache.shape
    for t, name in ((key_cache, 'key_cache'), (value_cache, 'value_cache')):
        _check(t, torch.float16, (kv_heads, max_seq, head_dim), name)
    if qkv.dim() != 2:
        raise ValueError(f'qkv must be [tokens, (q_heads + 2 kv_heads) * head_dim], got {tuple(qkv.shape)}')
    tokens = qkv.shape[0]
    _check(qkv, torch.float16, (tokens, (q_heads + 2 * kv_heads) * head_dim), 'qkv')
    for t, name in ((cos_rows, 'cos_rows'), (sin_rows, 'sin_rows')):
        _check(t, torch.float16, (tokens, head_dim), name)
    for t, name in ((q_norm, 'q_norm'), (k_norm, 'k_norm')):
        if t is not None:
            _check(t, torch.float16, (head_dim,), name)
    if q_out is None:
        q_out = torch.empty(tokens, q_heads, head_dim, dtype=torch.float16, device=device)
    else:
        _check(q_out, torch.float16, (tokens, q_heads, head_dim), 'q_out')
    _call('wq_prefill_qk_rope', _ptr(qkv), tokens, q_heads, kv_heads, head_dim, _ptr(q_norm), _ptr(k_norm),
          float(eps), _ptr(cos_rows), _ptr(sin_rows), int(start), _ptr(key_cache), _ptr(value_cache), max_seq,
          _ptr(q_out), _stream(device))
    return q_out


def lm_head_workspace_size(k: int, vocab: int) -> int:
    b = ctypes.c_size_t()
    _call('wq_lm_head_workspace_size', k, vocab, ctypes.byref(b))
    return b.value


def lm_head(x: torch.Tensor, weight: torch.Tensor, *, logits: torch.Tensor | None = None,
            token: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
            want_logits: bool = True, want_token: bool = True, norm_weight: torch.Tensor | None = None,
            sumsq_in: torch.Tensor | None = None, eps: float = 1e-6) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """fp16 LM head of one token (``x`` [k], ``weight`` [vocab, k]) and its
    greedy token (``torch.argmax`` over the fp16 logits) in one pass:
    ``wq_lm_head``.  Returns ``(logits [vocab] fp16, token [1] int64)``.
    With ``norm_weight`` and ``sumsq_in`` (fp32 sums of squares of ``x`` over
    16-element tiles) ``x`` is the final residual stream and the kernel forms
    the final RMSNorm itself (``wq_lm_head_rmsnorm``)."""
    device = _require_gpu(x, weight, logits, token, workspace, norm_weight, sumsq_in)
    if (norm_weight is None) != (sumsq_in is None):
        raise ValueError('norm_weight and sumsq_in go together')
    if weight.dim() != 2:
        raise ValueError(f'weight must be [vocab, k], got {tuple(weight.shape)}')
    vocab, k = weight.shape
    _check(weight, torch.float16, (vocab, k), 'weight')
    if x.dtype != torch.float16 or not x.is_contiguous() or x.numel() != k:
        raise ValueError(f'x must be contiguous float16 with {k} elements')
    if logits is None and want_logits:
        logits = torch.empty(vocab, dtype=torch.float16, device=device)
    if logits is not None:
        _check(logits.view(-1), torch.float16, (vocab,), 'logits')
    if token is None and want_token:
        token = torch.empty(1, dtype=torch.int64, device=device)
    if token is not None and (token.dtype != torch.int64 or token.numel() != 1 or not token.is_contiguous()):
        raise ValueError('token must be one contiguous int64')
    if workspace is None and token is not None:
        workspace = shared_workspace(device, lm_head_workspace_size(k, vocab), ('lm_head', k, vocab))
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(),
                                                             workspace.numel() * workspace.element_size())
    if norm_weight is None:
        _call('wq_lm_head', _ptr(_aligned(x)), k, _ptr(weight), vocab, _ptr(logits), _ptr(token), ws_ptr, ws_bytes,
              _stream(device))
    else:
        _check(norm_weight.view(-1), torch.float16, (k,), 'norm_weight')
        if sumsq_in.dtype != torch.float32 or not sumsq_in.is_contiguous():
            raise ValueError('sumsq_in must be a contiguous float32 tensor')
        _call('wq_lm_head_rmsnorm', _ptr(_aligned(x)), k, _ptr(_aligned(norm_weight)), _ptr(sumsq_in),
              sumsq_in.numel(), float(eps), _ptr(weight), vocab, _ptr(logits), _ptr(token), ws_ptr, ws_bytes,
              _stream(device))
    return logits, token


def argmax_f16_workspace_size(n: int) -> int:
    b = ctypes.c_size_t()
    _call('wq_argmax_f16_workspace_size', n, ctypes.byref(b))
    return b.value


def argmax_f16(x: torch.Tensor, *, out: torch.Tensor | None = None,
               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``torch.argmax`` of a 1-D contiguous fp16 tensor (first index of the
    largest value, NaN the largest) as one int64 on the device:
    ``wq_argmax_f16``."""
    device = _require_gpu(x, out, workspace)
    if x.dtype != torch.float16 or not x.is_contiguous() or x.numel() < 1:
        raise ValueError('x must be a non-empty contiguous float16 tensor')
    n = x.numel()
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=device)
    elif out.dtype != torch.int64 or out.numel() != 1 or not out.is_contiguous():
        raise ValueError('out must be one contiguous int64')
    if workspace is None:
        workspace = shared_workspace(device, argmax_f16_workspace_size(n), ('argmax_f16', n))
    _call('wq_argmax_f16', _ptr(_aligned(x)), n, _ptr(out), workspace.data_ptr(),
          workspace.numel() * workspace.element_size(), _stream(device))
    return out


# ----------------------------------------------------------------------------- embedding

class HostTable(NamedTuple):
    """An fp16 ``[rows, cols]`` table kept in pinned host memory, with the
    address kernels read it at (``wq_host_device_pointer``)."""
    tensor: torch.Tensor     # pinned CPU fp16, contiguous
    device_ptr: int
    device: torch.device


def host_table(table: torch.Tensor, device: torch.device | str) -> HostTable:
    """``table`` (CPU fp16 2-D) in pinned host memory, mapped for ``device``'s
    kernels; a pinned contiguous table is used as it is, anything else is
    copied into a new pinned buffer."""
    if table.device.type != 'cpu' or table.dtype != torch.float16 or table.dim() != 2:
        raise ValueError(f'expected a 2-D float16 CPU table, got {table.dtype} {tuple(table.shape)} on {table.device}')
    device = torch.device(device)
    table = table.contiguous()
    if not table.is_pinned():
        table = table.pin_memory()
    ptr = ctypes.c_void_p()
    with torch.cuda.device(device):
        _call('wq_host_device_pointer', table.data_ptr(), ctypes.byref(ptr))
    return HostTable(table, int(ptr.value), device)


def embed_rows(table: 'HostTable | torch.Tensor', tokens: torch.Tensor, out: torch.Tensor | None = None,
               sumsq_out: torch.Tensor | None = None) -> torch.Tensor:
    """``out[r] = table[tokens[r]]`` (``wq_embed_rows``): the embedding rows of
    device int64 token ids from a ``HostTable`` (read over the host link) or a
    device fp16 table; an out-of-range id gives a NaN row.  ``sumsq_out``
    (fp32, ``rows * hidden / 16``) receives each row's sums of squares over
    16-element tiles, the input of the fused linears' RMSNorm prologue."""
    if isinstance(table, HostTable):
        vocab, hidden = table.tensor.shape
        tptr, tdev = table.device_ptr, table.device
    else:
        if table.dtype != torch.float16 or table.dim() != 2 or not table.is_contiguous():
            raise ValueError('table must be a contiguous 2-D float16 tensor')
        vocab, hidden = table.shape
        tptr, tdev = table.data_ptr(), _require_gpu(table)
    device = _require_gpu(tokens, out)
    if device != tdev:
        raise ValueError(f'table is mapped for {tdev}, tokens are on {device}')
    if tokens.dtype != torch.int64 or not tokens.is_contiguous():
        raise TypeError('tokens must be a contiguous int64 tensor')
    rows = tokens.numel()
    if out is None:
        out = torch.empty((rows, hidden), dtype=torch.float16, device=device)
    elif out.dtype != torch.float16 or out.numel() != rows * hidden or not out.is_contiguous():
        raise ValueError(f'out must be a contiguous float16 tensor of {rows * hidden} elements')
    if sumsq_out is not None:
        if (sumsq_out.device != device or sumsq_out.dtype != torch.float32 or not sumsq_out.is_contiguous()
                or hidden % 16 or sumsq_out.numel() != rows * (hidden // 16)):
            raise ValueError(f'sumsq_out must be a contiguous float32 tensor of {rows * (hidden // 16)} elements '
                             'on the tokens\' device (hidden % 16 == 0)')
    _call('wq_embed_rows', tptr, vocab, hidden, _ptr(tokens), rows, _ptr(out), _ptr(sumsq_out), _stream(device))
    return out
