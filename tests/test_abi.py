"""The C-ABI library loads, exports every symbol the header declares, and
rejects malformed requests before any GPU work (CPU-only checks)."""
import ctypes
import re
from pathlib import Path

import pytest

from ondeviceinfer_amd import _native

HEADERS = sorted((Path(__file__).resolve().parents[1] / 'include').glob('*.h'))


def declared_functions() -> list[str]:
    names = []
    for header in HEADERS:
        text = re.sub(r'/\*.*?\*/', '', header.read_text(), flags=re.S)
        names += re.findall(r'^\s*(?:const\s+char\s*\*|int)\s+(wq_\w+)\s*\(', text, flags=re.M)
    return names


def test_header_declares_the_bound_entry_points():
    names = declared_functions()
    assert len(names) == len(set(names)) >= 12
    assert set(names) == set(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.wq_abi_version() == _native.ABI_VERSION


def _status(fn, *args):
    return getattr(_native.load(), fn)(*args)


def test_shape_validation_happens_on_the_host():
    tb, mb = ctypes.c_size_t(), ctypes.c_size_t()
    assert _status('wq_w4_repack_size', 5120, 5120, 128, ctypes.byref(tb), ctypes.byref(mb)) == _native.WQ_OK
    assert tb.value == 5120 * 5120 // 2 and mb.value == 320 * 40 * 40
    assert _status('wq_w4_repack_size', 12, 5120, 128, ctypes.byref(tb), ctypes.byref(mb)) == _native.WQ_ERR_UNSUPPORTED
    assert b'n % 8' in _native.load().wq_last_error()
    assert _status('wq_w4_repack_size', 16, 5120, 64, ctypes.byref(tb), ctypes.byref(mb)) == _native.WQ_ERR_UNSUPPORTED
    assert _status('wq_w4_repack_size', 0, 5120, 128, ctypes.byref(tb), ctypes.byref(mb)) == \
        _native.WQ_ERR_INVALID_ARGUMENT
    # k not a multiple of the group -> rejected before any launch
    assert _status('wq_w4a16_linear', 1, 1, 200, 1, 1, 16, 128, 1, None, 0, None) == _native.WQ_ERR_UNSUPPORTED
    # null pointers -> rejected
    assert _status('wq_w4a16_linear', None, 1, 256, None, None, 16, 128, None, None, 0, None) == \
        _native.WQ_ERR_INVALID_ARGUMENT
    assert _status('wq_w8_quantize', None, 0, 4, None, None, None, None) == _native.WQ_ERR_INVALID_ARGUMENT


def test_status_maps_to_python_exceptions():
    with pytest.raises(ValueError, match='n % 8'):
        _native.w4_repack_size(12, 256, 128)
    assert _native.w4_repack_size(16, 256, 128) == (16 * 128, 2 * 40)
    assert _native.w4a16_workspace_size(1, 5120, 5120, 128) == 0


def test_prefill_k_split_workspace_follows_the_chain_length():
    """The deep-ring GEMM's k split, as the host sizes its workspace (no GPU
    needed): a 16 KiB counter region plus one fp32 partial tile set of
    4 waves x NT x MT KiB per (workgroup, split), NT = 1 and MT = 2 (32-row
    tiles) at these M.  Short chains (40 blocks) split only grids of at
    most 384 workgroups, long ones (64 blocks or more) up to 640."""
    counters, per_split_tile = 16384, 4 * 1 * 2 * 1024
    # down 17408->5120 (136 blocks): 80 n slices x 4 / 8 row blocks
    assert _native.w4a16_workspace_size(128, 5120, 17408, 128) == counters + 320 * 4 * per_split_tile
    assert _native.w4a16_workspace_size(256, 5120, 17408, 128) == counters + 640 * 2 * per_split_tile
    # q/o 5120->5120 (40 blocks) at M = 256: 640 workgroups keep the whole k range
    assert _native.w4a16_workspace_size(256, 5120, 5120, 128) == 0
    # fused QKV 5120->7168 (40 blocks): 112 n slices x 3 row blocks at M = 65 split
    # in four; 4 row blocks at M = 128 (448 workgroups) keep the whole k range
    assert _native.w4a16_workspace_size(65, 7168, 5120, 128) == counters + 336 * 4 * per_split_tile
    assert _native.w4a16_workspace_size(128, 7168, 5120, 128) == 0
    assert _native.w4a16_workspace_size(256, 5120, 5120, 128) == 0
    # 65 blocks, 16 n slices x 22 row blocks = 352 workgroups: four splits
    assert _native.w4a16_workspace_size(700, 1000, 8320, 128) == counters + 352 * 4 * per_split_tile
    # M = 257: 64-row tiles (400 workgroups), no deep ring, no split
    assert _native.w4a16_workspace_size(257, 5120, 17408, 128) == 0
