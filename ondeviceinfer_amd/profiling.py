"""Opt-in ROCTX ranges (``ONDEVICEINFER_NVTX=1``), mirroring ``ondeviceinfer/profiling.py:17-49``.

On PyTorch-ROCm ``torch.cuda.nvtx`` emits ROCTX markers that rocprofv3's
marker trace records.
"""
from __future__ import annotations

import contextlib
import os

import torch

_ENABLED = os.environ.get('ONDEVICEINFER_NVTX', '0') == '1'


@contextlib.contextmanager
def nvtx_range(name: str):
    if not _ENABLED or not torch.cuda.is_available():
        yield
        return
    torch.cuda.nvtx.range_push(name)
    try:
        yield
    finally:
        torch.cuda.nvtx.range_pop()
