"""Build ``libondeviceinfer_wq.so`` (gfx950) in-tree with hipcc.

Usage: ``python -m ondeviceinfer_amd.build`` (also called by
``__graft_entry__.build()``).  Each ``csrc/*.hip`` compiles to an object under
``ondeviceinfer_amd/_build/`` in parallel, then one shared library is linked
next to this file, where ``ondeviceinfer_amd._native`` loads it.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
BUILD = PKG / '_build'
LIB_NAME = 'libondeviceinfer_wq.so'
LIB_PATH = PKG / LIB_NAME
ARCH = 'gfx950'

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
HIP_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-fPIC', '-std=c++17', '-mcode-object-version=5',
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-function', f'-I{PKG.parent / "include"}',
]


def hipcc() -> str:
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError('hipcc not found; the HIP toolchain is required to build the library')


def _compile(src: Path, extra: list[str]) -> tuple[Path, str]:
    obj = BUILD / (src.stem + '.o')
    cmd = [hipcc(), *HIP_FLAGS, *extra, '-c', str(src), '-o', str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    log = '\n'.join(line for line in (proc.stdout + proc.stderr).splitlines()
                    if 'packed-fp32-ops' not in line)
    if proc.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{" ".join(cmd)}\n{log}')
    return obj, log


def build(verbose: bool = False, extra: list[str] | None = None) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    if not sources:
        raise RuntimeError(f'no HIP sources under {CSRC}')
    jobs = min(len(sources), int(os.environ.get('MAX_JOBS', '8')))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda s: _compile(s, extra or []), sources))
    for obj, log in results:
        if verbose and log.strip():
            print(f'[{obj.name}]\n{log}', file=sys.stderr)
    tmp = LIB_PATH.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', '-o', str(tmp), *[str(o) for o, _ in results]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f'link failed:\n{" ".join(cmd)}\n{proc.stdout}{proc.stderr}')
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == '__main__':
    path = build(verbose='-v' in sys.argv)
    print(path)
