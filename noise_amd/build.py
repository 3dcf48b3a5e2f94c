"""Builds libnoise_amd.so (every HIP source under csrc/) for gfx950 with hipcc, in-tree.

    python -m noise_amd.build          # or __graft_entry__.build()

The library lands next to this file so that it travels with the source tree; nothing is
installed into site-packages or a JIT cache.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / 'csrc'
LIB = PKG / 'libnoise_amd.so'
ARCH = 'gfx950'

FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++20', '-fPIC', '-Wall', '-Wno-unused-function',
    f'-I{ROOT / "include"}', f'-I{CSRC}',
    # Packed fp32 VALU forms are kept out of the generated code on purpose.
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
]


def hipcc():
    for cand in (os.environ.get('HIPCC'), shutil.which('hipcc'), '/opt/rocm/bin/hipcc'):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError('hipcc not found (ROCm is required to build libnoise_amd)')


def _compile(src, obj):
    cmd = [hipcc(), *FLAGS, '-c', str(src), '-o', str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{res.stderr}')
    return obj


def build(verbose=False):
    """Compile every csrc/*.hip and link libnoise_amd.so; returns the library path."""
    objdir = PKG / '_build'
    objdir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(lambda s: _compile(s, objdir / (s.stem + '.o')), sources))
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, objs), '-o', str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB} from {len(sources)} sources', file=sys.stderr)
    return LIB


if __name__ == '__main__':
    build(verbose=True)
