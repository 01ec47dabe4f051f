"""Builds the HIP library libtcq.so (gfx950) in-tree from yanlongvla_amd/csrc/*.hip with hipcc.

    python -m yanlongvla_amd.build          # or __graft_entry__.build()

Flags: -ffp-contract=off keeps every a * b + c un-contracted (the reference arithmetic is reproduced bit for bit, as the
reference compiled with --fmad=false); FP32 division and sqrt stay correctly rounded; packed-FP32 instructions are disabled
(-packed-fp32-ops) so every FP32 operation is a scalar IEEE operation.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
INCLUDE = PKG.parent / 'include'
LIB = PKG / 'libtcq.so'
BUILD = PKG.parent / '_build'
ARCH = os.environ.get('TCQ_OFFLOAD_ARCH', 'gfx950')

FLAGS = ['--offload-arch=' + ARCH, '-O3', '-fPIC', '-std=c++17', '-ffp-contract=off', '-fhip-fp32-correctly-rounded-divide-sqrt',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', '-Wno-unused-command-line-argument', '-I', str(INCLUDE)]


def hipcc():
    for c in (os.environ.get('HIPCC'), '/opt/rocm/bin/hipcc', 'hipcc'):
        if c and (os.path.sep not in c or Path(c).exists()):
            return c
    raise RuntimeError('hipcc not found')


def _compile(src, obj):
    cmd = [hipcc(), *FLAGS, '-c', str(src), '-o', str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}')
    return obj


def build(verbose=True):
    """Compile every csrc/*.hip and link libtcq.so. Always recompiles (the build check of a fresh tree)."""
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob('*.hip'))
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, BUILD / (s.stem + '.o')), srcs))
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [hipcc(), '--offload-arch=' + ARCH, '-shared', '-fPIC', *map(str, objs), '-o', str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'link failed:\n{r.stdout}\n{r.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB} from {len(srcs)} sources', file=sys.stderr)
    return LIB


if __name__ == '__main__':
    build()
