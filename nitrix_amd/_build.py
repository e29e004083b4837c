"""Build ``libnxattn.so`` (the HIP kernels plus the C ABI) for gfx950.

Every ``csrc/*.hip`` file is compiled with ``hipcc --offload-arch=gfx950``
into ``_build/`` and linked into ``nitrix_amd/libnxattn.so`` next to this
file.  ``python -m nitrix_amd._build`` runs it from the command line.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
BUILD = PKG / '_build'
LIB = PKG / 'libnxattn.so'
INCLUDE = PKG.parent / 'include'

ARCH = 'gfx950'

HIPCC_FLAGS = [
    f'--offload-arch={ARCH}',
    '-O3',
    '-std=c++17',
    '-fPIC',
    '-Wall',
    '-Wno-unused-result',
    # Packed-fp32 VALU forms stay off: plain fp32 arithmetic only.
    '-Xclang',
    '-target-feature',
    '-Xclang',
    '-packed-fp32-ops',
    f'-I{INCLUDE}',
]


# Code generation flags of single translation units, on top of HIPCC_FLAGS.
# The head-dim-256 kernels run at one wave per SIMD with 512 registers; for
# them these flags measured faster on the box (bf16 B4 H16 L4096 D256,
# same-box A/B): the forward 11 % with MFMA operands and results forced into
# VGPRs, dK/dV 7 % and dQ 6 % with the max-ILP machine scheduler.  Neither
# helps the head dim 64 / 128 kernels (max-ILP is 2-4 % slower at D = 64).
FILE_FLAGS = {
    'nxa_fwd16_wide.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form'],
    'nxa_bwd16_wide.hip': ['-mllvm', '-amdgpu-sched-strategy=max-ilp'],
}


def _hipcc() -> str:
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    cand = pathlib.Path(rocm) / 'bin' / 'hipcc'
    if cand.exists():
        return str(cand)
    found = shutil.which('hipcc')
    if not found:
        raise RuntimeError('hipcc not found (set ROCM_PATH)')
    return found


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), '-c', str(src), '-o', str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(
            f'hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}'
        )


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source and link ``libnxattn.so``; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    objs = [BUILD / (s.stem + '.o') for s in sources]
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        futs = [pool.submit(_compile, s, o) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [
        _hipcc(),
        f'--offload-arch={ARCH}',
        '-shared',
        '-fPIC',
        '-o',
        str(tmp),
        *map(str, objs),
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stdout}\n{res.stderr}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB}')
    return LIB


if __name__ == '__main__':
    build(verbose=True)
