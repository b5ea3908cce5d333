"""Compile the gfx950 HIP sources into the in-tree C-ABI library libw8a8.so.

    python minimax-h3-2xt4_amd/build_lib.py [--jobs N] [--verbose]

Each csrc/*.hip compiles to an object under _build/ (in parallel), then one
hipcc link produces w8a8/libw8a8.so next to the Python bindings.
csrc/gemm_inst.hip compiles once per (epilogue, output dtype) pair of the
GEMM (INST_VARIANTS), each with its own -D pair.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / 'csrc'
BUILD = PKG / '_build'
OUT = PKG / 'w8a8' / 'libw8a8.so'
ARCH = 'gfx950'

HIPCC_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC',
    # Every float expression is evaluated as written: no FMA contraction and
    # no fast-math reassociation or reciprocal division.
    '-ffp-contract=off', '-fno-fast-math',
    # Packed FP32 instructions stay off.
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wno-unused-command-line-argument',
    f'-I{ROOT / "include"}', f'-I{CSRC}',
]


# (epilogue, output dtype) pairs of gemm_inst.hip: epilogue 0 int32, 1 row,
# 2 column; output 1 f16, 2 bf16, 3 f32, 4 i32.
INST_VARIANTS = [(0, 4), (1, 1), (1, 2), (1, 3), (2, 1), (2, 2), (2, 3)]


# Per-file options. attention.hip: MFMA results in VGPRs (its scores feed
# VALU work every block; in AGPRs each block would copy them over).
FILE_FLAGS = {'attention.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form']}


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not Path(path).exists():
        raise RuntimeError('hipcc not found')
    return path


def _units():
    """(source, object name, extra flags) of every object in the library."""
    units = []
    for src in sorted(CSRC.glob('*.hip')):
        if src.name == 'gemm_inst.hip':
            for epi, out in INST_VARIANTS:
                units.append((src, f'{src.stem}_{epi}_{out}.o',
                              [f'-DW8A8_INST_EPI={epi}', f'-DW8A8_INST_OUT={out}']))
        else:
            units.append((src, src.stem + '.o', FILE_FLAGS.get(src.name, [])))
    return units


def _compile(unit, verbose):
    src, name, extra = unit
    obj = BUILD / name
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, '-c', str(src), '-o', str(obj)]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}')
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)
    return obj


def build(jobs=None, verbose=False):
    BUILD.mkdir(exist_ok=True)
    units = _units()
    jobs = jobs or min(len(units), max(1, os.cpu_count() or 4))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda u: _compile(u, verbose), units))
    tmp = OUT.with_suffix('.so.tmp')
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, objs), '-o', str(tmp)]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stdout}\n{res.stderr}')
    os.replace(tmp, OUT)
    return OUT


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('--jobs', type=int, default=None)
    ap.add_argument('--verbose', action='store_true')
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))
