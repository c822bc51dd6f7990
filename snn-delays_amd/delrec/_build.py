"""Compile ``libdelrec_hip.so`` for gfx950 in-tree with hipcc.

Flags: ``-ffp-contract=off`` keeps the LIF / triangle arithmetic separately rounded (the
same fp32 operation sequence as the PyTorch scans), and packed-fp32 instructions are
disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).

Each source compiles to its own object in a temporary directory (in parallel), then the
objects are linked into the shared library.
"""

import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / 'csrc'
INCLUDE = PKG.parent.parent / 'include'
OUT = PKG / 'libdelrec_hip.so'
SOURCES = ('abi.hip', 'axonal.hip', 'gemm.hip', 'lagmm.hip', 'synaptic.hip')
ARCH = os.environ.get('DELREC_OFFLOAD_ARCH', 'gfx950')


def _hipcc():
    return os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')


def compile_flags():
    return ['-O3', '-std=c++17', f'--offload-arch={ARCH}', '-fPIC', '-ffp-contract=off',
            '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops', f'-I{INCLUDE}']


def command(out=OUT):
    """One-shot compile-and-link command line (equivalent to build())."""
    return [_hipcc(), *compile_flags(), '-shared', *[str(CSRC / s) for s in SOURCES], '-o', str(out)]


def _run(cmd, verbose):
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f'hipcc failed ({res.returncode}): {cmd[-1]}')


def build(verbose=False, jobs=None):
    """Compile every HIP source into the shared library (always recompiles)."""
    jobs = jobs or min(len(SOURCES), max(1, os.cpu_count() or 1))
    with tempfile.TemporaryDirectory(prefix='delrec_build_') as tmpdir:
        objs = [os.path.join(tmpdir, Path(s).stem + '.o') for s in SOURCES]
        cmds = [[_hipcc(), *compile_flags(), '-c', str(CSRC / s), '-o', o] for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp = OUT.with_suffix('.so.tmp')
        _run([_hipcc(), f'--offload-arch={ARCH}', '-fPIC', '-shared', *objs, '-o', str(tmp)], verbose)
        os.replace(tmp, OUT)
    return OUT


if __name__ == '__main__':
    print(build(verbose=True))
