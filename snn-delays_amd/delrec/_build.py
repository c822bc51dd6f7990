"""Compile ``libdelrec_hip.so`` for gfx950 in-tree with hipcc.

Flags: ``-ffp-contract=off`` keeps the LIF / triangle arithmetic separately rounded (the
same fp32 operation sequence as the PyTorch scans), and packed-fp32 instructions are
disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / 'csrc'
INCLUDE = PKG.parent.parent / 'include'
OUT = PKG / 'libdelrec_hip.so'
SOURCES = ('abi.hip', 'axonal.hip', 'gemm.hip', 'lagmm.hip', 'synaptic.hip')
ARCH = os.environ.get('DELREC_OFFLOAD_ARCH', 'gfx950')


def command(out=OUT):
    hipcc = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
    return [hipcc, '-O3', '-std=c++17', f'--offload-arch={ARCH}', '-fPIC', '-shared',
            '-ffp-contract=off', '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
            f'-I{INCLUDE}', *[str(CSRC / s) for s in SOURCES], '-o', str(out)]


def build(verbose=False):
    """Compile every HIP source into the shared library (always recompiles)."""
    tmp = OUT.with_suffix('.so.tmp')
    cmd = command(tmp)
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f'hipcc failed ({res.returncode})')
    os.replace(tmp, OUT)
    return OUT


if __name__ == '__main__':
    print(build(verbose=True))
