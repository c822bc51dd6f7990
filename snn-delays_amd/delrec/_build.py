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
SOURCES = ('abi.hip', 'axonal.hip', 'farsparse.hip', 'gemm.hip', 'hybstep.hip', 'lagmm.hip', 'lagstep.hip', 'peaks.hip',
           'readout.hip', 'spikelinear.hip', 'synaptic.hip')
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


EXT_SOURCE = CSRC / 'torch_ext.cpp'
EXT_OUT = PKG / 'delrec_torch.so'


def extension_command(out=EXT_OUT):
    """Host-only compile of the C++ autograd Function (torch_ext.cpp) against torch and the
    HIP library, which it finds next to itself at run time (rpath $ORIGIN)."""
    import sysconfig
    import torch
    tdir = Path(torch.__file__).resolve().parent
    return [_hipcc(), '--cuda-host-only', '-O2', '-std=c++17', '-fPIC', '-shared', str(EXT_SOURCE), '-o', str(out),
            f'-I{tdir / "include"}', f'-I{tdir / "include" / "torch" / "csrc" / "api" / "include"}',
            f'-I{sysconfig.get_paths()["include"]}', f'-I{INCLUDE}',
            '-DTORCH_EXTENSION_NAME=delrec_torch', '-DTORCH_API_INCLUDE_EXTENSION_H',
            f'-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}',
            f'-L{tdir / "lib"}', '-ltorch', '-ltorch_cpu', '-ltorch_python', '-lc10', '-lc10_hip', '-ltorch_hip',
            f'-L{PKG}', '-ldelrec_hip', '-Wl,-rpath,$ORIGIN', f'-Wl,-rpath,{tdir / "lib"}']


def build(verbose=False, jobs=None):
    """Compile every HIP source into the shared library, then the C++ autograd extension
    that links it (always recompiles)."""
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
    tmp = EXT_OUT.with_suffix('.so.tmp')
    _run(extension_command(tmp), verbose)
    os.replace(tmp, EXT_OUT)
    return OUT


if __name__ == '__main__':
    print(build(verbose=True))
