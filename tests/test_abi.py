"""CPU checks of the C ABI: the library loads, exports every declared symbol, and its
argument structs have the same layout in C (as the compiler lays out include/delrec.h) and
in the ctypes binding. No kernel is launched."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'delrec.h')


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r'^\s*(?:int|const char\*)\s+(delrec_\w+)\s*\(', text, re.M)))


def test_header_declares_the_binding_exports():
    from delrec import _lib
    assert _declared_functions() == sorted(_lib.EXPORTS)


def test_library_loads_and_exports_every_symbol():
    from delrec import _lib
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert _lib.version().startswith('delrec-mi355x')
    # the binding's struct layouts are those of the header's ABI version
    hdr = re.search(r'#define DELREC_ABI_VERSION "([^"]+)"', open(HEADER).read()).group(1)
    assert hdr == _lib.ABI_VERSION and _lib.version().split()[1] == hdr
    assert lib.delrec_strerror(0) == b'ok'
    assert b'workspace' in lib.delrec_strerror(3)


def test_query_workspace_and_argument_errors_without_gpu():
    from delrec import _lib
    lib = _lib.load()
    size = ctypes.c_size_t(0)
    assert lib.delrec_query_workspace(_lib.WS_AXONAL_BWD, 128, 128, 256, 36, 0, ctypes.byref(size)) == 0
    assert size.value >= 128 * 128 * 256 * 4
    assert lib.delrec_query_workspace(99, 1, 1, 1, 2, 0, ctypes.byref(size)) == 1       # bad kind
    assert lib.delrec_query_workspace(_lib.WS_SYN_FWD, 0, 1, 1, 2, 0, ctypes.byref(size)) == 1
    # null / inconsistent arguments are rejected before anything touches the device
    assert lib.delrec_axonal_fwd(None, None) == 1
    args = _lib.AxonalFwdArgs(T=4, B=1, N=8, L=3)
    assert lib.delrec_axonal_fwd(ctypes.byref(args), None) == 1          # null tensors
    assert lib.delrec_syn_bwd(None, None) == 1
    assert lib.delrec_delay_grad(None, None, None, 0.0, 4, 3, None, None) == 1
    ticket, value = ctypes.c_uint32(0), ctypes.c_float(0.0)
    assert lib.delrec_max_post(None, 4, ctypes.byref(ticket), None) == 1     # null vector
    assert lib.delrec_max_take(0, ctypes.byref(value), 10) == 1              # ticket 0 is never issued
    assert lib.delrec_max_take(5, None, 10) == 1


_STRUCTS = ['delrec_lif', 'delrec_axonal_fwd_args', 'delrec_axonal_bwd_args', 'delrec_syn_fwd_args',
            'delrec_syn_bwd_args', 'delrec_lif_fwd_args', 'delrec_lif_bwd_args', 'delrec_spike_linear_args',
            'delrec_spike_linear_dw_args', 'delrec_readout_ce_args']


def _c_layout():
    """sizeof / offsetof of every field, as gcc lays out the header."""
    from delrec import _lib
    classes = {'delrec_lif': _lib.Lif, 'delrec_axonal_fwd_args': _lib.AxonalFwdArgs,
               'delrec_axonal_bwd_args': _lib.AxonalBwdArgs, 'delrec_syn_fwd_args': _lib.SynFwdArgs,
               'delrec_syn_bwd_args': _lib.SynBwdArgs, 'delrec_lif_fwd_args': _lib.LifFwdArgs,
               'delrec_lif_bwd_args': _lib.LifBwdArgs, 'delrec_spike_linear_args': _lib.SpikeLinearArgs,
               'delrec_spike_linear_dw_args': _lib.SpikeLinearDwArgs, 'delrec_readout_ce_args': _lib.ReadoutCeArgs}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', 'int main(void) {']
    for st in _STRUCTS:
        lines.append(f'  printf("{st} size %zu\\n", sizeof({st}));')
        for fname, _ in classes[st]._fields_:
            lines.append(f'  printf("{st} {fname} %zu\\n", offsetof({st}, {fname}));')
    lines += ['  return 0;', '}']
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = os.path.join(tmp, 'probe.c'), os.path.join(tmp, 'probe')
        open(src, 'w').write('\n'.join(lines))
        subprocess.run(['gcc', '-std=c11', src, '-o', exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return classes, dict((' '.join(l.split()[:2]), int(l.split()[2])) for l in out.splitlines())


def test_struct_layout_matches_ctypes():
    classes, c = _c_layout()
    for st, cls in classes.items():
        assert c[f'{st} size'] == ctypes.sizeof(cls), st
        for fname, _ in cls._fields_:
            assert c[f'{st} {fname}'] == getattr(cls, fname).offset, f'{st}.{fname}'


def test_torch_extension_loads_and_exposes_the_axonal_function():
    """The C++ autograd extension is built next to the HIP library, links it, and exposes
    the axonal layer's Function (no GPU call is made)."""
    from delrec import _lib
    ext = _lib.torch_ext()
    assert ext is not None, f'{_lib.EXT_PATH} is not built'
    assert callable(ext.axonal_common)
    doc = ext.axonal_common.__doc__
    for arg in ('x', 'W', 'd', 'bias', 'drop', 'sigma', 'tau', 'vth', 'surrogate', 'gamma', 'alpha', 'detach'):
        assert f'{arg}:' in doc


def test_synaptic_scan_form_follows_the_taps_per_connection():
    """Rings too large for LDS take the lag-stacked GEMM scans only where a connection's
    taps are a fair share of the window (flags bits 8..15 = ceil(2 s_max)): a synaptic
    layer at sigma 4 (10 taps over 46 lags) does, a hybrid at sigma 0 (2 taps over 65 lags)
    keeps the per-connection gathers; the lag-stacked workspace holds the (L-1) N^2 lag
    weights and is far larger."""
    from delrec import _lib
    lib = _lib.load()
    T, B, N = 32, 8, 1024

    def size(kind, L, flags, taps):
        n = ctypes.c_size_t(0)
        assert lib.delrec_query_workspace(kind, T, B, N, L, flags | (taps << 8), ctypes.byref(n)) == 0
        return n.value

    assert _lib.lag_taps(5.0) == 10 and _lib.lag_taps(1.0) == 2 and _lib.lag_taps(1.25) == 3
    planes = 2 * 46 * N * N * 2                       # two bf16 planes of M_l, 46 lags
    for kind in (_lib.WS_SYN_FWD, _lib.WS_SYN_BWD):
        wide = size(kind, 47, 0, _lib.lag_taps(5.0))         # synaptic, sigma 4
        narrow = size(kind, 66, 2, _lib.lag_taps(1.0))       # hybrid, sigma 0
        assert wide >= planes > narrow
