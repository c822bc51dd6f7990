"""ctypes binding of ``libdelrec_hip.so`` (the C ABI declared in ``include/delrec.h``).

The library is loaded once, after ``torch`` (so both share torch's HIP runtime). There is
no fallback: if the shared object is missing or a call returns a non-zero status, a
``DelrecError`` is raised. Tensors are passed as raw device pointers on torch's current
stream; scratch memory comes from torch's caching allocator, sized by
``delrec_query_workspace``.
"""

import ctypes
import math
import os
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get('DELREC_HIP_LIB', _HERE / 'libdelrec_hip.so'))

c_f32 = ctypes.c_float
c_i32 = ctypes.c_int32
c_vp = ctypes.c_void_p
c_size = ctypes.c_size_t

DELREC_TAPS_SOFT, DELREC_TAPS_ROUND, DELREC_TAPS_INTERP = 0, 1, 2
DELREC_BWD_SOFT, DELREC_BWD_STRAIGHT = 0, 1
DELREC_ERR_WINDOW = 5
DELREC_ERR_SCRATCH = 9
WS_AXONAL_FWD, WS_AXONAL_BWD, WS_SYN_FWD, WS_SYN_BWD, WS_SPIKE_LINEAR = 1, 2, 3, 4, 5
WS_SPIKE_LINEAR_DW, WS_READOUT_CE = 6, 7
READOUT_SUM, READOUT_MEAN, READOUT_MAX = 0, 1, 2

# Every symbol include/delrec.h declares (checked by the CPU test suite).
EXPORTS = ('delrec_axonal_fwd', 'delrec_axonal_bwd', 'delrec_axonal_bwd_noalloc', 'delrec_syn_fwd',
           'delrec_syn_bwd', 'delrec_spike_linear_fwd',
           'delrec_lif_fwd', 'delrec_lif_bwd', 'delrec_delay_grad', 'delrec_query_workspace',
           'delrec_strerror', 'delrec_version', 'delrec_scan_timing', 'delrec_scan_timing_read',
           'delrec_max_post', 'delrec_max_take', 'delrec_peak_mfma', 'delrec_spike_linear_dw',
           'delrec_spike_linear_dx_split', 'delrec_readout_ce')


class DelrecError(RuntimeError):
    """A non-zero ``delrec_status`` from the HIP library."""

    def __init__(self, fn, status, message):
        super().__init__(f'{fn} failed: status {status} ({message})')
        self.status = status


class Lif(ctypes.Structure):
    _fields_ = [('tau', c_f32), ('decay', c_f32), ('v_threshold', c_f32), ('v_reset', c_f32),
                ('soft_reset', c_i32), ('decay_input', c_i32), ('detach_reset', c_i32),
                ('surrogate', c_i32), ('gamma', c_f32), ('alpha', c_f32)]


class AxonalFwdArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('N', c_i32), ('L', c_i32),
                ('x', c_vp), ('W', c_vp), ('w_bf16', c_i32), ('bias', c_vp), ('d', c_vp),
                ('s', c_vp), ('s_uniform', c_f32), ('drop', c_vp), ('taps', c_i32),
                ('lag', c_vp), ('frac', c_vp), ('lif', Lif),
                ('y', c_vp), ('u', c_vp), ('rec', c_vp), ('z', c_vp), ('bits', c_vp),
                ('workspace', c_vp), ('workspace_bytes', c_size),
                ('dmax_ticket', ctypes.POINTER(ctypes.c_uint32))]


class AxonalBwdArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('N', c_i32), ('L', c_i32),
                ('gy', c_vp), ('u', c_vp), ('bits', c_vp), ('z', c_vp), ('W', c_vp),
                ('w_bf16', c_i32), ('d', c_vp), ('s', c_vp), ('s_uniform', c_f32), ('drop', c_vp),
                ('mode', c_i32), ('lag', c_vp), ('lif', Lif),
                ('dx', c_vp), ('dW', c_vp), ('db', c_vp), ('dd', c_vp), ('ds', c_vp),
                ('workspace', c_vp), ('workspace_bytes', c_size)]


class SynFwdArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('N', c_i32), ('L', c_i32),
                ('x', c_vp), ('W', c_vp), ('w_bf16', c_i32), ('bias', c_vp), ('d', c_vp),
                ('base', c_vp), ('offsets', c_vp), ('s', c_vp), ('s_uniform', c_f32),
                ('s_max', c_f32), ('drop', c_vp), ('lif', Lif), ('y', c_vp), ('u', c_vp), ('bits', c_vp),
                ('workspace', c_vp), ('workspace_bytes', c_size),
                ('d_min', c_f32), ('off_min', c_i32), ('off_count', c_i32)]


class SynBwdArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('N', c_i32), ('L', c_i32),
                ('gy', c_vp), ('u', c_vp), ('y', c_vp), ('bits', c_vp), ('W', c_vp),
                ('w_bf16', c_i32), ('d', c_vp), ('base', c_vp), ('offsets', c_vp), ('s', c_vp),
                ('s_uniform', c_f32), ('s_max', c_f32), ('drop', c_vp), ('lif', Lif),
                ('dx', c_vp), ('dW', c_vp), ('dd', c_vp), ('ds', c_vp), ('db', c_vp),
                ('workspace', c_vp), ('workspace_bytes', c_size),
                ('d_min', c_f32), ('off_min', c_i32), ('off_count', c_i32),
                ('near_known', c_i32), ('near_lt4', c_i32), ('near_lt2', c_i32)]


class SpikeLinearArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('K', c_i32), ('M', c_i32), ('bits', c_vp), ('W', c_vp),
                ('bias', c_vp), ('out', c_vp), ('workspace', c_vp), ('workspace_bytes', c_size)]


class SpikeLinearDwArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('K', c_i32), ('M', c_i32), ('bits', c_vp), ('g', c_vp),
                ('dW', c_vp), ('workspace', c_vp), ('workspace_bytes', c_size)]


class ReadoutCeArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('C', c_i32), ('logits', c_vp), ('labels', c_vp),
                ('reduce', c_i32), ('integrator', c_i32), ('tau', c_f32), ('out', c_vp), ('dlogits', c_vp),
                ('loss', c_vp), ('workspace', c_vp), ('workspace_bytes', c_size)]


class LifFwdArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('N', c_i32), ('x', c_vp), ('lif', Lif),
                ('y', c_vp), ('u', c_vp)]


class LifBwdArgs(ctypes.Structure):
    _fields_ = [('T', c_i32), ('B', c_i32), ('N', c_i32), ('gy', c_vp), ('u', c_vp), ('y', c_vp),
                ('lif', Lif), ('dx', c_vp)]


# the DELREC_ABI_VERSION of include/delrec.h these ctypes structs mirror
ABI_VERSION = '0.5.0'

_lib = None


def load():
    """Load the HIP library (once). Raises ImportError with the build hint if missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f'{LIB_PATH} is not built: run `python -c "import __graft_entry__ as g; '
                          f'g.build()"` from the repository root')
    lib = ctypes.CDLL(str(LIB_PATH))
    for name in ('delrec_axonal_fwd', 'delrec_axonal_bwd', 'delrec_axonal_bwd_noalloc', 'delrec_syn_fwd',
                 'delrec_syn_bwd', 'delrec_spike_linear_fwd', 'delrec_spike_linear_dw', 'delrec_readout_ce',
                 'delrec_lif_fwd', 'delrec_lif_bwd'):
        getattr(lib, name).restype = c_i32
        getattr(lib, name).argtypes = [c_vp, c_vp]
    lib.delrec_delay_grad.restype = c_i32
    lib.delrec_delay_grad.argtypes = [c_vp, c_vp, c_vp, c_f32, c_i32, c_i32, c_vp, c_vp]
    lib.delrec_query_workspace.restype = c_i32
    lib.delrec_query_workspace.argtypes = [c_i32] * 6 + [ctypes.POINTER(c_size)]
    lib.delrec_strerror.restype = ctypes.c_char_p
    lib.delrec_strerror.argtypes = [c_i32]
    lib.delrec_version.restype = ctypes.c_char_p
    lib.delrec_scan_timing.restype = c_i32
    lib.delrec_scan_timing.argtypes = [c_i32]
    lib.delrec_scan_timing_read.restype = c_i32
    lib.delrec_scan_timing_read.argtypes = [ctypes.POINTER(c_f32), ctypes.POINTER(c_i32), c_i32]
    lib.delrec_max_post.restype = c_i32
    lib.delrec_max_post.argtypes = [c_vp, c_i32, ctypes.POINTER(ctypes.c_uint32), c_vp]
    lib.delrec_max_take.restype = c_i32
    lib.delrec_max_take.argtypes = [ctypes.c_uint32, ctypes.POINTER(c_f32), c_i32]
    lib.delrec_peak_mfma.restype = c_i32
    lib.delrec_peak_mfma.argtypes = [c_i32, c_i32, c_vp, c_size, ctypes.POINTER(ctypes.c_double), c_vp]
    lib.delrec_spike_linear_dx_split.restype = c_i32
    lib.delrec_spike_linear_dx_split.argtypes = [c_vp, ctypes.c_int64, c_i32, c_vp, c_vp]
    got = lib.delrec_version().decode()
    if got.split()[1:2] != [ABI_VERSION]:
        raise ImportError(f'{LIB_PATH} reports "{got}"; this binding lays out the argument structs of '
                          f'ABI {ABI_VERSION}: rebuild the library')
    _lib = lib
    return lib


_EXT = []
EXT_PATH = _HERE / 'delrec_torch.so'


def torch_ext():
    """The C++ autograd extension (``delrec_torch.so``, built next to the HIP library), or
    None when it has not been built. It calls the same C ABI; without it the layers use the
    Python ``autograd.Function``s over the ctypes binding."""
    if not _EXT:
        mod = None
        if EXT_PATH.exists():
            import importlib.util
            load()
            spec = importlib.util.spec_from_file_location('delrec_torch', str(EXT_PATH))
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
        _EXT.append(mod)
    return _EXT[0]


def _check(fn, status):
    if status != 0:
        raise DelrecError(fn, status, load().delrec_strerror(status).decode())


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def make_lif(tau, v_threshold, v_reset, decay_input, detach_reset, surr_id, gamma, alpha):
    """``delrec_lif`` from the neuron constants; ``v_reset=None`` means soft reset."""
    tau = float(tau)
    return Lif(tau=tau, decay=float(1.0 - 1.0 / tau), v_threshold=float(v_threshold),
               v_reset=0.0 if v_reset is None else float(v_reset),
               soft_reset=1 if v_reset is None else 0, decay_input=int(bool(decay_input)),
               detach_reset=int(bool(detach_reset)), surrogate=int(surr_id),
               gamma=float(gamma), alpha=float(alpha))


_WS_SIZES = {}


def lag_taps(s_max):
    """ceil(2 s_max) on the float32 value the C ABI receives (the most lags of non-zero weight
    per connection), for bits 8..15 of the synaptic workspace flags."""
    s32 = ctypes.c_float(float(s_max)).value
    return min(255, max(0, math.ceil(2.0 * s32)))


_FORM_ENV = ('DELREC_SYN_LAGSTEP', 'DELREC_SYN_HYBSTEP', 'DELREC_HYB_FWD')


def workspace_bytes(kind, T, B, N, L, flags):
    """``delrec_query_workspace`` (memoised: the size is a function of the arguments and of
    DELREC_SYN_LAGSTEP / DELREC_SYN_HYBSTEP / DELREC_HYB_FWD, which pick the synaptic scans'
    form)."""
    key = (kind, T, B, N, L, flags) + tuple(os.environ.get(v) for v in _FORM_ENV)
    n = _WS_SIZES.get(key)
    if n is None:
        size = c_size(0)
        _check('delrec_query_workspace', load().delrec_query_workspace(kind, T, B, N, L, flags,
                                                                       ctypes.byref(size)))
        n = _WS_SIZES[key] = max(int(size.value), 1)
    return n


def workspace(kind, T, B, N, L, flags, device):
    return torch.empty(workspace_bytes(kind, T, B, N, L, flags), dtype=torch.uint8, device=device)


class _Timing:
    """Optional HIP-event brackets around every library call (used by the benchmark):
    events are recorded on the same stream the kernels are launched on."""

    active = None   # list of (entry point, start event, end event) while timing

    def __enter__(self):
        _Timing.active = []
        return _Timing.active

    def __exit__(self, *exc):
        _Timing.active = None
        return False


def timing():
    return _Timing()


def call(name, args, stream):
    rec = _Timing.active
    if rec is not None:
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        _check(name, getattr(load(), name)(ctypes.byref(args), stream))
        e.record()
        rec.append((name, s, e))
        return
    _check(name, getattr(load(), name)(ctypes.byref(args), stream))


SCAN_KINDS = {1: 'axonal_fwd_scan', 2: 'axonal_bwd_scan', 3: 'syn_fwd_scan', 4: 'syn_bwd_scan'}


class scan_timing:
    """HIP-event durations of the time-scan kernels launched inside the block (at most
    ``capacity`` launches): ``with scan_timing(n) as st: ...`` then ``st.launches`` is a
    list of (kind name, ms)."""

    def __init__(self, capacity):
        self.capacity = int(capacity)
        self.launches = []

    def __enter__(self):
        _check('delrec_scan_timing', load().delrec_scan_timing(self.capacity))
        return self

    def __exit__(self, *exc):
        lib = load()
        ms = (c_f32 * self.capacity)()
        kinds = (c_i32 * self.capacity)()
        n = lib.delrec_scan_timing_read(ms, kinds, self.capacity)
        lib.delrec_scan_timing(0)
        if n < 0:
            _check('delrec_scan_timing_read', -n)
        self.launches = [(SCAN_KINDS.get(kinds[k], str(kinds[k])), ms[k]) for k in range(n)]
        return False


DELREC_OK = 0


class PostedMax:
    """max of a contiguous fp32 device vector, written into pinned host memory by a kernel
    queued on the current stream (``delrec_max_post``); ``value()`` waits for that kernel's
    store only, and reads the maximum again (synchronously) if the slot was reused by later
    posts or the value did not arrive."""

    def __init__(self, t, ticket=None):
        """Post max(t) now, or adopt the ``ticket`` an entry point returned for max(t)."""
        assert t.dtype == torch.float32 and t.is_contiguous() and t.numel() > 0
        self.t = t
        if ticket is None:
            tk = ctypes.c_uint32(0)
            _check('delrec_max_post', load().delrec_max_post(ptr(t), t.numel(), ctypes.byref(tk),
                                                             stream_of(t)))
            ticket = tk.value
        self.ticket = int(ticket)

    def value(self):
        out = c_f32(0.0)
        if load().delrec_max_take(self.ticket, ctypes.byref(out), 10000) == DELREC_OK:
            return float(out.value)
        return float(self.t.max())


def delay_grad(C, W, d, sigma, N, Lm, out, stream):
    _check('delrec_delay_grad', load().delrec_delay_grad(ptr(C), ptr(W), ptr(d), float(sigma), N,
                                                         Lm, ptr(out), stream))


def spike_linear_dx_split(g2, out, stream):
    """``out`` (rows, 3M) bf16 = [hi | lo | hi] of ``g2`` (rows, M) fp32."""
    rows, M = g2.shape
    _check('delrec_spike_linear_dx_split', load().delrec_spike_linear_dx_split(ptr(g2), rows, M, ptr(out), stream))


def version():
    return load().delrec_version().decode()


def peak_mfma(kind, iters, sink, stream):
    """Launch the register-only MFMA loop (kind 0: bf16, 1: fp32) on ``stream``; returns the
    flops the launch issues (the caller times it)."""
    flops = ctypes.c_double(0.0)
    _check('delrec_peak_mfma', load().delrec_peak_mfma(kind, iters, ptr(sink), sink.numel() * sink.element_size(),
                                                        ctypes.byref(flops), stream))
    return flops.value
