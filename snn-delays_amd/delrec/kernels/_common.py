"""Host helpers shared by the autograd Functions: device checks, neuron constants,
surrogate ids, window length, dropout-mask normalisation."""

import math
import time

import numpy as np
import torch

from .. import _lib
from .surrogate import surrogate_id


def require_device(x, what='input'):
    """The layer runs only on the GPU: a CPU tensor is an error, never a fallback."""
    if not x.is_cuda:
        raise RuntimeError(f'delrec-mi355x runs the delayed-LIF scan with HIP kernels on the GPU; '
                           f'{what} is on {x.device}. The pure-PyTorch scans of the reference are '
                           f'not part of this build.')


def lif_struct(neuron, surrogate_function, gamma=None):
    """``delrec_lif`` of a LIFNode-like object plus the config's surrogate."""
    sid, g, alpha = surrogate_id(surrogate_function, gamma)
    return _lib.make_lif(neuron.tau, neuron.v_threshold, neuron.v_reset,
                         getattr(neuron, 'decay_input', False), getattr(neuron, 'detach_reset', False),
                         sid, g, alpha)


_PINNED = {}


# read_scalars polls its event without pause this long, then sleeps between polls (a long
# wait would otherwise hold a host core for its whole duration)
_SPIN_S, _NAP_S = 5e-3, 5e-5


def read_scalars(*vals):
    """Copy a few 0-dim device tensors to the host through a pinned buffer and wait for them
    by polling an event: the one device-to-host read of a forward, which waits for the GPU
    work queued before it (a previous backward: 0.1 to 5 ms at the small and mid-size shapes,
    100 ms at the largest). Waits up to 5 ms are spun for the earliest wake-up; past that the
    thread sleeps 50 us between polls, which adds at most one nap (about 0.1 ms with the
    kernel's timer slack) to a wait of 5 ms or more."""
    dev = vals[0].device
    buf = _PINNED.get(dev)
    if buf is None:
        buf = _PINNED[dev] = (torch.empty(8, dtype=torch.float32, pin_memory=True),
                              torch.cuda.Event())
    host, ev = buf
    n = len(vals)
    stacked = vals[0].reshape(1) if n == 1 else torch.stack([v.reshape(()) for v in vals])
    host[:n].copy_(stacked.to(torch.float32), non_blocking=True)
    ev.record()
    t0 = time.perf_counter()
    while not ev.query():
        if time.perf_counter() - t0 > _SPIN_S:
            time.sleep(_NAP_S)
    return host[:n].tolist()


def window_length_f32(d_max, s_max):
    """``L = ceil(1 + max d + max s) + 1`` with the sum rounded to fp32 after each addition,
    as the reference's fp32 tensors compute it (``delays.build_mask``, reference
    ``triton_kernels/delays.py:26``)."""
    v = np.float32(np.float32(1.0) + np.float32(d_max)) + np.float32(s_max)
    return int(math.ceil(float(np.float32(v)))) + 1


def round_half_even_f32(v):
    """``torch.round`` of an fp32 value (half to even), as an int."""
    return int(np.round(np.float32(v)))


def window_length_f64(d_max, s_max):
    """The same in double precision, as ``EventDrivenSyn`` / ``HybridSynDelay`` compute it
    (``synaptic_eventdriven.py:391``, ``synaptic_hybrid.py:148``)."""
    return int(math.ceil(1.0 + float(d_max) + float(s_max))) + 1


def drop_bn(drop, T, B, N):
    """Normalise a recurrent-dropout multiplier to a contiguous ``(B, N)`` fp32 tensor, or
    ``None`` when absent. A ``(T, B, N)`` argument must hold the same mask at every step
    (the fixed-mask semantics of the reference, ``delay_layers_triton.py:37-48``)."""
    if drop is None:
        return None
    drop = drop.detach()
    if drop.dim() == 3:
        if drop.shape != (T, B, N):
            raise ValueError(f'drop has shape {tuple(drop.shape)}, expected {(T, B, N)}')
        first = drop[0]
        if drop.stride(0) != 0 and T > 1 and not torch.equal(drop, first.unsqueeze(0).expand_as(drop)):
            raise ValueError('drop must be the same (B, N) mask at every time step')
        drop = first
    if drop.shape != (B, N):
        raise ValueError(f'drop has shape {tuple(drop.shape)}, expected {(B, N)}')
    return drop.to(torch.float32).contiguous()


def weights(W):
    """Contiguous device weights and the bf16 flag (fp32 and bf16 are native)."""
    W = W.detach()
    if W.dtype == torch.bfloat16:
        return W.contiguous(), 1
    return W.to(torch.float32).contiguous(), 0


def bits_shape(T, B, N):
    return (B, (T + 31) // 32, N)
