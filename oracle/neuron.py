"""LIF neuron and surrogate gradients, restated for the oracle (test infrastructure only).

The reference's layers call a spikingjelly ``LIFNode`` in single-step mode
(``src/delrec/delay_layers_pytorch.py:179,310``), built at ``src/delrec/delay_layers.py:100-109``
with ``tau, decay_input, v_reset, v_threshold, surrogate_function, detach_reset``.
spikingjelly (git d4fee3a1715bf42ce15f52fde1b1d4709d7ea25e) is not installed here; this
module restates its published LIF:

  charge   decay_input=False, v_reset in {None, 0}:  h = v * (1 - 1/tau) + x
           decay_input=False, v_reset != 0:          h = v - (v - v_reset)/tau + x
           decay_input=True,  v_reset in {None, 0}:  h = v + (x - v)/tau
           decay_input=True,  v_reset != 0:          h = v + (x - (v - v_reset))/tau
  fire     spike = surrogate(h - v_threshold)        (Heaviside forward, H(0) = 1)
  reset    soft (v_reset None): v = h - spike_d * v_threshold
           hard:                v = (1 - spike_d) * h + spike_d * v_reset
           spike_d = spike.detach() when detach_reset
  state    v starts at v_reset (0 when v_reset is None)

The first branch is the one every configuration here uses; it is pinned by the
reference's own comment ``configs/perf_HAR.py:71-73`` ("LIFNode with decay_input=False,
v_reset=0 gives v = (1-1/tau)*v + x") and by ``triton_kernels/lif.py:25-33``. All four are
pinned by their closed forms at zero recurrent weight (a constant input relaxes the
membrane geometrically from v_reset to its fixed point, and a hard reset restarts the same
curve; tests/test_oracle_scans.py). What stays unpinned (spikingjelly absent) is only
spikingjelly's fp32 operation order inside the decay_input / v_reset != 0 forms.
"""

import math

import torch


class ATanSurrogate(torch.autograd.Function):
    """Heaviside forward, ATan backward ``(alpha/2) / (1 + (pi/2 * alpha * x)^2)``.

    Restates spikingjelly ``surrogate.ATan`` (used by ``configs/perf_MEM.py:40``) as the
    reference's kernels state it at ``triton_kernels/surrogate.py:25-27``. Pinned by that
    closed form (tests/test_oracle_math.py).
    """

    @staticmethod
    def forward(ctx, x, alpha):
        ctx.save_for_backward(x)
        ctx.alpha = float(alpha)
        return (x >= 0).to(x.dtype)

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        a = ctx.alpha
        z = (math.pi / 2 * a) * x
        return (a / 2) / (1 + z * z) * grad, None


class TriangleSurrogate(torch.autograd.Function):
    """Heaviside forward, triangle backward ``(1/gamma^2) * max(0, gamma - |x|)``.

    Restates ``delrec.utils.Triangle`` (``src/delrec/utils.py:23-41``). Pinned by that
    closed form (tests/test_oracle_math.py).
    """

    @staticmethod
    def forward(ctx, x, gamma):
        ctx.save_for_backward(x)
        ctx.gamma = float(gamma)
        return (x >= 0).to(x.dtype)

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        g = ctx.gamma
        return grad * ((1 / g) * (1 / g) * (g - x.abs()).clamp(min=0)), None


class LIFParams:
    """Neuron constants of one layer. ``surrogate`` is ``('atan', alpha)`` or
    ``('triangle', gamma)``."""

    def __init__(self, tau=2.0, v_threshold=1.0, v_reset=0.0, decay_input=False,
                 detach_reset=False, surrogate=('atan', 2.0)):
        self.tau = float(tau)
        self.v_threshold = float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.decay_input = bool(decay_input)
        self.detach_reset = bool(detach_reset)
        kind, width = surrogate
        assert kind in ('atan', 'triangle'), kind
        self.surrogate = (kind, float(width))

    def fire(self, h):
        kind, width = self.surrogate
        fn = ATanSurrogate if kind == 'atan' else TriangleSurrogate
        return fn.apply(h - self.v_threshold, width)


def lif_initial_v(p, like):
    """spikingjelly's reset state: ``v = v_reset`` (0 for soft reset)."""
    v0 = 0.0 if p.v_reset is None else p.v_reset
    return torch.full_like(like, v0)


def lif_step(p, x, v, forced=None):
    """One single-step LIF update. Returns ``(spike, h, v_next)``; ``h`` is the pre-reset
    membrane the BPTT needs.

    ``forced`` (teacher forcing, a test device of this oracle, not of the reference): the
    spike takes the given 0/1 values instead of ``h >= v_threshold`` while its gradient is
    still the surrogate's at ``h``; the reset uses the forced spike. A run forced with a
    kernel's own spike train follows that train's membrane trajectory exactly, so the
    kernel's spikes can be checked at every step against ``h >= v_threshold`` of that run."""
    tau = p.tau
    reset0 = p.v_reset is None or p.v_reset == 0.0
    if p.decay_input:
        h = v + (x - v) / tau if reset0 else v + (x - (v - p.v_reset)) / tau
    else:
        h = v * (1.0 - 1.0 / tau) + x if reset0 else v - (v - p.v_reset) / tau + x
    spike = p.fire(h)
    if forced is not None:
        spike = spike + (forced.to(spike.dtype) - spike).detach()
    spike_d = spike.detach() if p.detach_reset else spike
    if p.v_reset is None:
        v_next = h - spike_d * p.v_threshold
    else:
        v_next = (1.0 - spike_d) * h + spike_d * p.v_reset
    return spike, h, v_next
