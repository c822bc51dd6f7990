"""Neuron, surrogate and dropout modules the DelRec layers are built from.

The reference builds its layers from spikingjelly (``spikingjelly.activation_based``:
``neuron.LIFNode``, ``base.MemoryModule``, ``layer.Dropout``, ``surrogate.ATan``;
``src/delrec/delay_layers.py:21``, ``configs/perf_MEM.py:7``). spikingjelly is not a
dependency of this build: these classes keep the constructor arguments and attributes
the layers, model classes and configs read (``tau``, ``v_threshold``, ``v_reset``,
``decay_input``, ``surrogate_function``, ``detach_reset``, ``step_mode``, ``store_v_seq``)
and run their multi-step forward through the HIP LIF kernel.
"""

import torch

from .kernels.lif import lif_sequence


class MemoryModule(torch.nn.Module):
    """A module with resettable state (``reset()`` restores every registered memory)."""

    def __init__(self):
        super().__init__()
        self._memories = {}

    def register_memory(self, name, value):
        self._memories[name] = value
        setattr(self, name, value)

    def reset(self):
        for name, value in self._memories.items():
            setattr(self, name, value)


class ATan(torch.nn.Module):
    """ATan surrogate descriptor: Heaviside forward, ``(alpha/2)/(1+(pi/2*alpha*x)^2)``
    backward (the reference's surrogate id 1, ``triton_kernels/surrogate.py:25-27``)."""

    surrogate_kind = 'atan'

    def __init__(self, alpha=2.0, spiking=True):
        super().__init__()
        self.alpha = float(alpha)
        self.spiking = spiking

    def forward(self, x):
        from .utils import ATanFunction
        return ATanFunction.apply(x, self.alpha)


class surrogate:  # noqa: N801 - namespace mirroring spikingjelly.activation_based.surrogate
    ATan = ATan


class LIFNode(MemoryModule):
    """Leaky integrate-and-fire neuron (spikingjelly ``LIFNode`` semantics).

    charge: ``h = v*(1-1/tau) + x`` (``decay_input=False``, ``v_reset`` 0 or None),
    ``h = v - (v - v_reset)/tau + x``, ``h = v + (x - v)/tau`` or
    ``h = v + (x - (v - v_reset))/tau``; fire ``y = H(h - v_threshold)``; reset hard to
    ``v_reset`` or soft (``v_reset=None``) by subtracting ``v_threshold``.
    Multi-step forward runs ``delrec_lif_fwd`` on the GPU; every call starts from the
    reset state.
    """

    def __init__(self, tau=2.0, decay_input=True, v_threshold=1.0, v_reset=0.0,
                 surrogate_function=None, detach_reset=False, step_mode='s', backend='torch',
                 store_v_seq=False):
        super().__init__()
        if float(tau) <= 1.0 and not decay_input:
            pass  # allowed: leak factor (1 - 1/tau) may be <= 0, as in the reference configs
        self.tau = float(tau)
        self.decay_input = bool(decay_input)
        self.v_threshold = float(v_threshold)
        self.v_reset = None if v_reset is None else float(v_reset)
        self.surrogate_function = surrogate_function if surrogate_function is not None else ATan()
        self.detach_reset = bool(detach_reset)
        self.step_mode = step_mode
        self.backend = backend
        self.store_v_seq = store_v_seq
        self.register_memory('v', 0.0 if v_reset is None else float(v_reset))

    def forward(self, x_seq):
        if self.step_mode != 'm':
            raise NotImplementedError('LIFNode: only multi-step mode (step_mode="m") runs on the HIP kernel')
        return lif_sequence(x_seq, self)

    def extra_repr(self):
        return (f'tau={self.tau}, v_threshold={self.v_threshold}, v_reset={self.v_reset}, '
                f'decay_input={self.decay_input}, detach_reset={self.detach_reset}, '
                f'step_mode={self.step_mode}')


class Dropout(MemoryModule):
    """Dropout whose mask is drawn once and kept until ``reset()`` (spikingjelly
    ``layer.Dropout``): single-step mode masks each step with the same ``(B, N)`` mask,
    multi-step mode masks all of ``(T, B, N)`` with one ``(B, N)`` mask."""

    def __init__(self, p=0.5, step_mode='s'):
        super().__init__()
        assert 0.0 <= p < 1.0
        self.p = float(p)
        self.step_mode = step_mode
        self.register_memory('mask', None)

    def _draw(self, like):
        return torch.nn.functional.dropout(torch.ones_like(like), self.p, training=True)

    def forward(self, x):
        if not self.training or self.p == 0.0:
            return x
        if self.step_mode == 'm':
            if self.mask is None:
                self.mask = self._draw(x[0].detach())
            return x * self.mask
        if self.mask is None:
            self.mask = self._draw(x.detach())
        return x * self.mask

    def extra_repr(self):
        return f'p={self.p}, step_mode={self.step_mode}'


class neuron:  # noqa: N801 - namespace mirroring spikingjelly.activation_based.neuron
    LIFNode = LIFNode


class layer:  # noqa: N801 - namespace mirroring spikingjelly.activation_based.layer
    Dropout = Dropout


class base:  # noqa: N801 - namespace mirroring spikingjelly.activation_based.base
    MemoryModule = MemoryModule
