"""Recurrent spiking layers with learnable transmission delays (module API of
``src/delrec/delay_layers.py``).

    axonal_recdel     one delay per presynaptic neuron, ``recurrent_delays`` (N,)
    synaptic_recdel   one delay per connection, ``recurrent_delays`` (N, N)
    common_recdel     one delay shared by the whole layer, ``recurrent_delays`` (1,)
    vanilla_recurrent plain recurrent LIF without delays

A spike of neuron j at step t reaches its targets at t + 1 + d; d is relaxed to the reals
and spread over neighbouring steps by a triangle of half-width 1 + sigma. Tensors are
time-major ``(T, B, N)``. Parameters, initialisation, sigma annealing and clamping follow
the reference (``delay_layers.py:86-304``) so seeded models are initialised identically.

Execution: every forward runs the HIP kernels on the GPU. ``forward_version`` accepts the
reference's names: ``'triton_exact'`` (default for axonal), ``'triton_approx'``,
``'triton_ste'``, ``'eventdriven'`` (default for synaptic) and ``'hybrid_triton'`` (default
for hybrid-tagged synaptic layers) select the corresponding HIP modes. ``'v1'`` / ``'v2'``,
the reference's pure-PyTorch scans, are not part of this build and raise; so does a CPU
input. There is no silent fallback: a kernel error propagates to the caller.
"""

import torch

from .delay_layers_hip import AxonalHipScans, SynapticHipScans, SynapticHybridScans
from .neuron import LIFNode, MemoryModule, Dropout

# Default forward of each layer kind; the names are the reference's (delay_layers.py:82-83).
AXONAL_CUDA_DEFAULT = 'triton_exact'
SYNAPTIC_CUDA_DEFAULT = 'eventdriven'

_TORCH_SCANS_MSG = ("forward_version {!r} is the reference's pure-PyTorch scan, which this "
                    "build does not ship; use the default (HIP) forward")


def _make_recurrent_dropout(config):
    """Recurrent dropout whose mask is fixed over the time steps of one sequence."""
    return Dropout(config.recurrent_dropout_rate, step_mode='s')


def _make_neuron(config, neuron_module):
    return neuron_module(
        tau=config.tau,
        decay_input=config.decay_input,
        v_reset=config.v_reset,
        v_threshold=config.v_threshold,
        surrogate_function=config.surrogate_function,
        detach_reset=config.detach_reset,
        step_mode='s',
        backend=config.backend,
    )


class vanilla_recurrent(AxonalHipScans, MemoryModule):
    """Delay-free recurrent LIF, ``rec[t] = y[t-1] @ W`` (reference
    ``delay_layers_pytorch.py:18-47``). Runs as an axonal layer with every delay 0 and
    sigma 0 (a single exact tap at lag 1) on ``W^T``; recurrent dropout acts on the
    spikes in the reference, so an active recurrent dropout is rejected here."""

    def __init__(self, config, neurons, neuron_module=LIFNode):
        super().__init__()
        self.config = config
        self.step_mode = config.step_mode
        self.store_v_seq = config.store_v_seq
        self.neuron_module = _make_neuron(config, neuron_module)
        self.neurons = neurons
        self.recurrent_weights = torch.nn.Parameter(torch.zeros(neurons, neurons), requires_grad=True)
        self.dropout = _make_recurrent_dropout(config)
        self.init_recurrent_weights()

    def init_recurrent_weights(self):
        torch.nn.init.orthogonal_(self.recurrent_weights, gain=1.0)

    def forward(self, x_seq):
        if self.step_mode == 's':
            raise NotImplementedError('single-step mode is not supported; use step_mode="m"')
        if self.training and self.config.recurrent_dropout_rate > 0:
            raise NotImplementedError('vanilla_recurrent with recurrent dropout (mask on the spikes)')
        from .kernels import AxonalRecdelHip
        from .kernels.surrogate import surrogate_id
        N = self.neurons
        sid, gamma, alpha = surrogate_id(self.config.surrogate_function,
                                         getattr(self.config, 'surrogate_gamma', None))
        zeros = torch.zeros(N, device=x_seq.device, dtype=torch.float32)
        nm = self.neuron_module
        y = AxonalRecdelHip.apply(
            x_seq, self.recurrent_weights.t(), None, zeros, zeros, None, 0.0, nm.tau,
            nm.v_threshold, nm.v_reset, False, self.config.detach_reset, sid, gamma, False, 0,
            alpha, getattr(nm, 'decay_input', False))
        self.x_seq = x_seq
        return y


class axonal_recdel(AxonalHipScans, MemoryModule):
    def __init__(self, config, neurons, neuron_module=LIFNode):
        super().__init__()
        self.config = config
        self.step_mode = config.step_mode
        self.store_v_seq = config.store_v_seq
        self.neuron_module = _make_neuron(config, neuron_module)
        self.neurons = neurons
        self.sigma = float(self.config.sigma_init)
        # STE on the delay discretisation: forward taps at round(d), gradient passes to d.
        self.round_delays = getattr(config, 'round_delays', False)
        self.recurrent_weights = torch.nn.Parameter(torch.zeros(neurons, neurons), requires_grad=True)
        self.recurrent_delays = torch.nn.Parameter(torch.zeros(neurons), requires_grad=True)
        self.dropout = _make_recurrent_dropout(config)
        self.use_sig_p = config.use_sig_p
        if self.use_sig_p:
            self.p_spread = torch.nn.Parameter(torch.zeros(neurons), requires_grad=True)
        self.use_rec_bias = getattr(config, 'use_rec_bias', False)
        if self.use_rec_bias:
            self.recurrent_bias = torch.nn.Parameter(torch.zeros(neurons), requires_grad=True)
        self.init_recurrent_weights()
        self.init_recurrent_delays()

    def init_recurrent_weights(self):
        init_mode = getattr(self.config, 'init_rec_weights', 'orthogonal')
        if init_mode == 'orthogonal':
            torch.nn.init.orthogonal_(self.recurrent_weights, gain=self.config.rec_delay_init_gain)
        elif init_mode == 'kaiming_uniform':
            torch.nn.init.kaiming_uniform_(self.recurrent_weights, a=5 ** 0.5)
        else:
            raise ValueError(f"Unknown init_rec_weights '{init_mode}' "
                             f"(expected 'orthogonal' or 'kaiming_uniform').")
        if getattr(self, 'use_rec_bias', False):
            bound = 1.0 / (self.recurrent_weights.shape[1] ** 0.5)
            torch.nn.init.uniform_(self.recurrent_bias, -bound, bound)

    def init_recurrent_delays(self):
        with torch.no_grad():
            mode = self.config.init_rec_delay
            if mode == 'half_normal':
                half_normal = torch.abs(torch.randn_like(self.recurrent_delays) * self.config.delay_std_init)
                self.recurrent_delays.copy_(half_normal)
                self.recurrent_delays.clamp_(min=0.0)
            elif mode == 'uniform_integer':
                maximum = self.config.hybrid_offset_scale
                if int(maximum) != maximum or maximum < 0:
                    raise ValueError('hybrid_offset_scale must be a nonnegative integer')
                self.recurrent_delays.copy_(torch.randint(
                    0, int(maximum) + 1, self.recurrent_delays.shape,
                    device=self.recurrent_delays.device))
            elif mode == 'uniform':
                torch.nn.init.uniform_(self.recurrent_delays, a=self.config.init_recdel_offset,
                                       b=self.config.max_rec_delay)
                self.recurrent_delays.clamp_(min=0.0)

    def update_sigma(self, current_epoch):
        """Anneal the spread: ``sigma = sigma_init * (sigma_decay ** (100/epochs)) ** epoch``.
        ``sigma`` is a plain attribute, not part of the ``state_dict``."""
        decay_per_epoch = self.config.sigma_decay ** (100 / self.config.epochs)
        self.sigma = self.config.sigma_init * (decay_per_epoch ** current_epoch)

    def clamp_recurrent_delays(self):
        with torch.no_grad():
            self.recurrent_delays.clamp_(min=0)

    def recurrent_dropout_mask(self, B, N, like):
        """The fixed ``(B, N)`` recurrent-dropout multiplier of this forward, or ``None``."""
        if self.training and self.config.recurrent_dropout_rate > 0:
            return self.dropout(torch.ones(B, N, device=like.device, dtype=like.dtype))
        return None

    def forward(self, x_seq):
        if self.step_mode == 's':
            raise NotImplementedError('single-step mode is not supported; use step_mode="m"')
        fv = getattr(self, 'forward_version', None)
        if fv is None:
            fv = AXONAL_CUDA_DEFAULT
        if fv in ('v1', 'v2'):
            raise NotImplementedError(_TORCH_SCANS_MSG.format(fv))
        if fv in ('eventdriven', 'eventdriven_torch'):
            raise ValueError("axonal_recdel has no event-driven kernel in this release. "
                             "Use 'triton_exact' (the default).")
        if fv in ('triton_exact', 'hip'):
            return self.multi_step_forward_triton(x_seq, approx=False)
        if fv == 'triton_approx':
            return self.multi_step_forward_triton(x_seq, approx=True)
        if fv == 'triton_ste':
            return self.multi_step_forward_triton(x_seq, ste_mode=1)
        raise ValueError(f'unknown forward_version {fv!r}')


class synaptic_recdel(SynapticHipScans, SynapticHybridScans, axonal_recdel):
    def __init__(self, config, neurons, neuron_module=LIFNode):
        super().__init__(config=config, neurons=neurons, neuron_module=neuron_module)
        # one delay d_ij per connection: (N_in, N_out)
        self.recurrent_delays = torch.nn.Parameter(torch.zeros(neurons, neurons), requires_grad=True)
        self.init_recurrent_delays()

    def forward(self, x_seq):
        if self.step_mode == 's':
            raise NotImplementedError('single-step mode is not supported; use step_mode="m"')
        fv = getattr(self, 'forward_version', None)
        if fv is None:
            if getattr(self, '_hybrid_delay', False):
                from .kernels.synaptic_hybrid import hybrid_kernel_usable
                fv = 'hybrid_triton' if hybrid_kernel_usable(self, x_seq) else SYNAPTIC_CUDA_DEFAULT
            else:
                fv = SYNAPTIC_CUDA_DEFAULT
        if fv in ('v1', 'v2'):
            raise NotImplementedError(_TORCH_SCANS_MSG.format(fv))
        if fv == 'eventdriven_torch':
            raise ValueError("the pure-PyTorch event-driven reference was removed from this "
                             "release, use 'eventdriven' (the default).")
        if fv == 'hybrid_triton':
            return self.multi_step_forward_hybrid_triton(x_seq)
        if fv in ('eventdriven', 'hip'):
            return self.multi_step_forward_eventdriven(x_seq)
        raise ValueError(f'unknown forward_version {fv!r}')


class common_recdel(axonal_recdel):
    """``axonal_recdel`` with a single learnable delay shared by all neurons of the layer
    (``recurrent_delays`` shape (1,), broadcast to (N,); its gradient is the sum)."""

    def __init__(self, config, neurons, neuron_module=LIFNode):
        super().__init__(config=config, neurons=neurons, neuron_module=neuron_module)
        self.recurrent_delays = torch.nn.Parameter(torch.zeros(1), requires_grad=True)
        self.init_recurrent_delays()
        self.forward_version = None
