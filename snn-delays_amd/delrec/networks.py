"""Model classes that stack the recurrent delay layers (reference ``src/delrec/networks.py``).

A hidden block is ``Linear -> Dropout -> neuron -> spike_registrator [-> BatchNorm]``; the
stack ends with a ``Linear`` readout. The recurrent classes kept here are the ones whose
hot path this build implements: axonal, synaptic, common, vanilla, fixed and hybrid
recurrent delays (``networks.py:140-400, 802-984, 1128-1204``). Layers are created in the
reference's order, so a seeded model draws the same initial parameters.

Feedforward-delay classes ride DCLS's convolution, not this path, and are not provided;
``dcls_module`` exists only so ``isinstance`` checks in callers keep working.
"""

import torch

from .spike_linear import SpikeLinear

from .delay_layers import axonal_recdel, synaptic_recdel, common_recdel
from .neuron import Dropout


class dcls_module(torch.nn.Module):
    """Placeholder for the reference's DCLS feedforward-delay convolution (out of scope)."""

    def __init__(self, *args, **kwargs):
        raise NotImplementedError('feedforward (DCLS) delays are not part of this build')


class spike_registrator(torch.nn.Module):
    """Pass-through that keeps a copy of the spike trains (firing-rate penalties, analyses)."""

    def __init__(self):
        super().__init__()
        self.spikes = None

    def forward(self, x):
        assert x.dim() == 3  # (T, B, N)
        self.spikes = x.clone()
        return x


def _plain_neuron(config):
    return config.neuron_module(
        tau=config.tau, decay_input=config.decay_input, v_reset=config.v_reset,
        v_threshold=config.v_threshold, surrogate_function=config.surrogate_function,
        detach_reset=config.detach_reset, step_mode=config.step_mode, backend=config.backend,
        store_v_seq=config.store_v_seq)


def _batch_norm(config, dim):
    raise NotImplementedError('use_batch_norm=True: spikingjelly BatchNorm1d is not part of this build')


class SNN(torch.nn.Module):
    def __init__(self, config):
        super().__init__()
        assert config.dataset in ['SSC', 'PSMNIST', 'HAR', 'AL', 'MG', 'MEM'], "Unsupported SNN dataset."
        self.config = config
        layers = []
        dim_buffer = config.input_size
        for layer_dim in config.hidden_layers:
            layers.append(torch.nn.Linear(dim_buffer, layer_dim, bias=config.bias))
            dim_buffer = layer_dim
            layers.append(Dropout(config.feedforward_dropout_rate, step_mode='m'))
            layers.append(_plain_neuron(config))
            layers.append(spike_registrator())
            if config.use_batch_norm:
                layers.append(_batch_norm(config, layer_dim))
        layers.append(torch.nn.Linear(dim_buffer, config.output_size, bias=config.bias))
        self.layers = torch.nn.Sequential(*layers)
        self.init_weights()

    def forward(self, x):
        assert x.dim() == 3  # (T, B, N)
        return self.layers(x)

    def init_weights(self):
        for m in self.layers:
            if isinstance(m, torch.nn.Linear):
                if self.config.init_ff_weights == 'kaiming':
                    torch.nn.init.kaiming_uniform_(m.weight, nonlinearity='relu')
                elif self.config.init_ff_weights == 'normal':
                    torch.nn.init.normal_(m.weight, mean=0.0, std=0.1)

    def log_params(self):
        logs = {}
        for idx, layer in enumerate(self.layers):
            if isinstance(layer, torch.nn.Linear):
                logs[f'w_linear_{idx}'] = torch.abs(layer.weight).mean()
                logs[f'w_linear_grad_max_{idx}'] = (layer.weight.grad.abs().max().item()
                                                    if layer.weight.grad is not None else 0.0)
        return logs


def _recurrent_stack(model, config, make_recurrent):
    layers = []
    dim_buffer = config.input_size
    for idx, layer_dim in enumerate(config.hidden_layers):
        # the Linear after a recurrent layer takes its spikes: the binary-activation GEMM
        linear = torch.nn.Linear if idx == 0 else SpikeLinear
        layers.append(linear(dim_buffer, layer_dim, bias=config.bias))
        dim_buffer = layer_dim
        layers.append(Dropout(config.feedforward_dropout_rate, step_mode='m'))
        is_last_hidden = idx == len(config.hidden_layers) - 1
        if is_last_hidden and getattr(config, 'no_recurrence_in_last_layer', False):
            layers.append(_plain_neuron(config))
        else:
            layers.append(make_recurrent(config, layer_dim, config.neuron_module))
        layers.append(spike_registrator())
        if config.use_batch_norm:
            layers.append(_batch_norm(config, layer_dim))
    layers.append(SpikeLinear(dim_buffer, config.output_size, bias=config.bias))
    model.layers = torch.nn.Sequential(*layers)
    model.init_weights()


class SNN_axonal_recurrent_delays(SNN):
    """Recurrent SNN with one learned delay per presynaptic neuron."""

    def __init__(self, config):
        super().__init__(config)
        self.config = config
        _recurrent_stack(self, config, axonal_recdel)

    def clamp_delays(self):
        for m in self.layers:
            if isinstance(m, axonal_recdel):
                m.clamp_recurrent_delays()

    def round_pos(self):
        """Project the recurrent delays onto the integer grid (nearest or stochastic)."""
        stochastic = getattr(self.config, 'round_mode', 'nearest') == 'stochastic'
        with torch.no_grad():
            for m in self.layers:
                if isinstance(m, axonal_recdel):
                    d = m.recurrent_delays
                    if stochastic:
                        d.copy_(torch.floor(d + torch.rand_like(d)))
                    else:
                        d.round_()
                    m.clamp_recurrent_delays()

    def log_params(self):
        logs = super().log_params()
        for idx, layer in enumerate(self.layers):
            if isinstance(layer, axonal_recdel):
                logs[f'sigma_rec{idx}'] = layer.sigma
                logs[f'pos_rec{idx}'] = layer.recurrent_delays.detach().cpu().numpy().mean()
                w = layer.recurrent_weights
                logs[f'recurrent_w_{idx}'] = torch.abs(w).mean()
                logs[f'recurrent_w_grad_max_{idx}'] = w.grad.abs().max().item() if w.grad is not None else 0.0
                d = layer.recurrent_delays
                logs[f'recurrent_delay_grad_max_{idx}'] = d.grad.abs().max().item() if d.grad is not None else 0.0
        return logs


class SNN_synaptic_recurrent_delays(SNN_axonal_recurrent_delays):
    """Per-connection delays (``synaptic_recdel``, ``recurrent_delays`` (N, N))."""

    def __init__(self, config):
        SNN.__init__(self, config)
        self.config = config
        _recurrent_stack(self, config, synaptic_recdel)


class SNN_common_recurrent_delays(SNN_axonal_recurrent_delays):
    """One delay shared by each recurrent layer (``common_recdel``)."""

    def __init__(self, config):
        SNN.__init__(self, config)
        self.config = config
        _recurrent_stack(self, config, common_recdel)


def _freeze_delays(layer, round_first):
    if round_first:
        with torch.no_grad():
            layer.recurrent_delays.round_()
            layer.clamp_recurrent_delays()
    layer.recurrent_delays.requires_grad = False
    layer.sigma = 0.0
    layer.config.sigma_init = 0.0
    layer.use_sig_p = False
    if hasattr(layer, 'p_spread'):
        del layer.p_spread


class SNN_vanilla_recurrent(SNN_axonal_recurrent_delays):
    """Axonal stack with every delay frozen at 0 and no spread."""

    def __init__(self, config):
        super().__init__(config)
        for layer in self.layers:
            if isinstance(layer, axonal_recdel):
                with torch.no_grad():
                    layer.recurrent_delays.fill_(0.0)
                _freeze_delays(layer, round_first=False)


class SNN_fixed_recurrent_delays(SNN_axonal_recurrent_delays):
    """Axonal delays frozen at their rounded initial values, no spread."""

    def __init__(self, config):
        super().__init__(config)
        for layer in self.layers:
            if isinstance(layer, axonal_recdel):
                _freeze_delays(layer, round_first=True)


class SNN_fixed_synaptic_recurrent_delays(SNN_synaptic_recurrent_delays):
    """Per-connection delays frozen at their rounded initial values, no spread."""

    def __init__(self, config):
        super().__init__(config)
        for layer in self.layers:
            if isinstance(layer, axonal_recdel):
                _freeze_delays(layer, round_first=True)


# ---------------------------------------------------------------- hybrid delays ---------

class _AxonalWithFixedOffsets(torch.nn.Module):
    """Parametrise a delay tensor as ``axonal + position_shift + position_sign * offsets``:
    one learned value per source plus frozen integer per-connection offsets (a buffer).
    On the recurrent path ``position_shift=0`` and ``position_sign=1``."""

    def __init__(self, offsets, position_shift=0.0, position_sign=1.0):
        super().__init__()
        self.register_buffer('offsets', offsets)
        self.position_shift = position_shift
        self.position_sign = position_sign

    def forward(self, axonal):
        assert torch.broadcast_shapes(axonal.shape, self.offsets.shape) == self.offsets.shape, (
            f'axonal {tuple(axonal.shape)} does not broadcast into offsets {tuple(self.offsets.shape)}')
        return axonal + self.position_shift + self.position_sign * self.offsets


def learned_delay_parameter(module, name):
    """The leaf parameter behind ``module.<name>``, also when it is parametrised."""
    from torch.nn.utils import parametrize
    if parametrize.is_parametrized(module, name):
        return getattr(module.parametrizations, name).original
    return getattr(module, name)


_HYBRID_OFFSET_DISTRIBUTIONS = ('uniform', 'gaussian', 'triangular')


def _hybrid_params(config):
    """Validated ``(maximum, seed, distribution, sigma)`` of the hybrid offsets."""
    maximum = getattr(config, 'hybrid_offset_scale', 4)
    if int(maximum) != maximum or maximum < 0:
        raise ValueError('hybrid_offset_scale must be a nonnegative integer')
    if config.kernel_count != 1:
        raise ValueError('hybrid delay models require kernel_count=1 (one delay per axon/synapse).')
    distribution = getattr(config, 'hybrid_offset_distribution', 'uniform')
    if distribution not in _HYBRID_OFFSET_DISTRIBUTIONS:
        raise ValueError(f'hybrid_offset_distribution must be one of {_HYBRID_OFFSET_DISTRIBUTIONS}, '
                         f'got {distribution!r}')
    sigma = getattr(config, 'hybrid_offset_sigma', None)
    if distribution == 'gaussian' and not (sigma is not None and sigma > 0):
        raise ValueError("distribution 'gaussian' requires a positive hybrid_offset_sigma")
    return int(maximum), getattr(config, 'hybrid_delay_seed', 123), distribution, sigma


def _draw_offsets(shape, maximum, generator, distribution='uniform', sigma=None):
    """Frozen integer offsets in ``[0, maximum]`` (zeros when ``maximum == 0``)."""
    if maximum == 0:
        return torch.zeros(shape)
    if distribution == 'uniform':
        return torch.randint(maximum + 1, shape, generator=generator).float()
    if distribution == 'gaussian':
        draws = torch.normal(maximum / 2.0, float(sigma), size=shape, generator=generator)
        return draws.round().clamp_(0, maximum)
    if distribution == 'triangular':
        u = torch.rand(shape, generator=generator)
        draws = torch.where(u < 0.5, maximum * torch.sqrt(u / 2.0),
                            maximum * (1.0 - torch.sqrt((1.0 - u) / 2.0)))
        return draws.round().clamp_(0, maximum)
    raise ValueError(f'Unknown distribution {distribution!r} (expected one of {_HYBRID_OFFSET_DISTRIBUTIONS}).')


def hybrid_centered_base(base, config, *, pathway):
    """Shift the base so the mean effective delay equals the base itself when
    ``config.hybrid_base_centering == 'centered'`` (recurrent: ``base - maximum/2``)."""
    if getattr(config, 'hybrid_base_centering', 'normal') != 'centered':
        return base
    half = getattr(config, 'hybrid_offset_scale', 4) / 2.0
    return base + half if pathway == 'feedforward' else base - half


def _reparametrize_recurrent_delay(module, maximum, generator, config, distribution='uniform', sigma=None):
    """Tie a ``synaptic_recdel``'s (N, N) delays to one learned (N,) base (row 0 of the
    initial delays, optionally centred) plus frozen offsets; tag it ``_hybrid_delay``."""
    from torch.nn.utils import parametrize
    offsets = _draw_offsets(module.recurrent_delays.shape, maximum, generator, distribution, sigma)
    base = hybrid_centered_base(module.recurrent_delays[0].detach().clone(), config, pathway='recurrent')
    parametrize.register_parametrization(module, 'recurrent_delays', _AxonalWithFixedOffsets(offsets),
                                         unsafe=True)
    module.parametrizations.recurrent_delays.original = torch.nn.Parameter(base)
    module._hybrid_delay = True
    module.forward_version = None


class SNN_recurrent_hybrid_delays(SNN_axonal_recurrent_delays):
    """Recurrent hybrid delays: ``d(i, j) = d_j + delta_ij`` with one learned axonal delay
    per source and frozen integer per-connection offsets. ``hybrid_offset_scale == 0`` is
    exactly ``SNN_axonal_recurrent_delays``."""

    def __init__(self, config):
        maximum, seed, distribution, sigma = _hybrid_params(config)
        self._hybrid_max = maximum
        if maximum == 0:
            super().__init__(config)
            return
        SNN_synaptic_recurrent_delays.__init__(self, config)
        generator = torch.Generator().manual_seed(seed)
        for module in self.layers:
            if isinstance(module, axonal_recdel):
                _reparametrize_recurrent_delay(module, maximum, generator, config, distribution, sigma)

    def clamp_delays(self):
        if self._hybrid_max == 0:
            return super().clamp_delays()
        with torch.no_grad():
            for module in self.layers:
                if isinstance(module, axonal_recdel):
                    learned_delay_parameter(module, 'recurrent_delays').clamp_(min=0)

    def round_pos(self):
        if self._hybrid_max == 0:
            return super().round_pos()
        with torch.no_grad():
            for module in self.layers:
                if isinstance(module, axonal_recdel):
                    learned_delay_parameter(module, 'recurrent_delays').round_()
        self.clamp_delays()


class SNN_fixed_hybrid_recurrent_delays(SNN_recurrent_hybrid_delays):
    """Hybrid delays with the rounded base frozen at initialisation; weights train."""

    def __init__(self, config):
        super().__init__(config)
        self.round_pos()
        for layer in self.layers:
            if isinstance(layer, axonal_recdel):
                learned_delay_parameter(layer, 'recurrent_delays').requires_grad_(False)
                layer.sigma = 0.0
                layer.config.sigma_init = 0.0
                layer.use_sig_p = False
                if hasattr(layer, 'p_spread'):
                    del layer.p_spread
