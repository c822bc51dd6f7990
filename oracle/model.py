"""Oracle forward of a whole ``SNN_*`` stack (test infrastructure only).

``reference_forward(model, x)`` walks ``model.layers`` (the ``nn.Sequential`` the
reference's ``SNN.forward`` runs, ``networks.py:111-114``) and evaluates every module with
plain torch ops on the module's own parameters, replacing each recurrent delay layer
by the oracle scan (``scans.axonal_v2`` / ``scans.synaptic_v2``) and each plain LIF layer
by ``scans.lif_layer``. Autograd therefore lands in the same ``.grad`` fields a fused run
fills, which is how the reference's ``tests/check_hybrid_kernel.py:59-69`` compares its
``'v2'`` and fused paths. Modules are recognised by their attributes (duck typing), so
this file does not import the product.
"""

import torch

from . import scans
from .neuron import LIFParams


def lif_params_of(neuron_module, surrogate_function=None):
    """Oracle ``LIFParams`` from a product ``LIFNode`` (tau, v_threshold, v_reset,
    decay_input, detach_reset, surrogate)."""
    surr = surrogate_function if surrogate_function is not None else neuron_module.surrogate_function
    kind = getattr(surr, 'surrogate_kind', None)
    if kind is None:
        kind = 'atan' if 'atan' in type(surr).__name__.lower() else 'triangle'
    width = getattr(surr, 'alpha', 2.0) if kind == 'atan' else getattr(surr, 'gamma', 1.0)
    return LIFParams(tau=neuron_module.tau, v_threshold=neuron_module.v_threshold,
                     v_reset=neuron_module.v_reset, decay_input=neuron_module.decay_input,
                     detach_reset=neuron_module.detach_reset, surrogate=(kind, width))


def recurrent_layer_forward(layer, x, version='v2'):
    """Oracle scan of one recurrent delay layer with the layer's parameters; returns
    ``(y, extras)``."""
    lif = lif_params_of(layer.neuron_module)
    W = layer.recurrent_weights
    d = layer.recurrent_delays
    T, B, N = x.shape
    if d.dim() == 1 and d.numel() == 1 and N > 1:      # common_recdel: one shared delay
        d = d.expand(N)
    bias = layer.recurrent_bias if getattr(layer, 'use_rec_bias', False) else None
    p = layer.p_spread if getattr(layer, 'use_sig_p', False) else None
    drop = layer.recurrent_dropout_mask(B, N, x) if hasattr(layer, 'recurrent_dropout_mask') else None
    kw = dict(sigma=float(layer.sigma), bias=bias, drop=drop, p_spread=p,
              use_sig_p=bool(getattr(layer, 'use_sig_p', False)),
              round_delays=bool(getattr(layer, 'round_delays', False)))
    if d.dim() == 1:
        fn = scans.axonal_v2 if version == 'v2' else scans.axonal_v1
    else:
        fn = scans.synaptic_v2 if version == 'v2' else scans.synaptic_v1
    return fn(x, W, d, lif, **kw)


def reference_forward(model, x, version='v2'):
    """Oracle forward of an ``SNN_*`` model on ``x (T, B, C_in)``."""
    for m in model.layers:
        if hasattr(m, 'recurrent_weights') and hasattr(m, 'recurrent_delays'):
            x, _ = recurrent_layer_forward(m, x, version)
        elif hasattr(m, 'recurrent_weights'):
            raise NotImplementedError('vanilla_recurrent: use oracle.scans.vanilla directly')
        elif isinstance(m, torch.nn.Linear):
            x = torch.nn.functional.linear(x, m.weight, m.bias)
        elif hasattr(m, 'v_threshold') and hasattr(m, 'tau'):
            x, _ = scans.lif_layer(x, lif_params_of(m))
        elif type(m).__name__ == 'spike_registrator':
            pass
        elif type(m).__name__ == 'Dropout':
            if m.training and m.p > 0:
                raise NotImplementedError('oracle forward with active feedforward dropout')
        else:
            raise NotImplementedError(f'oracle forward: unsupported module {type(m).__name__}')
    return x
