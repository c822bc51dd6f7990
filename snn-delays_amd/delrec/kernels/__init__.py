"""HIP kernels of the delayed-LIF recurrent layer, behind the reference's operator API.

    recdel_base           axonal scan: ``AxonalRecdelHip`` (alias ``AxonalRecdelTriton``)
    synaptic_eventdriven  per-connection delays: ``EventDrivenSyn``,
                          ``eventdriven_trainable_forward``
    synaptic_hybrid       hybrid delays: ``HybridSynDelay``, ``hybrid_trainable_forward``,
                          ``hybrid_kernel_usable``, ``_delay_grad``
    delays                ``build_mask``, ``build_lag``, ``build_lag_interp``, ``build_syn_mask``
    surrogate             surrogate ids (0 = triangle, 1 = ATan)
    lif                   the plain multi-step LIF layer

The entry points mirror ``delrec.triton_kernels`` (reference
``src/delrec/triton_kernels/__init__.py:64-73``); the compute is in ``libdelrec_hip.so``.
"""

from .recdel_base import AxonalRecdelHip, AxonalRecdelTriton
from .synaptic_eventdriven import EventDrivenSyn, eventdriven_trainable_forward
from .synaptic_hybrid import HybridSynDelay, hybrid_trainable_forward, hybrid_kernel_usable, _delay_grad
from .delays import build_mask, build_lag, build_lag_interp, build_syn_mask
from .surrogate import _SURR_ID, surrogate_id
from .lif import LIFSequence

__all__ = [
    'AxonalRecdelHip', 'AxonalRecdelTriton',
    'EventDrivenSyn', 'eventdriven_trainable_forward',
    'HybridSynDelay', 'hybrid_trainable_forward', 'hybrid_kernel_usable',
    'build_mask', 'build_lag', 'build_lag_interp', 'build_syn_mask',
    'LIFSequence',
]
