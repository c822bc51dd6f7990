"""Import path kept for callers of the reference's ``delrec.triton_kernels`` package.

There is no Triton in this build: every name resolves to the HIP implementation in
``delrec.kernels`` (the reference's list of public names is
``src/delrec/triton_kernels/__init__.py:64-73``).
"""

from ..kernels import *  # noqa: F401,F403
from ..kernels import (AxonalRecdelTriton, EventDrivenSyn, eventdriven_trainable_forward,  # noqa: F401
                       HybridSynDelay, hybrid_trainable_forward, hybrid_kernel_usable,
                       build_mask, build_lag, build_lag_interp, build_syn_mask, _SURR_ID)
from . import delays, synaptic_hybrid, synaptic_eventdriven, recdel_base, surrogate  # noqa: F401,E402
