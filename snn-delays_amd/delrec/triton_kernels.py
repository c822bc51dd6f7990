"""The reference's import path ``delrec.triton_kernels`` (public names:
``src/delrec/triton_kernels/__init__.py:64-73``). There is no Triton in this build: the name
is a second name of ``delrec.kernels``, the HIP implementation, submodules included, so that
``from delrec.triton_kernels.synaptic_hybrid import HybridSynDelay`` and the like resolve to
the same objects."""

import sys

from . import kernels as _kernels
from .kernels import delays, recdel_base, surrogate, synaptic_eventdriven, synaptic_hybrid  # noqa: F401

for _name in ('delays', 'recdel_base', 'surrogate', 'synaptic_eventdriven', 'synaptic_hybrid'):
    sys.modules[f'{__name__}.{_name}'] = getattr(_kernels, _name)
sys.modules[__name__] = _kernels
