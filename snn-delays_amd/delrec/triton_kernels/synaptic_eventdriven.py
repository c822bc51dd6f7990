"""Import path of the reference's ``delrec.triton_kernels.synaptic_eventdriven``; resolves to ``delrec.kernels.synaptic_eventdriven``."""

from ..kernels.synaptic_eventdriven import *  # noqa: F401,F403
from ..kernels import synaptic_eventdriven as _impl

globals().update({k: v for k, v in vars(_impl).items() if not k.startswith('__')})
