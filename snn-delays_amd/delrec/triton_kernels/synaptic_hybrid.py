"""Import path of the reference's ``delrec.triton_kernels.synaptic_hybrid``; resolves to ``delrec.kernels.synaptic_hybrid``."""

from ..kernels.synaptic_hybrid import *  # noqa: F401,F403
from ..kernels import synaptic_hybrid as _impl

globals().update({k: v for k, v in vars(_impl).items() if not k.startswith('__')})
