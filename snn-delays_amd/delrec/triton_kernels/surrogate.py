"""Import path of the reference's ``delrec.triton_kernels.surrogate``; resolves to ``delrec.kernels.surrogate``."""

from ..kernels.surrogate import *  # noqa: F401,F403
from ..kernels import surrogate as _impl

globals().update({k: v for k, v in vars(_impl).items() if not k.startswith('__')})
