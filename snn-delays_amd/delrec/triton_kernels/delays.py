"""Import path of the reference's ``delrec.triton_kernels.delays``; resolves to ``delrec.kernels.delays``."""

from ..kernels.delays import *  # noqa: F401,F403
from ..kernels import delays as _impl

globals().update({k: v for k, v in vars(_impl).items() if not k.startswith('__')})
