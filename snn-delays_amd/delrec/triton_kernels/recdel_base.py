"""Import path of the reference's ``delrec.triton_kernels.recdel_base``; resolves to ``delrec.kernels.recdel_base``."""

from ..kernels.recdel_base import *  # noqa: F401,F403
from ..kernels import recdel_base as _impl

globals().update({k: v for k, v in vars(_impl).items() if not k.startswith('__')})
