"""Plain multi-step LIF layer on the GPU (``delrec_lif_fwd`` / ``delrec_lif_bwd``).

The ``SNN_*`` stacks place ordinary LIF layers around the recurrent one (the
non-recurrent last layer, ``networks.py:148-160``); this runs them with the same neuron
arithmetic as the recurrent kernels. The reference's charge/fire/reset helpers are
``triton_kernels/lif.py:25-56``.
"""

import torch

from .. import _lib
from ._common import require_device


class LIFSequence(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, lif):
        require_device(x)
        x = x.detach().to(torch.float32).contiguous()
        T, B, N = x.shape
        y = torch.empty_like(x)
        u = torch.empty_like(x)
        args = _lib.LifFwdArgs(T=T, B=B, N=N, x=_lib.ptr(x), lif=lif, y=_lib.ptr(y), u=_lib.ptr(u))
        _lib.call('delrec_lif_fwd', args, _lib.stream_of(x))
        ctx.save_for_backward(u, y)
        ctx.lif = lif
        return y

    @staticmethod
    def backward(ctx, gy):
        u, y = ctx.saved_tensors
        gy = gy.to(torch.float32).contiguous()
        T, B, N = u.shape
        dx = torch.empty_like(u)
        args = _lib.LifBwdArgs(T=T, B=B, N=N, gy=_lib.ptr(gy), u=_lib.ptr(u), y=_lib.ptr(y),
                               lif=ctx.lif, dx=_lib.ptr(dx))
        _lib.call('delrec_lif_bwd', args, _lib.stream_of(gy))
        return dx, None


def lif_sequence(x_seq, node):
    from ._common import lif_struct
    lif = lif_struct(node, node.surrogate_function, getattr(node, 'surrogate_gamma', None))
    return LIFSequence.apply(x_seq, lif)
