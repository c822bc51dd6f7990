"""The loss end of the SNN_* stacks over ``delrec_readout_ce``: the readout Linear's output
(T, B, C) reduced over time, optionally through a non-spiking leaky integrator, then the
cross-entropy against the labels -- forward and gradient in one fused pass.

Reference forms (``src/delrec/utils.py``): ``calc_loss_SSC`` sums the readout over time,
``calc_loss_HAR`` / ``calc_loss_AL`` average it, ``calc_loss_SHD`` takes its maximum; all
then apply ``torch.nn.CrossEntropyLoss`` (mean over the batch). The SHD stack reads out the
membrane of a LIF with an unreachable threshold (``networks_shd.py:187-199``): with
``v_reset = 0`` and ``decay_input=False`` its charge is ``v = v (1 - 1/tau) + x``, with
``decay_input=True`` it is ``v = v + (x - v) / tau`` (spikingjelly ``LIFNode``).
"""

import torch

from . import _lib
from .kernels._common import require_device

_REDUCE = {'sum': _lib.READOUT_SUM, 'mean': _lib.READOUT_MEAN, 'max': _lib.READOUT_MAX}


class ReadoutCE(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, labels, reduce, tau, decay_input):
        require_device(logits, 'logits')
        T, B, C = logits.shape
        x = logits.detach().to(torch.float32).contiguous()
        lab = labels.detach().to(device=x.device, dtype=torch.int64).contiguous()
        dl = torch.empty_like(x)
        loss = torch.empty(1, device=x.device, dtype=torch.float32)
        integrator = 0 if tau is None else (2 if decay_input else 1)
        ws = _lib.workspace(_lib.WS_READOUT_CE, T, B, C, 1, 0, x.device)
        args = _lib.ReadoutCeArgs(T=T, B=B, C=C, logits=_lib.ptr(x), labels=_lib.ptr(lab), reduce=_REDUCE[reduce],
                                  integrator=integrator, tau=0.0 if tau is None else float(tau), out=None,
                                  dlogits=_lib.ptr(dl), loss=_lib.ptr(loss), workspace=_lib.ptr(ws),
                                  workspace_bytes=ws.numel())
        _lib.call('delrec_readout_ce', args, _lib.stream_of(x))
        ctx.save_for_backward(dl)
        ctx.dtype = logits.dtype
        return loss.reshape(())

    @staticmethod
    def backward(ctx, g):
        (dl,) = ctx.saved_tensors
        return (dl * g).to(ctx.dtype), None, None, None, None


def readout_ce(logits, labels, reduce='mean', tau=None, decay_input=False):
    """Cross-entropy of the readout ``logits`` (T, B, C) reduced over time by ``reduce``
    ('sum', 'mean' or 'max'), after a leaky integrator of time constant ``tau`` when given."""
    if reduce not in _REDUCE:
        raise ValueError(f'reduce must be one of {sorted(_REDUCE)}, got {reduce!r}')
    return ReadoutCE.apply(logits, labels, reduce, tau, decay_input)


def calc_loss_SSC(output, y):
    """``utils.calc_loss_SSC``: sum over time, then cross-entropy."""
    return readout_ce(output, y, 'sum')


def calc_loss_HAR(output, y):
    """``utils.calc_loss_HAR``: mean over time, then cross-entropy."""
    return readout_ce(output, y, 'mean')


calc_loss_AL = calc_loss_HAR


def calc_loss_SHD(output, y):
    """``utils.calc_loss_SHD``: maximum over time, then cross-entropy."""
    return readout_ce(output, y, 'max')
