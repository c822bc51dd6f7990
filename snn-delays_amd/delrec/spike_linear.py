"""Linear layer on spike inputs over ``delrec_spike_linear_fwd``.

In the SNN_* stacks a ``torch.nn.Linear`` follows every recurrent layer (reference
``networks.py:140-181``: Linear -> Dropout -> recurrent layer -> spike_registrator -> the
next Linear). Its input is the layer's spike train, so its forward is a binary-activation
GEMM; the recurrent layers' autograd Functions attach their spike bits to their output
(``_delrec_bits``), and ``SpikeLinear`` reads those bits instead of the fp32 spikes. Any
other input (no bits attached -- an input projection of analog data, a batch-normalised
train, a CPU tensor) takes ``torch.nn.functional.linear``, the reference's own operation.
The backward is two plain GEMMs (``dx = g W``, ``dW = g^T x``) and ``db = sum g``.
"""

import torch

from . import _lib


def attach_bits(y, bits):
    """Mark ``y`` (T, B, N) as a spike train whose bits (B, ceil(T/32), N) are ``bits``."""
    y._delrec_bits = bits
    return y


class SpikeLinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, bits):
        T, B, K = x.shape
        M = weight.shape[0]
        W = weight.detach().to(torch.float32).contiguous()
        b = None if bias is None else bias.detach().to(torch.float32).contiguous()
        out = torch.empty(T, B, M, device=x.device, dtype=torch.float32)
        ws = _lib.workspace(_lib.WS_SPIKE_LINEAR, T, B, K, M, 0, x.device)
        args = _lib.SpikeLinearArgs(T=T, B=B, K=K, M=M, bits=_lib.ptr(bits), W=_lib.ptr(W), bias=_lib.ptr(b),
                                    out=_lib.ptr(out), workspace=_lib.ptr(ws), workspace_bytes=ws.numel())
        _lib.call('delrec_spike_linear_fwd', args, _lib.stream_of(x))
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        g2 = g.reshape(-1, g.shape[-1])
        dx = dW = db = None
        if ctx.needs_input_grad[0]:
            dx = (g2 @ weight.to(g2.dtype)).reshape(x.shape)
        if ctx.needs_input_grad[1]:
            dW = (g2.t() @ x.reshape(-1, x.shape[-1]).to(g2.dtype)).to(weight.dtype)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = g2.sum(0)
        return dx, dW, db, None


class SpikeLinear(torch.nn.Linear):
    """``torch.nn.Linear`` that runs the binary-activation GEMM on a recurrent layer's spike
    output (same parameters, initialisation and state dict as ``torch.nn.Linear``)."""

    def forward(self, x):
        bits = getattr(x, '_delrec_bits', None)
        if (bits is None or not x.is_cuda or x.dim() != 3 or self.weight.dtype != torch.float32
                or x.dtype != torch.float32 or tuple(bits.shape) != (x.shape[1], (x.shape[0] + 31) // 32, x.shape[2])):
            return torch.nn.functional.linear(x, self.weight, self.bias)
        return SpikeLinearFn.apply(x, self.weight, self.bias, bits)
