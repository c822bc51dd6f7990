"""Linear layer on spike inputs over ``delrec_spike_linear_fwd`` / ``delrec_spike_linear_dw``.

In the SNN_* stacks a ``torch.nn.Linear`` follows every recurrent layer (reference
``networks.py:140-181``: Linear -> Dropout -> recurrent layer -> spike_registrator -> the
next Linear). Its input is the layer's spike train, so its forward and its weight gradient
are binary-activation GEMMs; the recurrent layers' autograd Functions attach their spike
bits to their output (``attach_bits``), and ``SpikeLinear`` reads those bits instead of the
fp32 spikes: the forward ``out = y W^T + b`` and the weight gradient ``dW = g^T y`` both run on
the bits. The input gradient ``dy = g W`` is a plain GEMM: for GEMMs of at least 2^40 flops
(C5's inter-layer Linear: 4.4 * 10^12) one bf16 GEMM with fp32 output (torch's
``mm(..., out_dtype=float32)``) over g split into ``[hi | lo | hi]`` by
``delrec_spike_linear_dx_split`` and W stacked ``[W_hi; W_hi; W_lo]`` (about 2^-16 relative
per product, within the gradients' rtol 1e-4), where the device's torch offers that GEMM;
otherwise torch's fp32 GEMM, the reference's own (``DELREC_LINEAR_DX_SPLIT=1`` / ``=0``
takes the split GEMM at any size / never); ``db = sum g``.

The bits are used only while they still describe the tensor: ``attach_bits`` records the
tensor's version counter, and an input that was modified in place since (or any other input
without bits -- an input projection of analog data, a batch-normalised train, a CPU tensor,
or sizes past the kernels' 32-bit addressing) takes ``torch.nn.functional.linear``, the
reference's own operation.
"""

import os

import torch

from . import _lib

_LIMIT = 1 << 31   # the kernels address the spike words and W planes with 32-bit byte offsets


def attach_bits(y, bits):
    """Mark ``y`` (T, B, N) as a spike train whose bits (B, ceil(T/32), N) are ``bits``, as of
    its current version."""
    y._delrec_bits = (bits, y._version)
    return y


def spike_bits(x):
    """The spike bits attached to ``x``, or ``None`` when there are none or ``x`` was
    modified in place after they were attached."""
    tag = getattr(x, '_delrec_bits', None)
    if tag is None:
        return None
    bits, version = tag
    return bits if x._version == version else None


def bits_path_fits(T, B, K, M):
    """The 32-bit byte-offset limits of ``delrec_spike_linear_fwd`` (spike words; three bf16
    planes of W^T, K rounded up to 32 and M to 128)."""
    kp, mp = (K + 31) // 32 * 32, (M + 127) // 128 * 128
    return B * ((T + 31) // 32) * K * 4 < _LIMIT and 3 * kp * mp * 2 < _LIMIT


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
        ctx.save_for_backward(weight, bits)
        ctx.shape = (T, B, K, M)
        ctx.x_dtype = x.dtype
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, g):
        weight, bits = ctx.saved_tensors
        T, B, K, M = ctx.shape
        g = g.to(torch.float32).contiguous()
        g2 = g.reshape(-1, M)
        dx = dW = db = None
        if ctx.needs_input_grad[0]:
            dx = input_grad(g2, weight.to(torch.float32)).reshape(T, B, K).to(ctx.x_dtype)
        if ctx.needs_input_grad[1]:
            dW = spike_linear_dw(g, bits, K).to(weight.dtype)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = g2.sum(0)
        return dx, dW, db, None


_MM_OUT_DTYPE = {}


def _mm_out_dtype(device):
    """Whether torch runs a bf16 x bf16 GEMM with fp32 output on ``device`` (checked once)."""
    ok = _MM_OUT_DTYPE.get(device)
    if ok is None:
        try:
            a = torch.ones(16, 16, device=device, dtype=torch.bfloat16)
            ok = torch.mm(a, a, out_dtype=torch.float32).dtype == torch.float32
        except (RuntimeError, TypeError, NotImplementedError):
            ok = False
        _MM_OUT_DTYPE[device] = ok
    return ok


_SPLIT_FLOPS = 1 << 40


def input_grad(g2, W):
    """``dy = g2 W`` (rows, K) for g2 (rows, M) and W (M, K) fp32: at 2^40 flops or more one
    bf16 GEMM with fp32 accumulation and output over ``[g_hi | g_lo | g_hi]`` and
    ``[W_hi; W_hi; W_lo]``, else -- or where the device's torch has no fp32-output bf16 GEMM --
    the fp32 GEMM the reference's ``torch.nn.Linear`` backward runs."""
    rows, M = g2.shape
    mode = os.environ.get('DELREC_LINEAR_DX_SPLIT')
    big = 2 * rows * M * W.shape[1] >= _SPLIT_FLOPS
    if mode == '0' or (mode != '1' and not big) or not (g2.is_cuda and _mm_out_dtype(g2.device)):
        return g2 @ W
    gs = torch.empty(rows, 3 * M, device=g2.device, dtype=torch.bfloat16)
    _lib.spike_linear_dx_split(g2, gs, _lib.stream_of(g2))
    w_hi = W.to(torch.bfloat16)
    w_lo = (W - w_hi.to(torch.float32)).to(torch.bfloat16)
    return torch.mm(gs, torch.cat([w_hi, w_hi, w_lo], 0), out_dtype=torch.float32)


def spike_linear_dw(g, bits, K):
    """``dW[m, k] = sum_{t,b} g[t, b, m] y[t, b, k]`` (M, K) from the spike bits of y."""
    T, B, M = g.shape
    dW = torch.empty(M, K, device=g.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.WS_SPIKE_LINEAR_DW, T, B, K, M, 0, g.device)
    args = _lib.SpikeLinearDwArgs(T=T, B=B, K=K, M=M, bits=_lib.ptr(bits), g=_lib.ptr(g), dW=_lib.ptr(dW),
                                  workspace=_lib.ptr(ws), workspace_bytes=ws.numel())
    _lib.call('delrec_spike_linear_dw', args, _lib.stream_of(g))
    return dW


class SpikeLinear(torch.nn.Linear):
    """``torch.nn.Linear`` that runs the binary-activation GEMMs on a recurrent layer's spike
    output (same parameters, initialisation and state dict as ``torch.nn.Linear``)."""

    def forward(self, x):
        bits = spike_bits(x)
        if (bits is None or not x.is_cuda or x.dim() != 3 or self.weight.dtype != torch.float32
                or x.dtype != torch.float32 or tuple(bits.shape) != (x.shape[1], (x.shape[0] + 31) // 32, x.shape[2])
                or not bits_path_fits(x.shape[0], x.shape[1], x.shape[2], self.weight.shape[0])):
            return torch.nn.functional.linear(x, self.weight, self.bias)
        return SpikeLinearFn.apply(x, self.weight, self.bias, bits)
