"""Hybrid recurrent delays ``d[i,j] = base[j] + offsets[i,j]`` over ``delrec_syn_fwd/bwd``.

Drop-in for ``HybridSynDelay`` / ``hybrid_trainable_forward`` / ``hybrid_kernel_usable`` /
``_delay_grad`` (reference ``triton_kernels/synaptic_hybrid.py``):
``HybridSynDelay.apply(x, W, d, bias, drop, layer) -> y`` with backward
``(dx, dW, dd, dbias, None, None)``, where ``d`` is the materialised ``(N, N)`` delay and
its gradient reaches the learned ``(N,)`` base through the module's parametrisation.

When the layer carries the hybrid parametrisation (``_AxonalWithFixedOffsets``) and the
delays are not STE-rounded, the kernels read the delay as ``base[j] + int8 offset[i,j]``
(5 bytes per connection less traffic than a float tensor) and compute the same fp32 sum
the parametrisation does. Otherwise the materialised ``d`` is used.
"""

import os

import torch

from .. import _lib
from ..spike_linear import attach_bits
from ._common import drop_bn, require_device
from .synaptic_eventdriven import layer_lif, recurrent_drop, syn_backward, syn_forward


def hybrid_kernel_usable(layer, x_seq):
    """Host-side gate of the dedicated hybrid path (reference ``synaptic_hybrid.py:49-58``);
    ``decay_input`` is supported by the HIP kernels, ``use_sig_p`` is not part of the
    hybrid Function's signature (it has no ``p_spread``)."""
    return (x_seq.is_cuda
            and not os.environ.get('DELREC_DISABLE_HYBRID_KERNEL')
            and not getattr(layer, 'use_sig_p', False))


def _int8_offsets(layer):
    """``(base, int8 offsets, (smallest offset, offset count))`` read from the hybrid
    parametrisation, or ``(None, None, None)``. The offsets are frozen: their int8 copy and
    range are computed once per tensor version."""
    from torch.nn.utils import parametrize
    if layer.round_delays or not parametrize.is_parametrized(layer, 'recurrent_delays'):
        return None, None, None
    plist = layer.parametrizations.recurrent_delays
    if len(plist) != 1:
        return None, None, None
    par = plist[0]
    if not hasattr(par, 'offsets') or getattr(par, 'position_shift', 0.0) != 0.0 \
            or getattr(par, 'position_sign', 1.0) != 1.0:
        return None, None, None
    off = par.offsets
    cache = getattr(layer, '_delrec_off8', None)
    key = (off.data_ptr(), off._version, off.device)
    if cache is None or cache[0] != key:
        ok = bool(((off == off.round()) & (off >= -128) & (off <= 127)).all())
        off8 = off.detach().to(torch.int8).contiguous() if ok else None
        rng = None
        if off8 is not None:
            lo, hi = (int(v) for v in torch.stack([off8.min(), off8.max()]).tolist())
            rng = (lo, hi - lo + 1)
        cache = (key, off8, rng)
        layer._delrec_off8 = cache
    if cache[1] is None:
        return None, None, None
    base = plist.original
    if base.dim() != 1:
        return None, None, None
    return base.detach().to(torch.float32).contiguous(), cache[1], cache[2]


class HybridSynDelay(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, d, bias, drop, layer):
        assert not layer.use_sig_p, "hybrid kernel: use_sig_p not supported"
        require_device(x)
        T, B, N = x.shape
        d_det = d.detach()
        d_eff = (d_det.round() if layer.round_delays else d_det).to(torch.float32).contiguous()
        base, off8, off_range = _int8_offsets(layer)
        s = 1.0 + float(layer.sigma)
        m = drop_bn(drop, T, B, N)
        bc = None if bias is None else bias.detach().to(torch.float32).contiguous()
        lif = layer_lif(layer)
        d_arg = None if base is not None else d_eff
        y, u, bits, L, Wc, w_bf16, _, hyb = syn_forward(x, W, d_arg, base, off8, None, s, d_eff, bc, m, lif,
                                                        off_range=off_range)
        ctx.save_for_backward(u, y, bits, Wc, d_arg, base, off8, m)
        ctx.meta = (L, w_bf16, s, bias is not None, W.dtype, hyb)
        ctx.lif = lif
        return attach_bits(y, bits)

    @staticmethod
    def backward(ctx, gy):
        u, y, bits, Wc, d_arg, base, off8, m = ctx.saved_tensors
        L, w_bf16, s, use_bias, w_dtype, hyb = ctx.meta
        dx, dW, dd, _, db = syn_backward(
            gy, u, y, bits, Wc, w_bf16, d_arg, base, off8, None, s, s, m, ctx.lif, L,
            ctx.needs_input_grad[1], ctx.needs_input_grad[2], False,
            use_bias and ctx.needs_input_grad[3], hyb=hyb)
        if dW is not None and w_dtype != torch.float32:
            dW = dW.to(w_dtype)
        return dx, dW, dd, db, None, None


def _delay_grad(Cstack, W, d_eff, sigma, Lm):
    """``dd[i,o] = W[i,o] * sum_{l=1}^{Lm-1} Cstack[i,o,l] * sign(l-1-d)[|l-1-d| <= s] / s^2``
    on the GPU (the reference's closed-form test hook, ``synaptic_hybrid.py:116-126``)."""
    require_device(W, 'W')
    N = W.shape[0]
    C = Cstack.detach().to(torch.float32).contiguous()
    Wc = W.detach().to(torch.float32).contiguous()
    dc = d_eff.detach().to(torch.float32).contiguous()
    out = torch.empty(N, N, device=W.device, dtype=torch.float32)
    _lib.delay_grad(C, Wc, dc, float(sigma), N, int(Lm), out, _lib.stream_of(Wc))
    return out


_ANNOUNCED = set()


def hybrid_trainable_forward(layer, x_seq):
    """Autograd-enabled hybrid forward; gradients reach ``recurrent_weights``, the learned
    delay base (through the parametrisation), ``recurrent_bias`` and ``x``."""
    T, B, N = x_seq.shape
    if N not in _ANNOUNCED:
        _ANNOUNCED.add(N)
        print(f'[delrec] hybrid recurrent delay: HIP kernel active (N={N}, T={T}, B={B})', flush=True)
    drop = recurrent_drop(layer, x_seq)
    bias = layer.recurrent_bias if layer.use_rec_bias else None
    y = HybridSynDelay.apply(x_seq, layer.recurrent_weights, layer.recurrent_delays, bias, drop, layer)
    layer.x_seq = x_seq
    layer.rec_now_seq = None
    if layer.store_v_seq:
        layer.v_seq = None
    return y
