"""Synaptic (per-connection) delayed-LIF layer over ``delrec_syn_fwd/bwd``.

Drop-in for ``EventDrivenSyn`` / ``eventdriven_trainable_forward`` (reference
``triton_kernels/synaptic_eventdriven.py:379-488``): ``EventDrivenSyn.apply(x, W, d,
p_spread, bias, drop, layer) -> y`` with backward ``(dx, dW, dd, dp, dbias, None, None)``.
The forward is the spike-sparse scatter scan; the backward is the dense reverse BPTT scan
followed by the lag-correlation GEMM, which folds ``dW = sum_l h * C_l`` and
``dd = W * sum_l dh/dd * C_l`` (and ``ds``) into its epilogue instead of materialising the
``(N, N, L)`` lag stack.
"""

import numpy as np
import torch

from .. import _lib
from ..spike_linear import attach_bits
from ._common import bits_shape, drop_bn, lif_struct, read_scalars, require_device, weights, window_length_f64


def _spread(layer, device):
    """Per-source half-width (``use_sig_p``) or ``None`` for the uniform ``1 + sigma``."""
    if layer.use_sig_p:
        return (1.0 + 2.0 * float(layer.sigma) * torch.sigmoid(
            layer.p_spread.detach().to(device=device, dtype=torch.float32))).contiguous()
    return None


def hybrid_form(d_min, s_uniform, off_range):
    """The hybrid's scan-form fields: ``(d_min, off_min, off_count, flags)`` for the argument
    structs and the workspace query (bit 2: every source's taps at lags >= 1, i.e.
    d_min = min_j base_j + off_min >= s - 1 in float32 as the entry point compares; bits
    16..23: the offset count); zeros when the offset range is unknown (``off_range`` None)."""
    if off_range is None:
        return 0.0, 0, 0, 0
    off_min, off_count = off_range
    d32, s32 = np.float32(d_min), np.float32(s_uniform)
    lags_ok = bool(d32 >= np.float32(s32 - np.float32(1.0)))
    return float(d32), int(off_min), int(off_count), (4 if lags_ok else 0) | (min(int(off_count), 255) << 16)


def syn_forward(x, W, d_eff, base, offsets, s_vec, s_uniform, d_all, bias, drop, lif, off_range=None):
    """Launch ``delrec_syn_fwd`` with per-connection delays ``d_eff`` (N, N), or with the
    hybrid ``base`` (N) + int8 ``offsets`` (N, N) when ``d_eff`` is None; ``d_all`` is a
    device tensor holding every effective delay (for the window length); ``off_range`` =
    (smallest offset, offset count) of the hybrid's int8 offsets. Returns
    ``(y, u, bits, L, Wc, w_bf16, s_max, hyb)`` with ``hyb`` the hybrid's scan-form fields
    (``hybrid_form``) and its first-lag counts (below 4, below 2; -1 when not hybrid) for the
    backward."""
    require_device(x)
    T, B, N = x.shape
    dev = x.device
    xc = x.detach().to(torch.float32).contiguous()
    Wc, w_bf16 = weights(W)
    y = torch.empty(T, B, N, device=dev, dtype=torch.float32)
    u = torch.empty_like(y)
    bits = torch.empty(bits_shape(T, B, N), device=dev, dtype=torch.int32)
    # the window length needs max d (and max s): the one device-to-host read of the call,
    # taken after the host work above so that it overlaps the GPU work still queued
    if s_vec is not None:
        d_max, s_max = read_scalars(d_all.max(), s_vec.max())
        d_min = d_max
    elif off_range is not None:
        # the offset-stacked and arrival forms give every source the triangle of its
        # smallest possible delay, base_j + (smallest offset): they apply when that is
        # >= s - 1 for every source, i.e. min_j base_j + off_min in fp32 (a bound of the
        # smallest delay that also covers a source without a connection at off_min)
        # The same read carries the backward's split of the sources by first lag: how many
        # start below lag 4 and below lag 2, by the entry point's own fp32 formula
        # max(1, floor(1 + (base_j + off_min) - s) + 1), so that the backward needs no read
        lof = (torch.floor((1.0 + (base + float(off_range[0]))) - float(s_uniform)) + 1.0).clamp(min=1.0)
        (d_max, d_min, n4, n2) = read_scalars(d_all.max(), base.min() + float(off_range[0]),
                                              (lof < 4).sum().float(), (lof < 2).sum().float())
        s_max = s_uniform
        near = (int(n4), int(n2))
    else:
        (d_max,), s_max = read_scalars(d_all.max()), s_uniform
        d_min = d_max
    L = max(window_length_f64(d_max, s_max), 2)
    hyb = hybrid_form(d_min, s_uniform, off_range if d_eff is None and s_vec is None else None)
    hyb = tuple(hyb) + (near if off_range is not None and s_vec is None and d_eff is None else (-1, -1))
    # the scan form follows the taps per connection: the entry point's smax (the largest
    # per-column half-width, or the uniform one)
    smax = float(s_max) if s_vec is not None else max(float(s_max), float(s_uniform))
    flags = w_bf16 | (2 if d_eff is None else 0) | (_lib.lag_taps(smax) << 8) | hyb[3]
    ws = _lib.workspace(_lib.WS_SYN_FWD, T, B, N, L, flags, dev)
    args = _lib.SynFwdArgs(
        T=T, B=B, N=N, L=L, x=_lib.ptr(xc), W=_lib.ptr(Wc), w_bf16=w_bf16, bias=_lib.ptr(bias),
        d=_lib.ptr(d_eff), base=_lib.ptr(base), offsets=_lib.ptr(offsets), s=_lib.ptr(s_vec),
        s_uniform=float(s_uniform), s_max=float(s_max), drop=_lib.ptr(drop), lif=lif, y=_lib.ptr(y),
        u=_lib.ptr(u), bits=_lib.ptr(bits), workspace=_lib.ptr(ws), workspace_bytes=ws.numel(),
        d_min=hyb[0], off_min=hyb[1], off_count=hyb[2])
    _lib.call('delrec_syn_fwd', args, _lib.stream_of(xc))
    return y, u, bits, L, Wc, w_bf16, float(s_max), hyb


def syn_backward(gy, u, y, bits, Wc, w_bf16, d_eff, base, offsets, s_vec, s_uniform, s_max, drop, lif,
                 L, need_W, need_d, need_s, need_b, hyb=(0.0, 0, 0, 0, -1, -1)):
    """Launch ``delrec_syn_bwd`` (``hyb``: the forward's hybrid scan-form fields and first-lag
    counts). Returns
    ``(dx, dW, dd, ds, db)`` (``None`` where not requested)."""
    T, B, N = u.shape
    dev = u.device
    gy = gy.to(torch.float32).contiguous()
    dx = torch.empty_like(gy)
    dW = torch.empty(N, N, device=dev, dtype=torch.float32) if need_W else None
    dd = torch.empty(N, N, device=dev, dtype=torch.float32) if need_d else None
    ds = torch.empty(N, device=dev, dtype=torch.float32) if need_s else None
    db = torch.empty(N, device=dev, dtype=torch.float32) if need_b else None
    smax = float(s_uniform) if d_eff is None else (float(s_max) if s_vec is not None
                                                   else max(float(s_max), float(s_uniform)))
    flags = w_bf16 | (2 if d_eff is None else 0) | (_lib.lag_taps(smax) << 8) | hyb[3]
    ws = _lib.workspace(_lib.WS_SYN_BWD, T, B, N, L, flags, dev)
    args = _lib.SynBwdArgs(
        T=T, B=B, N=N, L=L, gy=_lib.ptr(gy), u=_lib.ptr(u), y=_lib.ptr(y), bits=_lib.ptr(bits),
        W=_lib.ptr(Wc), w_bf16=w_bf16, d=_lib.ptr(d_eff), base=_lib.ptr(base),
        offsets=_lib.ptr(offsets), s=_lib.ptr(s_vec), s_uniform=float(s_uniform), s_max=float(s_max),
        drop=_lib.ptr(drop), lif=lif, dx=_lib.ptr(dx), dW=_lib.ptr(dW), dd=_lib.ptr(dd), ds=_lib.ptr(ds), db=_lib.ptr(db),
        workspace=_lib.ptr(ws), workspace_bytes=ws.numel(), d_min=hyb[0], off_min=hyb[1], off_count=hyb[2],
        near_known=int(len(hyb) > 5 and hyb[4] >= 0), near_lt4=max(hyb[4], 0) if len(hyb) > 5 else 0,
        near_lt2=max(hyb[5], 0) if len(hyb) > 5 else 0)
    _lib.call('delrec_syn_bwd', args, _lib.stream_of(gy))
    return dx, dW, dd, ds, db


def layer_lif(layer):
    cfg = layer.config
    return lif_struct(layer.neuron_module, cfg.surrogate_function, getattr(cfg, 'surrogate_gamma', None))


class EventDrivenSyn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, d, p_spread, bias, drop, layer):
        T, B, N = x.shape
        dev = x.device
        d_eff = (d.detach().round() if layer.round_delays else d.detach()).to(torch.float32).contiguous()
        s_vec = _spread(layer, dev)
        s_uniform = 1.0 + float(layer.sigma)
        m = drop_bn(drop, T, B, N)
        bc = None if bias is None else bias.detach().to(torch.float32).contiguous()
        lif = layer_lif(layer)
        y, u, bits, L, Wc, w_bf16, s_max, _ = syn_forward(x, W, d_eff, None, None, s_vec, s_uniform, d_eff,
                                                          bc, m, lif)
        ctx.save_for_backward(u, y, bits, Wc, d_eff, s_vec, m, p_spread)
        ctx.meta = (L, w_bf16, s_uniform, s_max, float(layer.sigma), bool(layer.use_sig_p),
                    bias is not None, W.dtype)
        ctx.lif = lif
        return attach_bits(y, bits)

    @staticmethod
    def backward(ctx, gy):
        u, y, bits, Wc, d_eff, s_vec, m, p_spread = ctx.saved_tensors
        L, w_bf16, s_uniform, s_max, sigma, use_sig_p, use_bias, w_dtype = ctx.meta
        need_p = use_sig_p and ctx.needs_input_grad[3]
        dx, dW, dd, ds, db = syn_backward(
            gy, u, y, bits, Wc, w_bf16, d_eff, None, None, s_vec, s_uniform, s_max, m, ctx.lif, L,
            ctx.needs_input_grad[1], ctx.needs_input_grad[2], need_p,
            use_bias and ctx.needs_input_grad[4])
        dp = None
        if need_p:
            with torch.enable_grad():
                p_ = p_spread.detach().to(torch.float32).requires_grad_(True)
                (dp,) = torch.autograd.grad(1.0 + 2.0 * sigma * torch.sigmoid(p_), p_, ds)
        if dW is not None and w_dtype != torch.float32:
            dW = dW.to(w_dtype)
        return dx, dW, dd, dp, db, None, None


def recurrent_drop(layer, x_seq):
    """The layer's fixed recurrent-dropout mask ``(B, N)``, or ``None`` when inactive
    (reference ``synaptic_eventdriven.py:479-483``)."""
    T, B, N = x_seq.shape
    if layer.training and getattr(layer.config, 'recurrent_dropout_rate', 0.0) > 0:
        return layer.dropout(torch.ones(B, N, device=x_seq.device, dtype=x_seq.dtype))
    return None


def eventdriven_trainable_forward(layer, x_seq):
    """Autograd-enabled synaptic forward; gradients reach ``recurrent_weights``,
    ``recurrent_delays``, ``recurrent_bias``, ``p_spread`` and ``x``."""
    T, B, N = x_seq.shape
    drop = recurrent_drop(layer, x_seq)
    bias = layer.recurrent_bias if layer.use_rec_bias else None
    p_spread = (layer.p_spread if layer.use_sig_p
                else torch.zeros(N, device=x_seq.device, dtype=x_seq.dtype))
    return EventDrivenSyn.apply(x_seq, layer.recurrent_weights, layer.recurrent_delays,
                                p_spread, bias, drop, layer)
