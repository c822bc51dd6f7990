"""Axonal delayed-LIF layer: the autograd Function over ``delrec_axonal_fwd/bwd``.

Drop-in for ``AxonalRecdelTriton`` (reference ``triton_kernels/recdel_base.py:349-439``):
same argument order and meaning, ``(x, W, bias, d, p_spread, drop, sigma, tau, v_th,
v_reset, use_sig_p, detach_reset, surr_id, gamma, approx, ste_mode, alpha)``, plus an
optional trailing ``decay_input`` (the reference routes ``decay_input=True`` to its
PyTorch scan; the HIP kernel implements that charge form). The backward returns the
gradients of ``x, W, bias, d, p_spread`` and ``None`` for the rest.

Modes (reference ``recdel_base.py:361-383``):
  exact      soft triangle taps forward and backward, ``dd`` / ``dp`` from the
             closed-form kernel derivative accumulated in the scan;
  approx     one rounded tap forward, the single-tap backward and the straight-through
             ``dd = sum gz * (y[t-lag-1] - y[t-lag])``;
  ste_mode   1: rounded tap forward, 2: two-tap interpolated forward; soft backward.

Windows of more than 256 lags (the spike history the axonal kernels hold in registers) take
the per-connection scans of the synaptic layer with every connection of source j at the
source's delay, ``d[i, j] = d[j]``: the same triangle taps and the same sums, the delay
gradient ``dd[j] = sum_i dd[i, j]``; the hard-tap modes there run the soft scan at the tap's
own delay with a half-width of 1 (``_long_window_forward``).
"""

import ctypes
import os
import threading

import torch

from .. import _lib
from ..spike_linear import attach_bits
from ._common import (bits_shape, drop_bn, read_scalars, require_device, round_half_even_f32, weights,
                      window_length_f32, window_length_f64)
from .delays import build_lag, build_lag_interp


STRAIGHT_LINE_MAX_ELEMS = 1 << 28   # (T, B, N) fp32 outputs addressed with 32-bit offsets
REGISTER_LAGS = 256                 # spike history the axonal kernels hold (lags 1 .. 256)



def _straight_line_forward(N, sigma, use_sig_p, approx, ste_mode, decay_input, v_reset, TB=1):
    """The calls the C ABI's straight-line forward takes without a window length (L = 0):
    soft taps of a uniform half-width with at most 8 lags of non-zero weight, decay charge,
    hard reset to 0, N <= 256, T * B * N <= 2^28 (each output at most 1 GiB)."""
    return (N <= 256 and TB * N <= STRAIGHT_LINE_MAX_ELEMS and not use_sig_p and not approx
            and not ste_mode and not decay_input
            and v_reset is not None and float(v_reset) == 0.0 and 0.0 <= float(sigma) <= 3.0
            and os.environ.get('DELREC_AXONAL_FWD') != 'tiled')


def deferred_read_safe(dmax_hint, sigma, margin=16.0):
    """Whether the straight-line forward may run before max d is read: a known recent max d
    (``dmax_hint``, None when unknown) leaves ``margin`` steps of the register history to
    spare. A window that jumps past it anyway still fails loudly (NaN outputs, an error in the
    backward)."""
    return dmax_hint is not None and window_length_f32(float(dmax_hint) + margin, 1.0 + float(sigma)) - 1 <= REGISTER_LAGS


# per thread: the caller's grad mode at apply() (forward() itself runs with gradients disabled,
# and ctx.needs_input_grad follows the inputs' requires_grad even under torch.no_grad()); the
# caller's max-delay hint for this call (``dmax_hint``, set by the layer); the max d the
# forward read (``last_dmax``, for the layer)
_APPLY_STATE = threading.local()


def apply_with_hint(dmax_hint, *args):
    """``AxonalRecdelHip.apply`` with a known recent max d; returns ``(y, max d read or None)``."""
    _APPLY_STATE.dmax_hint = dmax_hint
    _APPLY_STATE.last_dmax = None
    try:
        y = AxonalRecdelHip.apply(*args)
    finally:
        _APPLY_STATE.dmax_hint = None
    return y, _APPLY_STATE.last_dmax


class AxonalRecdelHip(torch.autograd.Function):
    @classmethod
    def apply(cls, *args, **kwargs):
        _APPLY_STATE.grad = torch.is_grad_enabled()
        return super().apply(*args, **kwargs)

    @staticmethod
    def forward(ctx, x, W, bias, d, p_spread, drop, sigma, tau, v_th, v_reset, use_sig_p,
                detach_reset, surr_id, gamma=1.0, approx=False, ste_mode=0, alpha=2.0,
                decay_input=False):
        require_device(x)
        T, B, N = x.shape
        dev = x.device
        xc = x.detach().to(torch.float32).contiguous()
        Wc, w_bf16 = weights(W)
        dc = d.detach().to(torch.float32).contiguous()
        sigma = float(sigma)
        s_vec = None
        if use_sig_p:
            s_vec = (1.0 + 2.0 * sigma * torch.sigmoid(p_spread.detach().to(torch.float32))).contiguous()
        m = drop_bn(drop, T, B, N)
        bc = None if bias is None else bias.detach().to(torch.float32).contiguous()
        lif = _lib.make_lif(tau, v_th, v_reset, decay_input, detach_reset, surr_id, gamma, alpha)
        y = torch.empty(T, B, N, device=dev, dtype=torch.float32)
        u = torch.empty_like(y)
        z = torch.empty_like(y)
        bits = torch.empty(bits_shape(T, B, N), device=dev, dtype=torch.int32)
        ws = _lib.workspace(_lib.WS_AXONAL_FWD, T, B, N, 2, w_bf16, dev)   # size does not depend on L
        args = _lib.AxonalFwdArgs(
            T=T, B=B, N=N, L=2, x=_lib.ptr(xc), W=_lib.ptr(Wc), w_bf16=w_bf16, bias=_lib.ptr(bc),
            d=_lib.ptr(dc), s=_lib.ptr(s_vec), s_uniform=1.0 + sigma, drop=_lib.ptr(m), taps=0,
            lif=lif, y=_lib.ptr(y), u=_lib.ptr(u), rec=None, z=_lib.ptr(z), bits=_lib.ptr(bits),
            workspace=_lib.ptr(ws), workspace_bytes=ws.numel())
        stream = _lib.stream_of(xc)

        # The straight-line forward sizes its spike history from d itself, so when gradients
        # are wanted the window length is not read here: the scan's first workgroup writes
        # max d into pinned host memory, and the backward reads it (by then it has long
        # arrived). Without gradients the read stays synchronous so that an over-long window
        # raises.
        if (getattr(_APPLY_STATE, 'grad', True) and any(ctx.needs_input_grad[:5])
                and deferred_read_safe(getattr(_APPLY_STATE, 'dmax_hint', None), sigma)
                and _straight_line_forward(N, sigma, use_sig_p, approx, ste_mode, decay_input, v_reset,
                                           T * B)):
            ticket = ctypes.c_uint32(0)
            args.L = 0
            args.taps = _lib.DELREC_TAPS_SOFT
            args.dmax_ticket = ctypes.pointer(ticket)
            _lib.call('delrec_axonal_fwd', args, stream)
            pending = _lib.PostedMax(dc, ticket.value)
            ctx.save_for_backward(u, z, bits, Wc, dc, s_vec, m, None, p_spread)
            ctx.meta = (T, B, N, pending, w_bf16, sigma, bool(use_sig_p), _lib.DELREC_BWD_SOFT, W.dtype)
            ctx.lif = lif
            return attach_bits(y, bits)

        # The window length needs max d (and max s): the one device-to-host read of the call,
        # taken after the host work above so that it overlaps the GPU work still queued.
        if use_sig_p:
            d_max, s_max = read_scalars(dc.max(), s_vec.max())
        else:
            (d_max,), s_max = read_scalars(dc.max()), 1.0 + sigma
        _APPLY_STATE.last_dmax = float(d_max)
        if window_length_f32(d_max, s_max) - 1 > REGISTER_LAGS:
            hard = 'approx' if approx and not ste_mode else ('round' if ste_mode == 1 else
                                                             'interp' if ste_mode else None)
            return _long_window_forward(ctx, x, W, d, dc, s_vec, sigma, bc, m, lif, p_spread, hard,
                                        d_max, s_max)
        lag = frac = None
        if ste_mode:
            L = window_length_f32(d_max, s_max)
            if ste_mode == 1:
                lag, taps = build_lag(dc, L), _lib.DELREC_TAPS_ROUND
            else:
                (lag, frac), taps = build_lag_interp(dc, L), _lib.DELREC_TAPS_INTERP
            approx = False
            mode = _lib.DELREC_BWD_SOFT
        elif approx:
            L = round_half_even_f32(d_max) + 2          # max(round(d)) = round(max(d))
            lag, taps, mode = build_lag(dc, L), _lib.DELREC_TAPS_ROUND, _lib.DELREC_BWD_STRAIGHT
        else:
            L = window_length_f32(d_max, s_max)
            taps, mode = _lib.DELREC_TAPS_SOFT, _lib.DELREC_BWD_SOFT
        args.L = max(L, 2)
        args.taps = taps
        if lag is not None:
            args.lag = lag.data_ptr()
        if frac is not None:
            args.frac = frac.data_ptr()
        _lib.call('delrec_axonal_fwd', args, stream)
        L = args.L

        ctx.save_for_backward(u, z, bits, Wc, dc, s_vec, m, lag, p_spread)
        ctx.meta = (T, B, N, L, w_bf16, sigma, bool(use_sig_p), mode, W.dtype)
        ctx.lif = lif
        return attach_bits(y, bits)

    @staticmethod
    def backward(ctx, gy):
        if ctx.meta[0] == 'long':
            return _long_window_backward(ctx, gy)
        u, z, bits, Wc, dc, s_vec, m, lag, p_spread = ctx.saved_tensors
        T, B, N, L, w_bf16, sigma, use_sig_p, mode, w_dtype = ctx.meta
        if isinstance(L, _lib.PostedMax):
            d_max = L.value()
            if d_max != d_max:
                # a NaN delay, or a window the forward could not hold without its length
                # (it then wrote NaN outputs)
                raise _lib.DelrecError('delrec_axonal_bwd', _lib.DELREC_ERR_WINDOW,
                                       'delay window beyond the 256 lags the forward holds, or a NaN delay')
            L = max(window_length_f32(d_max, 1.0 + sigma), 2)
        dev = u.device
        gy = gy.to(torch.float32).contiguous()
        need_W, need_b, need_d = ctx.needs_input_grad[1], ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        need_p = use_sig_p and ctx.needs_input_grad[4] and mode == _lib.DELREC_BWD_SOFT
        dx = torch.empty_like(gy)
        dW = torch.empty(N, N, device=dev, dtype=torch.float32) if need_W else None
        db = torch.empty(N, device=dev, dtype=torch.float32) if need_b else None
        dd = torch.empty(N, device=dev, dtype=torch.float32) if need_d else None
        ds = torch.empty(N, device=dev, dtype=torch.float32) if need_p else None
        ws = _lib.workspace(_lib.WS_AXONAL_BWD, T, B, N, L, w_bf16, dev)
        args = _lib.AxonalBwdArgs(
            T=T, B=B, N=N, L=L, gy=_lib.ptr(gy), u=_lib.ptr(u), bits=_lib.ptr(bits), z=_lib.ptr(z),
            W=_lib.ptr(Wc), w_bf16=w_bf16, d=_lib.ptr(dc), s=_lib.ptr(s_vec), s_uniform=1.0 + sigma,
            drop=_lib.ptr(m), mode=mode, lag=_lib.ptr(lag), lif=ctx.lif, dx=_lib.ptr(dx),
            dW=_lib.ptr(dW), db=_lib.ptr(db), dd=_lib.ptr(dd), ds=_lib.ptr(ds),
            workspace=_lib.ptr(ws), workspace_bytes=ws.numel())
        _lib.call('delrec_axonal_bwd', args, _lib.stream_of(gy))
        dp = None
        if need_p:
            with torch.enable_grad():
                p_ = p_spread.detach().to(torch.float32).requires_grad_(True)
                s_ = 1.0 + 2.0 * sigma * torch.sigmoid(p_)
                (dp,) = torch.autograd.grad(s_, p_, ds)
            dp = dp.to(p_spread.dtype)
        if dW is not None and w_dtype != torch.float32:
            dW = dW.to(w_dtype)
        return (dx, dW, db, dd, dp) + (None,) * 13


def _long_window_forward(ctx, x, W, d, dc, s_vec, sigma, bc, m, lif, p_spread, hard, d_max, s_max):
    """The axonal layer through the synaptic scans with d[i, j] = d[j] (windows beyond the
    register history).

    The hard-tap forwards are the soft scan with a half-width of 1 at a delay of the tap's
    own: weight max(0, 1 - |l - (1 + d')|) is 1 at lag l = 1 + d' for an integer d' = lag - 1
    (``approx``, ``ste_round``: the rounded tap), and 1 - frac, frac at lags floor(1 + d) and
    the next for d' = max(d, 0) (``ste_interp``: ``frac = 1 + d - lag`` is exact in fp32, so
    the weights are the reference's own; d < 0 clamps to the one tap at lag 1). The STE
    backward is the soft one at the layer's own delays and spread, except for dW, which pairs
    the gradient of rec with the hard trace the forward used; ``approx`` back-propagates
    through its one tap and takes the straight-through delay gradient
    ``dd[j] = sum_{t,b} gz[t,b,j] (y[t-lag_j-1, b, j] - y[t-lag_j, b, j])`` with
    ``gz = (dx m) W`` the gradient of the delayed trace."""
    from .synaptic_eventdriven import syn_forward
    N = x.shape[-1]
    expand = lambda v: v.unsqueeze(0).expand(N, N).contiguous()
    d_syn = expand(dc)
    if hard is None:
        d_fwd, s_fwd, s_uni = dc, s_vec, 1.0 + sigma
    else:
        if hard == 'interp':
            d_fwd = dc.clamp(min=0.0)
        else:
            L_h = round_half_even_f32(d_max) + 2 if hard == 'approx' else window_length_f32(d_max, s_max)
            d_fwd = (build_lag(dc, L_h) - 1).to(torch.float32)
        s_fwd, s_uni = None, 1.0
    y, u, bits, L, Wc, w_bf16, s_fmax, _ = syn_forward(x, W, d_syn if hard is None else expand(d_fwd), None, None,
                                                       s_fwd, s_uni, d_fwd, bc, m, lif)
    if hard is None or hard == 'approx':
        d_bwd, s_bwd, L_bwd, s_bmax = (d_syn, s_vec, L, s_fmax) if hard is None else (expand(d_fwd), None, L, 1.0)
    else:
        d_bwd, s_bwd, s_bmax = d_syn, s_vec, float(s_max)
        L_bwd = max(window_length_f64(d_max, s_max), 2)
    ctx.save_for_backward(u, y, bits, Wc, d_bwd, s_bwd, m, p_spread, None if hard is None else d_fwd)
    ctx.meta = ('long', L_bwd, w_bf16, sigma, s_bmax, W.dtype, s_vec is not None, hard)
    ctx.lif = lif
    return attach_bits(y, bits)


def _long_window_backward(ctx, gy):
    from .synaptic_eventdriven import syn_backward
    u, y, bits, Wc, d_syn, s_vec, m, p_spread, d_tap = ctx.saved_tensors
    _, L, w_bf16, sigma, s_max, w_dtype, use_sig_p, hard = ctx.meta
    approx = hard == 'approx'
    need_d = ctx.needs_input_grad[3]
    need_p = use_sig_p and ctx.needs_input_grad[4] and not approx
    s_uni = 1.0 if approx else 1.0 + sigma
    ste = hard is not None and not approx
    dx, dW, dd, ds, db = syn_backward(gy, u, y, bits, Wc, w_bf16, d_syn, None, None, None if approx else s_vec,
                                      s_uni, s_max, m, ctx.lif, L, ctx.needs_input_grad[1] and not ste,
                                      need_d and not approx, need_p, ctx.needs_input_grad[2])
    if dd is not None:
        dd = dd.sum(0)          # every connection of source j carries d[j]
    if approx and need_d:
        dd = _straight_through_dd(dx, m, Wc, y, d_tap)
    if ste and ctx.needs_input_grad[1]:
        dW = _hard_trace_dw(dx, m, y, d_tap)
    dp = None
    if need_p:
        with torch.enable_grad():
            p_ = p_spread.detach().to(torch.float32).requires_grad_(True)
            (dp,) = torch.autograd.grad(1.0 + 2.0 * sigma * torch.sigmoid(p_), p_, ds)
        dp = dp.to(p_spread.dtype)
    if dW is not None and w_dtype != torch.float32:
        dW = dW.to(w_dtype)
    return (dx, dW, db, dd, dp) + (None,) * 13


def _delayed(y, lag):
    """y[t - lag_j, b, j] (0 before the first step) for a per-source lag (N,) >= 0."""
    T, B, N = y.shape
    pad = int(lag.max())
    yp = torch.cat([torch.zeros(pad, B, N, device=y.device, dtype=y.dtype), y])
    idx = (torch.arange(T, device=y.device).view(T, 1) + pad - lag.view(1, N)).view(T, 1, N).expand(T, B, N)
    return yp.gather(0, idx)


def _straight_through_dd(dx, m, Wc, y, d_tap):
    """``approx``'s delay gradient for the long-window route (see ``_long_window_forward``):
    the gradient of the delayed trace z_j (rec_i = sum_j W_ij z_j enters the LIF input times
    the dropout mask, as x does) against the difference of the spikes one lag past the tap
    and at it."""
    T, B, N = y.shape
    g = dx if m is None else dx * m
    gz = (g.reshape(T * B, N) @ Wc.float()).view(T, B, N)
    lag = d_tap.to(torch.long) + 1
    return (gz * (_delayed(y, lag + 1) - _delayed(y, lag))).sum((0, 1))


def _hard_trace_dw(dx, m, y, d_tap):
    """The STE modes' weight gradient for the long-window route: dW[i, j] = sum_{t,b}
    gr[t,b,i] z[t,b,j] with gr = dx m the gradient of rec and z the forward's hard trace
    (the value the straight-through trace carries), z_j = (1 - frac) y[t - lag_j] +
    frac y[t - lag_j - 1] for the tap's delay d' = lag - 1 + frac (frac = 0: the rounded
    tap)."""
    T, B, N = y.shape
    g = dx if m is None else dx * m
    pos = 1.0 + d_tap
    lag = torch.floor(pos)
    frac = pos - lag
    lag = lag.to(torch.long)
    z = (1.0 - frac) * _delayed(y, lag) + frac * _delayed(y, lag + 1)
    return g.reshape(T * B, N).t() @ z.reshape(T * B, N)


# The reference's name for this Function (``delrec.triton_kernels.AxonalRecdelTriton``).
AxonalRecdelTriton = AxonalRecdelHip
