"""Delay-kernel and tap builders (reference ``triton_kernels/delays.py``).

The HIP kernels evaluate the triangular weights on the fly and never materialise a mask;
these host functions keep the reference's public helpers (``build_mask``, ``build_lag``,
``build_lag_interp``, ``build_syn_mask``) for callers and checks that use them, and
produce the hard lags of the rounded / interpolated forward modes.
"""

import torch

from ._common import window_length_f32


def _spread(sigma, p_spread, use_sig_p, like):
    if use_sig_p:
        s = 1.0 + 2.0 * sigma * torch.sigmoid(p_spread).to(device=like.device, dtype=like.dtype)
        return s, float(s.detach().max())
    s = torch.tensor(1.0 + float(sigma), device=like.device, dtype=like.dtype)
    return s, float(s)


def build_mask(d, sigma, p_spread, use_sig_p):
    """``(N, L)`` triangular kernel ``max(0, s - |l - (1 + d)|)/s^2`` and ``L``;
    differentiable in ``d`` and ``p_spread``."""
    s, s_max = _spread(sigma, p_spread, use_sig_p, d)
    L = window_length_f32(float(d.detach().max()), s_max)
    lags = torch.arange(L, device=d.device, dtype=d.dtype)
    if use_sig_p:
        s = s.unsqueeze(1)
    return torch.clamp(s - torch.abs(lags[None, :] - (1.0 + d)[:, None]), min=0.0) / (s * s), L


def build_lag(d, L):
    """Integer tap of the rounded forward: ``round(d) + 1`` clamped to ``[1, L-1]``."""
    return (torch.round(d).long() + 1).clamp_(1, max(1, L - 1)).to(torch.int32)


def build_lag_interp(d, L):
    """Two-tap interpolated forward: lower lag ``floor(1 + d)`` clamped to ``[1, L-1]`` and
    the weight of the next lag, ``clamp(1 + d - lag, 0, 1)``."""
    pos = 1.0 + d
    lag = torch.floor(pos).long().clamp_(1, max(1, L - 1))
    frac = (pos - lag.to(d.dtype)).clamp_(0.0, 1.0)
    return lag.to(torch.int32), frac.to(torch.float32)


def build_syn_mask(d, sigma, p_spread, use_sig_p):
    """``(N_in, N_out, L)`` per-connection triangular kernel and ``L`` (half-width indexed
    by the source under ``use_sig_p``)."""
    s, s_max = _spread(sigma, p_spread, use_sig_p, d)
    L = window_length_f32(float(d.detach().max()), s_max)
    lags = torch.arange(L, device=d.device, dtype=d.dtype)
    if use_sig_p:
        s = s.view(1, -1, 1)
    return torch.clamp(s - torch.abs(lags.view(1, 1, L) - (1.0 + d)[:, :, None]), min=0.0) / (s * s), L
