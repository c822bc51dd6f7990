"""Pure-PyTorch recurrent delay scans, restated for the oracle (test infrastructure only).

Functional forms of the reference's scans; every tensor argument is explicit so the tests
can run them on copies of a layer's parameters and differentiate with autograd (BPTT):

  axonal_v2     ``AxonalTorchScans.multi_step_forward_v2``  (delay_layers_pytorch.py:121-194)
  axonal_v1     ``AxonalTorchScans.multi_step_forward_v1``  (delay_layers_pytorch.py:53-119)
  synaptic_v2   ``SynapticTorchScans.multi_step_forward_v2`` (delay_layers_pytorch.py:271-325)
  synaptic_v1   ``SynapticTorchScans.multi_step_forward_v1`` (delay_layers_pytorch.py:220-269)
  vanilla       ``VanillaTorchScans.multi_step_forward``     (delay_layers_pytorch.py:18-47)

Conventions (time-major ``(T, B, N)``; ``W[i, j]`` is the weight from source j to receiver
i): a spike of j at step t reaches i at t + l with weight ``h(l; d)`` for lags
``l = 1 .. L-1``; the recurrent input of step t is ``rec = W z (+ bias)`` where
``z[j] = sum_l h[j, l] y[t-l, j]`` (axonal) or ``rec[i] = sum_j sum_l W[i,j] h[i,j,l] y[t-l, j]``
(synaptic); the neuron input is ``x[t] + drop * rec``. The sliding window keeps the
last ``L-1`` spike vectors oldest-first and pairs them with the lag-reversed kernel, the
same layout the reference uses (kept alike so the fp32 reduction order is the same).

Each function returns ``(y, extras)`` with ``extras = {'u': pre-reset membranes,
'rec': recurrent inputs before dropout, 'L': window length}``.
Pinned by: the closed-form delay semantics and triangle weights, W = 0 closed forms,
v1 == v2, hybrid(offsets=0) == axonal, broadcast synaptic == axonal, integer-offset time
shift, an independent hand-written scalar BPTT (tests/test_oracle_*.py), and hand-derived
golden vectors (tests/golden/, written by tests/golden/make_fixtures.py from closed forms;
nothing of the reference is run).
"""

import torch

from .delays import axonal_mask, syn_mask
from .neuron import lif_initial_v, lif_step


def _ste_round(d, round_delays):
    return d + (d.round() - d).detach() if round_delays else d


def _drop(drop, B, N, like):
    return torch.ones(B, N, dtype=like.dtype, device=like.device) if drop is None else drop


def hard_lags(d, L, taps):
    """Per-source integer lag (and interpolation weight) of the reference's hard-tap
    forwards (``triton_kernels/delays.py:32-44``): ``approx`` / ``ste_round``:
    lag = clamp(round(d) + 1, 1, L - 1) (round half to even, as ``torch.round``);
    ``ste_interp``: lag = clamp(floor(1 + d), 1, L - 1), frac = clamp(1 + d - lag, 0, 1)."""
    d = d.detach()
    if taps in ('approx', 'ste_round'):
        return (torch.round(d).long() + 1).clamp(1, max(1, L - 1)), None
    pos = 1.0 + d
    lag = torch.floor(pos).long().clamp(1, max(1, L - 1))
    return lag, (pos - lag.to(d.dtype)).clamp(0.0, 1.0)


def axonal_v2(x, W, d, lif, sigma=0.0, bias=None, drop=None, p_spread=None,
              use_sig_p=False, round_delays=False, forced=None, taps='soft'):
    """Dense sliding-window axonal scan. ``drop`` is the fixed ``(B, N)`` recurrent
    dropout multiplier (ones when off), applied to ``rec`` (after the bias). ``forced``: an
    optional ``(T, B, N)`` spike train the neurons are teacher-forced with (``lif_step``).

    ``taps`` selects the reference fused kernel's forward modes (``recdel_base.py:55-99,
    361-383``): ``soft`` the triangle over every lag; ``approx`` one rounded tap
    z = y(t - lag) with the window of ``round(max d) + 2`` lags, its single-tap backward
    and the straight-through delay gradient dz/dd = y(t - lag - 1) - y(t - lag)
    (``recdel_base.py:219-224, 266-285``), no spread gradient; ``ste_round`` / ``ste_interp``
    the rounded tap or the two-tap interpolation (1 - frac) y(t - lag) + frac y(t - lag - 1)
    in the forward with the soft triangle's gradients in the backward
    (``recdel_base.py:363-378``)."""
    T, B, N = x.shape
    assert taps in ('soft', 'approx', 'ste_round', 'ste_interp'), taps
    d = _ste_round(d.to(x.dtype), round_delays)
    mask, L = axonal_mask(d, sigma, p_spread, use_sig_p)        # (N, L)
    lag = frac = None
    if taps == 'approx':
        L = int(torch.round(d.detach()).max().item()) + 2
    if taps != 'soft':
        # the hard taps read their own history of lags 1 .. Lh (the reference kernel loads
        # y(t - lag - 1) from the whole spike tensor, one lag past its window)
        lag, frac = hard_lags(d, L, taps)
        Lh = int(lag.max()) + 1
        hist = torch.zeros(B, N, Lh, dtype=x.dtype, device=x.device)       # oldest .. newest
        idx0 = (Lh - lag).view(1, N, 1).expand(B, N, 1)      # slot of y(t - lag)
        idx1 = idx0 - 1                                      # slot of y(t - lag - 1)
    m = _drop(drop, B, N, x)
    v = lif_initial_v(lif, x[0])
    ys, us, recs = [], [], []
    if L >= 2:
        k_rev = mask[:, 1:L].flip(-1).unsqueeze(0) if taps != 'approx' else None   # lag L-1 .. 1
        window = torch.zeros(B, N, L - 1, dtype=x.dtype, device=x.device)          # oldest .. newest
    for t in range(T):
        if L >= 2:
            if taps == 'soft':
                z = (k_rev * window).sum(-1)                      # (B, N)
            else:
                y0 = hist.gather(-1, idx0).squeeze(-1)
                y1 = hist.gather(-1, idx1).squeeze(-1)
                if taps == 'approx':
                    z = y0 + (d - d.detach()) * (y1 - y0).detach()
                else:
                    hard = y0 if taps == 'ste_round' else (1.0 - frac) * y0 + frac * y1
                    soft = (k_rev * window).sum(-1)
                    z = soft + (hard - soft).detach()
            rec = torch.matmul(W.unsqueeze(0), z.unsqueeze(-1)).squeeze(-1)
        else:
            rec = torch.zeros(B, N, dtype=x.dtype, device=x.device)
        if bias is not None:
            rec = rec + bias
        recs.append(rec)
        y, h, v = lif_step(lif, x[t] + rec * m, v, None if forced is None else forced[t])
        if L >= 2:
            window = torch.cat([window[..., 1:], y.unsqueeze(-1)], dim=-1)
            if taps != 'soft':
                hist = torch.cat([hist[..., 1:], y.unsqueeze(-1)], dim=-1)
        ys.append(y)
        us.append(h)
    return torch.stack(ys), {'u': torch.stack(us), 'rec': torch.stack(recs), 'L': L}


def synaptic_v2(x, W, d, lif, sigma=0.0, bias=None, drop=None, p_spread=None,
                use_sig_p=False, round_delays=False, forced=None):
    """Dense sliding-window synaptic scan: one ``B x N(L-1)`` by ``N(L-1) x N`` product per
    step against the lag-reversed ``W * h`` stack. Hybrid delays are passed materialised,
    ``d = base[None, :] + offsets``. ``forced``: as in ``axonal_v2``."""
    T, B, N = x.shape
    d = _ste_round(d.to(x.dtype), round_delays)
    mask, L = syn_mask(d, sigma, p_spread, use_sig_p)           # (N, N, L)
    m = _drop(drop, B, N, x)
    v = lif_initial_v(lif, x[0])
    ys, us, recs = [], [], []
    if L >= 2:
        wk = (W.unsqueeze(-1) * mask)[..., 1:L].flip(-1).reshape(N, N * (L - 1))
        window = torch.zeros(B, N, L - 1, dtype=x.dtype, device=x.device)
    for t in range(T):
        if L >= 2:
            rec = window.reshape(B, N * (L - 1)) @ wk.t()
        else:
            rec = torch.zeros(B, N, dtype=x.dtype, device=x.device)
        if bias is not None:
            rec = rec + bias
        recs.append(rec)
        y, h, v = lif_step(lif, x[t] + rec * m, v, None if forced is None else forced[t])
        if L >= 2:
            window = torch.cat([window[..., 1:], y.unsqueeze(-1)], dim=-1)
        ys.append(y)
        us.append(h)
    return torch.stack(ys), {'u': torch.stack(us), 'rec': torch.stack(recs), 'L': L}


def _ring_scan(x, lif, bias, drop, L, emit):
    """Circular-buffer scan shared by the v1 forms: ``emit(y) -> (B, N, L)`` is the
    contribution of the spikes of this step to the next ``L-1`` steps (lag 1..L-1)."""
    T, B, N = x.shape
    m = _drop(drop, B, N, x)
    ring = torch.zeros(B, N, L, dtype=x.dtype, device=x.device)
    ptr = 0
    v = lif_initial_v(lif, x[0])
    ys, us = [], []
    for t in range(T):
        rec = ring[:, :, ptr]
        if bias is not None:
            rec = rec + bias
        y, h, v = lif_step(lif, x[t] + rec * m, v)
        contrib = emit(y)
        ring = ring.clone()
        ring[:, :, ptr] = 0.0
        ptr = (ptr + 1) % L
        for l in range(1, L):
            slot = (ptr + l - 1) % L
            ring[:, :, slot] = ring[:, :, slot] + contrib[:, :, l]
        ys.append(y)
        us.append(h)
    return torch.stack(ys), {'u': torch.stack(us), 'L': L}


def axonal_v1(x, W, d, lif, sigma=0.0, bias=None, drop=None, p_spread=None,
              use_sig_p=False, round_delays=False):
    """Circular-buffer axonal scan (the paper's Algorithm 1)."""
    d = _ste_round(d.to(x.dtype), round_delays)
    mask, L = axonal_mask(d, sigma, p_spread, use_sig_p)
    return _ring_scan(x, lif, bias, drop, L,
                      lambda y: torch.matmul(W.unsqueeze(0), y.unsqueeze(2) * mask.unsqueeze(0)))


def synaptic_v1(x, W, d, lif, sigma=0.0, bias=None, drop=None, p_spread=None,
                use_sig_p=False, round_delays=False):
    """Circular-buffer synaptic scan."""
    d = _ste_round(d.to(x.dtype), round_delays)
    mask, L = syn_mask(d, sigma, p_spread, use_sig_p)
    return _ring_scan(x, lif, bias, drop, L,
                      lambda y: torch.einsum('bo,io,iol->bil', y, W, mask))


def vanilla(x, W, lif, drop=None, forced=None):
    """Delay-free recurrent LIF: ``rec[t] = y[t-1] W`` (note the product order of the
    reference, ``delay_layers_pytorch.py:34``). ``forced``: as in ``axonal_v2``."""
    T, B, N = x.shape
    m = _drop(drop, B, N, x)
    v = lif_initial_v(lif, x[0])
    ys, us = [], []
    prev = torch.zeros(B, N, dtype=x.dtype, device=x.device)
    for t in range(T):
        rec = torch.matmul(prev * m, W)
        y, h, v = lif_step(lif, x[t] + rec, v, None if forced is None else forced[t])
        prev = y
        ys.append(y)
        us.append(h)
    return torch.stack(ys), {'u': torch.stack(us)}


def lif_layer(x, lif, forced=None):
    """A plain multi-step LIF layer (no recurrence). ``forced``: as in ``axonal_v2``."""
    v = lif_initial_v(lif, x[0])
    ys, us = [], []
    for t in range(x.shape[0]):
        y, h, v = lif_step(lif, x[t], v, None if forced is None else forced[t])
        ys.append(y)
        us.append(h)
    return torch.stack(ys), {'u': torch.stack(us)}
