"""Triangular delay kernel and its derivatives, restated for the oracle (test infrastructure).

Eq. 7 of the paper as the reference states it (``delay_layers_pytorch.py:143-151``,
``:200-218``; ``triton_kernels/delays.py:13-63``):

    s          = 1 + sigma                 (or per source 1 + 2*sigma*sigmoid(p) with use_sig_p)
    L          = ceil(1 + max d + max s) + 1
    h[.., l]   = max(0, s - |l - (1 + d)|) / s^2      for l = 0 .. L-1   (l = 0 is never used)

The delay gradient of a per-connection kernel, in closed form (``synaptic_hybrid.py:93-113``):

    dd[i,j] = W[i,j] * sum_{l>=1} C[i,j,l] * sign(l-1-d) * [ |l-1-d| <= s ] / s^2

(sign(0) = 0 and an inclusive support edge: the subgradients torch's ``abs`` and
``clamp(min=0)`` take). Pinned by the known-answer inputs of
``tests/check_hybrid_kernel.py:143-152`` with hand-computed expected values, and against
autograd through ``syn_mask`` (tests/test_oracle_math.py).
"""

import math

import torch


def spread(sigma, p_spread=None, use_sig_p=False, *, dtype=torch.float32, device=None):
    """Half-width ``s`` of the triangle: a 0-d tensor, or a per-source ``(N,)`` tensor
    under ``use_sig_p``. Returns ``(s, s_max_float)``."""
    if use_sig_p:
        s = 1.0 + 2.0 * float(sigma) * torch.sigmoid(p_spread.to(dtype))
        return s, float(s.detach().max())
    s = torch.tensor(1.0 + float(sigma), dtype=dtype, device=device)
    return s, float(s)


def window_length(d_max, s_max):
    """``L = ceil(1 + max d + max s) + 1``, evaluated in fp32 like the reference's
    ``torch.ceil`` on an fp32 tensor (``delay_layers_pytorch.py:145``)."""
    v = torch.tensor(1.0, dtype=torch.float32) + torch.tensor(float(d_max), dtype=torch.float32) \
        + torch.tensor(float(s_max), dtype=torch.float32)
    return int(torch.ceil(v).item()) + 1


def axonal_mask(d, sigma, p_spread=None, use_sig_p=False):
    """``(N, L)`` triangular kernel for per-source delays ``d (N,)`` and ``L``.
    Differentiable in ``d`` and ``p_spread``."""
    s, s_max = spread(sigma, p_spread, use_sig_p, dtype=d.dtype, device=d.device)
    L = window_length(float(d.detach().max()), s_max)
    lags = torch.arange(L, dtype=d.dtype, device=d.device)
    if use_sig_p:
        s = s[:, None]
    mask = torch.clamp(s - torch.abs(lags[None, :] - (1.0 + d)[:, None]), min=0.0) / (s * s)
    return mask, L


def syn_mask(d, sigma, p_spread=None, use_sig_p=False):
    """``(N_in, N_out, L)`` triangular kernel for per-connection delays ``d (N, N)``
    (receiver i, source j); the half-width is indexed by the source under use_sig_p."""
    s, s_max = spread(sigma, p_spread, use_sig_p, dtype=d.dtype, device=d.device)
    L = window_length(float(d.detach().max()), s_max)
    lags = torch.arange(L, dtype=d.dtype, device=d.device)
    if use_sig_p:
        s = s.view(1, -1, 1)
    mask = torch.clamp(s - torch.abs(lags.view(1, 1, L) - (1.0 + d)[:, :, None]), min=0.0) / (s * s)
    return mask, L


def dmask_dd(d, sigma, L):
    """Closed-form ``d h / d d`` on lags ``0..L-1`` for a uniform half-width:
    ``sign(l-1-d) * [|l-1-d| <= s] / s^2``."""
    s = 1.0 + float(sigma)
    a = torch.arange(L, dtype=d.dtype, device=d.device).view(*([1] * d.dim()), L) - 1.0 - d.unsqueeze(-1)
    return torch.sign(a) * (a.abs() <= s).to(d.dtype) / (s * s)


def delay_grad_closed_form(C, W, d, sigma):
    """``dd[i,j] = W[i,j] * sum_{l>=1} C[i,j,l] * dh/dd(l; d_ij)``; ``C`` is the
    ``(N, N, Lm)`` lag-correlation stack (lag 0 ignored, as ``range(1, Lm)`` in the
    reference's kernel)."""
    Lm = C.shape[-1]
    g = dmask_dd(d, sigma, Lm)
    g[..., 0] = 0.0
    return W * (C * g).sum(-1)


def hybrid_delays(base, offsets):
    """Effective hybrid delays ``d[i,j] = base[j] + 0.0 + 1.0 * offsets[i,j]``, the
    recurrent parametrisation ``_AxonalWithFixedOffsets.forward`` (``networks.py:823-829``)
    with ``position_shift=0`` and ``position_sign=1``."""
    return base + 0.0 + 1.0 * offsets


def draw_offsets(shape, maximum, generator):
    """Frozen integer offsets uniform on ``{0..maximum}`` as ``networks.py:873-895`` draws
    them (``randint(maximum + 1)`` from a seeded generator); zeros when ``maximum == 0``."""
    if maximum == 0:
        return torch.zeros(shape)
    return torch.randint(maximum + 1, shape, generator=generator).float()


def taps_range(d, s):
    """Integer lags ``l >= 1`` with a non-zero triangle weight for delay ``d`` and
    half-width ``s`` (python floats): ``|l - 1 - d| < s``."""
    lo = max(1, math.floor(1.0 + d - s) + 1)
    hi = math.ceil(1.0 + d + s) - 1
    return lo, hi
