"""Shared helpers of the parity tests: seeded inputs, oracle runs, comparisons."""

import torch

from oracle import neuron as oneuron, scans
from oracle.delays import axonal_mask, dmask_dd, syn_mask


def gen(seed):
    return torch.Generator().manual_seed(seed)


def first_flip(y_hip, y_ref, u_ref, v_th, tol=1e-5):
    """Index of the first time step whose spikes differ, or None.

    A flip is allowed only at a unit whose oracle membrane lies within ``tol`` of the
    threshold (a different fp32 reduction order can move it across); everything after
    that step may legitimately diverge.
    """
    diff = (y_hip != y_ref)
    if not bool(diff.any()):
        return None
    t = int(diff.any(dim=(1, 2)).nonzero()[0])
    near = (u_ref[t] - v_th).abs() < tol
    bad = diff[t] & ~near
    assert not bool(bad.any()), (
        f'spike mismatch at t={t} for units away from threshold: '
        f'min |u-th| there = {float((u_ref[t] - v_th).abs()[diff[t]].min()):.3e}')
    return t


def max_err(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    abs_err = (a - b).abs().max().item()
    rel = ((a - b).abs() / (b.abs() + 1e-6)).max().item()
    return abs_err, rel


def assert_close(actual, expected, rtol, atol, name):
    a, e = actual.detach().float().cpu(), expected.detach().float().cpu()
    ae, re = max_err(a, e)
    print(f'  {name}: max abs err {ae:.3e}, max rel err {re:.3e}, |ref|max {e.abs().max().item():.3e}')
    torch.testing.assert_close(a, e, rtol=rtol, atol=atol, msg=lambda m: f'{name}: {m}')


def lif_params(tau=2.0, v_th=1.0, v_reset=0.0, decay_input=False, detach_reset=False,
               surrogate=('atan', 2.0)):
    return oneuron.LIFParams(tau=tau, v_threshold=v_th, v_reset=v_reset, decay_input=decay_input,
                             detach_reset=detach_reset, surrogate=surrogate)


def _cast(t, dtype):
    return t if t is None or dtype is None else t.detach().cpu().to(dtype)


def oracle_axonal(x, W, d, lif, sigma, gy, bias=None, p=None, use_sig_p=False, drop=None,
                  round_delays=False, dtype=None, forced=None):
    """Oracle forward + BPTT. Returns (y, u, grads dict). ``dtype``: every tensor cast to it
    first (float64: the reference the device gradients are held to); ``forced``: the spike
    train the neurons are teacher-forced with (``oracle.neuron.lif_step``)."""
    x, W, d, gy, bias, p, drop, forced = (_cast(t, dtype) for t in (x, W, d, gy, bias, p, drop, forced))
    leaves = {'x': x.clone().requires_grad_(True), 'W': W.clone().requires_grad_(True),
              'd': d.clone().requires_grad_(True)}
    if bias is not None:
        leaves['bias'] = bias.clone().requires_grad_(True)
    if p is not None:
        leaves['p'] = p.clone().requires_grad_(True)
    y, ext = scans.axonal_v2(leaves['x'], leaves['W'], leaves['d'], lif, sigma=sigma,
                             bias=leaves.get('bias'), drop=drop, p_spread=leaves.get('p'),
                             use_sig_p=use_sig_p, round_delays=round_delays, forced=forced)
    (y * gy).sum().backward()
    return y.detach(), ext['u'].detach(), {k: v.grad for k, v in leaves.items()}


def oracle_synaptic(x, W, d, lif, sigma, gy, bias=None, p=None, use_sig_p=False, drop=None,
                    base=None, offsets=None, round_delays=False, dtype=None, forced=None):
    """Oracle synaptic forward + BPTT. With ``base``/``offsets`` the delay is the hybrid
    parametrisation and the gradient is reported for ``base``. ``dtype`` / ``forced``: as in
    ``oracle_axonal``; a hybrid delay is the parametrisation's fp32 sum ``base + offsets``
    in every dtype (exact in float64), its gradient flowing to ``base``."""
    d32 = None if base is None else base.detach().cpu().float() + 0.0 + 1.0 * offsets.detach().cpu().float()
    x, W, d, gy, bias, p, drop, base, forced = (_cast(t, dtype)
                                                for t in (x, W, d, gy, bias, p, drop, base, forced))
    leaves = {'x': x.clone().requires_grad_(True), 'W': W.clone().requires_grad_(True)}
    if base is not None:
        leaves['base'] = base.clone().requires_grad_(True)
        if dtype is None or dtype == torch.float32:
            dd = leaves['base'] + 0.0 + 1.0 * offsets
        else:
            dd = leaves['base'] + (d32.to(dtype) - leaves['base'].detach())
    else:
        leaves['d'] = d.clone().requires_grad_(True)
        dd = leaves['d']
    if bias is not None:
        leaves['bias'] = bias.clone().requires_grad_(True)
    if p is not None:
        leaves['p'] = p.clone().requires_grad_(True)
    y, ext = scans.synaptic_v2(leaves['x'], leaves['W'], dd, lif, sigma=sigma, bias=leaves.get('bias'),
                               drop=drop, p_spread=leaves.get('p'), use_sig_p=use_sig_p,
                               round_delays=round_delays, forced=forced)
    (y * gy).sum().backward()
    return y.detach(), ext['u'].detach(), {k: v.grad for k, v in leaves.items()}


class OracleModel(torch.nn.Module):
    """An ``SNN_*`` model evaluated by the oracle (``oracle.model.reference_forward``) on
    its own parameters, so a training harness can step it like the HIP model: the
    optimiser sees the wrapped model's parameters, ``clamp_delays`` reaches them, and the
    input is cast to the parameters' dtype (float64 runs)."""

    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def forward(self, x):
        from oracle.model import reference_forward
        return reference_forward(self.inner, x.to(next(self.inner.parameters()).dtype))

    def clamp_delays(self):
        self.inner.clamp_delays()


# Per-element error budget of a weight gradient, beyond the fixed rtol / atol: an fp32 (or
# split-bf16) computation of dW[i, j] = sum_k term_k carries rounding of each term's operands
# and of the accumulation. Modelled as independent relative errors of at most EPS per term,
# the error of the sum has a standard deviation of about EPS * sqrt(Q) / sqrt(3) with
# Q = sum_k term_k^2 -- a per-element figure from that element's own terms. KAPPA * EPS *
# sqrt(Q) with KAPPA = 4 is about 7 standard deviations; a dropped term or a wrong index gives
# an error of the size of a whole term, about sqrt(Q / n) for n terms, which is
# 1 / (KAPPA EPS sqrt(n)) > 50 times that budget for every n below 10^6 at EPS = 2^-15.
#   EPS = 2^-15 for bf16 W: the backward takes gr as two bf16 planes (2^-16 per term) in the
#         future-gradient product and again in the lag correlation behind dW;
#   EPS = 2^-20 for fp32 W: three bf16 planes (2^-24) plus gr's own deviation from float64
#         after an fp32 BPTT chain (about 1e-6 relative).
#   EPS = 2^-15 for the lag- and offset-stacked per-step product scans with fp32 W (taken where
#         the rings do not fit LDS): as for bf16 W, gr enters their future-gradient products and
#         the correlation behind dW as hi + lo bf16 planes, hi*hi + hi*lo + lo*hi (about 2^-16
#         per term each time), and W.h as two planes (2^-17).
# The same budget bounds a delay gradient's element, dd[i, j] = W[i, j] sum_l dh/dd C_l[i, j]
# (dbase[j]: the sum over the column's receivers i), from its own terms.
GRAD_KAPPA = 4.0
STACKED_EPS = 2.0 ** -15


def grad_eps(w_bf16):
    return 2.0 ** -15 if w_bf16 else 2.0 ** -20


def dw_term_sq_synaptic(gr, y, h, idx):
    """Q[i, j] = sum_l h[i, j, l]^2 sum_{t >= l, b} gr[t, b, i]^2 y[t - l, b, j] for the
    (i, j) pairs ``idx`` (two index tensors): the squared terms of a synaptic / hybrid
    dW = sum_l h * C_l, C_l = sum gr(t) y(t - l)^T (spikes are 0 / 1). ``h``: (N, N, L)."""
    ii, jj = idx
    g2 = gr[:, :, ii].double() ** 2            # (T, B, m)
    yy = y[:, :, jj].double()                  # (T, B, m)
    T, L = g2.shape[0], h.shape[-1]
    q = torch.zeros(ii.numel(), dtype=torch.float64)
    for l in range(1, min(L, T)):
        c = (g2[l:] * yy[:T - l]).sum(dim=(0, 1))
        q += h[ii, jj, l].double() ** 2 * c
    return q


def dw_term_sq_axonal(gr, y, h, idx):
    """Q[i, j] = sum_{t, b} gr[t, b, i]^2 z[t, b, j]^2 with the delayed trace
    z[t, b, j] = sum_l h[j, l] y[t - l, b, j] (``h``: (N, L)) for the pairs ``idx``."""
    ii, jj = idx
    T, L = y.shape[0], h.shape[-1]
    yy = y[:, :, jj].double()
    z = torch.zeros_like(yy)
    for l in range(1, min(L, T)):
        z[l:] += h[jj, l].double() * yy[:T - l]
    return ((gr[:, :, ii].double() ** 2) * z ** 2).sum(dim=(0, 1))


def check_elementwise(name, got, ref64, rtol, atol, ref32=None, term_sq=None, eps=None):
    """``|got - ref64| <= atol + rtol |ref64| + floor`` per element. Where the fixed
    tolerance alone is missed, the element's floor is the larger of: the fp32 oracle's own
    distance from float64 at that element (``ref32``: a callable returning that tensor; an
    fp32 computation is not held closer than the fp32 restatement gets there), and, for a
    weight gradient, ``GRAD_KAPPA * eps * sqrt(Q)`` from that element's own terms
    (``term_sq``: a callable of the missing elements' index tuple returning Q). Prints the
    counts; asserts."""
    got = got.detach().double().cpu()
    ref = ref64.detach().double().cpu()
    err = (got - ref).abs()
    bound = atol + rtol * ref.abs()
    miss = err > bound
    n_miss = int(miss.sum())
    fl32 = flq = 0.0
    if n_miss:
        idx = miss.nonzero(as_tuple=True)
        floor = torch.zeros(n_miss, dtype=torch.float64)
        if ref32 is not None:
            d32 = (ref32().detach().double().cpu() - ref)[idx].abs()
            floor = torch.maximum(floor, d32)
            fl32 = float(d32.max())
        if term_sq is not None:
            fq = GRAD_KAPPA * eps * term_sq(idx).sqrt()
            floor = torch.maximum(floor, fq)
            flq = float(fq.max())
        ok = err[idx] <= bound[idx] + floor
        still = int((~ok).sum())
    else:
        still = 0
    print(f'  {name}: max abs err {float(err.max()):.3e}, |ref|max {float(ref.abs().max()):.3e}; '
          f'{n_miss} of {err.numel()} elements past rtol {rtol:g} / atol {atol:g}; per-element floors up '
          f'to {fl32:.3e} (fp32 oracle) / {flq:.3e} (term budget); {still} past their floor', flush=True)
    if still:
        ok_all = torch.ones_like(miss)
        ok_all[idx] = ok
        worst = int((err - bound).masked_fill(ok_all, -1.0).argmax())
        at = tuple(int(i) for i in torch.unravel_index(torch.tensor(worst), ref.shape))
        raise AssertionError(f'{name}: {still} of {err.numel()} elements differ; at {at}: got '
                             f'{float(got.reshape(-1)[worst]):.6e} ref {float(ref.reshape(-1)[worst]):.6e}')


def grads64(run, leaves, gy, forced):
    """The oracle's gradients in float64 on the fp32 leaves' values, teacher-forced with the
    device's spike train ``forced``: ``run(l, forced)`` is the oracle forward on the leaves
    ``l`` (name -> float64 tensor) returning y. Returns name -> gradient."""
    l64 = {k: v.detach().cpu().double().requires_grad_(True) for k, v in leaves.items()}
    y = run(l64, forced.detach().cpu().double())
    (y * gy.detach().cpu().double()).sum().backward()
    return {k: v.grad for k, v in l64.items()}


def check_grads(got, g64, g32, rtol, atol=1e-5, budget=None, eps=None):
    """Each device gradient in ``got`` (name -> tensor) against the float64 oracle's
    (``g64``) at the fixed, unscaled ``rtol`` / ``atol``. An element that misses them gets the
    floor of ``check_elementwise``: the fp32 oracle's (``g32``) own distance from float64 at
    that element and, for a name in ``budget`` (name -> ``term_sq`` callable), the rounding
    budget of that element's own terms at ``eps`` per term."""
    budget = budget or {}
    for k, v in got.items():
        check_elementwise('d' + k, v, g64[k], rtol, atol, ref32=lambda k=k: g32[k],
                          term_sq=budget.get(k), eps=eps)


def syn_budget(gr, y, d, sigma, W=None, drop=None, hybrid=False):
    """``term_sq`` callables of a synaptic / hybrid run with one uniform spread: 'W' always and,
    with ``W`` given, the delay gradient -- 'd' per connection, or 'base' (``hybrid``) per
    source. ``gr``: the float64 oracle's dx; ``y``: the spike train; ``d``: the (N, N) delays;
    ``drop``: the (B, N) dropout multiplier the recurrent input is scaled by."""
    gr = gr.detach().cpu().double()
    if drop is not None:
        gr = gr * drop.detach().cpu().double()[None]
    y = y.detach().cpu()
    d = d.detach().cpu().float()
    h, L = syn_mask(d, sigma)
    out = {'W': lambda idx: dw_term_sq_synaptic(gr, y, h, idx)}
    if W is not None:
        dh = dmask_dd(d.double(), sigma, L)
        g2, yy, T = gr ** 2, y.double(), y.shape[0]
        qd = torch.zeros(d.shape, dtype=torch.float64)
        for l in range(1, min(L, T)):
            qd += dh[:, :, l] ** 2 * torch.einsum('tbi,tbj->ij', g2[l:], yy[:T - l])
        qd *= W.detach().cpu().double() ** 2
        if hybrid:
            qb = qd.sum(0)
            out['base'] = lambda idx: qb[idx[0]]
        else:
            out['d'] = lambda idx: qd[idx]
    return out


def axonal_budget(gr, y, d, sigma):
    """``term_sq`` of an axonal dW (no dropout, one spread); ``d`` the (N,) delays."""
    h, _ = axonal_mask(d.detach().cpu().float(), sigma)
    y = y.detach().cpu()
    return {'W': lambda idx: dw_term_sq_axonal(gr, y, h, idx)}


def gemm_term_sq(A, B):
    """``term_sq`` of a product C = A @ B: Q[i, j] = sum_k (A[i, k] B[k, j])^2 for the pairs
    ``idx``, in chunks of 256 pairs."""
    A2, B2 = A.detach().cpu().double() ** 2, B.detach().cpu().double() ** 2

    def q(idx):
        ii, jj = idx
        return torch.cat([(A2[ii[s:s + 256]] * B2[:, jj[s:s + 256]].t()).sum(1)
                          for s in range(0, ii.numel(), 256)])
    return q
