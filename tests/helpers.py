"""Shared helpers of the parity tests: seeded inputs, oracle runs, comparisons."""

import torch

from oracle import neuron as oneuron, scans


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


def oracle_axonal(x, W, d, lif, sigma, gy, bias=None, p=None, use_sig_p=False, drop=None,
                  round_delays=False):
    """Oracle forward + BPTT. Returns (y, u, grads dict)."""
    leaves = {'x': x.clone().requires_grad_(True), 'W': W.clone().requires_grad_(True),
              'd': d.clone().requires_grad_(True)}
    if bias is not None:
        leaves['bias'] = bias.clone().requires_grad_(True)
    if p is not None:
        leaves['p'] = p.clone().requires_grad_(True)
    y, ext = scans.axonal_v2(leaves['x'], leaves['W'], leaves['d'], lif, sigma=sigma,
                             bias=leaves.get('bias'), drop=drop, p_spread=leaves.get('p'),
                             use_sig_p=use_sig_p, round_delays=round_delays)
    (y * gy).sum().backward()
    return y.detach(), ext['u'].detach(), {k: v.grad for k, v in leaves.items()}


def oracle_synaptic(x, W, d, lif, sigma, gy, bias=None, p=None, use_sig_p=False, drop=None,
                    base=None, offsets=None, round_delays=False):
    """Oracle synaptic forward + BPTT. With ``base``/``offsets`` the delay is the hybrid
    parametrisation and the gradient is reported for ``base``."""
    leaves = {'x': x.clone().requires_grad_(True), 'W': W.clone().requires_grad_(True)}
    if base is not None:
        leaves['base'] = base.clone().requires_grad_(True)
        dd = leaves['base'] + 0.0 + 1.0 * offsets
    else:
        leaves['d'] = d.clone().requires_grad_(True)
        dd = leaves['d']
    if bias is not None:
        leaves['bias'] = bias.clone().requires_grad_(True)
    if p is not None:
        leaves['p'] = p.clone().requires_grad_(True)
    y, ext = scans.synaptic_v2(leaves['x'], leaves['W'], dd, lif, sigma=sigma, bias=leaves.get('bias'),
                               drop=drop, p_spread=leaves.get('p'), use_sig_p=use_sig_p,
                               round_delays=round_delays)
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
