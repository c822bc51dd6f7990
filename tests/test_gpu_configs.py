"""GPU parity at the shapes of the benchmark workloads (bench.py WORKLOADS C1..C5), through
the product modules the benchmark times, against the CPU oracle.

C1 and C2 run whole. C3, C4 and C5 keep the workload's N, delays, half-width and W dtype
(so the dispatcher picks the kernels the benchmark times) and shorten the run: T long
enough for the longest delays to arrive; C4 keeps B = 256 (its GEMM splits follow B), C5
takes 32 batch rows (its kernels are per row or tile the batch). Each shape runs its step
twice, and the second must reproduce the first bit for bit (spikes, membrane, every gradient).

The oracle runs teacher-forced with the kernel's spike train (``oracle.neuron.lif_step``):
it then follows the kernel's trajectory exactly, so every spike of every step can be
checked against the oracle's membrane -- a kernel spike must equal ``u >= threshold`` of
the oracle except at units whose oracle membrane lies within 1e-5 of the threshold (a
different fp32 summation order may move them across). Membranes and every gradient are
compared with the tolerance of the workload's weight type, unscaled: fp32 W rtol 1e-4,
atol 1e-5; bf16 W rtol 2e-2, atol 1e-5. The upstream gradient is N(0, 1).

The oracle runs in float64 on the same (fp32 / bf16) values: a weight gradient here sums
10^4 products, and the fp32 v2 scan's own rounding of such a sum reaches about 1e-5, the
size of the atol, so the fp32 oracle is itself only an fp32 approximation of the value both
computations aim at; the float64 run is that value to about 1e-12. An element that misses
the tolerance against the float64 oracle gets a floor of its own (``helpers.check_elementwise``):
the larger of the fp32 oracle's distance from float64 at that element and, for dW, the
rounding budget of that element's own terms (4 * eps * sqrt(sum of its squared terms), eps
the stated per-term error of the kernel's operand split) -- never a whole-tensor figure, so a
dropped term, a wrong index or sign still lands far outside. The counts are printed.
"""

import pytest
import torch

import bench
from helpers import check_elementwise, dw_term_sq_axonal, dw_term_sq_synaptic, gen, grad_eps, lif_params
from oracle import scans
from oracle.delays import axonal_mask, syn_mask

CASES = [
    # workload, T (None: the workload's), B (None: the workload's)
    ('C1', None, None),
    ('C2', None, None),
    ('C3', 64, None),
    ('C4', 56, None),
    ('C5', 80, 32),
]

THRESHOLD_BAND = 1e-5


def _tolerance(w):
    return (2e-2, 1e-5) if w['w_bf16'] else (1e-4, 1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize('case', CASES, ids=[c[0] for c in CASES])
def test_workload_shape_matches_oracle(dev, case, monkeypatch):
    name, T, B = case
    w = bench.WORKLOADS[name]
    print(f'workload {name} T={T or w["T"]} B={B or w["B"]} N={w["N"]}', flush=True)
    m = bench.build(w, dev, T=T, B=B)
    layer = m.layers[0]
    x = m.x
    T, B, N = x.shape
    gy = torch.randn(T, B, N, generator=gen(77))

    # the product path (the module the benchmark times); the synaptic / hybrid forward
    # launcher is wrapped to keep the membrane it returns
    from delrec.kernels import synaptic_eventdriven, synaptic_hybrid
    seen = {}

    def keep(fwd):
        def run(*a, **k):
            out = fwd(*a, **k)
            seen['u'] = out[1].detach()
            return out
        return run

    monkeypatch.setattr(synaptic_hybrid, 'syn_forward', keep(synaptic_hybrid.syn_forward))
    monkeypatch.setattr(synaptic_eventdriven, 'syn_forward', keep(synaptic_eventdriven.syn_forward))
    xg = x.detach().clone().requires_grad_(True)
    layer.zero_grad(set_to_none=True)
    y = layer(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    y_hip = y.detach().cpu()
    assert bool(((y_hip == 0) | (y_hip == 1)).all()), 'spikes are not 0/1'
    print(f'  firing rate {float(y_hip.mean()):.4f}', flush=True)

    # the same step once more: spikes, membrane and every gradient bit-identical (the kernels
    # add their partial sums in a fixed order; no floating-point atomics)
    first = {n: q.grad.detach().clone() for n, q in layer.named_parameters() if q.grad is not None}
    first['x'], u1 = xg.grad.detach().clone(), seen.get('u')
    u1 = None if u1 is None else u1.clone()
    xg2 = x.detach().clone().requires_grad_(True)
    layer.zero_grad(set_to_none=True)
    y2 = layer(xg2)
    (y2 * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    again = {n: q.grad for n, q in layer.named_parameters() if q.grad is not None}
    again['x'] = xg2.grad
    assert torch.equal(y2.detach().cpu(), y_hip), 'spikes differ between two identical steps'
    assert u1 is None or torch.equal(seen['u'], u1), 'membranes differ between two identical steps'
    assert sorted(again) == sorted(first)
    for n in first:
        assert torch.equal(again[n], first[n]), f'{n} gradient differs between two identical steps'
    print(f'  a second identical step: bit-identical ({", ".join(sorted(first))})', flush=True)
    if w['kind'] == 'axonal':
        # the C++ Function keeps its membrane to itself: the same scan through the Python
        # Function, whose saved tensors start with it
        from delrec import _lib
        monkeypatch.setattr(_lib, 'torch_ext', lambda: None)
        y2 = layer(x.detach().clone().requires_grad_(True))
        torch.cuda.synchronize()
        assert torch.equal(y2.detach().cpu(), y_hip), 'the two axonal entry paths differ'
        seen['u'] = y2.grad_fn.saved_tensors[0].detach()
    u_hip = seen['u'].cpu()

    # the oracle on the same parameters, teacher-forced with the kernel's spikes
    lif = lif_params(tau=w['tau'])
    f64 = torch.float64
    W = layer.recurrent_weights.detach().cpu().to(f64)
    leaves = {'x': x.detach().cpu().to(f64).requires_grad_(True), 'W': W.clone().requires_grad_(True)}
    if w['kind'] == 'hybrid':
        par = layer.parametrizations.recurrent_delays
        leaves['base'] = par.original.detach().cpu().to(f64).requires_grad_(True)
        # the parametrisation's fp32 sum, then exact in float64
        d32 = par.original.detach().cpu() + 0.0 + 1.0 * par[0].offsets.detach().float().cpu()
        d = leaves['base'] + (d32.to(f64) - leaves['base'].detach())
        hip_grads = {'base': par.original.grad}
        fn = scans.synaptic_v2
    else:
        leaves['d'] = layer.recurrent_delays.detach().cpu().to(f64).requires_grad_(True)
        d = leaves['d']
        hip_grads = {'d': layer.recurrent_delays.grad}
        fn = scans.axonal_v2 if w['kind'] == 'axonal' else scans.synaptic_v2
    hip_grads.update({'x': xg.grad, 'W': layer.recurrent_weights.grad})
    y_ref, ext = fn(leaves['x'], leaves['W'], d, lif, sigma=w['sigma'], forced=y_hip.to(f64))
    (y_ref * gy.to(f64)).sum().backward()
    u_ref = ext['u'].detach()

    # every spike against the oracle's membrane on the kernel's trajectory
    gap = (u_ref - lif.v_threshold).abs()
    fired = u_ref >= lif.v_threshold
    wrong = (fired != (y_hip != 0)) & (gap >= THRESHOLD_BAND)
    print(f'  oracle min |u - threshold| = {float(gap.min()):.3e}; units within {THRESHOLD_BAND:g}: '
          f'{int((gap < THRESHOLD_BAND).sum())}; spikes that differ from the oracle membrane: '
          f'{int((fired != (y_hip != 0)).sum())}', flush=True)
    assert not bool(wrong.any()), (
        f'{int(wrong.sum())} spikes differ away from the threshold band; first at t='
        f'{int(wrong.any(dim=(1, 2)).nonzero()[0])}')

    rtol, atol = _tolerance(w)
    key = 'base' if w['kind'] == 'hybrid' else 'd'
    checks = [('u', u_hip, u_ref, None), ('dx', hip_grads['x'], leaves['x'].grad, 'x'),
              ('dW', hip_grads['W'], leaves['W'].grad, 'W'), ('d' + key, hip_grads[key], leaves[key].grad, key)]
    ref32 = {}

    def oracle32():
        """The same teacher-forced oracle in fp32: membrane and gradients, by leaf name."""
        if not ref32:
            l32 = {k: v.detach().float().requires_grad_(True) for k, v in leaves.items()}
            if w['kind'] == 'hybrid':
                d_ = l32['base'] + (d32 - l32['base'].detach())
            else:
                d_ = l32['d']
            y32, ext32 = fn(l32['x'], l32['W'], d_, lif, sigma=w['sigma'], forced=y_hip.float())
            (y32 * gy).sum().backward()
            ref32['u'] = ext32['u'].detach()
            ref32.update({k: v.grad for k, v in l32.items()})
        return ref32

    def term_sq(idx):
        """Q of the missing dW elements, from the float64 run's gr (= dx: no dropout) and
        the kernel's spike train."""
        gr = leaves['x'].grad
        if w['kind'] == 'axonal':
            h, _ = axonal_mask(d.detach(), w['sigma'])
            return dw_term_sq_axonal(gr, y_hip, h, idx)
        h, _ = syn_mask(d.detach(), w['sigma'])
        return dw_term_sq_synaptic(gr, y_hip, h, idx)

    for name, got, ref, leaf in checks:
        check_elementwise(name, got, ref, rtol, atol,
                          ref32=lambda leaf=leaf: oracle32()['u' if leaf is None else leaf],
                          term_sq=term_sq if leaf == 'W' else None, eps=grad_eps(w['w_bf16']))
