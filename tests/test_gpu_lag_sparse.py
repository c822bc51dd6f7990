"""GPU parity of the event-driven lag correlation (``lag_win_sp_kernel``, csrc/lagmm.hip): the
weight- and delay-gradient correlation for bf16 W when the batch fills 64-row chunks and the
dense grid has at least 4096 workgroups (forced here with DELREC_LAG_SPARSE=1). Spike
columns are ordered by class on the device -- silent (no products), sparse (at most two spikes
in any group of four batch rows: the exact compressed operand of the 4:2 sparse MFMA), dense
(the dense MFMA on 0/1 spikes) -- and put back by lag_finish.

Against the dense form (``DELREC_LAG_SPARSE=0``) on the same layer and inputs: dx identical
(the correlation does not touch it), dbase equal up to the order of fp32 sums (both forms are
exact in their bf16 operands: rtol 1e-5, atol 1e-6, unscaled), dW (returned in bf16) within one
bf16 rounding (rtol 2^-7, atol 1e-6; an element whose terms cancel gets the fp32 accumulation
budget of its own terms, ``helpers.check_elementwise``). Cases: the 6-,
8- and 10-lag passes, a 13-lag tile range (two 6-lag passes), three taps (sigma 0.5), rows
past B in the last chunk, a third of the neurons held silent, and firing rates up to ~30 %
where groups hold more than two spikes (the count is printed and required to be non-zero).
One case also against the oracle run in float64, teacher-forced with the device's spikes
(bf16 W: rtol 2e-2, atol 1e-5, with the per-element floors of ``helpers.check_grads``).
"""

import pytest
import torch

from helpers import (check_elementwise, check_grads, first_flip, gen, grad_eps, lif_params, oracle_synaptic,
                     syn_budget)
from test_gpu_synaptic import hybrid_layer

CASES = [
    # T, B, N, base range, max offset, sigma, input gain, oracle, silent third
    (40, 64, 200, (0.0, 20.0), 4, 0.0, 1.2, True, True),     # 6 lags per column
    (40, 128, 130, (0.0, 20.0), 6, 0.0, 3.0, False, False),  # 8 lags, high firing, two chunks
    (33, 100, 96, (0.0, 15.0), 8, 0.0, 2.0, False, True),    # 10 lags, rows 100 .. 127 padding
    (36, 64, 150, (0.0, 20.0), 11, 0.0, 2.5, False, False),  # 13 lags: two 6-lag passes
    (30, 64, 120, (1.0, 20.0), 4, 0.5, 2.0, False, True),    # three taps (8 lags)
    (24, 64, 600, (0.0, 30.0), 4, 0.0, 0.8, False, True),    # 10 column tiles, low firing
]


def _grads(layer, x, gy):
    layer.zero_grad(set_to_none=True)
    xg = x.detach().clone().requires_grad_(True)
    y = layer.multi_step_forward_hybrid_triton(xg)
    (y * gy).sum().backward()
    torch.cuda.synchronize()
    par = layer.parametrizations.recurrent_delays
    return (y.detach().clone(), xg.grad.detach().clone(), layer.recurrent_weights.grad.detach().float().clone(),
            par.original.grad.detach().clone())


def _overfull_groups(y):
    """Groups of four consecutive batch rows (within 64-row chunks) with more than two spikes
    at one step and column."""
    T, B, N = y.shape
    Bp = (B + 63) // 64 * 64
    yy = torch.zeros(T, Bp, N, device=y.device)
    yy[:, :B] = y
    return int((yy.view(T, Bp // 4, 4, N).sum(2) > 2).sum())


@pytest.mark.gpu
@pytest.mark.parametrize('case', CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}s{c[5]}g{c[6]}{"q" if c[8] else ""}' for c in CASES])
def test_sparse_lag_correlation_matches_dense(dev, case, monkeypatch, capfd):
    T, B, N, (lo, hi), K, sigma, gain, with_oracle, silent = case
    print(f'case {case}', flush=True)
    g = gen(31)
    x = torch.randn(T, B, N, generator=g) * gain + 0.3
    if silent:   # neurons spread over the columns that never fire
        x[:, :, torch.randperm(N, generator=g)[:N // 3]] = -5.0
    W = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).bfloat16().float()
    base = lo + torch.rand(N, generator=g) * (hi - lo)
    offsets = torch.randint(K + 1, (N, N), generator=g).float()
    gy = torch.randn(T, B, N, generator=g)
    layer = hybrid_layer(N, W, base, offsets, dev, bf16=True, sigma_init=sigma)
    xd, gyd = x.to(dev), gy.to(dev)
    monkeypatch.setenv('DELREC_LOG_PLAN', '1')
    monkeypatch.setenv('DELREC_LAG_SPARSE', '1')   # these grids are below the form's own threshold
    y, dx, dW, dbase = _grads(layer, xd, gyd)
    plan = capfd.readouterr().err
    assert 'lag correlation: event-driven spikes' in plan, plan
    rate = float(y.mean())
    over = _overfull_groups(y)
    quiet = int((y.sum((0, 1)) == 0).sum())
    print(f'  firing rate {rate:.3f}, silent neurons {quiet}, groups with more than two spikes: {over}', flush=True)
    if silent:
        assert quiet >= N // 3
    if gain >= 2.0:
        assert over > 0, 'the case must exercise the residual product'
    monkeypatch.setenv('DELREC_LAG_SPARSE', '0')
    y2, dx2, dW2, dbase2 = _grads(layer, xd, gyd)
    plan = capfd.readouterr().err
    assert 'lag correlation: dense spikes' in plan, plan
    assert torch.equal(y, y2) and torch.equal(dx, dx2)
    d = base[None, :] + 0.0 + 1.0 * offsets
    check_elementwise('dbase sparse vs dense', dbase, dbase2, 1e-5, 1e-6)
    check_elementwise('dW sparse vs dense', dW, dW2, 2.0 ** -7, 1e-6, eps=grad_eps(False),
                      term_sq=syn_budget(dx, y, d, sigma)['W'])
    if with_oracle:
        lif = lif_params()
        y_ref, u_ref, gref = oracle_synaptic(x, W, None, lif, sigma, gy, base=base, offsets=offsets)
        flip = first_flip(y.cpu(), y_ref, u_ref, lif.v_threshold)
        assert flip is None, f'near-threshold flip at t={flip}'
        _, _, g64 = oracle_synaptic(x, W, None, lif, sigma, gy, base=base, offsets=offsets,
                                    dtype=torch.float64, forced=y)
        check_grads({'W': dW, 'base': dbase}, g64, gref, 2e-2, 1e-5, eps=grad_eps(True),
                    budget=syn_budget(g64['x'], y, d, sigma, W=W, hybrid=True))
