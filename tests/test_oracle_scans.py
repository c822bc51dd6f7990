"""CPU pins of the oracle's scans: delay semantics, LIF closed forms, BPTT, invariants.

* single-spike propagation against hand-derived arrival weights (tests/golden/single_spike.json)
* W = 0: each neuron is an independent LIF, checked against an explicit scalar recurrence
* the backward against an independent scalar reverse recursion written from the BPTT
  equations (not autograd)
* v1 (circular buffer) == v2 (sliding window); hybrid with zero offsets == axonal;
  synaptic with d[i, j] = d[j] == axonal; an integer offset k == a time shift by k
"""

import json
import math
import os

import pytest
import torch

from oracle import neuron, scans

GOLDEN = os.path.join(os.path.dirname(__file__), 'golden')


def _cases():
    with open(os.path.join(GOLDEN, 'single_spike.json')) as f:
        return json.load(f)


@pytest.mark.parametrize('case', _cases(), ids=lambda c: f"d{c['d']}s{c['sigma']}")
@pytest.mark.parametrize('kind', ['axonal', 'synaptic'])
def test_single_spike_arrives_at_t_plus_1_plus_d(case, kind):
    T, w = case['T'], case['w']
    x = torch.zeros(T, 1, 2, dtype=torch.float64)
    x[0, 0, 0] = 10.0                       # source 0 fires once, at t = 0
    W = torch.zeros(2, 2, dtype=torch.float64)
    W[1, 0] = w                             # source 0 -> receiver 1
    lif = neuron.LIFParams(tau=2.0, v_threshold=1.0, v_reset=0.0)
    if kind == 'axonal':
        d = torch.tensor([case['d'], 0.0], dtype=torch.float64)
        y, ext = scans.axonal_v2(x, W, d, lif, sigma=case['sigma'])
    else:
        d = torch.tensor([[0.0, 0.0], [case['d'], 0.0]], dtype=torch.float64)
        y, ext = scans.synaptic_v2(x, W, d, lif, sigma=case['sigma'])
    assert y[:, 0, 0].tolist() == [1.0] + [0.0] * (T - 1)
    torch.testing.assert_close(ext['rec'][:, 0, 1], torch.tensor(case['expected_rec'], dtype=torch.float64),
                               rtol=1e-12, atol=1e-12)


def test_zero_weights_give_independent_lif():
    g = torch.Generator().manual_seed(3)
    T, B, N = 30, 2, 5
    x = torch.rand(T, B, N, generator=g, dtype=torch.float64) * 1.3
    lif = neuron.LIFParams(tau=2.0, v_threshold=1.0, v_reset=0.0)
    y, ext = scans.axonal_v2(x, torch.zeros(N, N, dtype=torch.float64), torch.rand(N, dtype=torch.float64) * 4,
                             lif, sigma=0.5)
    for b in range(B):
        for n in range(N):
            v = 0.0
            for t in range(T):
                u = 0.5 * v + float(x[t, b, n])
                s = 1.0 if u >= 1.0 else 0.0
                assert float(ext['u'][t, b, n]) == pytest.approx(u, abs=1e-14)
                assert float(y[t, b, n]) == s
                v = 0.0 if s else u


def _scalar_axonal(x, W, d, sigma, gy, tau=2.0, th=1.0):
    """Forward and BPTT of the axonal layer, hard reset to 0, ATan(2), written as explicit
    scalar recursions from the equations (no autograd)."""
    T, N = len(x), len(W)
    s = 1.0 + sigma
    decay = 1.0 - 1.0 / tau
    L = int(math.ceil(1.0 + max(d) + s)) + 1
    h = [[max(0.0, s - abs(l - 1.0 - d[j])) / (s * s) for l in range(L)] for j in range(N)]
    dh = [[(1 if l - 1.0 - d[j] > 0 else -1 if l - 1.0 - d[j] < 0 else 0)
           * (1.0 if abs(l - 1.0 - d[j]) <= s else 0.0) / (s * s) for l in range(L)] for j in range(N)]
    y = [[0.0] * N for _ in range(T)]
    u = [[0.0] * N for _ in range(T)]
    z = [[0.0] * N for _ in range(T)]
    v = [0.0] * N
    for t in range(T):
        for j in range(N):
            z[t][j] = sum(h[j][l] * y[t - l][j] for l in range(1, L) if t - l >= 0)
        for i in range(N):
            r = sum(W[i][j] * z[t][j] for j in range(N))
            u[t][i] = v[i] * decay + x[t][i] + r
            y[t][i] = 1.0 if u[t][i] - th >= 0 else 0.0
            v[i] = 0.0 if y[t][i] else u[t][i]
    gz = [[0.0] * N for _ in range(T)]
    dx = [[0.0] * N for _ in range(T)]
    lam = [0.0] * N
    for t in range(T - 1, -1, -1):
        gr = [0.0] * N
        for j in range(N):
            gfut = sum(h[j][l] * gz[t + l][j] for l in range(1, L) if t + l < T)
            xs = u[t][j] - th
            sg = 1.0 / (1.0 + (math.pi * xs) ** 2)
            gS = gy[t][j] + gfut - lam[j] * u[t][j]
            du = lam[j] * (1.0 - y[t][j]) + gS * sg
            lam[j] = decay * du
            dx[t][j] = du
            gr[j] = du
        for j in range(N):
            gz[t][j] = sum(gr[i] * W[i][j] for i in range(N))
        for j in range(N):  # keep gr for dW
            pass
        if t == T - 1:
            grs = [None] * T
        grs[t] = gr
    dW = [[sum(grs[t][i] * z[t][j] for t in range(T)) for j in range(N)] for i in range(N)]
    dd = [sum(dh[j][l] * sum(gz[t][j] * y[t - l][j] for t in range(T) if t - l >= 0) for l in range(1, L))
          for j in range(N)]
    return y, dx, dW, dd


@pytest.mark.parametrize('sigma', [0.0, 0.7])
def test_bptt_matches_scalar_reverse_recursion(sigma):
    g = torch.Generator().manual_seed(11)
    T, N = 9, 4
    x = torch.rand(T, 1, N, generator=g, dtype=torch.float64) * 1.6
    W = torch.randn(N, N, generator=g, dtype=torch.float64) * 0.8
    d = torch.rand(N, generator=g, dtype=torch.float64) * 3.0
    gy = torch.randn(T, 1, N, generator=g, dtype=torch.float64)
    lif = neuron.LIFParams(tau=2.0, v_threshold=1.0, v_reset=0.0)
    xr, Wr, dr = (t.clone().requires_grad_(True) for t in (x, W, d))
    y, _ = scans.axonal_v2(xr, Wr, dr, lif, sigma=sigma)
    (y * gy).sum().backward()
    ys, dx, dW, dd = _scalar_axonal(x[:, 0].tolist(), W.tolist(), d.tolist(), sigma, gy[:, 0].tolist())
    assert y.detach()[:, 0].tolist() == ys
    assert 0 < sum(map(sum, ys)) < T * N      # some but not all units spike
    torch.testing.assert_close(xr.grad[:, 0], torch.tensor(dx, dtype=torch.float64), rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(Wr.grad, torch.tensor(dW, dtype=torch.float64), rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(dr.grad, torch.tensor(dd, dtype=torch.float64), rtol=1e-10, atol=1e-12)


def _inputs(seed, T=16, B=3, N=6, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, B, N, generator=g, dtype=dtype) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g, dtype=dtype) * 0.6
    return g, x, W


@pytest.mark.parametrize('sigma', [0.0, 0.5, 1.0])
def test_v1_equals_v2(sigma):
    g, x, W = _inputs(1)
    d = torch.rand(6, generator=g, dtype=torch.float64) * 5
    lif = neuron.LIFParams()
    y1, e1 = scans.axonal_v1(x, W, d, lif, sigma=sigma)
    y2, e2 = scans.axonal_v2(x, W, d, lif, sigma=sigma)
    assert torch.equal(y1, y2)
    torch.testing.assert_close(e1['u'], e2['u'], rtol=1e-12, atol=1e-12)
    D = torch.rand(6, 6, generator=g, dtype=torch.float64) * 5
    y1, e1 = scans.synaptic_v1(x, W, D, lif, sigma=sigma)
    y2, e2 = scans.synaptic_v2(x, W, D, lif, sigma=sigma)
    assert torch.equal(y1, y2)
    torch.testing.assert_close(e1['u'], e2['u'], rtol=1e-12, atol=1e-12)


def test_broadcast_synaptic_equals_axonal_and_grads_sum():
    g, x, W = _inputs(2)
    d = torch.rand(6, generator=g, dtype=torch.float64) * 5
    lif = neuron.LIFParams()
    gy = torch.randn(x.shape, generator=g, dtype=torch.float64)
    da = d.clone().requires_grad_(True)
    ya, _ = scans.axonal_v2(x, W, da, lif, sigma=0.6)
    (ya * gy).sum().backward()
    ds = d.clone().requires_grad_(True)
    ysyn, _ = scans.synaptic_v2(x, W, ds.unsqueeze(0).expand(6, 6), lif, sigma=0.6)
    (ysyn * gy).sum().backward()
    assert torch.equal(ya, ysyn)
    torch.testing.assert_close(da.grad, ds.grad, rtol=1e-10, atol=1e-12)


def test_hybrid_zero_offsets_equal_axonal():
    from oracle.delays import hybrid_delays
    g, x, W = _inputs(3)
    base = torch.rand(6, generator=g, dtype=torch.float64) * 5
    lif = neuron.LIFParams()
    ya, _ = scans.axonal_v2(x, W, base, lif, sigma=0.0)
    yh, _ = scans.synaptic_v2(x, W, hybrid_delays(base, torch.zeros(6, 6, dtype=torch.float64)), lif, sigma=0.0)
    assert torch.equal(ya, yh)


@pytest.mark.parametrize('k', [1, 3])
def test_integer_offset_is_a_time_shift(k):
    """Adding the integer k to every delay equals delaying every spike k more steps: the
    hybrid with constant offsets k matches the axonal model with delays d + k."""
    from oracle.delays import hybrid_delays
    g, x, W = _inputs(4)
    base = torch.rand(6, generator=g, dtype=torch.float64) * 4
    lif = neuron.LIFParams()
    ya, ea = scans.axonal_v2(x, W, base + k, lif, sigma=0.5)
    yh, eh = scans.synaptic_v2(x, W, hybrid_delays(base, torch.full((6, 6), float(k), dtype=torch.float64)),
                               lif, sigma=0.5)
    assert torch.equal(ya, yh)
    torch.testing.assert_close(ea['rec'], eh['rec'], rtol=1e-12, atol=1e-12)


def test_soft_reset_and_bias_and_dropout_plumbing():
    g, x, W = _inputs(5)
    d = torch.rand(6, generator=g, dtype=torch.float64) * 3
    bias = torch.randn(6, generator=g, dtype=torch.float64) * 0.1
    drop = (torch.rand(3, 6, generator=g) > 0.3).double() / 0.7
    lif = neuron.LIFParams(v_reset=None)
    y, e = scans.axonal_v2(x, W, d, lif, sigma=0.3, bias=bias, drop=drop)
    # recompute step by step from the recorded recurrent input: a = x + drop * rec
    v = torch.zeros(3, 6, dtype=torch.float64)
    for t in range(x.shape[0]):
        u = v * 0.5 + x[t] + e['rec'][t] * drop
        torch.testing.assert_close(e['u'][t], u, rtol=1e-12, atol=1e-12)
        s = (u - 1.0 >= 0).double()
        v = u - s * 1.0
    assert torch.equal(y, torch.stack([(e['u'][t] - 1.0 >= 0).double() for t in range(x.shape[0])]))
