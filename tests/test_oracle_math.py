"""CPU pins of the oracle's delay kernel, surrogates and closed-form delay gradient.

Each check is against something the oracle's code does not restate: hand-derived known
answers (tests/golden/*.json), autograd on a differently written mask, textbook identities
of the triangle, or finite differences.
"""

import json
import math
import os

import pytest
import torch

from oracle import delays, neuron

GOLDEN = os.path.join(os.path.dirname(__file__), 'golden')


def _load(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.mark.parametrize('case', _load('known_answer_delay_grad.json'), ids=lambda c: f"sigma{c['sigma']}")
def test_closed_form_delay_grad_known_answer(case):
    """The reference's known-answer inputs (check_hybrid_kernel.py:143-152) against the
    hand-computed closed form, and against autograd through the triangle mask."""
    sigma = case['sigma']
    d = torch.tensor(case['d_row'], dtype=torch.float64).repeat(5, 1)
    W = torch.arange(1, 26, dtype=torch.float64).reshape(5, 5) / 25
    dr = d.clone().requires_grad_(True)
    mask, L = delays.syn_mask(dr, sigma)
    assert L == case['L']
    C = torch.arange(L, dtype=torch.float64).square().expand(5, 5, L).contiguous()
    (auto,) = torch.autograd.grad((mask * W.unsqueeze(-1) * C).sum(), dr)
    closed = delays.delay_grad_closed_form(C, W, d, sigma)
    expected = torch.tensor(case['expected_dd'], dtype=torch.float64)
    torch.testing.assert_close(closed, expected, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(auto, expected, rtol=1e-12, atol=1e-12)
    assert expected[:, :3].abs().max() > 0   # integer delays exercise the inclusive edge


@pytest.mark.parametrize('sigma', [0.0, 0.5, 1.3])
def test_closed_form_matches_autograd_random(sigma):
    """The reference's test_hybrid_delay_grad_closed_form_matches_autograd
    (tests/test_hybrid_delay_invariance.py:145-162): d away from the kinks."""
    g = torch.Generator().manual_seed(0)
    N, lm = 12, 6
    d = 0.3 + 3.0 * torch.rand(N, N, generator=g, dtype=torch.float64)
    W = torch.randn(N, N, generator=g, dtype=torch.float64)
    C = torch.randn(N, N, lm, generator=g, dtype=torch.float64)
    C[:, :, 0] = 0.0
    dr = d.clone().requires_grad_(True)
    s = 1.0 + sigma
    # a differently written kernel: piecewise-linear hat evaluated lag by lag
    lags = torch.arange(lm, dtype=torch.float64)
    hat = torch.relu(s - (lags - 1.0 - dr.unsqueeze(-1)).abs()) / s ** 2
    (auto,) = torch.autograd.grad(hat, dr, grad_outputs=W.unsqueeze(-1) * C)
    torch.testing.assert_close(delays.delay_grad_closed_form(C, W, d, sigma), auto, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize('d,sigma', [(3.25, 0.0), (3.25, 0.5), (7.6, 1.0), (5.0, 2.0), (10.3, 4.0)])
def test_triangle_weights_are_a_partition_of_unity(d, sigma):
    """For s >= 1 the integer samples of the unit-area triangle sum to exactly 1 (the spike
    is spread, not scaled); for an integer half-width they also reproduce linear functions,
    so their centre of mass sits exactly at 1 + d (not shifted)."""
    mask, L = delays.axonal_mask(torch.tensor([d], dtype=torch.float64), sigma)
    w = mask[0]
    lags = torch.arange(L, dtype=torch.float64)
    assert abs(float(w.sum()) - 1.0) < 1e-12
    if float(1.0 + sigma).is_integer():
        assert abs(float((w * lags).sum()) - (1.0 + d)) < 1e-12
    assert float(w[0]) == 0.0


def test_triangle_hand_values():
    """h(l; d=1.25, sigma=0.5): s = 1.5, centre 2.25 -> (0.25, 1.25, 0.75) / 2.25."""
    mask, L = delays.axonal_mask(torch.tensor([1.25], dtype=torch.float64), 0.5)
    assert L == math.ceil(1 + 1.25 + 1.5) + 1
    expected = [0.0, 0.25 / 2.25, 1.25 / 2.25, 0.75 / 2.25] + [0.0] * (L - 4)
    torch.testing.assert_close(mask[0], torch.tensor(expected, dtype=torch.float64))


def test_window_length_formula():
    assert delays.window_length(16.0, 1.0) == 19      # C1: ceil(1+16+1)+1
    assert delays.window_length(32.0, 2.0) == 36      # C2
    assert delays.window_length(48.0, 1.0) == 51      # C3
    assert delays.window_length(41.0, 5.0) == 48
    assert delays.window_length(0.0, 1.0) == 3


def test_use_sig_p_spread_derivative_finite_difference():
    """d mask / d p through s = 1 + 2 sigma sigmoid(p), checked by central differences."""
    d = torch.tensor([2.3, 4.1, 0.7], dtype=torch.float64)
    p = torch.tensor([0.2, -1.0, 0.5], dtype=torch.float64, requires_grad=True)
    G = torch.randn(3, 9, dtype=torch.float64, generator=torch.Generator().manual_seed(1))

    def f(pv):
        m, L = delays.axonal_mask(d, 1.5, pv, use_sig_p=True)
        return (m[:, :9] * G[:, :m.shape[1]]).sum() if m.shape[1] >= 9 else (m * G[:, :m.shape[1]]).sum()

    (auto,) = torch.autograd.grad(f(p), p)
    eps = 1e-6
    for k in range(3):
        e = torch.zeros(3, dtype=torch.float64)
        e[k] = eps
        fd = (f(p.detach() + e) - f(p.detach() - e)) / (2 * eps)
        assert abs(float(fd) - float(auto[k])) < 1e-6


def test_atan_surrogate_closed_form():
    x = torch.linspace(-2, 2, 41, dtype=torch.float64, requires_grad=True)
    y = neuron.ATanSurrogate.apply(x, 2.0)
    assert torch.equal(y, (x >= 0).double())
    (g,) = torch.autograd.grad(y.sum(), x)
    ref = [1.0 / (1.0 + (math.pi * float(v)) ** 2) for v in x.detach()]   # alpha=2: (2/2)/(1+(pi x)^2)
    torch.testing.assert_close(g, torch.tensor(ref, dtype=torch.float64))
    # the derivative of (1/pi) atan(pi x) + 1/2, the smooth step ATan stands for
    fd = ((torch.atan(math.pi * (x.detach() + 1e-6)) - torch.atan(math.pi * (x.detach() - 1e-6)))
          / math.pi / 2e-6)
    torch.testing.assert_close(g, fd, rtol=1e-6, atol=1e-8)


def test_triangle_surrogate_closed_form():
    x = torch.tensor([-1.5, -1.0, -0.5, 0.0, 0.25, 1.0, 2.0], dtype=torch.float64, requires_grad=True)
    y = neuron.TriangleSurrogate.apply(x, 1.0)
    (g,) = torch.autograd.grad(y.sum(), x)
    torch.testing.assert_close(g, torch.tensor([0.0, 0.0, 0.5, 1.0, 0.75, 0.0, 0.0], dtype=torch.float64))
    y2 = neuron.TriangleSurrogate.apply(x, 2.0)
    (g2,) = torch.autograd.grad(y2.sum(), x)
    torch.testing.assert_close(g2, torch.tensor([0.125, 0.25, 0.375, 0.5, 0.4375, 0.25, 0.0],
                                                dtype=torch.float64))


def test_hybrid_parametrisation_sum():
    base = torch.tensor([0.5, 1.25, -2.0])
    off = torch.tensor([[0.0, 1.0, 4.0], [2.0, 0.0, 3.0], [1.0, 1.0, 0.0]])
    d = delays.hybrid_delays(base, off)
    assert torch.equal(d, torch.tensor([[0.5, 2.25, 2.0], [2.5, 1.25, 1.0], [1.5, 2.25, -2.0]]))
    g = torch.Generator().manual_seed(123)
    o = delays.draw_offsets((64, 64), 4, g)
    assert o.min() >= 0 and o.max() <= 4 and torch.equal(o, o.round())
    assert torch.equal(delays.draw_offsets((3, 3), 0, g), torch.zeros(3, 3))
