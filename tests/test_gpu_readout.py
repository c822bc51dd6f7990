"""GPU parity of the fused readout loss (``delrec_readout_ce`` through
``delrec.readout.readout_ce``) against float64 autograd of the reference's own operations:
the time reduction of ``utils.calc_loss_SSC`` (sum), ``calc_loss_HAR`` / ``calc_loss_AL``
(mean) and ``calc_loss_SHD`` (max), optionally after the SHD stack's non-spiking LIF readout
(``networks_shd.py:187-199``: threshold 1e8, v_reset 0; charge ``v (1 - 1/tau) + x``, or
``v + (x - v) / tau`` with decay_input), then ``torch.nn.CrossEntropyLoss``. Loss and the
gradient with respect to the readout's output: fp32 rtol 1e-4, atol 1e-6 (the gradient's
entries are O(1/B)).
"""

import pytest
import torch

from helpers import gen

CASES = [
    # T, B, C, reduce, tau (None: no integrator), decay_input
    (32, 64, 4, 'mean', 2.0, False),          # C1's readout: LI integrator, time mean
    (32, 64, 4, 'mean', None, False),
    (50, 16, 20, 'sum', None, False),
    (50, 16, 35, 'max', None, False),
    (40, 8, 10, 'max', 2.0, False),
    (40, 8, 10, 'sum', 3.0, True),
    (1, 5, 300, 'mean', None, False),         # more classes than threads
    (1024, 4, 10, 'mean', 2.0, False),        # C5's readout length
]


def _reference(x, labels, reduce, tau, decay_input):
    v = torch.zeros_like(x[0])
    vs = []
    for t in range(x.shape[0]):
        if tau is None:
            v = x[t]
        elif decay_input:
            v = v + (x[t] - v) / tau
        else:
            v = v * (1.0 - 1.0 / tau) + x[t]
        vs.append(v)
    v = torch.stack(vs)
    m = v.sum(0) if reduce == 'sum' else (v.mean(0) if reduce == 'mean' else v.max(0)[0])
    return torch.nn.CrossEntropyLoss()(m, labels)


@pytest.mark.gpu
@pytest.mark.parametrize('case', CASES, ids=[f'T{c[0]}B{c[1]}C{c[2]}{c[3]}{"" if c[4] is None else "li" + str(c[4])}'
                                             f'{"di" if c[5] else ""}' for c in CASES])
def test_readout_ce_matches_autograd(dev, case):
    from delrec.readout import readout_ce
    T, B, C, reduce, tau, di = case
    print(f'case {case}', flush=True)
    g = gen(21)
    x = torch.randn(T, B, C, generator=g)
    labels = torch.randint(C, (B,), generator=g)
    xr = x.double().requires_grad_(True)
    ref = _reference(xr, labels, reduce, tau, di)
    ref.backward()
    xg = x.to(dev).requires_grad_(True)
    loss = readout_ce(xg, labels.to(dev), reduce, tau, di)
    (loss * 3.0).backward()
    torch.cuda.synchronize()
    print(f'  loss {float(loss):.6f} vs {float(ref):.6f}', flush=True)
    torch.testing.assert_close(loss.detach().cpu().double(), ref.detach(), rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(xg.grad.cpu().double(), 3.0 * xr.grad, rtol=1e-4, atol=1e-6)
