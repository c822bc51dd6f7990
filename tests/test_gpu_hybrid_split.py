"""The offset-stacked hybrid backward's split of the sources by first lag (near: first lag
below the block length) without a host read: the forward computes how many sources start
below lag 4 and below lag 2 with its own host read and hands the counts to the backward
(``near_known``), which partitions the sources on the device. Checked against the backward
that reads the first lags back itself (counts withheld): bit-identical gradients; and with
counts that contradict the device's: every output NaN, never a silently wrong split.
"""

import pytest
import torch

from helpers import gen
from test_gpu_synaptic import hybrid_layer


def _run(layer, x, gy):
    layer.zero_grad(set_to_none=True)
    xg = x.detach().clone().requires_grad_(True)
    y = layer.multi_step_forward_hybrid_triton(xg)
    (y * gy).sum().backward()
    torch.cuda.synchronize()
    par = layer.parametrizations.recurrent_delays
    return xg.grad.detach().clone(), layer.recurrent_weights.grad.detach().clone(), par.original.grad.detach().clone()


def _case(dev):
    T, B, N = 20, 3, 200
    g = gen(31)
    x = (torch.randn(T, B, N, generator=g) * 1.2 + 0.3).to(dev)
    W = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).bfloat16().float()
    base = torch.rand(N, generator=g) * 20.0          # about 15 % of the sources near
    offsets = torch.randint(5, (N, N), generator=g).float()
    gy = torch.randn(T, B, N, generator=g).to(dev)
    return hybrid_layer(N, W, base, offsets, dev, bf16=True, sigma_init=0.0), x, gy


@pytest.mark.gpu
def test_split_counts_from_the_forward_match_the_read_back(dev, monkeypatch, capfd):
    from delrec.kernels import synaptic_eventdriven as se
    import delrec.kernels.synaptic_hybrid as sh
    monkeypatch.setenv('DELREC_SYN_HYBSTEP', '1')
    monkeypatch.setenv('DELREC_LOG_PLAN', '1')
    layer, x, gy = _case(dev)
    seen = []
    real = se.syn_backward

    def spy(*a, **k):
        seen.append(k.get('hyb'))
        return real(*a, **k)

    monkeypatch.setattr(sh, 'syn_backward', spy)
    given = _run(layer, x, gy)
    hyb = seen[-1]
    print(f'  counts from the forward: first lag < 4: {hyb[4]}, < 2: {hyb[5]}', flush=True)
    assert len(hyb) == 6 and hyb[4] > 0 and 0 <= hyb[5] <= hyb[4]
    plan = capfd.readouterr().err
    assert f'near sources {hyb[4]} ' in plan, plan

    def withheld(*a, **k):   # the backward reads the first lags back itself
        k['hyb'] = tuple(k['hyb'][:4])
        return real(*a, **k)

    monkeypatch.setattr(sh, 'syn_backward', withheld)
    read = _run(layer, x, gy)
    for name, p, q in zip(('dx', 'dW', 'dbase'), given, read):
        assert torch.equal(p, q), f'{name} differs between the given and the read-back split'


@pytest.mark.gpu
def test_split_counts_that_contradict_the_device_give_nan(dev, monkeypatch):
    from delrec.kernels import synaptic_eventdriven as se
    import delrec.kernels.synaptic_hybrid as sh
    monkeypatch.setenv('DELREC_SYN_HYBSTEP', '1')
    layer, x, gy = _case(dev)
    real = se.syn_backward

    def wrong(*a, **k):
        h = k['hyb']
        k['hyb'] = tuple(h[:4]) + (h[4] + 1, h[5])   # one near source too many
        return real(*a, **k)

    monkeypatch.setattr(sh, 'syn_backward', wrong)
    dx, dW, dbase = _run(layer, x, gy)
    print(f'  NaN dx {int(dx.isnan().sum())} of {dx.numel()}', flush=True)
    assert bool(dx.isnan().all()) and bool(dW.float().isnan().any())
