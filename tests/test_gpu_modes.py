"""GPU parity of the secondary modes against the CPU oracle: the reference fused kernel's
hard-tap forwards (``triton_approx``, ``triton_ste`` with the rounded or the interpolated
tap), STE-rounded delays (``round_delays``), the delay-free ``vanilla_recurrent`` layer, the
plain multi-step LIF layer, and the kernel variants kept behind environment switches
(the dense tiled axonal forward, the synaptic per-connection forward and the general
hybrid backward). Tolerances as everywhere: spikes exact except within 1e-5 of the
threshold; gradients against the oracle run in float64 on the same values, teacher-forced
with the device's spike train, at the fixed, unscaled fp32 rtol 1e-4 / atol 1e-5, where an
element that misses them gets the fp32 oracle's own distance from float64 there as its
floor (``helpers.check_grads``).
"""

import pytest
import torch

from helpers import check_grads, first_flip, gen, grads64, lif_params
from oracle import neuron as oneuron, scans

RTOL, ATOL = 1e-4, 1e-5


def _check(got, run, leaves, gy, y):
    """``got`` (name -> device gradient) against the float64 run of ``run`` on ``leaves``
    (the fp32 oracle's leaves, their ``.grad`` the fp32 gradients)."""
    g64 = grads64(run, leaves, gy, y)
    check_grads(got, g64, {k: v.grad for k, v in leaves.items()}, RTOL, ATOL)


def _axonal_module(N, sigma, dmax, dev, seed, **cfg_kw):
    from configs.perf_MEM import Config
    from delrec.delay_layers import axonal_recdel
    cfg = Config()
    cfg.sigma_init = sigma
    cfg.max_rec_delay = dmax
    cfg.init_rec_weights = 'kaiming_uniform'
    for k, v in cfg_kw.items():
        setattr(cfg, k, v)
    torch.manual_seed(seed)
    layer = axonal_recdel(cfg, N)
    with torch.no_grad():
        layer.recurrent_weights.mul_(4.0)
    return layer.to(dev), cfg


MODES = [
    # forward_version, ste_round_forward, oracle taps, T, B, N, dmax, sigma
    ('triton_approx', True, 'approx', 24, 3, 48, 9.0, 0.0),
    ('triton_approx', True, 'approx', 20, 2, 130, 14.0, 0.7),
    ('triton_ste', True, 'ste_round', 24, 3, 48, 9.0, 0.5),
    ('triton_ste', False, 'ste_interp', 24, 3, 48, 9.0, 0.5),
    ('triton_ste', False, 'ste_interp', 20, 2, 64, 12.0, 1.0),
    # windows beyond the 256 lags of the axonal kernels' spike history: the synaptic scans
    # at the tap's own delay (forward) and the soft or straight-through backward
    ('triton_approx', True, 'approx', 300, 2, 40, 290.0, 0.0),
    ('triton_approx', True, 'approx', 300, 2, 40, 290.0, 0.6),
    ('triton_ste', True, 'ste_round', 300, 2, 40, 290.0, 0.5),
    ('triton_ste', False, 'ste_interp', 310, 2, 40, 300.0, 0.7),
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', MODES, ids=[f'{c[2]}-N{c[5]}s{c[7]}' for c in MODES])
def test_hard_tap_modes_match_oracle(dev, case):
    fv, ste_round, taps, T, B, N, dmax, sigma = case
    print(f'case {case}', flush=True)
    layer, cfg = _axonal_module(N, sigma, dmax, dev, seed=3, ste_round_forward=ste_round)
    layer.forward_version = fv
    g = gen(4)
    x = torch.randn(T, B, N, generator=g) * 1.1 + 0.35
    gy = torch.randn(T, B, N, generator=g)
    W, d = layer.recurrent_weights.detach().cpu(), layer.recurrent_delays.detach().cpu()
    lif = lif_params()
    xr, Wr, dr = (t.clone().requires_grad_(True) for t in (x, W, d))
    y_ref, ext = scans.axonal_v2(xr, Wr, dr, lif, sigma=sigma, taps=taps)
    (y_ref * gy).sum().backward()

    if T > 256:
        assert float(d.max()) > 256.0, 'the case must take the long-window route'
    xg = x.to(dev).requires_grad_(True)
    y = layer(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    flip = first_flip(y.detach().cpu(), y_ref.detach(), ext['u'].detach(), lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    print(f'  spikes identical ({int(y_ref.sum())} of {y_ref.numel()})', flush=True)
    _check({'x': xg.grad, 'W': layer.recurrent_weights.grad, 'd': layer.recurrent_delays.grad},
           lambda l, f: scans.axonal_v2(l['x'], l['W'], l['d'], lif, sigma=sigma, taps=taps, forced=f)[0],
           {'x': xr, 'W': Wr, 'd': dr}, gy, y)


@pytest.mark.gpu
@pytest.mark.parametrize('sigma', [0.0, 0.6])
def test_round_delays_match_oracle(dev, sigma):
    """``round_delays``: the forward uses round(d), the gradient flows straight through to d
    (reference delay_layers_triton.py:67-69)."""
    T, B, N = 24, 3, 40
    layer, _ = _axonal_module(N, sigma, 7.0, dev, seed=5, round_delays=True)
    g = gen(6)
    x = torch.randn(T, B, N, generator=g) * 1.1 + 0.35
    gy = torch.randn(T, B, N, generator=g)
    W, d = layer.recurrent_weights.detach().cpu(), layer.recurrent_delays.detach().cpu()
    lif = lif_params()
    xr, Wr, dr = (t.clone().requires_grad_(True) for t in (x, W, d))
    y_ref, ext = scans.axonal_v2(xr, Wr, dr, lif, sigma=sigma, round_delays=True)
    (y_ref * gy).sum().backward()
    xg = x.to(dev).requires_grad_(True)
    y = layer(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    flip = first_flip(y.detach().cpu(), y_ref.detach(), ext['u'].detach(), lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    _check({'x': xg.grad, 'W': layer.recurrent_weights.grad, 'd': layer.recurrent_delays.grad},
           lambda l, f: scans.axonal_v2(l['x'], l['W'], l['d'], lif, sigma=sigma, round_delays=True,
                                        forced=f)[0],
           {'x': xr, 'W': Wr, 'd': dr}, gy, y)


@pytest.mark.gpu
@pytest.mark.parametrize('N', [40, 300])
def test_vanilla_recurrent_matches_oracle(dev, N):
    """The delay-free recurrent layer (reference delay_layers_pytorch.py:18-47)."""
    from configs.perf_MEM import Config
    from delrec.delay_layers import vanilla_recurrent
    cfg = Config()
    torch.manual_seed(7)
    layer = vanilla_recurrent(cfg, N).to(dev)
    with torch.no_grad():
        layer.recurrent_weights.mul_(2.0)
    T, B = 20, 3
    g = gen(8)
    x = torch.randn(T, B, N, generator=g) * 1.1 + 0.35
    gy = torch.randn(T, B, N, generator=g)
    lif = lif_params()
    xr, Wr = x.clone().requires_grad_(True), layer.recurrent_weights.detach().cpu().clone().requires_grad_(True)
    y_ref, ext = scans.vanilla(xr, Wr, lif)
    (y_ref * gy).sum().backward()
    xg = x.to(dev).requires_grad_(True)
    y = layer(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    flip = first_flip(y.detach().cpu(), y_ref.detach(), ext['u'].detach(), lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    assert 0 < float(y_ref.mean()) < 1
    _check({'x': xg.grad, 'W': layer.recurrent_weights.grad},
           lambda l, f: scans.vanilla(l['x'], l['W'], lif, forced=f)[0], {'x': xr, 'W': Wr}, gy, y)


LIF_FORMS = [
    # tau, v_reset, decay_input, detach_reset, surrogate
    (2.0, 0.0, False, False, ('atan', 2.0)),
    (3.0, -0.2, False, False, ('atan', 2.0)),
    (2.5, 0.0, True, False, ('atan', 2.0)),
    (2.5, 0.3, True, True, ('triangle', 1.0)),
    (2.0, None, False, False, ('atan', 3.0)),
]


@pytest.mark.gpu
@pytest.mark.parametrize('form', LIF_FORMS, ids=[f'tau{f[0]}vr{f[1]}di{int(f[2])}det{int(f[3])}{f[4][0]}'
                                                 for f in LIF_FORMS])
def test_plain_lif_layer_matches_oracle(dev, form):
    """The multi-step LIF layer the SNN_* stacks place around the recurrent one (e.g. the
    last layer with no_recurrence_in_last_layer, reference networks.py:148-160)."""
    from delrec.neuron import ATan, LIFNode
    from delrec.utils import Triangle
    tau, v_reset, decay_input, detach, surr = form
    kind, width = surr
    sf = ATan(width) if kind == 'atan' else Triangle.apply
    node = LIFNode(tau=tau, decay_input=decay_input, v_threshold=1.0, v_reset=v_reset,
                   surrogate_function=sf, detach_reset=detach, step_mode='m')
    if kind == 'triangle':
        node.surrogate_gamma = width
    T, B, N = 30, 4, 70
    g = gen(9)
    x = torch.randn(T, B, N, generator=g) * 1.3 + (0.6 if decay_input else 0.4)
    gy = torch.randn(T, B, N, generator=g)
    lif = oneuron.LIFParams(tau=tau, v_threshold=1.0, v_reset=v_reset, decay_input=decay_input,
                            detach_reset=detach, surrogate=surr)
    xr = x.clone().requires_grad_(True)
    y_ref, ext = scans.lif_layer(xr, lif)
    (y_ref * gy).sum().backward()
    xg = x.to(dev).requires_grad_(True)
    y = node(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    flip = first_flip(y.detach().cpu(), y_ref.detach(), ext['u'].detach(), 1.0)
    assert flip is None, f'near-threshold flip at t={flip}'
    assert 0 < float(y_ref.mean()) < 1
    _check({'x': xg.grad}, lambda l, f: scans.lif_layer(l['x'], lif, forced=f)[0], {'x': xr}, gy, y)


# kernel variants kept behind environment switches, on the cases of the default paths
@pytest.mark.gpu
@pytest.mark.parametrize('idx', [0, 2, 3, 13])
def test_axonal_dense_tiled_forward_matches_oracle(dev, idx, monkeypatch):
    import test_gpu_axonal as ax
    monkeypatch.setenv('DELREC_AXONAL_FWD', 'tiled')
    ax.test_axonal_fwd_bwd_matches_oracle(dev, ax.CASES[idx], monkeypatch)


@pytest.mark.gpu
@pytest.mark.parametrize('idx', [0, 2, 6, 7])
def test_synaptic_per_connection_forward_matches_oracle(dev, idx, monkeypatch):
    import test_gpu_synaptic as sy
    monkeypatch.setenv('DELREC_SYN_SCATTER', '0')
    sy.test_synaptic_fwd_bwd_matches_oracle(dev, sy.SYN_CASES[idx])


@pytest.mark.gpu
@pytest.mark.parametrize('idx', [0, 2, 6])
def test_hybrid_general_backward_matches_oracle(dev, idx, monkeypatch):
    import test_gpu_synaptic as sy
    monkeypatch.setenv('DELREC_SYN_BWD_HYB', '0')
    monkeypatch.setenv('DELREC_SYN_SCATTER', '0')
    sy.test_hybrid_fwd_bwd_matches_oracle(dev, sy.HYB_CASES[idx])
