"""Whole-model parity on the GPU, the check the reference runs in tests/check_hybrid_kernel.py
(:44-128): the same SNN_* network evaluated by the oracle (its pure-PyTorch v2 scans) and
by the HIP layers, one forward + backward of ``out.pow(2).mean()``, output and every
parameter gradient compared with the reference's tolerances (forward 1e-4 / 1e-4,
gradients atol 2e-4 / rtol 2e-3). The config is the reference's: perf_MEM with one hidden
recurrent layer of 64, T = 24, B = 8, hybrid offsets up to 4, seed 0 for the model and 7
for the input.
"""

import copy

import pytest
import torch

from helpers import gen

T, B = 24, 8
FWD_ATOL, FWD_RTOL = 1e-4, 1e-4
GRAD_ATOL, GRAD_RTOL = 2e-4, 2e-3

MODELS = ['SNN_recurrent_hybrid_delays', 'SNN_axonal_recurrent_delays', 'SNN_synaptic_recurrent_delays',
          'SNN_common_recurrent_delays']


def _config(sigma=None):
    from configs.perf_MEM import Config
    cfg = Config()
    cfg.hidden_layers = [64]
    cfg.time_window = T
    cfg.batch_size = B
    cfg.use_batch_norm = False
    cfg.feedforward_dropout_rate = 0.0
    cfg.recurrent_dropout_rate = 0.0
    cfg.no_recurrence_in_last_layer = False     # keep a real recurrent layer in the hidden layer
    cfg.kernel_count = 1
    cfg.hybrid_offset_scale = 4
    if sigma is not None:
        cfg.sigma_init = sigma
    return cfg


def _grads(model):
    return {n: p.grad.detach().float().cpu().clone() for n, p in model.named_parameters()
            if p.grad is not None}


@pytest.mark.gpu
@pytest.mark.parametrize('sigma', [None, 1.0], ids=['config_sigma', 'sigma1'])
@pytest.mark.parametrize('name', MODELS)
def test_model_forward_backward_matches_oracle(dev, name, sigma):
    from delrec import networks
    from delrec.utils import reset_states
    from oracle.model import reference_forward
    print(f'model {name} sigma {sigma}', flush=True)
    cfg = _config(sigma)
    torch.manual_seed(0)
    model = getattr(networks, name)(cfg)
    model.eval()
    x = torch.randn(T, B, cfg.input_size, generator=gen(7))

    ref = copy.deepcopy(model)
    reset_states(ref)
    y_ref = reference_forward(ref, x.clone())
    y_ref.pow(2).mean().backward()
    g_ref = _grads(ref)
    assert torch.isfinite(y_ref).all() and all(torch.isfinite(g).all() for g in g_ref.values())

    hip = copy.deepcopy(model).to(dev)
    reset_states(hip)
    y = hip(x.to(dev))
    y.pow(2).mean().backward()
    torch.cuda.synchronize()
    g = _grads(hip)

    torch.testing.assert_close(y.detach().cpu(), y_ref.detach(), atol=FWD_ATOL, rtol=FWD_RTOL)
    assert set(g) == set(g_ref), set(g).symmetric_difference(g_ref)
    worst = 0.0
    for n in sorted(g_ref):
        torch.testing.assert_close(g[n], g_ref[n], atol=GRAD_ATOL, rtol=GRAD_RTOL, msg=lambda m: f'{n}: {m}')
        worst = max(worst, (g[n] - g_ref[n]).abs().max().item() / (g_ref[n].abs().max().item() + 1e-12))
    print(f'  OK, max relative gradient difference {worst:.2e} over {len(g)} parameters')


@pytest.mark.gpu
@pytest.mark.parametrize('name', MODELS[:3])
def test_delay_maintenance_on_device(dev, name):
    """The delay-parameter maintenance of a training loop run on device tensors (reference
    ``networks.py:183-199,910-933``, ``delay_layers.py:178-189``): clamp, the epoch's
    spread, nearest rounding give on the GPU what they give on the CPU; stochastic rounding
    lands on the floor or the ceiling; the model then still matches the oracle."""
    from delrec import networks
    from delrec.delay_layers import axonal_recdel
    from delrec.networks import learned_delay_parameter
    from delrec.training.mem import set_epoch
    from delrec.utils import reset_states
    from oracle.model import reference_forward
    print(f'delay maintenance {name}', flush=True)
    cfg = _config(sigma=1.0)
    cfg.epochs = 20
    torch.manual_seed(0)
    model = getattr(networks, name)(cfg)
    model.eval()
    layer = [m for m in model.layers if isinstance(m, axonal_recdel)][0]
    leaf = learned_delay_parameter(layer, 'recurrent_delays')
    with torch.no_grad():     # off the grid, a few below 0
        leaf.add_(torch.rand(leaf.shape, generator=gen(5)) * 3.0 - 1.0)
    ref, hip = copy.deepcopy(model), copy.deepcopy(model).to(dev)
    for m in (ref, hip):
        m.clamp_delays()
        set_epoch(m, cfg, 7)
    lay = lambda m: [x for x in m.layers if isinstance(x, axonal_recdel)][0]
    assert lay(hip).sigma == lay(ref).sigma == pytest.approx(cfg.sigma_init * cfg.sigma_decay ** (100 / 20 * 7))
    l_ref, l_hip = learned_delay_parameter(lay(ref), 'recurrent_delays'), learned_delay_parameter(lay(hip), 'recurrent_delays')
    assert l_hip.is_cuda and torch.equal(l_hip.detach().cpu(), l_ref.detach()) and float(l_ref.detach().min()) >= 0.0
    # stochastic rounding on device: every delay on its floor or ceiling
    before = l_hip.detach().clone()
    hip.config.round_mode = 'stochastic'
    hip.round_pos()
    after = l_hip.detach()
    assert torch.all((after == before.floor()) | (after == before.ceil()))
    # nearest rounding: the same on both devices
    with torch.no_grad():
        l_hip.copy_(before)
    hip.config.round_mode = 'nearest'
    for m in (ref, hip):
        m.round_pos()
    assert torch.equal(l_hip.detach().cpu(), l_ref.detach())
    # the maintained model against the oracle, one forward + backward
    x = torch.randn(T, B, cfg.input_size, generator=gen(7))
    reset_states(ref)
    y_ref = reference_forward(ref, x.clone())
    y_ref.pow(2).mean().backward()
    reset_states(hip)
    y = hip(x.to(dev))
    y.pow(2).mean().backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(y.detach().cpu(), y_ref.detach(), atol=FWD_ATOL, rtol=FWD_RTOL)
    g, g_ref = _grads(hip), _grads(ref)
    assert set(g) == set(g_ref)
    for n in sorted(g_ref):
        torch.testing.assert_close(g[n], g_ref[n], atol=GRAD_ATOL, rtol=GRAD_RTOL, msg=lambda m: f'{n}: {m}')
