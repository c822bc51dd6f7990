"""The memorisation training harness on the CPU (no GPU): the dataset's draws, the
optimiser's parameter groups, the per-epoch spread and a short run through the oracle
forward (``helpers.OracleModel``)."""

import copy
import math

import pytest
import torch

from helpers import OracleModel


def _config(model='SNN_axonal_recurrent_delays', epochs=3):
    from configs.perf_MEM import Config
    cfg = Config()
    cfg.model = model
    cfg.epochs = epochs
    cfg.input_gain = 3.0
    return cfg


def test_temporal_dataset_draws():
    from delrec.datasets import SpikeMemorization
    d = SpikeMemorization(40, 5, 12, 3, seed=4, input_gain=2.5)
    assert d.inputs.shape == (40, 12, 5) and len(d) == 40
    # one spike per (sample, input neuron), carrying the gain
    assert torch.equal((d.inputs != 0).sum(1), torch.ones(40, 5, dtype=torch.long))
    assert torch.equal(d.inputs.amax(1), torch.full((40, 5), 2.5))
    # spike times, then labels, from one generator seeded with the dataset seed
    g = torch.Generator().manual_seed(4)
    when = torch.randint(0, 12, (40, 5), generator=g)
    assert torch.equal(d.inputs.argmax(1), when)
    assert torch.equal(d.labels, torch.randint(0, 3, (40,), generator=g))
    x, y = d[7]
    assert x.shape == (12, 5) and int(y) == int(d.labels[7])
    again = SpikeMemorization(40, 5, 12, 3, seed=4, input_gain=2.5)
    assert torch.equal(again.inputs, d.inputs) and torch.equal(again.labels, d.labels)


def test_spatial_dataset_draws():
    from delrec.datasets import SpikeMemorization
    d = SpikeMemorization(16, 3, 6, 4, seed=2, input_gain=0.5, task_type='spatial')
    g = torch.Generator().manual_seed(2)
    level = torch.rand(16, 3, generator=g) * 0.5
    assert torch.equal(d.inputs, level.unsqueeze(1).expand(16, 6, 3))
    assert torch.equal(d.labels, torch.randint(0, 4, (16,), generator=g))
    with pytest.raises(ValueError):
        SpikeMemorization(16, 3, 6, 4, task_type='other')
    with pytest.raises(ValueError):
        SpikeMemorization(0, 3, 6, 4)


@pytest.mark.parametrize('name', ['SNN_axonal_recurrent_delays', 'SNN_recurrent_hybrid_delays'])
def test_optimizer_groups(name):
    from delrec import networks
    from delrec.delay_layers import axonal_recdel
    from delrec.networks import learned_delay_parameter
    from delrec.training.mem import make_optimizer
    cfg = _config(name)
    model = getattr(networks, name)(cfg)
    opt = make_optimizer(model, cfg)
    weights, positions = opt.param_groups
    rec = [m for m in model.modules() if isinstance(m, axonal_recdel)]
    assert len(rec) == 1
    assert [id(p) for p in positions['params']] == [id(learned_delay_parameter(m, 'recurrent_delays')) for m in rec]
    assert positions['lr'] == cfg.lr_positions and positions['weight_decay'] == 0.0
    assert weights['lr'] == cfg.lr_w and weights['weight_decay'] == cfg.weight_decay
    n_all = sum(1 for p in model.parameters() if p.requires_grad)
    assert len(weights['params']) + len(positions['params']) == n_all


def test_set_epoch_anneals_sigma():
    from delrec import networks
    from delrec.training.mem import set_epoch
    cfg = _config(epochs=20)
    cfg.sigma_init = 1.5
    model = networks.SNN_axonal_recurrent_delays(cfg)
    rec = [m for m in model.modules() if hasattr(m, 'recurrent_delays')][0]
    set_epoch(model, cfg, 0)
    assert rec.sigma == pytest.approx(1.5)
    set_epoch(model, cfg, 20)
    # after all epochs the spread has decayed by sigma_decay ** 100
    assert rec.sigma == pytest.approx(1.5 * cfg.sigma_decay ** 100, rel=1e-9)


def test_run_with_oracle_forward_learns():
    from delrec import networks
    from delrec.training.mem import run
    cfg = _config(epochs=12)
    torch.manual_seed(cfg.seed)
    model = networks.SNN_axonal_recurrent_delays(cfg)
    rows = []
    trained = OracleModel(copy.deepcopy(model))
    history, final = run(cfg, 'cpu', trained, log=rows.append)
    assert rows == history and [r['epoch'] for r in history] == list(range(1, 13))
    losses = [r['loss'] for r in history]
    assert all(math.isfinite(v) for v in losses)
    # four balanced-ish classes: chance level ln 4 at the start, below it after training
    assert abs(losses[0] - math.log(4)) < 0.02
    assert losses[-1] < losses[0] - 0.005
    assert final['num_samples'] == cfg.num_samples
    # the delays moved and stay clamped at >= 0
    d0 = model.layers[2].recurrent_delays.detach()
    d1 = trained.inner.layers[2].recurrent_delays.detach()
    assert not torch.equal(d0, d1) and float(d1.min()) >= 0.0
