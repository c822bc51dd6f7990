"""Training on the memorisation task: the optimiser, the per-epoch schedule and one epoch
over a loader (reference ``src/delrec/training/mem.py:12-81``), and a whole run
(reference ``experiments/train_mem.py:77-151``) without its files and plots.

The recurrent delay layers run on the HIP kernels; nothing here picks a device path: the
model's own forward does.
"""

import torch
from torch.nn import functional as F
from torch.utils.data import DataLoader

from ..datasets import SpikeMemorization
from ..delay_layers import axonal_recdel
from ..networks import learned_delay_parameter
from ..utils import reset_states, seed_everything


def make_optimizer(model, config):
    """AdamW over two groups: the delay positions (and ``p_spread``) of every recurrent
    delay layer at ``lr_positions`` without weight decay, every other trainable parameter
    at ``lr_w`` with ``weight_decay`` (reference ``mem.py:12-31``)."""
    positions = []
    for module in model.modules():
        if isinstance(module, axonal_recdel):
            positions.append(learned_delay_parameter(module, 'recurrent_delays'))
            if hasattr(module, 'p_spread'):
                positions.append(module.p_spread)
    taken = {id(p) for p in positions}
    weights = [p for p in model.parameters() if p.requires_grad and id(p) not in taken]
    return torch.optim.AdamW([
        {'params': weights, 'lr': config.lr_w, 'weight_decay': config.weight_decay},
        {'params': [p for p in positions if p.requires_grad], 'lr': config.lr_positions,
         'weight_decay': 0.0},
    ])


def set_epoch(model, config, epoch):
    """The epoch's spread of every recurrent delay layer (reference ``mem.py:34-40``)."""
    with torch.no_grad():
        for module in model.modules():
            if isinstance(module, axonal_recdel):
                module.update_sigma(epoch)


def readout_logits(outputs, config):
    """Logits from the ``(T, B, classes)`` outputs by the configured temporal readout."""
    if config.readout == 'mean':
        return outputs.mean(0)
    if config.readout == 'sum':
        return outputs.sum(0)
    if config.readout == 'last':
        return outputs[-1]
    raise ValueError(f'Unknown readout: {config.readout}')


def run_epoch(loader, model, device, config, optimizer=None):
    """One pass over ``loader``: a training epoch when ``optimizer`` is given (backward,
    gradient-norm clip, step, delay clamp per batch), else a measurement pass without
    gradients. Returns the mean loss, the accuracy and the counts (reference
    ``mem.py:43-81``)."""
    training = optimizer is not None
    model.train(training)
    loss_sum, correct, count = 0.0, 0, 0
    with torch.set_grad_enabled(training):
        for inputs, labels in loader:
            x = inputs.transpose(0, 1).contiguous().to(device)    # (T, B, C)
            labels = labels.to(device)
            reset_states(model)
            if training:
                optimizer.zero_grad(set_to_none=True)
            logits = readout_logits(model(x), config)
            loss = F.cross_entropy(logits, labels)
            if not torch.isfinite(loss):
                raise RuntimeError('Non-finite memorization loss')
            if training:
                loss.backward()
                if config.grad_clip > 0:
                    torch.nn.utils.clip_grad_norm_(model.parameters(), config.grad_clip)
                optimizer.step()
                if hasattr(model, 'clamp_delays'):
                    model.clamp_delays()
            n = labels.numel()
            loss_sum += loss.item() * n
            correct += int((logits.argmax(1) == labels).sum().item())
            count += n
    reset_states(model)
    return {'loss': loss_sum / count, 'accuracy_percent': 100.0 * correct / count,
            'correct': correct, 'num_samples': count}


def make_loaders(config):
    """The training loader (shuffled by a generator seeded with ``config.seed``) and the
    in-order measurement loader over the same dataset (reference ``train_mem.py:80-87``)."""
    data = SpikeMemorization(config.num_samples, config.input_size, config.time_window,
                             config.output_size, config.dataset_seed, config.input_gain,
                             config.task_type)
    train = DataLoader(data, batch_size=config.batch_size, shuffle=True,
                       generator=torch.Generator().manual_seed(config.seed), num_workers=0)
    measure = DataLoader(data, batch_size=config.batch_size, shuffle=False, num_workers=0)
    return train, measure


def run(config, device, model=None, *, log=None):
    """Train ``model`` (default: ``config.model`` built after seeding with ``config.seed``)
    for ``config.epochs`` epochs and measure it after each one. Returns the history (one
    ``{'epoch', 'loss', 'accuracy_percent', 'online_loss'}`` per epoch) and the final
    measurement. ``log(row)`` is called after each epoch when given."""
    seed_everything(config.seed)
    train, measure = make_loaders(config)
    if model is None:
        from .. import networks
        model = getattr(networks, config.model)(config)
    model = model.to(device)
    optimizer = make_optimizer(model, config)
    scheduler = torch.optim.lr_scheduler.CosineAnnealingLR(optimizer, T_max=config.epochs)
    history, final = [], None
    for epoch in range(config.epochs):
        set_epoch(model, config, epoch)
        online = run_epoch(train, model, device, config, optimizer)
        final = run_epoch(measure, model, device, config)
        row = {'epoch': epoch + 1, 'loss': final['loss'], 'accuracy_percent': final['accuracy_percent'],
               'online_loss': online['loss']}
        history.append(row)
        if log is not None:
            log(row)
        scheduler.step()
    return history, final
