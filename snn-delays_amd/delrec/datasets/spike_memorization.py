"""The memorisation task: fixed random input patterns with independent random labels
(reference ``src/delrec/datasets/spike_memorization.py:7-46``).

A seed fixes the whole set. The draws follow the reference's order on one CPU generator,
so a seed gives the same samples here as there: for ``temporal`` patterns, one spike time
per (sample, input neuron) from ``randint(0, seq_length)``, the spike carrying
``input_gain``; for ``spatial`` patterns, one constant current per (sample, input neuron)
from ``rand * input_gain``; then the labels from ``randint(0, n_classes)``.
"""

import torch
from torch.utils.data import Dataset


class SpikeMemorization(Dataset):
    """``(x, label)`` pairs, ``x`` of shape ``(seq_length, n_input)``."""

    def __init__(self, num_samples, n_input, seq_length, n_classes, seed=0, input_gain=1.0,
                 task_type='temporal'):
        self.num_samples, self.n_input = int(num_samples), int(n_input)
        self.seq_length, self.n_classes = int(seq_length), int(n_classes)
        self.input_gain, self.task_type = float(input_gain), task_type
        if min(self.num_samples, self.n_input, self.seq_length, self.n_classes) < 1:
            raise ValueError('Sample, input, time and class counts must be positive.')
        gen = torch.Generator().manual_seed(int(seed))
        S, C, T = self.num_samples, self.n_input, self.seq_length
        if task_type == 'temporal':
            when = torch.randint(0, T, (S, C), generator=gen)
            x = torch.zeros(S, T, C)
            # one spike per (sample, input neuron), at time when[s, c]
            x.scatter_(1, when.unsqueeze(1), torch.full((S, 1, C), self.input_gain))
        elif task_type == 'spatial':
            level = torch.rand(S, C, generator=gen) * self.input_gain
            x = level.unsqueeze(1).repeat(1, T, 1)
        else:
            raise ValueError(f"Unknown task_type: {task_type!r}. Use 'temporal' or 'spatial'.")
        self.inputs = x
        self.labels = torch.randint(0, self.n_classes, (S,), generator=gen).long()

    def __len__(self):
        return self.num_samples

    def __getitem__(self, idx):
        return self.inputs[idx], self.labels[idx]
