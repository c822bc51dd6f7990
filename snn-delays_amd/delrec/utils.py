"""Surrogate functions and state helpers of the DelRec API (reference ``src/delrec/utils.py``).

Only the pieces the recurrent-layer path uses are provided: ``Triangle`` (the reference's
surrogate id 0, ``utils.py:23-41``), ``reset_states`` (``utils.py:43-46``) and the
seeding helper. Losses, metrics and progress bars belong to the reference's training
drivers and are not part of this build.
"""

import math
import random

import numpy as np
import torch


class Triangle(torch.autograd.Function):
    """Heaviside forward, ``(1/gamma^2) * max(0, gamma - |x|)`` backward."""

    @staticmethod
    def forward(ctx, input, gamma=1.0):
        ctx.save_for_backward(input)
        ctx.gamma = float(gamma)
        return input.ge(0.0).to(input.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        (x,) = ctx.saved_tensors
        g = ctx.gamma
        return grad_output * ((1 / g) * (1 / g) * (g - x.abs()).clamp(min=0)), None


class ATanFunction(torch.autograd.Function):
    """Heaviside forward, ``(alpha/2) / (1 + (pi/2 * alpha * x)^2)`` backward."""

    @staticmethod
    def forward(ctx, x, alpha):
        ctx.save_for_backward(x)
        ctx.alpha = float(alpha)
        return (x >= 0).to(x.dtype)

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        a = ctx.alpha
        z = (math.pi / 2 * a) * x
        return (a / 2) / (1 + z * z) * grad, None


def reset_states(model):
    """Call ``reset()`` on every submodule that has one (neuron state, dropout masks)."""
    for m in model.modules():
        if hasattr(m, 'reset'):
            m.reset()


def seed_everything(seed):
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)
