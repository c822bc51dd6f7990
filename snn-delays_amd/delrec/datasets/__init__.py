"""Synthetic datasets of the DelRec experiments that this package trains on."""

from .spike_memorization import SpikeMemorization

__all__ = ['SpikeMemorization']
