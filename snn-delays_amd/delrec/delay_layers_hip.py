"""Layer-side glue between the delay-layer modules and the HIP autograd Functions.

Counterpart of the reference's ``delrec/delay_layers_triton.py`` mixins
(``AxonalTritonScans.multi_step_forward_triton`` :21-79,
``SynapticTritonScans.multi_step_forward_eventdriven`` :85-96,
``SynapticHybridScans.multi_step_forward_hybrid_triton`` :108-112): it reads the layer's
configuration (surrogate id and width, recurrent dropout mask fixed over time, optional
bias and learned spread, STE-rounded delays) and calls the Function. The method names
are the reference's, so code that calls them directly keeps working.
"""

import os

import torch

from . import _lib
from .kernels import AxonalRecdelHip, eventdriven_trainable_forward, hybrid_trainable_forward
from .kernels._common import require_device
from .kernels.recdel_base import STRAIGHT_LINE_MAX_ELEMS, apply_with_hint, deferred_read_safe
from .kernels.surrogate import surrogate_id


class AxonalHipScans:
    """Fused scans for per-neuron (axonal) delays."""

    def multi_step_forward_triton(self, x_seq, approx=False, ste_mode=0):
        require_device(x_seq)
        T, B, N = x_seq.shape
        gamma_cfg = getattr(self.config, 'surrogate_gamma', None)
        sid, gamma, alpha = surrogate_id(self.config.surrogate_function, gamma_cfg)
        if self.training and self.config.recurrent_dropout_rate > 0:
            drop = self.dropout(torch.ones(B, N, device=x_seq.device, dtype=x_seq.dtype))
        else:
            drop = None
        if self.use_sig_p:
            p_spread = self.p_spread
        else:
            # a zero spread the Function differentiates nothing against: kept, not re-made
            p_spread = getattr(self, '_zero_spread', None)
            if p_spread is None or p_spread.shape != (N,) or p_spread.device != x_seq.device \
                    or p_spread.dtype != x_seq.dtype:
                p_spread = torch.zeros(N, device=x_seq.device, dtype=x_seq.dtype)
                self._zero_spread = p_spread
        bias = self.recurrent_bias if self.use_rec_bias else None
        if ste_mode:
            ste_mode = 1 if getattr(self.config, 'ste_round_forward', True) else 2
        d_in = self.recurrent_delays
        if d_in.numel() == 1 and N > 1:       # common_recdel: one delay shared by the layer
            d_in = d_in.expand(N)
        if self.round_delays:
            d_in = d_in + (d_in.round() - d_in).detach()
        nm = self.neuron_module
        hint = self._refresh_dmax_hint(d_in)
        ext = _lib.torch_ext()
        if ext is not None and self._cpp_function_applies(x_seq, d_in, bias, approx, ste_mode, hint):
            if not getattr(self, '_dmax_from_ext', False):
                ext.forget_dmax(d_in.detach())
                self._dmax_from_ext = True
            # the common regime: the C++ autograd Function over the same C ABI (no Python on
            # the forward or backward path, no window-length read in the forward)
            y = ext.axonal_common(x_seq, self.recurrent_weights, d_in, bias, drop, float(self.sigma),
                                  float(nm.tau), float(nm.v_threshold), int(sid), float(gamma),
                                  float(alpha), bool(self.config.detach_reset))
        else:
            y = self._axonal_function(x_seq, d_in, bias, drop, p_spread, sid, gamma, alpha, approx,
                                      ste_mode, hint)
        self.x_seq = x_seq
        self.rec_now_seq = None
        if self.store_v_seq:
            self.v_seq = None
        return y

    def _refresh_dmax_hint(self, d_in):
        """The largest delay of a recent call, which lets the forward run before reading the
        window length (None: unknown). The Python Function's read sets it; after a call of
        the C++ Function it is the max d that Function's backward took for these delays --
        kept by the extension per delay storage, whose entry the layer clears when it first
        hands its delays over (an entry written before could belong to freed memory that the
        delays now occupy)."""
        ext = _lib.torch_ext()
        d = d_in.detach()
        if ext is not None and getattr(self, '_dmax_from_ext', False) and d.is_cuda:
            v = ext.seen_dmax(d)
            if v == v:
                self._dmax_hint = float(v)
        return getattr(self, '_dmax_hint', None)

    def _cpp_function_applies(self, x_seq, d_in, bias, approx, ste_mode, dmax_hint=None):
        """Whether the call takes the C++ autograd Function: the common regime (soft taps of
        a uniform half-width up to 8 lags of non-zero weight, decay charge, hard reset to 0,
        N <= 256) and gradients wanted. Its forward does not read the window length (its
        backward does, and rejects a window the forward could not hold); without gradients
        the Python Function reads the window length first, so an over-long window raises at
        the forward."""
        nm = self.neuron_module
        N = x_seq.shape[-1]
        wants_grad = torch.is_grad_enabled() and (
            x_seq.requires_grad or self.recurrent_weights.requires_grad or d_in.requires_grad
            or (bias is not None and bias.requires_grad))
        return (wants_grad and not approx and not ste_mode and not self.use_sig_p and N <= 256
                and deferred_read_safe(dmax_hint, self.sigma)
                and x_seq.numel() <= STRAIGHT_LINE_MAX_ELEMS and x_seq.dtype == torch.float32
                and nm.v_reset is not None and float(nm.v_reset) == 0.0
                and not getattr(nm, 'decay_input', False) and 0.0 <= float(self.sigma) <= 3.0
                and os.environ.get('DELREC_AXONAL_FWD') != 'tiled')

    def _axonal_function(self, x_seq, d_in, bias, drop, p_spread, sid, gamma, alpha, approx, ste_mode,
                         dmax_hint=None):
        nm = self.neuron_module
        y, dmax = apply_with_hint(
            dmax_hint, x_seq, self.recurrent_weights, bias, d_in, p_spread, drop,
            float(self.sigma), nm.tau, nm.v_threshold, nm.v_reset, self.use_sig_p,
            self.config.detach_reset, sid, gamma, approx, ste_mode, alpha,
            getattr(nm, 'decay_input', False))
        if dmax is not None:
            self._dmax_hint = dmax
        return y


class SynapticHipScans:
    """Spike-sparse scan for per-connection (synaptic) delays."""

    def multi_step_forward_eventdriven(self, x_seq):
        require_device(x_seq)
        y = eventdriven_trainable_forward(self, x_seq)
        self.x_seq = x_seq
        self.rec_now_seq = None
        if self.store_v_seq:
            self.v_seq = None
        return y


class SynapticHybridScans:
    """Scan for hybrid recurrent delays (learned per-source base + frozen integer offsets)."""

    def multi_step_forward_hybrid_triton(self, x_seq):
        require_device(x_seq)
        return hybrid_trainable_forward(self, x_seq)
