"""CPU tests of the module / model API (no kernel launch).

Mirrors the CPU part of the reference's tests/test_hybrid_delay_invariance.py for the
recurrent classes (its feedforward half needs DCLS and is out of scope): state_dict and
initial values of the hybrid at ``hybrid_offset_scale == 0`` equal the axonal model's,
offsets are frozen integer buffers, invalid knobs raise; the forward comparisons run
through the oracle. Also the dispatch and error conventions of this build.
"""

import pytest
import torch

from oracle.model import reference_forward

T, B = 10, 4


def base_config(maximum):
    from configs.perf_MEM import Config
    cfg = Config()
    cfg.input_size = 8
    cfg.output_size = 3
    cfg.hidden_layers = [16]
    cfg.time_window = T
    cfg.batch_size = B
    cfg.use_batch_norm = False
    cfg.feedforward_dropout_rate = 0.0
    cfg.recurrent_dropout_rate = 0.0
    cfg.no_recurrence_in_last_layer = False
    cfg.kernel_count = 1
    cfg.hybrid_offset_scale = maximum
    cfg.hybrid_delay_seed = 123
    return cfg


def _probe(cfg):
    return torch.randn(cfg.time_window, B, cfg.input_size, generator=torch.Generator().manual_seed(7))


def test_maximum_zero_is_the_axonal_model():
    from delrec import networks
    cfg = base_config(0)
    torch.manual_seed(0)
    hybrid = networks.SNN_recurrent_hybrid_delays(cfg)
    torch.manual_seed(0)
    axonal = networks.SNN_axonal_recurrent_delays(cfg)
    hs, as_ = hybrid.state_dict(), axonal.state_dict()
    assert set(hs) == set(as_)
    for key in as_:
        assert torch.equal(hs[key], as_[key]), key
    x = _probe(cfg)
    hybrid.eval()
    axonal.eval()
    torch.testing.assert_close(reference_forward(hybrid, x), reference_forward(axonal, x), atol=1e-6, rtol=0)


def test_maximum_positive_keeps_axonal_delay_budget():
    from delrec import networks
    from delrec.delay_layers import axonal_recdel
    from delrec.networks import learned_delay_parameter
    cfg = base_config(4)
    torch.manual_seed(0)
    hybrid = networks.SNN_recurrent_hybrid_delays(cfg)
    torch.manual_seed(0)
    axonal = networks.SNN_axonal_recurrent_delays(base_config(0))
    h = [learned_delay_parameter(m, 'recurrent_delays') for m in hybrid.layers if isinstance(m, axonal_recdel)]
    a = [learned_delay_parameter(m, 'recurrent_delays') for m in axonal.layers if isinstance(m, axonal_recdel)]
    assert len(h) == len(a) == 1
    assert h[0].requires_grad and h[0].numel() == a[0].numel()
    offsets = [b for n, b in hybrid.named_buffers() if n.endswith('.offsets')]
    assert offsets and all(not b.requires_grad for b in offsets)
    assert all(int(b.max()) <= 4 and int(b.min()) >= 0 for b in offsets)
    hybrid.eval()
    out = reference_forward(hybrid, _probe(cfg))
    assert out.shape == (T, B, cfg.output_size) and torch.isfinite(out).all()


def test_hybrid_base_is_row_zero_of_the_initial_delays_centred():
    from delrec import networks
    cfg = base_config(4)
    cfg.hybrid_base_centering = 'centered'
    torch.manual_seed(0)
    syn = networks.SNN_synaptic_recurrent_delays(cfg)
    torch.manual_seed(0)
    hyb = networks.SNN_recurrent_hybrid_delays(cfg)
    d0 = syn.layers[2].recurrent_delays[0].detach()
    base = hyb.layers[2].parametrizations.recurrent_delays.original.detach()
    torch.testing.assert_close(base, d0 - 2.0)
    d = hyb.layers[2].recurrent_delays
    off = hyb.layers[2].parametrizations.recurrent_delays[0].offsets
    assert torch.equal(d, base[None, :] + off)


@pytest.mark.parametrize('bad', [-1, 1.5])
def test_maximum_must_be_nonnegative_integer(bad):
    from delrec import networks
    with pytest.raises(ValueError):
        networks.SNN_recurrent_hybrid_delays(base_config(bad))


def test_kernel_count_must_be_one():
    from delrec import networks
    cfg = base_config(4)
    cfg.kernel_count = 2
    with pytest.raises(ValueError):
        networks.SNN_recurrent_hybrid_delays(cfg)


def test_offset_distributions():
    from delrec.networks import _draw_offsets
    g = torch.Generator().manual_seed(0)
    for dist, sig in (('uniform', None), ('gaussian', 2.0), ('triangular', None)):
        o = _draw_offsets((50, 50), 6, g, dist, sig)
        assert o.min() >= 0 and o.max() <= 6 and torch.equal(o, o.round())
    with pytest.raises(ValueError):
        _draw_offsets((2, 2), 3, g, 'cauchy')


def test_forward_dispatch_and_errors():
    from delrec.delay_layers import axonal_recdel, synaptic_recdel
    cfg = base_config(0)
    ax = axonal_recdel(cfg, 8)
    x = torch.zeros(4, 2, 8)
    with pytest.raises(RuntimeError, match='GPU'):
        ax(x)                                      # CPU input: no fallback, a loud error
    ax.forward_version = 'v2'
    with pytest.raises(NotImplementedError):
        ax(x)
    ax.forward_version = 'eventdriven'
    with pytest.raises(ValueError):
        ax(x)
    syn = synaptic_recdel(cfg, 8)
    syn.forward_version = 'eventdriven_torch'
    with pytest.raises(ValueError):
        syn(x)
    syn.forward_version = 'nonsense'
    with pytest.raises(ValueError):
        syn(x)


def test_surrogate_ids():
    from delrec.kernels.surrogate import surrogate_id
    from delrec.neuron import ATan
    from delrec.utils import Triangle
    assert surrogate_id(ATan(3.0)) == (1, 1.0, 3.0)
    assert surrogate_id(Triangle.apply, 0.7) == (0, 0.7, 2.0)
    with pytest.raises(ValueError):
        surrogate_id(torch.sigmoid)


def test_drop_mask_normalisation():
    from delrec.kernels._common import drop_bn
    m = torch.rand(3, 5)
    assert torch.equal(drop_bn(m, 4, 3, 5), m)
    assert torch.equal(drop_bn(m.unsqueeze(0).expand(4, 3, 5), 4, 3, 5), m)
    assert drop_bn(None, 4, 3, 5) is None
    varying = torch.rand(4, 3, 5)
    with pytest.raises(ValueError):
        drop_bn(varying, 4, 3, 5)


def test_hard_lag_builders():
    from delrec.kernels.delays import build_lag, build_lag_interp
    d = torch.tensor([0.0, 0.4, 0.6, 2.5, 9.7])
    assert build_lag(d, 6).tolist() == [1, 1, 2, 3, 5]          # round half to even, clamp to L-1
    lag, frac = build_lag_interp(d, 12)
    assert lag.tolist() == [1, 1, 1, 3, 10]
    torch.testing.assert_close(frac, torch.tensor([0.0, 0.4, 0.6, 0.5, 0.7]))


def test_long_window_approx_delay_gradient_matches_the_oracle():
    """The long-window route's straight-through delay gradient of ``approx`` (host tensor
    algebra over the backward's dx and the spikes), fed the oracle's own dx and spikes, equals
    the oracle's autograd dd -- with dropout, and a negative delay clamped to lag 1."""
    from helpers import gen, lif_params
    from oracle import scans
    from delrec.kernels.delays import build_lag
    from delrec.kernels.recdel_base import _straight_through_dd
    T, B, N = 60, 2, 24
    g = gen(1)
    x = torch.randn(T, B, N, generator=g) * 1.1 + 0.35
    W = torch.randn(N, N, generator=g) * (4 / N ** 0.5)
    d = torch.rand(N, generator=g) * 40
    d[3] = -0.7
    drop = (torch.rand(B, N, generator=g) > 0.2).float() / 0.8
    xr, Wr, dr = (t.clone().requires_grad_(True) for t in (x, W, d))
    y, _ = scans.axonal_v2(xr, Wr, dr, lif_params(), sigma=0.0, taps='approx', drop=drop)
    (y * torch.randn(T, B, N, generator=g)).sum().backward()
    lag = build_lag(d, int(torch.round(d).max()) + 2)
    dd = _straight_through_dd(xr.grad, drop, W, y.detach(), (lag - 1).float())
    assert float(dr.grad.abs().max()) > 1.0
    torch.testing.assert_close(dd, dr.grad, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize('taps', ['ste_round', 'ste_interp'])
def test_long_window_ste_weight_gradient_matches_the_oracle(taps):
    """The long-window route's STE weight gradient (the gradient of rec against the forward's
    hard trace, host tensor algebra), fed the oracle's own dx and spikes, equals the oracle's
    autograd dW -- with dropout and a spread, whose soft taps the trace must not use."""
    from helpers import gen, lif_params
    from oracle import scans
    from delrec.kernels.delays import build_lag
    from delrec.kernels.recdel_base import _hard_trace_dw
    from delrec.kernels._common import window_length_f32
    T, B, N = 60, 2, 24
    g = gen(2)
    x = torch.randn(T, B, N, generator=g) * 1.1 + 0.35
    W = torch.randn(N, N, generator=g) * (4 / N ** 0.5)
    d = torch.rand(N, generator=g) * 40
    d[5] = -0.4
    drop = (torch.rand(B, N, generator=g) > 0.2).float() / 0.8
    xr, Wr, dr = (t.clone().requires_grad_(True) for t in (x, W, d))
    y, _ = scans.axonal_v2(xr, Wr, dr, lif_params(), sigma=0.7, taps=taps, drop=drop)
    (y * torch.randn(T, B, N, generator=g)).sum().backward()
    if taps == 'ste_round':
        d_tap = (build_lag(d, window_length_f32(float(d.max()), 1.7)) - 1).float()
    else:
        d_tap = d.clamp(min=0.0)
    dW = _hard_trace_dw(xr.grad, drop, y.detach(), d_tap)
    torch.testing.assert_close(dW, Wr.grad, rtol=1e-5, atol=1e-5)


def test_sigma_schedule_clamp_and_round():
    from delrec import networks
    from delrec.delay_layers import axonal_recdel
    cfg = base_config(0)
    cfg.sigma_init, cfg.sigma_decay, cfg.epochs = 2.0, 0.95, 50
    torch.manual_seed(0)
    model = networks.SNN_axonal_recurrent_delays(cfg)
    layer = [m for m in model.layers if isinstance(m, axonal_recdel)][0]
    layer.update_sigma(10)
    assert layer.sigma == pytest.approx(2.0 * (0.95 ** (100 / 50)) ** 10)
    assert 'sigma' not in ''.join(model.state_dict())
    with torch.no_grad():
        layer.recurrent_delays[:3] = torch.tensor([-1.0, 2.4, 2.6])
    model.round_pos()
    assert layer.recurrent_delays[:3].tolist() == [0.0, 2.0, 3.0]


def _round_up_share(model, layer, d, reps):
    """Fraction of stochastic roundings of ``d`` that went up, over ``reps`` calls."""
    ups, total = 0, 0
    for _ in range(reps):
        with torch.no_grad():
            layer.recurrent_delays.copy_(d)
        model.round_pos()
        r = layer.recurrent_delays.detach()
        assert torch.all((r == torch.floor(d)) | (r == torch.ceil(d)))
        ups += int((r > d).sum())
        total += r.numel()
    return ups / total


def test_stochastic_round_pos():
    """``round_mode = 'stochastic'``: ``floor(d + U[0, 1))``, so a delay goes up with
    probability frac(d), integers stay, negative ones clamp to 0 (reference
    ``networks.py:183-199``)."""
    from delrec import networks
    from delrec.delay_layers import axonal_recdel
    cfg = base_config(0)
    cfg.round_mode = 'stochastic'
    torch.manual_seed(0)
    model = networks.SNN_axonal_recurrent_delays(cfg)
    layer = [m for m in model.layers if isinstance(m, axonal_recdel)][0]
    n = layer.recurrent_delays.numel()
    d = torch.full((n,), 3.25)
    share = _round_up_share(model, layer, d, 400)        # 6400 draws: sd 0.0054
    assert abs(share - 0.25) < 0.025, share
    with torch.no_grad():
        layer.recurrent_delays.copy_(torch.linspace(-2.0, 5.0, n).round())
    ints = layer.recurrent_delays.detach().clone()
    model.round_pos()
    assert torch.equal(layer.recurrent_delays.detach(), ints.clamp(min=0))


def test_common_recdel_has_one_shared_delay():
    from delrec import networks
    cfg = base_config(0)
    torch.manual_seed(0)
    model = networks.SNN_common_recurrent_delays(cfg)
    layer = model.layers[2]
    assert layer.recurrent_delays.shape == (1,) and layer.forward_version is None


def test_fixed_models_freeze_delays():
    from delrec import networks
    cfg = base_config(4)
    torch.manual_seed(0)
    for cls in (networks.SNN_fixed_recurrent_delays, networks.SNN_fixed_synaptic_recurrent_delays,
                networks.SNN_fixed_hybrid_recurrent_delays, networks.SNN_vanilla_recurrent):
        model = cls(base_config(4))
        layer = model.layers[2]
        from delrec.networks import learned_delay_parameter
        leaf = learned_delay_parameter(layer, 'recurrent_delays')
        assert not leaf.requires_grad and layer.sigma == 0.0
        assert torch.equal(leaf, leaf.round())


def test_straight_line_forward_keeps_outputs_within_32_bit_offsets():
    """The straight-line axonal forward (L = 0, no host read of max d) addresses each
    (T, B, N) fp32 output with 32-bit byte offsets: larger calls take the general forward."""
    from delrec.kernels.recdel_base import STRAIGHT_LINE_MAX_ELEMS, _straight_line_forward
    assert STRAIGHT_LINE_MAX_ELEMS * 4 <= 1 << 30
    args = (256, 1.0, False, False, 0, False, 0.0)
    assert _straight_line_forward(*args, TB=128 * 128)
    assert _straight_line_forward(*args, TB=STRAIGHT_LINE_MAX_ELEMS // 256)
    assert not _straight_line_forward(*args, TB=STRAIGHT_LINE_MAX_ELEMS // 256 + 1)
    assert not _straight_line_forward(257, 1.0, False, False, 0, False, 0.0, TB=1)


def test_cpp_function_only_when_gradients_are_wanted():
    """The C++ autograd Function's forward does not read the window length (its backward
    rejects a window the forward could not hold), so it is taken only when gradients are
    wanted and the last max d seen for the delays leaves the register history room; otherwise
    the Python Function reads the window first (and routes a long one to the synaptic scans)."""
    from delrec.delay_layers import axonal_recdel
    cfg = base_config(0)
    cfg.sigma_init = 1.0
    layer = axonal_recdel(cfg, 32)
    x = torch.zeros(T, B, 32)
    d = layer.recurrent_delays
    # without a known max d (no earlier call) the window is read first
    assert not layer._cpp_function_applies(x.requires_grad_(True), d, None, False, 0, None)
    # a known max d whose window comes near the register history
    assert not layer._cpp_function_applies(x, d, None, False, 0, 240.0)
    assert layer._cpp_function_applies(x, d, None, False, 0, 20.0)
    assert layer._cpp_function_applies(torch.zeros(T, B, 32), d, None, False, 0, 20.0)   # W, d require grad
    with torch.no_grad():
        assert not layer._cpp_function_applies(x, d, None, False, 0, 20.0)
    for p in layer.parameters():
        p.requires_grad_(False)
    assert not layer._cpp_function_applies(torch.zeros(T, B, 32), d, None, False, 0, 20.0)
    for p in layer.parameters():
        p.requires_grad_(True)
    assert not layer._cpp_function_applies(x, d, None, True, 0, 20.0)      # approx
    assert not layer._cpp_function_applies(x, d, None, False, 1, 20.0)     # STE


def test_reference_import_path_resolves_to_the_hip_modules():
    """``delrec.triton_kernels`` (the reference's package, src/delrec/triton_kernels/
    __init__.py:64-73) names the HIP implementation's modules and objects."""
    import delrec.kernels as k
    from delrec.triton_kernels import AxonalRecdelTriton, build_syn_mask
    from delrec.triton_kernels.synaptic_hybrid import HybridSynDelay, hybrid_trainable_forward
    from delrec.triton_kernels.synaptic_eventdriven import EventDrivenSyn
    import delrec.triton_kernels.delays as tk_delays
    assert AxonalRecdelTriton is k.AxonalRecdelTriton and build_syn_mask is k.build_syn_mask
    assert HybridSynDelay is k.synaptic_hybrid.HybridSynDelay
    assert hybrid_trainable_forward is k.synaptic_hybrid.hybrid_trainable_forward
    assert EventDrivenSyn is k.synaptic_eventdriven.EventDrivenSyn
    assert tk_delays is k.delays


def test_spike_linear_falls_back_to_linear_without_bits():
    """Without spike bits (a CPU tensor, an analog input) SpikeLinear is torch's Linear."""
    from delrec.spike_linear import SpikeLinear
    torch.manual_seed(0)
    lin = SpikeLinear(12, 5)
    ref = torch.nn.Linear(12, 5)
    ref.load_state_dict(lin.state_dict())
    x = torch.rand(4, 3, 12)
    torch.testing.assert_close(lin(x), ref(x))
    assert isinstance(lin, torch.nn.Linear)


def test_spike_bits_follow_the_tensor_version():
    """Bits attached to a spike train are dropped once the tensor is modified in place, and
    the bits path is refused past the kernels' 32-bit addressing (CPU: no kernel runs)."""
    import torch
    from delrec.spike_linear import attach_bits, bits_path_fits, spike_bits
    y = torch.zeros(4, 2, 3)
    bits = torch.zeros(2, 1, 3, dtype=torch.int32)
    attach_bits(y, bits)
    assert spike_bits(y) is bits
    y.add_(1.0)
    assert spike_bits(y) is None
    assert spike_bits(torch.zeros(1)) is None
    assert bits_path_fits(1024, 512, 2048, 2048)
    assert not bits_path_fits(32 * 2048, 512, 2048, 2048)      # spike words past 2 GiB
    assert not bits_path_fits(32, 1, 40000, 40000)              # W planes past 2 GiB
