"""GPU parity of the synaptic and hybrid layers against the CPU oracle.

Spikes: identical to the fp32 oracle's except within 1e-5 of the threshold (none occur on
these seeds). Gradients: against the oracle run in float64 on the same values,
teacher-forced with the device's spike train, at fixed, unscaled tolerances -- fp32 W rtol
1e-4, bf16 W rtol 2e-2, atol 1e-5 -- where an element that misses them gets a floor of its
own (``helpers.check_grads``): the fp32 oracle's own distance from float64 there and, for
dW, dd and dbase, the rounding budget of that element's own terms (per-term error 2^-20 for
fp32 W, 2^-15 for bf16 W and for the stacked per-step product scans forced at these sizes
with fp32 W). The counts are printed.
"""

import pytest
import torch

from helpers import (STACKED_EPS, axonal_budget, check_grads, first_flip, gen, grad_eps, lif_params,
                     oracle_axonal, oracle_synaptic, syn_budget)

RTOL, ATOL = 1e-4, 1e-5

SYN_CASES = [
    # T,  B,  N,  dmax, sigma, extra
    (20, 3, 32, 6.0, 0.0, {}),
    (20, 3, 32, 6.0, 0.5, {}),
    (16, 2, 64, 10.0, 1.0, {'bias': True}),
    (16, 2, 48, 6.0, 0.8, {'sig_p': True}),
    (16, 2, 48, 6.0, 0.8, {'soft': True, 'triangle': True}),
    (16, 2, 48, 6.0, 0.8, {'decay_input': True}),
    (18, 3, 40, 6.0, 0.5, {'drop': True, 'bias': True}),   # fixed-mask recurrent dropout
    (12, 2, 96, 4.0, 4.0, {}),                  # wide triangle
    (12, 2, 40, 6.0, 8.0, {}),                  # half-width 9: runtime tap count
    (70, 2, 700, 60.0, 1.0, {}),                # rings too large for LDS: gather forward, workspace ring
    (130, 2, 400, 110.0, 1.0, {}),              # as above with a two-word spike history
]


def _syn_inputs(T, B, N, dmax, extra, seed):
    g = gen(seed)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    d = torch.rand(N, N, generator=g) * dmax
    gy = torch.randn(T, B, N, generator=g)
    bias = torch.randn(N, generator=g) * 0.1 if extra.get('bias') else None
    p = torch.randn(N, generator=g) if extra.get('sig_p') else None
    return x, W, d, gy, bias, p


class _Layer:
    """Minimal stand-in carrying what EventDrivenSyn / HybridSynDelay read from a layer."""

    def __init__(self, sigma, lif, use_sig_p=False, p=None, round_delays=False):
        from delrec.neuron import LIFNode, ATan
        from delrec.utils import Triangle

        class Cfg:
            pass

        cfg = Cfg()
        kind, width = lif.surrogate
        cfg.surrogate_function = ATan(width) if kind == 'atan' else Triangle.apply
        cfg.surrogate_gamma = width if kind == 'triangle' else 1.0
        cfg.detach_reset = lif.detach_reset
        cfg.recurrent_dropout_rate = 0.0
        self.config = cfg
        self.neuron_module = LIFNode(tau=lif.tau, decay_input=lif.decay_input,
                                     v_threshold=lif.v_threshold, v_reset=lif.v_reset,
                                     detach_reset=lif.detach_reset)
        self.sigma = sigma
        self.use_sig_p = use_sig_p
        self.p_spread = p
        self.round_delays = round_delays
        self.training = False


@pytest.mark.gpu
@pytest.mark.parametrize('case', SYN_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}d{c[3]}s{c[4]}{"".join(c[5])}'
                                                for c in SYN_CASES])
def test_synaptic_fwd_bwd_matches_oracle(dev, case, eps=None):
    from delrec.kernels import EventDrivenSyn
    T, B, N, dmax, sigma, extra = case
    print(f'case {case}', flush=True)
    x, W, d, gy, bias, p = _syn_inputs(T, B, N, dmax, extra, seed=1)
    drop = (torch.rand(B, N, generator=gen(7)) > 0.2).float() / 0.8 if extra.get('drop') else None
    v_reset = None if extra.get('soft') else 0.0
    surr = ('triangle', 1.0) if extra.get('triangle') else ('atan', 2.0)
    lif = lif_params(v_reset=v_reset, decay_input=extra.get('decay_input', False), surrogate=surr)
    y_ref, u_ref, gref = oracle_synaptic(x, W, d, lif, sigma, gy, bias=bias, p=p, use_sig_p=p is not None,
                                         drop=drop)

    xg, Wg, dg = (t.to(dev).requires_grad_(True) for t in (x, W, d))
    bg = bias.to(dev).requires_grad_(True) if bias is not None else None
    pg = p.to(dev).requires_grad_(True) if p is not None else torch.zeros(N, device=dev)
    layer = _Layer(sigma, lif, use_sig_p=p is not None, p=pg if p is not None else None)
    y = EventDrivenSyn.apply(xg, Wg, dg, pg, bg, drop.to(dev) if drop is not None else None, layer)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    flip = first_flip(y.detach().cpu(), y_ref, u_ref, lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    print(f'  spikes identical ({int(y_ref.sum())} spikes of {y_ref.numel()})')
    got = {'x': xg.grad, 'W': Wg.grad, 'd': dg.grad}
    if bg is not None:
        got['bias'] = bg.grad
    if p is not None:
        got['p'] = pg.grad
    _, _, g64 = oracle_synaptic(x, W, d, lif, sigma, gy, bias=bias, p=p, use_sig_p=p is not None, drop=drop,
                                dtype=torch.float64, forced=y)
    # the spread indexed by the source under sig_p is not modelled: dW's budget there is none
    budget = syn_budget(g64['x'], y, d, sigma, W=W, drop=drop) if p is None else None
    check_grads(got, g64, gref, RTOL, ATOL, budget=budget, eps=eps or grad_eps(False))


# the lag-stacked per-step GEMM scans (taken by default only where the rings do not fit
# LDS, the last two cases above) forced at every size; the same oracle and tolerances
LAGSTEP_CASES = [SYN_CASES[i] for i in (0, 1, 2, 3, 4, 5, 6, 7, 8)] + [
    (5, 2, 64, 20.0, 1.0, {}),     # a run shorter than one 8-step block, far lags present
    (40, 3, 200, 30.0, 2.0, {}),   # several blocks, N not a multiple of the 128-wide tiles
    (14, 2, 50, 8.0, 1.0, {'bias': True}),   # N not a multiple of 4: one neuron per LIF thread
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', LAGSTEP_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}d{c[3]}s{c[4]}{"".join(c[5])}'
                                                    for c in LAGSTEP_CASES])
def test_synaptic_lagstep_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_LAGSTEP', '1')
    test_synaptic_fwd_bwd_matches_oracle(dev, case, eps=STACKED_EPS)


# the per-connection gather forward and workspace-ring backward at the sizes that take the
# lag-stacked scans by default
@pytest.mark.gpu
@pytest.mark.parametrize('case', SYN_CASES[-2:], ids=[f'T{c[0]}B{c[1]}N{c[2]}d{c[3]}' for c in SYN_CASES[-2:]])
def test_synaptic_gather_path_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_LAGSTEP', '0')
    test_synaptic_fwd_bwd_matches_oracle(dev, case)


HYB_CASES = [
    # T, B, N, base range (lo, hi), max offset, bf16 weights, sigma
    (20, 3, 32, (0.0, 8.0), 4, False, 0.0),
    (20, 3, 64, (-2.0, 6.0), 4, False, 0.0),     # centred base: negative effective delays
    (16, 2, 48, (0.0, 10.0), 8, True, 0.0),      # bf16 W_rec, fp32 state
    (16, 2, 40, (-1.0, 7.0), 3, False, 0.7),     # mid-anneal triangle, four taps per column
    (12, 2, 32, (0.0, 6.0), 3, False, 8.0),      # half-width 9: runtime tap count
    (80, 2, 700, (0.0, 55.0), 8, True, 0.0),     # gather forward (two history words), workspace ring
    (24, 2, 300, (0.0, 20.0), 5, True, 0.0),     # split backward: 640 threads, an odd chunk count
]


def mem_config(**kw):
    from configs.perf_MEM import Config
    cfg = Config()
    for k, v in kw.items():
        setattr(cfg, k, v)
    return cfg


def hybrid_layer(N, W, base, offsets, dev, bf16=False, **cfg_kw):
    """A product ``synaptic_recdel`` carrying the hybrid parametrisation with the given
    weights, base and offsets."""
    from delrec.delay_layers import synaptic_recdel
    from delrec.networks import _reparametrize_recurrent_delay
    cfg = mem_config(hybrid_base_centering='normal', **cfg_kw)
    layer = synaptic_recdel(cfg, N)
    _reparametrize_recurrent_delay(layer, int(offsets.max().item()) or 1, gen(5), cfg)
    with torch.no_grad():
        layer.parametrizations.recurrent_delays.original.copy_(base)
        layer.parametrizations.recurrent_delays[0].offsets.copy_(offsets)
    layer.recurrent_weights = torch.nn.Parameter(W.bfloat16() if bf16 else W.clone())
    return layer.to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize('case', HYB_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}{"bf16" if c[5] else ""}s{c[6]}'
                                                for c in HYB_CASES])
def test_hybrid_fwd_bwd_matches_oracle(dev, case, eps=None):
    """Hybrid delays through the base + int8-offset kernel path of a parametrised layer."""
    import delrec.kernels.synaptic_hybrid as sh
    T, B, N, (lo, hi), K, bf16, sigma = case[:7]
    k0 = case[7] if len(case) > 7 else 0     # smallest offset (offsets uniform in k0 .. K)
    wide = len(case) > 8 and case[8]         # weights over a wide range of magnitudes
    print(f'case {case}', flush=True)
    g = gen(2)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    if wide:   # columns scaled by 2^-20 .. 2^4, entries within a column by 2^-12 .. 1
        W = W * torch.exp2(torch.randint(-20, 5, (1, N), generator=g).float()) \
              * torch.exp2(torch.randint(-12, 1, (N, N), generator=g).float())
    if bf16:
        W = W.bfloat16().float()
    base = lo + torch.rand(N, generator=g) * (hi - lo)
    offsets = (k0 + torch.randint(K - k0 + 1, (N, N), generator=g)).float()
    gy = torch.randn(T, B, N, generator=g)
    lif = lif_params()
    y_ref, u_ref, gref = oracle_synaptic(x, W, None, lif, sigma, gy, base=base, offsets=offsets)

    layer = hybrid_layer(N, W, base, offsets, dev, bf16=bf16, sigma_init=sigma)
    assert layer.sigma == sigma
    base8, _, _ = sh._int8_offsets(layer)
    assert base8 is not None, 'the base + int8 offsets path was not taken'
    xg = x.to(dev).requires_grad_(True)
    y = layer.multi_step_forward_hybrid_triton(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    flip = first_flip(y.detach().cpu(), y_ref, u_ref, lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    print(f'  spikes identical ({int(y_ref.sum())} spikes of {y_ref.numel()})')
    _check_hybrid_grads(xg.grad, layer, y, x, W, base, offsets, lif, sigma, gy, gref, bf16, eps)


def _check_hybrid_grads(dx, layer, y, x, W, base, offsets, lif, sigma, gy, gref, bf16, eps=None):
    """dx, dW and dbase of a hybrid layer's run against the float64 oracle (module docstring);
    ``eps``: dW's per-term budget where it exceeds the weight type's."""
    _, _, g64 = oracle_synaptic(x, W, None, lif, sigma, gy, base=base, offsets=offsets,
                                dtype=torch.float64, forced=y)
    got = {'x': dx, 'W': layer.recurrent_weights.grad.float(),
           'base': layer.parametrizations.recurrent_delays.original.grad}
    d = base[None, :] + 0.0 + 1.0 * offsets
    check_grads(got, g64, gref, 2e-2 if bf16 else RTOL, ATOL, eps=max(eps or 0.0, grad_eps(bf16)),
                budget=syn_budget(g64['x'], y, d, sigma, W=W, hybrid=True))


# the reference's invariant (tests/test_hybrid_delay_invariance.py:59-78) across the two HIP
# paths: the hybrid layer with every offset 0 is the axonal layer with d = base -- the same
# spikes, and dx, dW and dd (axonal) = dbase (hybrid) to the fp32 tolerance
@pytest.mark.gpu
@pytest.mark.parametrize('case', [(24, 3, 64, (0.0, 12.0), 0.0), (24, 2, 96, (1.0, 6.0), 1.0)],
                         ids=['T24B3N64s0', 'T24B2N96s1'])
def test_hybrid_zero_offsets_equal_axonal_on_device(dev, case):
    from delrec.kernels import AxonalRecdelHip
    T, B, N, (lo, hi), sigma = case
    g = gen(3)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    base = lo + torch.rand(N, generator=g) * (hi - lo)
    gy = torch.randn(T, B, N, generator=g)
    lif = lif_params()

    layer = hybrid_layer(N, W, base, torch.zeros(N, N), dev, sigma_init=sigma)
    xh = x.to(dev).requires_grad_(True)
    yh = layer.multi_step_forward_hybrid_triton(xh)
    (yh * gy.to(dev)).sum().backward()

    xa, Wa, da = (t.to(dev).requires_grad_(True) for t in (x, W, base))
    ya = AxonalRecdelHip.apply(xa, Wa, None, da, torch.zeros(N, device=dev), None, sigma, lif.tau,
                               lif.v_threshold, lif.v_reset, False, lif.detach_reset, 1, 1.0, False, 0,
                               2.0, lif.decay_input)
    (ya * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(yh.detach(), ya.detach()), 'spike trains differ'
    print(f'  spikes identical ({int(ya.sum())} spikes of {ya.numel()})')
    # both paths against the one axonal oracle (d = base), the gradients in float64
    y_ref, u_ref, g32 = oracle_axonal(x, W, base, lif, sigma, gy)
    flip = first_flip(ya.detach().cpu(), y_ref, u_ref, lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    _, _, g64 = oracle_axonal(x, W, base, lif, sigma, gy, dtype=torch.float64, forced=ya)
    budget = axonal_budget(g64['x'], ya, base, sigma)
    for path, got in (('hybrid', {'x': xh.grad, 'W': layer.recurrent_weights.grad.float(),
                                  'd': layer.parametrizations.recurrent_delays.original.grad}),
                      ('axonal', {'x': xa.grad, 'W': Wa.grad, 'd': da.grad})):
        print(f' {path}:')
        check_grads(got, g64, g32, RTOL, ATOL, budget=budget, eps=grad_eps(False))


@pytest.mark.gpu
@pytest.mark.parametrize('case', HYB_CASES[:5] + HYB_CASES[6:], ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}{"bf16" if c[5] else ""}s{c[6]}'
                                                    for c in HYB_CASES[:5] + HYB_CASES[6:]])
def test_hybrid_lagstep_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_LAGSTEP', '1')
    test_hybrid_fwd_bwd_matches_oracle(dev, case, eps=STACKED_EPS)


@pytest.mark.gpu
def test_hybrid_gather_path_matches_oracle(dev, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_LAGSTEP', '0')
    test_hybrid_fwd_bwd_matches_oracle(dev, HYB_CASES[5])


# the offset-stacked hybrid scans (taken by default where the rings do not fit LDS, as at
# N = 2048) forced at small sizes: bases >= s - 1 (every tap at a lag >= 1), offsets up to 8,
# fp32 and bf16 weights, one and two spike-history words (windows of 65+ lags), a triangle of
# three taps (sigma 0.5); the backward's split of the sources by first lag (near: lof < 4,
# per-step product; far: per-block product) with both parts, only far sources (bases >= 10)
# and only near ones (bases < 2.5), runs of T not a multiple of the block
HYBSTEP_CASES = [HYB_CASES[i] for i in (0, 2, 5, 6)] + [
    (20, 2, 64, (1.0, 12.0), 4, False, 0.5),
    (33, 3, 130, (0.0, 25.0), 2, True, 0.0),
    (21, 2, 96, (10.0, 20.0), 3, False, 0.0),
    (19, 3, 80, (0.0, 2.5), 3, True, 0.0),
    # bf16 W, 9 offsets at N = 288: the far product's 81 k-stages over 10 splits of 9, the
    # last split empty (its partial must come out zero)
    (20, 2, 288, (0.0, 25.0), 9, True, 0.0),
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', HYBSTEP_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}{"bf16" if c[5] else ""}s{c[6]}'
                                                    for c in HYBSTEP_CASES])
def test_hybrid_offset_stacked_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_HYBSTEP', '1')
    monkeypatch.setenv('DELREC_HYB_FWD', '0')    # the offset-stacked forward, not the arrival scatter
    test_hybrid_fwd_bwd_matches_oracle(dev, case, eps=STACKED_EPS)


# the hybrid forward as a scatter on arrival (the default for bf16 W, bases >= s - 1, at most
# 16 offsets, 4 taps and 2048 neurons): two and four compiled taps (sigma 0.5 runs three taps
# on the four-tap kernel), one and two spike-history words, two neurons per lane (N > 1024,
# the second half of the lanes partly idle), a smallest offset of 2 under negative bases. The
# offset field holds slot bytes where the ring's R slots are 2^16 bytes: 16 slots of one
# neuron per lane (9 offsets with two and with four taps), 8 slots of two (N = 1100); the
# other cases take the offset byte
ARRIVE_CASES = [
    (20, 3, 64, (0.0, 8.0), 4, True, 0.0),
    HYB_CASES[2],
    (20, 2, 64, (1.0, 12.0), 4, True, 0.5),
    (24, 2, 96, (1.0, 6.0), 4, True, 1.0),
    HYB_CASES[5],
    (12, 2, 1100, (0.0, 30.0), 4, True, 0.0),
    (20, 2, 64, (-1.5, 6.0), 6, True, 0.0, 2),
    (20, 2, 64, (0.0, 8.0), 9, True, 0.0),
    (24, 2, 96, (1.0, 6.0), 9, True, 1.0),
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', ARRIVE_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}s{c[6]}k{c[7] if len(c) > 7 else 0}'
                                                   for c in ARRIVE_CASES])
def test_hybrid_arrival_forward_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_HYB_FWD', '1')
    test_hybrid_fwd_bwd_matches_oracle(dev, case)


# the per-connection forwards on the bf16 cases the arrival scatter takes by default
@pytest.mark.gpu
@pytest.mark.parametrize('idx', [2, 5, 6])
def test_hybrid_per_connection_forward_matches_oracle(dev, idx, monkeypatch):
    monkeypatch.setenv('DELREC_HYB_FWD', '0')
    test_hybrid_fwd_bwd_matches_oracle(dev, HYB_CASES[idx])


# the hybrid backward with one lane per source (the split form is the default for N <= 512)
@pytest.mark.gpu
@pytest.mark.parametrize('case', [HYB_CASES[i] for i in (0, 2, 3, 6)],
                         ids=[f'T{c[0]}B{c[1]}N{c[2]}' for c in [HYB_CASES[i] for i in (0, 2, 3, 6)]])
def test_hybrid_unsplit_backward_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_BWD_SPLIT', '0')
    monkeypatch.setenv('DELREC_SYN_BWD_HYB_G', '0')
    test_hybrid_fwd_bwd_matches_oracle(dev, case)


# the split hybrid backward in its per-tap gather form, on the cases the offset-stacked form
# takes by default (every lag >= 1, at most 12 offsets)
@pytest.mark.gpu
@pytest.mark.parametrize('case', [HYB_CASES[i] for i in (0, 2, 6)],
                         ids=[f'T{c[0]}B{c[1]}N{c[2]}' for c in [HYB_CASES[i] for i in (0, 2, 6)]])
def test_hybrid_tap_gather_backward_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_SYN_BWD_HYB_G', '0')
    test_hybrid_fwd_bwd_matches_oracle(dev, case)


# the offset-stacked hybrid backward (G_j(t + 1) per step, a G history per source; taken by
# default where every lag is >= 1 and the offsets span at most 12): four taps at half-widths
# 1.5 and 2 (fp32 and bf16 W), offsets spanning 6 and 12 steps (ring pitches 16 and 24), an odd
# chunk count, bases from 0 (a zero-weight tap at lag 0), bf16 weights spread over 2^-32 .. 2^4;
# HYB_CASES 0, 2 and 6 take it too
HYB_G_CASES = [
    (20, 3, 64, (1.0, 12.0), 4, False, 0.5),
    (24, 2, 96, (1.0, 6.0), 4, True, 1.0),
    (30, 2, 80, (0.0, 14.0), 11, True, 0.0),
    (18, 3, 200, (0.0, 9.0), 5, False, 0.0),
    (20, 2, 128, (0.0, 10.0), 6, True, 0.0, 0, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', HYB_G_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}s{c[6]}{"w" if len(c) > 8 else ""}'
                                                   for c in HYB_G_CASES])
def test_hybrid_offset_stacked_backward_matches_oracle(dev, case, monkeypatch):
    monkeypatch.setenv('DELREC_HYB_FWD', '0')
    test_hybrid_fwd_bwd_matches_oracle(dev, case)


@pytest.mark.gpu
def test_delay_grad_known_answer(dev):
    """The reference's known-answer inputs (tests/check_hybrid_kernel.py:143-152) with the
    expected values worked out by hand: for s = 1 the closed form picks the two or three
    lags around 1 + d with signs -1 / 0 / +1, and C[..., l] = l^2."""
    from delrec.kernels import _delay_grad
    from delrec.kernels.delays import build_syn_mask
    values = torch.tensor([0.0, 1.0, 2.0, 0.25, 1.5])
    d = values.repeat(5, 1)
    W = torch.arange(1, 26).float().reshape(5, 5) / 25
    # sigma = 0: d=0 -> C2-C0 = 4; d=1 -> C3-C1 = 8; d=2 -> C4-C2 = 12; d=.25 -> C2-C1 = 3; d=1.5 -> C3-C2 = 5
    expected = W * torch.tensor([4.0, 8.0, 12.0, 3.0, 5.0])
    for sigma in (0.0, 0.5, 1.0):
        mask, L = build_syn_mask(d.clone().requires_grad_(True), sigma, None, False)
        C = torch.arange(L).float().square().expand(5, 5, L).contiguous()
        dr = d.clone().requires_grad_(True)
        m2, _ = build_syn_mask(dr, sigma, None, False)
        ref, = torch.autograd.grad((m2 * W.unsqueeze(-1) * C).sum(), dr)
        actual = _delay_grad(C.to(dev), W.to(dev), d.to(dev), sigma, L).cpu()
        torch.testing.assert_close(actual, ref, atol=2e-5, rtol=2e-5)
        assert ref[:, :3].abs().max() > 0
        if sigma == 0.0:
            torch.testing.assert_close(actual, expected, atol=1e-6, rtol=1e-6)


def _negative_base_without_smallest_offset(N, K, seed):
    """Bases in [0, 8) except source 0 at -0.5, whose column has no connection at the
    smallest offset 0 (every offset in column 0 is 1 .. K): its materialised delays are all
    >= 0.5, so the smallest materialised delay (0.5 or more) is >= s - 1 = 0, while the
    source's delay at the smallest offset, base_0 + 0 = -0.5, is not."""
    g = gen(seed)
    base = torch.rand(N, generator=g) * 8.0
    base[0] = -0.5
    offsets = torch.randint(K + 1, (N, N), generator=g).float()
    offsets[:, 0] = 1.0 + torch.randint(K, (N,), generator=g).float()
    assert bool((offsets[:, 1:] == 0).any())
    return base, offsets


def _hybrid_run(dev, T, B, N, W, base, offsets, bf16, sigma, x, gy):
    layer = hybrid_layer(N, W, base, offsets, dev, bf16=bf16, sigma_init=sigma)
    xg = x.to(dev).requires_grad_(True)
    y = layer.multi_step_forward_hybrid_triton(xg)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    return y.detach().cpu(), xg.grad.cpu(), layer


# the source whose base is the smallest has no connection at the smallest offset: the
# offset-stacked and arrival forms (which give a source the triangle of base_j + smallest
# offset) must not be taken on the smallest *materialised* delay -- whatever form each
# setting selects must match the oracle
NEG_BASE_FORMS = [{}, {'DELREC_HYB_FWD': '1'}, {'DELREC_SYN_HYBSTEP': '1', 'DELREC_HYB_FWD': '0'},
                  {'DELREC_SYN_HYBSTEP': '1'}, {'DELREC_SYN_BWD_HYB_G': '1'}]


@pytest.mark.gpu
@pytest.mark.parametrize('bf16', [True, False], ids=['bf16', 'fp32'])
@pytest.mark.parametrize('env', NEG_BASE_FORMS, ids=['default', 'arrival', 'hybstep', 'hybstep_arrival', 'hyb_g'])
def test_hybrid_negative_base_without_smallest_offset(dev, env, bf16, monkeypatch):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    T, B, N, K = 20, 3, 64, 4
    print(f'forms {env} bf16={bf16}', flush=True)
    base, offsets = _negative_base_without_smallest_offset(N, K, seed=4)
    g = gen(6)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    x[:, :, 0] += 1.5                      # source 0 fires often
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    if bf16:
        W = W.bfloat16().float()
    gy = torch.randn(T, B, N, generator=g)
    lif = lif_params()
    y_ref, u_ref, gref = oracle_synaptic(x, W, None, lif, 0.0, gy, base=base, offsets=offsets)
    assert float(y_ref[:, :, 0].sum()) > 0
    y, dx, layer = _hybrid_run(dev, T, B, N, W, base, offsets, bf16, 0.0, x, gy)
    flip = first_flip(y, y_ref, u_ref, lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    _check_hybrid_grads(dx, layer, y, x, W, base, offsets, lif, 0.0, gy, gref, bf16)


# the same case handed to the C ABI with a d_min that wrongly claims every source's taps
# at lags >= 1 (the smallest materialised delay instead of min_j base_j + off_min): the
# forms that rely on it write NaN where the dropped taps would have landed -- never a
# silently wrong result
@pytest.mark.gpu
@pytest.mark.parametrize('env', [{'DELREC_HYB_FWD': '1'}, {'DELREC_SYN_HYBSTEP': '1', 'DELREC_HYB_FWD': '0'},
                                 {'DELREC_SYN_BWD_HYB_G': '1'}], ids=['arrival', 'hybstep', 'hyb_g'])
def test_hybrid_wrong_d_min_gives_nan(dev, env, monkeypatch):
    from delrec.kernels import synaptic_eventdriven as se
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    real = se.hybrid_form
    monkeypatch.setattr(se, 'hybrid_form', lambda d_min, s, rng: real(0.5, s, rng))
    T, B, N, K = 20, 3, 64, 4
    base, offsets = _negative_base_without_smallest_offset(N, K, seed=4)
    g = gen(6)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    x[:, :, 0] += 1.5
    W = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).bfloat16().float()
    gy = torch.randn(T, B, N, generator=g)
    seen = {}
    fwd = se.syn_forward

    def keep(*a, **k):
        out = fwd(*a, **k)
        seen['u'] = out[1].detach()
        return out

    import delrec.kernels.synaptic_hybrid as sh
    monkeypatch.setattr(sh, 'syn_forward', keep)
    y, dx, _ = _hybrid_run(dev, T, B, N, W, base, offsets, True, 0.0, x, gy)
    u = seen['u'].cpu()
    print(f'  NaN membranes {int(u.isnan().sum())}, NaN dx {int(dx.isnan().sum())}', flush=True)
    if env.get('DELREC_SYN_BWD_HYB_G'):
        assert bool(dx.isnan().all())                # the whole backward refuses
    else:
        assert bool(u.isnan().any()) and bool(dx.isnan().any())


# the same layer handed to the C ABI with an offset range one short of the offsets' own (a
# caller's out-of-contract off_count): the forward packs each connection at the largest
# offset as a NaN weight in its receiver's own ring column, so those receivers' membranes
# turn NaN once the source fires -- never a silently dropped or misplaced connection
@pytest.mark.gpu
def test_hybrid_arrival_offsets_past_the_stated_range_give_nan(dev, monkeypatch):
    from delrec.kernels import synaptic_eventdriven as se
    monkeypatch.setenv('DELREC_HYB_FWD', '1')
    real = se.hybrid_form
    monkeypatch.setattr(se, 'hybrid_form', lambda d_min, s, rng: real(d_min, s, None if rng is None else (rng[0], rng[1] - 1)))
    T, B, N, K = 20, 3, 96, 4
    print(f'T={T} B={B} N={N}, offsets 0..{K}, stated {K} offsets', flush=True)
    g = gen(8)
    x = torch.randn(T, B, N, generator=g) * 1.5 + 0.5
    W = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).bfloat16().float()
    base = 1.0 + torch.rand(N, generator=g) * 6.0
    offsets = torch.randint(K + 1, (N, N), generator=g).float()
    seen = {}
    fwd = se.syn_forward

    def keep(*a, **k):
        out = fwd(*a, **k)
        seen['u'] = out[1].detach()
        return out

    import delrec.kernels.synaptic_hybrid as sh
    monkeypatch.setattr(sh, 'syn_forward', keep)
    gy = torch.randn(T, B, N, generator=g)
    _hybrid_run(dev, T, B, N, W, base, offsets, True, 0.0, x, gy)
    u = seen['u'].cpu()
    print(f'  NaN membranes {int(u.isnan().sum())} of {u.numel()}', flush=True)
    assert bool(u.isnan().any())
    assert not bool(u[0].isnan().any()), 'no input has arrived at step 0: its membranes are finite'


# bases exactly 0 (where training clamps them): the source's first tap sits at lag 0 with
# weight 0, which the offset-stacked backward reads as a zero-weight tap, not as a tap below
# lag 1 (its safety net must not fire)
@pytest.mark.gpu
@pytest.mark.parametrize('bf16', [True, False], ids=['bf16', 'fp32'])
def test_hybrid_zero_base_edge_tap(dev, bf16):
    T, B, N, K = 20, 3, 64, 4
    g = gen(8)
    base = torch.rand(N, generator=g) * 6.0
    base[::3] = 0.0
    offsets = torch.randint(K + 1, (N, N), generator=g).float()
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    if bf16:
        W = W.bfloat16().float()
    gy = torch.randn(T, B, N, generator=g)
    lif = lif_params()
    y_ref, u_ref, gref = oracle_synaptic(x, W, None, lif, 0.0, gy, base=base, offsets=offsets)
    y, dx, layer = _hybrid_run(dev, T, B, N, W, base, offsets, bf16, 0.0, x, gy)
    flip = first_flip(y, y_ref, u_ref, lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    assert bool(torch.isfinite(dx).all())
    _check_hybrid_grads(dx, layer, y, x, W, base, offsets, lif, 0.0, gy, gref, bf16)
