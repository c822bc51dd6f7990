"""GPU parity of the axonal layer (HIP kernels through the C ABI) against the CPU oracle.

Spikes must match exactly except at units whose oracle membrane is within 1e-5 of the
threshold (none occur on these seeds). Every gradient is held to the oracle run in float64
on the same values, teacher-forced with the device's spike train, at the fixed, unscaled
fp32 tolerance rtol 1e-4 / atol 1e-5; an element that misses it gets a floor of its own
(``helpers.check_grads``): the fp32 oracle's own distance from float64 there and, for dW,
the rounding budget of that element's terms. The forward's membrane and recurrent input,
read straight from the C ABI, are held to the fp32 oracle at the same unscaled tolerance.
The counts are printed.
"""

import pytest
import torch

from helpers import (assert_close, axonal_budget, check_grads, first_flip, gen, grad_eps, grads64,
                     lif_params, oracle_axonal)

RTOL, ATOL = 1e-4, 1e-5

CASES = [
    # T,  B,  N,  dmax, sigma, extra
    (24, 4, 32, 8.0, 0.0, {}),
    (24, 4, 32, 8.0, 0.5, {}),
    (20, 3, 64, 16.0, 1.0, {}),
    (16, 2, 256, 32.0, 1.0, {}),
    (16, 3, 48, 6.0, 1.3, {'bias': True}),
    (16, 3, 40, 6.0, 0.7, {'soft': True}),
    (16, 3, 40, 6.0, 0.7, {'decay_input': True}),
    (16, 3, 40, 6.0, 0.7, {'triangle': True}),
    (16, 3, 40, 6.0, 0.7, {'detach': True}),
    (16, 3, 40, 6.0, 0.7, {'sig_p': True}),
    (16, 3, 40, 6.0, 0.7, {'v_reset': -0.2}),
    (16, 2, 200, 20.0, 1.0, {'bias': True}),     # 4 x 32 tiles with padded rows (128 < N < 256)
    (16, 2, 136, 12.0, 0.6, {'sig_p': True}),
    (16, 2, 256, 32.0, 1.0, {'cj16': True}),     # the 8 x 16 tile layout at the same size
    (16, 2, 300, 10.0, 0.5, {}),                 # streamed-weight layout (N > 256)
    (12, 2, 24, 70.0, 0.0, {}),                  # window > 64 lags: two history words
    # straight-line kernels (soft taps, ATan, hard reset): long sequences crossing the
    # 32-step spike words and the prefetch blocks with a ragged tail, recurrent dropout
    (75, 2, 256, 32.0, 1.0, {}),
    (45, 3, 100, 12.0, 0.5, {'drop': True}),
    (37, 2, 160, 3.0, 0.0, {'bias': True, 'drop': True}),   # many sources with a lag-1 tap
    # T * B >= 1024: the dW GEMM's k splits come in multiples of 8, so the tiles of one k
    # chunk are grouped on one XCD (one 64-wide tile; then 2 x 2 tiles of 128)
    (32, 32, 64, 8.0, 1.0, {}),
    (64, 64, 256, 32.0, 1.0, {}),
]


def _run(dev, T, B, N, dmax, sigma, extra, seed=0, hint=False):
    from delrec.kernels import AxonalRecdelHip
    g = gen(seed)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    d = torch.rand(N, generator=g) * dmax
    gy = torch.randn(T, B, N, generator=g)
    bias = torch.randn(N, generator=g) * 0.1 if extra.get('bias') else None
    p = torch.randn(N, generator=g) if extra.get('sig_p') else None
    v_reset = None if extra.get('soft') else extra.get('v_reset', 0.0)
    surr = ('triangle', 1.0) if extra.get('triangle') else ('atan', 2.0)
    lif = lif_params(tau=2.0, v_reset=v_reset, decay_input=extra.get('decay_input', False),
                     detach_reset=extra.get('detach', False), surrogate=surr)
    drop = (torch.rand(B, N, generator=g) > 0.2).float() / 0.8 if extra.get('drop') else None
    y_ref, u_ref, gref = oracle_axonal(x, W, d, lif, sigma, gy, bias=bias, p=p,
                                       use_sig_p=p is not None, drop=drop)

    def oracle64(forced):
        """Float64 gradients teacher-forced with ``forced``, and dW's term budget (None under
        dropout or a learned spread, whose terms the budget does not model)."""
        g64 = oracle_axonal(x, W, d, lif, sigma, gy, bias=bias, p=p, use_sig_p=p is not None, drop=drop,
                            dtype=torch.float64, forced=forced)[2]
        plain = drop is None and p is None
        return g64, axonal_budget(g64['x'], forced, d, sigma) if plain else None

    leaves = [t.to(dev).requires_grad_(True) for t in (x, W, d)]
    bg = bias.to(dev).requires_grad_(True) if bias is not None else None
    pg = p.to(dev).requires_grad_(True) if p is not None else torch.zeros(N, device=dev)
    dg = drop.to(dev) if drop is not None else None
    # hint: a known max d, so the forward may run before reading the window length
    from delrec.kernels.recdel_base import apply_with_hint
    y, _ = apply_with_hint(float(d.max()) if hint else None,
                           leaves[0], leaves[1], bg, leaves[2], pg, dg, sigma, lif.tau,
                           lif.v_threshold, lif.v_reset, p is not None, lif.detach_reset,
                           0 if surr[0] == 'triangle' else 1, 1.0, False, 0, 2.0,
                           lif.decay_input)
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    return y.detach().cpu(), y_ref, u_ref, gref, leaves, bg, pg, lif, oracle64


# windows beyond the 256 lags of spike history the axonal kernels hold: the per-connection
# synaptic scans with d[i, j] = d[j] (soft taps), incl. a learned spread, bias, soft reset
LONG_CASES = [
    (320, 2, 48, 300.0, 0.5, {}),
    (300, 2, 40, 290.0, 0.7, {'sig_p': True}),
    (300, 2, 40, 280.0, 0.0, {'bias': True, 'soft': True}),
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', CASES + LONG_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}d{c[3]}s{c[4]}{"".join(c[5])}'
                                                          for c in CASES + LONG_CASES])
def test_axonal_fwd_bwd_matches_oracle(dev, case, monkeypatch):
    _check_case(dev, case, monkeypatch)


# the same with the largest delay already known (the deferred window read of the common regime)
@pytest.mark.gpu
@pytest.mark.parametrize('case', [CASES[i] for i in (1, 3, 16, 17, 18)],
                         ids=[f'T{c[0]}B{c[1]}N{c[2]}d{c[3]}' for c in [CASES[i] for i in (1, 3, 16, 17, 18)]])
def test_axonal_deferred_window_read_matches_oracle(dev, case, monkeypatch):
    _check_case(dev, case, monkeypatch, hint=True)


def _check_case(dev, case, monkeypatch, hint=False):
    T, B, N, dmax, sigma, extra = case
    print(f'case {case} hint={hint}', flush=True)
    if extra.get('cj16'):
        monkeypatch.setenv('DELREC_AXONAL_CJ', '16')
    y, y_ref, u_ref, gref, leaves, bg, pg, lif, oracle64 = _run(dev, T, B, N, dmax, sigma, extra, hint=hint)
    flip = first_flip(y, y_ref, u_ref, lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}; pick another seed'
    print(f'  spikes identical ({int(y.sum())} spikes of {y.numel()})')
    got = {'x': leaves[0].grad, 'W': leaves[1].grad, 'd': leaves[2].grad}
    if bg is not None:
        got['bias'] = bg.grad
    if 'p' in gref:
        got['p'] = pg.grad
    g64, budget = oracle64(y)
    check_grads(got, g64, gref, RTOL, ATOL, budget=budget, eps=grad_eps(False))


@pytest.mark.gpu
def test_axonal_forward_membrane_and_trace_via_abi(dev):
    """Membrane u and the saved delayed trace z, read straight from the C ABI outputs."""
    from delrec import _lib
    from delrec.kernels._common import bits_shape
    from oracle import scans
    T, B, N, sigma = 20, 3, 64, 1.0
    g = gen(3)
    x = torch.randn(T, B, N, generator=g) * 1.2 + 0.3
    W = torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)
    d = torch.rand(N, generator=g) * 10.0
    lif = lif_params()
    y_ref, ext = scans.axonal_v2(x, W, d, lif, sigma=sigma)
    L = ext['L']
    xs, Ws, ds = x.to(dev), W.to(dev), d.to(dev)
    y = torch.empty(T, B, N, device=dev)
    u = torch.empty_like(y)
    z = torch.empty_like(y)
    rec = torch.empty_like(y)
    bits = torch.zeros(bits_shape(T, B, N), device=dev, dtype=torch.int32)
    ws = _lib.workspace(_lib.WS_AXONAL_FWD, T, B, N, L, 0, dev)
    args = _lib.AxonalFwdArgs(T=T, B=B, N=N, L=L, x=_lib.ptr(xs), W=_lib.ptr(Ws), w_bf16=0,
                              bias=None, d=_lib.ptr(ds), s=None, s_uniform=1.0 + sigma, drop=None,
                              taps=0, lag=None, frac=None,
                              lif=_lib.make_lif(2.0, 1.0, 0.0, False, False, 1, 1.0, 2.0),
                              y=_lib.ptr(y), u=_lib.ptr(u), rec=_lib.ptr(rec), z=_lib.ptr(z),
                              bits=_lib.ptr(bits), workspace=_lib.ptr(ws), workspace_bytes=ws.numel())
    _lib.call('delrec_axonal_fwd', args, _lib.stream_of(xs))
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), y_ref)
    assert_close(u, ext['u'], RTOL, ATOL, 'u')
    assert_close(rec, ext['rec'], RTOL, ATOL, 'rec')
    # the bitmask holds the same spikes
    b = bits.cpu().to(torch.int64) & 0xFFFFFFFF
    t = torch.arange(T)
    unpacked = (b[:, t // 32, :] >> (t % 32).view(1, T, 1)) & 1         # (B, T, N)
    assert torch.equal(unpacked.permute(1, 0, 2).float(), y_ref)


@pytest.mark.gpu
def test_posted_max_matches_torch_max_and_detects_reused_slots(dev):
    """delrec_max_post / delrec_max_take (the forward's host read of max d, taken by the
    backward): the value torch.max gives, NaN included, for several posts outstanding at
    once and taken in reverse order; a slot reused by later posts is reported stale and
    PostedMax.value() then reads the maximum again."""
    import ctypes
    import math

    from delrec import _lib

    g = torch.Generator(device=dev).manual_seed(5)
    xs = [torch.randn(n, device=dev, generator=g) * 10 for n in (1, 7, 256, 1000, 4099)]
    xs.append(torch.full((5,), -3.0, device=dev))
    posts = [_lib.PostedMax(x) for x in xs]
    for x, p in reversed(list(zip(xs, posts))):
        assert p.value() == float(x.max())
    nan = torch.tensor([1.0, float('nan'), 2.0], device=dev)
    assert math.isnan(_lib.PostedMax(nan).value())

    first = _lib.PostedMax(xs[2])
    for _ in range(256):                       # DELREC_MAX_SLOTS later posts
        _lib.PostedMax(xs[0])
    torch.cuda.synchronize()
    out = ctypes.c_float(0.0)
    assert _lib.load().delrec_max_take(first.ticket, ctypes.byref(out), 1000) == 8   # DELREC_ERR_STALE
    assert first.value() == float(xs[2].max())
    # a ticket not posted yet: the wait ends at its time limit
    assert _lib.load().delrec_max_take(first.ticket + 100000, ctypes.byref(out), 50) == 7   # DELREC_ERR_PENDING


@pytest.mark.gpu
@pytest.mark.parametrize('fused', [True, False], ids=['in-scan', 'before-scan'])
def test_axonal_forward_posts_max_delay(dev, fused):
    """delrec_axonal_fwd with dmax_ticket: max d arrives in its readback slot, written by the
    straight-line scan's first workgroup (L = 0) or by the small kernel ahead of another
    scan (here the recurrent-input output rules out the straight-line form)."""
    import ctypes

    from delrec import _lib
    from delrec.kernels._common import bits_shape
    T, B, N, sigma = 20, 3, 64, 1.0
    g = gen(4)
    xs = (torch.randn(T, B, N, generator=g) * 1.2 + 0.3).to(dev)
    Ws = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).to(dev)
    ds = (torch.rand(N, generator=g) * 10.0).to(dev)
    y = torch.empty(T, B, N, device=dev)
    u, z, rec = torch.empty_like(y), torch.empty_like(y), torch.empty_like(y)
    bits = torch.zeros(bits_shape(T, B, N), device=dev, dtype=torch.int32)
    L = 0 if fused else 14
    ws = _lib.workspace(_lib.WS_AXONAL_FWD, T, B, N, max(L, 2), 0, dev)
    ticket = ctypes.c_uint32(0)
    args = _lib.AxonalFwdArgs(T=T, B=B, N=N, L=L, x=_lib.ptr(xs), W=_lib.ptr(Ws), w_bf16=0,
                              bias=None, d=_lib.ptr(ds), s=None, s_uniform=1.0 + sigma, drop=None,
                              taps=0, lag=None, frac=None,
                              lif=_lib.make_lif(2.0, 1.0, 0.0, False, False, 1, 1.0, 2.0),
                              y=_lib.ptr(y), u=_lib.ptr(u), rec=None if fused else _lib.ptr(rec),
                              z=_lib.ptr(z), bits=_lib.ptr(bits), workspace=_lib.ptr(ws),
                              workspace_bytes=ws.numel(), dmax_ticket=ctypes.pointer(ticket))
    _lib.call('delrec_axonal_fwd', args, _lib.stream_of(xs))
    assert ticket.value != 0
    out = ctypes.c_float(0.0)
    assert _lib.load().delrec_max_take(ticket.value, ctypes.byref(out), 5000) == 0
    assert out.value == float(ds.max())


@pytest.mark.gpu
def test_window_beyond_256_lags_through_the_layer(dev):
    """A layer whose delays reach 300 steps: the first call reads the window and takes the
    synaptic scans (parity with the oracle), and a wrong max-delay hint (the window jumped
    past the register history between two calls) still fails loudly: NaN outputs and an
    error in the backward, never silent spikes. (The hard-tap modes at such windows:
    test_gpu_modes.py.)"""
    from delrec.delay_layers import axonal_recdel
    from delrec import _lib
    from configs.perf_MEM import Config
    from oracle import scans
    cfg = Config()
    cfg.sigma_init = 0.5
    torch.manual_seed(0)
    layer = axonal_recdel(cfg, 64).to(dev)
    with torch.no_grad():
        layer.recurrent_delays[5] = 300.0
    x = torch.randn(310, 2, 64, generator=gen(3)) * 1.2 + 0.4
    print('forward + backward through the layer', flush=True)
    xg = x.to(dev).requires_grad_(True)
    y = layer(xg)
    gy = torch.randn(310, 2, 64, generator=gen(4))
    (y * gy.to(dev)).sum().backward()
    torch.cuda.synchronize()
    lif = lif_params(tau=float(layer.neuron_module.tau))
    xr = x.clone().requires_grad_(True)
    Wr = layer.recurrent_weights.detach().cpu().clone().requires_grad_(True)
    dr = layer.recurrent_delays.detach().cpu().clone().requires_grad_(True)
    y_ref, ext = scans.axonal_v2(xr, Wr, dr, lif, sigma=float(layer.sigma))
    (y_ref * gy).sum().backward()
    assert ext['L'] > 258
    flip = first_flip(y.detach().cpu(), y_ref.detach(), ext['u'].detach(), lif.v_threshold)
    assert flip is None, f'near-threshold flip at t={flip}'
    sigma = float(layer.sigma)
    g64 = grads64(lambda l, f: scans.axonal_v2(l['x'], l['W'], l['d'], lif, sigma=sigma, forced=f)[0],
                  {'x': xr, 'W': Wr, 'd': dr}, gy, y)
    check_grads({'x': xg.grad, 'W': layer.recurrent_weights.grad, 'd': layer.recurrent_delays.grad},
                g64, {'x': xr.grad, 'W': Wr.grad, 'd': dr.grad}, RTOL, ATOL,
                budget=axonal_budget(g64['x'], y, dr, sigma), eps=grad_eps(False))
    print('stale max-delay hint', flush=True)
    layer.zero_grad(set_to_none=True)
    assert layer._dmax_hint == 300.0
    layer._dmax_hint = 10.0
    xg = x[:20].to(dev).requires_grad_(True)
    y = layer(xg)
    torch.cuda.synchronize()
    assert bool(torch.isnan(y).all()), 'the forward must not return spikes it could not compute'
    with pytest.raises(Exception, match='256 lags'):
        y.sum().backward()
    torch.cuda.synchronize()
