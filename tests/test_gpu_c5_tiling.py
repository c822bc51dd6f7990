"""C5 (two stacked hybrid layers, N = 2048, bf16 W) at the benchmark's own batch of 512 rows,
so that every kernel runs the tiling the benchmark times: the far product's 16 row tiles of
128 (on the sparse MFMA, its XCD-grouped form) at its 2 k-splits, the far LIF's 32 tiles of 16
rows, the near product's 16 row tiles of 128 at 16 k-splits, the near chain's 256 workgroups of 2 rows, the lag
correlation's 16 chunks of 32 rows (a batch of 32 runs one far row tile instead).

Batch rows are independent through the whole recurrence, and a row whose upstream
gradient is 0 contributes exactly 0 to every gradient. So the upstream gradient is N(0, 1)
on 8 rows spread over those tiles and 0 elsewhere, and the float64 oracle runs on those 8
rows only (teacher-forced with the kernel's spikes, as in test_gpu_configs.py): membranes
and dx of those rows, dx = 0 on all others, dW and dbase of the whole layer. The second
layer takes the first layer's output through the HIP Linear on its spike bits, times the
workload's gain, exactly as the benchmark feeds it. Each layer also runs twice: every
output must be bit-identical between the runs (the kernels add their partial sums in a
fixed order).
"""

import pytest
import torch

import bench
from helpers import check_elementwise, dw_term_sq_synaptic, gen, grad_eps, lif_params
from oracle import scans
from oracle.delays import syn_mask

ROWS = [0, 63, 64, 255, 256, 320, 448, 511]     # edges of the 64-, 128- and 256-row tiles
T_RUN = 80                                      # > the longest delay (61 + 4 offsets + 2)
THRESHOLD_BAND = 1e-5


def _run_layer(layer, x, gy, dev):
    """Forward + backward of one product layer; returns (y with its spike bits, u, dx, dW,
    dbase) on the device."""
    from delrec.kernels import synaptic_hybrid
    seen = {}
    fwd = synaptic_hybrid.syn_forward

    def keep(*a, **k):
        out = fwd(*a, **k)
        seen['u'] = out[1].detach().clone()
        return out

    synaptic_hybrid.syn_forward = keep
    try:
        layer.zero_grad(set_to_none=True)
        xg = x.detach().clone().requires_grad_(True)
        y = layer(xg)
        y.backward(gy)
        torch.cuda.synchronize()
    finally:
        synaptic_hybrid.syn_forward = fwd
    par = layer.parametrizations.recurrent_delays
    return (y.detach(), seen['u'], xg.grad.detach().clone(), layer.recurrent_weights.grad.detach().clone(),
            par.original.grad.detach().clone())


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_c5_at_benchmark_tiling_both_layers(dev, monkeypatch, capfd):
    monkeypatch.setenv('DELREC_LOG_PLAN', '1')
    w = bench.WORKLOADS['C5']
    m = bench.build(w, dev, T=T_RUN)
    T, B, N = m.x.shape
    assert B == 512 and N == 2048
    rows = torch.tensor(ROWS)
    lif = lif_params(tau=w['tau'])
    f64 = torch.float64
    x_in = m.x
    y_prev = None
    for k, layer in enumerate(m.layers):
        if k > 0:
            with torch.no_grad():
                x_in = (m.inter[k - 1](y_prev) * w['gain2']).contiguous()
        print(f'C5 layer {k + 1}: T={T} B={B} N={N}, upstream gradient on rows {ROWS}', flush=True)
        gy = torch.zeros(T, B, N)
        gy[:, rows] = torch.randn(T, len(ROWS), N, generator=gen(90 + k))
        gyd = gy.to(dev)
        first = _run_layer(layer, x_in, gyd, dev)
        second = _run_layer(layer, x_in, gyd, dev)
        for name, a, b in zip(('y', 'u', 'dx', 'dW', 'dbase'), first, second):
            assert torch.equal(a, b), f'layer {k + 1}: {name} differs between two identical runs'
        y, u, dx, dW, dbase = first
        plan = capfd.readouterr().err
        print(plan, flush=True)
        assert 'far sources' in plan and 'product KS=2, sparse 128x256 tiles, 16 row tiles' in plan, plan
        assert 'near sources' in plan and '(product KS=16 block, 16 row tiles' in plan, plan
        y_prev = y
        y_rows = y[:, rows].cpu()
        print(f'  firing rate {float(y.mean()):.4f} (rows: {float(y_rows.mean()):.4f})', flush=True)
        dx_cpu = dx.cpu()
        others = torch.ones(B, dtype=torch.bool)
        others[rows] = False
        assert bool((dx_cpu[:, others] == 0).all()), 'dx is not 0 on rows without upstream gradient'

        # the oracle on the 8 rows, float64, teacher-forced with the kernel's spikes
        par = layer.parametrizations.recurrent_delays
        leaves = {'x': x_in[:, rows].detach().cpu().to(f64).requires_grad_(True),
                  'W': layer.recurrent_weights.detach().cpu().to(f64).requires_grad_(True),
                  'base': par.original.detach().cpu().to(f64).requires_grad_(True)}
        d32 = par.original.detach().cpu() + 0.0 + 1.0 * par[0].offsets.detach().float().cpu()
        d = leaves['base'] + (d32.to(f64) - leaves['base'].detach())
        y_ref, ext = scans.synaptic_v2(leaves['x'], leaves['W'], d, lif, sigma=w['sigma'],
                                       forced=y_rows.to(f64))
        (y_ref * gy[:, rows].to(f64)).sum().backward()
        u_ref = ext['u'].detach()
        gap = (u_ref - lif.v_threshold).abs()
        fired = u_ref >= lif.v_threshold
        wrong = (fired != (y_rows != 0)) & (gap >= THRESHOLD_BAND)
        print(f'  oracle min |u - threshold| = {float(gap.min()):.3e}; units within {THRESHOLD_BAND:g}: '
              f'{int((gap < THRESHOLD_BAND).sum())}', flush=True)
        assert not bool(wrong.any()), f'{int(wrong.sum())} spikes differ away from the threshold band'

        ref32 = {}

        def oracle32():
            if not ref32:
                l32 = {n: v.detach().float().requires_grad_(True) for n, v in leaves.items()}
                y32, e32 = scans.synaptic_v2(l32['x'], l32['W'], l32['base'] + (d32 - l32['base'].detach()),
                                             lif, sigma=w['sigma'], forced=y_rows.float())
                (y32 * gy[:, rows]).sum().backward()
                ref32['u'] = e32['u'].detach()
                ref32.update({n: v.grad for n, v in l32.items()})
            return ref32

        def term_sq(idx):
            h, _ = syn_mask(d.detach(), w['sigma'])
            return dw_term_sq_synaptic(leaves['x'].grad, y_rows, h, idx)

        rtol, atol = 2e-2, 1e-5
        eps = grad_eps(True)
        check_elementwise('u', u[:, rows], u_ref, rtol, atol, ref32=lambda: oracle32()['u'])
        check_elementwise('dx', dx_cpu[:, rows], leaves['x'].grad, rtol, atol, ref32=lambda: oracle32()['x'])
        check_elementwise('dW', dW, leaves['W'].grad, rtol, atol, ref32=lambda: oracle32()['W'],
                          term_sq=term_sq, eps=eps)
        check_elementwise('dbase', dbase, leaves['base'].grad, rtol, atol, ref32=lambda: oracle32()['base'])
        del leaves, ref32
