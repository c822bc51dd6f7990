"""GPU parity of the hybrid backward's products on the 4:2 sparse MFMA (``far_sparse_kernel``,
csrc/farsparse.hip): the default for the far sources in the offset-stacked scans with bf16
W, blocks of 4 steps and 3 .. 6 offsets (one to three sparse products per 32 receivers), and
for the near ones with DELREC_NEAR_SPARSE=1 (set in every test here).

Against the float64 oracle (``test_gpu_synaptic.test_hybrid_fwd_bwd_matches_oracle``, offset-stacked scans
forced): each offset count of the form, one and two 256-column tiles, row tiles past the
batch's last row, a triangle of three taps, T not a multiple of the block. On a batch of 128
rows, where the tiles take the XCD-grouped order, against the dense far product with the
near-block product (``DELREC_FAR_SPARSE=0``) and against both products as plain strided GEMMs
(``DELREC_NEAR_BLOCK=0`` too): the same gradients up to the order of fp32 sums (both products are exact
in their bf16 operands), and bit-identical results from two runs of the sparse form.
"""

import pytest
import torch

from helpers import gen
from test_gpu_synaptic import hybrid_layer
from test_gpu_synaptic import test_hybrid_fwd_bwd_matches_oracle as hybrid_parity   # (not collected here)

SPARSE_CASES = [
    # T, B, N, base range (lo, hi), max offset, bf16 weights, sigma
    (21, 3, 300, (0.0, 25.0), 4, True, 0.0),     # 5 offsets (three products), two column tiles
    (18, 2, 200, (0.0, 20.0), 2, True, 0.0),     # 3 offsets (two products)
    (20, 2, 130, (1.0, 25.0), 5, True, 0.5),     # 6 offsets, three taps (bases >= s - 1)
    (17, 3, 96, (0.0, 15.0), 3, True, 0.0),      # 4 offsets, one column tile
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', SPARSE_CASES, ids=[f'T{c[0]}B{c[1]}N{c[2]}K{c[4]}s{c[6]}' for c in SPARSE_CASES])
def test_far_sparse_matches_oracle(dev, case, monkeypatch, capfd):
    monkeypatch.setenv('DELREC_SYN_HYBSTEP', '1')
    monkeypatch.setenv('DELREC_NEAR_SPARSE', '1')
    monkeypatch.setenv('DELREC_HYB_FWD', '0')
    monkeypatch.setenv('DELREC_LOG_PLAN', '1')
    hybrid_parity(dev, case)
    plan = capfd.readouterr().err
    print(plan, flush=True)
    assert 'sparse 128x256 tiles' in plan, plan
    if 'near sources 0 ' not in plan:
        assert ' sparse, ' in plan, plan   # the near product on the sparse MFMA as well


def _grads(layer, x, gy):
    layer.zero_grad(set_to_none=True)
    xg = x.detach().clone().requires_grad_(True)
    y = layer.multi_step_forward_hybrid_triton(xg)
    (y * gy).sum().backward()
    torch.cuda.synchronize()
    par = layer.parametrizations.recurrent_delays
    return (y.detach().clone(), xg.grad.detach().clone(), layer.recurrent_weights.grad.detach().float().clone(),
            par.original.grad.detach().clone())


@pytest.mark.gpu
def test_far_sparse_matches_dense_product(dev, monkeypatch, capfd):
    T, B, N = 14, 128, 520
    print(f'T={T} B={B} N={N}, 5 offsets, bf16 W', flush=True)
    g = gen(21)
    x = (torch.randn(T, B, N, generator=g) * 1.2 + 0.3).to(dev)
    W = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).bfloat16().float()
    base = torch.rand(N, generator=g) * 30.0
    offsets = torch.randint(5, (N, N), generator=g).float()
    gy = torch.randn(T, B, N, generator=g).to(dev)
    layer = hybrid_layer(N, W, base, offsets, dev, bf16=True, sigma_init=0.0)
    monkeypatch.setenv('DELREC_SYN_HYBSTEP', '1')
    monkeypatch.setenv('DELREC_NEAR_SPARSE', '1')
    monkeypatch.setenv('DELREC_LOG_PLAN', '1')
    sparse = _grads(layer, x, gy)
    again = _grads(layer, x, gy)
    plan = capfd.readouterr().err
    assert 'sparse 128x256 tiles, 4 row tiles' in plan, plan
    monkeypatch.setenv('DELREC_FAR_SPARSE', '0')
    monkeypatch.delenv('DELREC_NEAR_SPARSE')
    block = _grads(layer, x, gy)          # dense far product, near-block product
    plan = capfd.readouterr().err
    assert 'far sources' in plan and 'sparse' not in plan and ' block, ' in plan, plan
    monkeypatch.setenv('DELREC_NEAR_BLOCK', '0')
    dense = _grads(layer, x, gy)          # both products as plain strided GEMMs
    plan = capfd.readouterr().err
    assert 'far sources' in plan and 'sparse' not in plan and ' block, ' not in plan, plan
    for name, a, b, c, d in zip(('y', 'dx', 'dW', 'dbase'), sparse, again, block, dense):
        assert torch.equal(a, b), f'{name} differs between two runs of the sparse product'
        ref = float(d.abs().max())
        for other, label in ((a, 'sparse'), (c, 'near-block')):
            err = float((other - d).abs().max())
            print(f'  {name}: max |{label} - dense| {err:.3e} (|dense| max {ref:.3e})', flush=True)
            if name == 'y':
                assert torch.equal(other, d), 'the forward differs'
            elif name == 'dW':
                # returned in bf16 (W's dtype): fp32 sums a few ulps apart may round to adjacent
                # bf16 values, one bf16 ulp (2^-7 relative at most) apart
                torch.testing.assert_close(other, d, rtol=2.0 ** -7, atol=1e-5 * ref)
            else:
                torch.testing.assert_close(other, d, rtol=1e-4, atol=1e-5 * ref)
