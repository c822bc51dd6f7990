"""GPU parity of the binary-activation Linear (``delrec_spike_linear_fwd`` and
``delrec_spike_linear_dw`` through ``delrec.spike_linear.SpikeLinear``) against
``torch.nn.functional.linear`` and its autograd in float64 on the same spikes and weights.
The spikes are exact; W (forward) and g (weight gradient) enter as bf16 hi + mid + lo (about
2^-25 relative), so the tolerance is fp32's: rtol 1e-5, atol 1e-6, unscaled (gradients rtol
1e-4, atol 1e-5), where an element whose terms cancel gets the fp32 accumulation budget of its
own terms, 4 * 2^-20 * sqrt(sum of its squared terms) (``helpers.check_elementwise``; 2^-16
per term for the split bf16 input gradient). Shapes cover T, K and M off their tile multiples (128 steps, 32
neurons, 128 outputs), with and without bias, inputs mostly or wholly silent (the kernels take
the input neurons in activity order and skip the silent ones), and the bits attached by a
recurrent layer.
"""

import numpy as np
import pytest
import torch

from helpers import check_elementwise, gemm_term_sq, gen, grad_eps


def pack_bits(y):
    """(T, B, K) {0, 1} -> (B, ceil(T/32), K) spike words (bit t % 32 of word t // 32)."""
    T, B, K = y.shape
    TW = (T + 31) // 32
    yy = np.zeros((TW * 32, B, K), dtype=np.uint64)
    yy[:T] = y.numpy().astype(np.uint64)
    words = np.zeros((B, TW, K), dtype=np.uint64)
    for i in range(32):
        words |= yy[i::32].transpose(1, 0, 2) << np.uint64(i)
    return torch.from_numpy(words.astype(np.uint32).view(np.int32))


CASES = [
    # T, B, K, M, bias, firing rate, silent input fraction
    (64, 3, 64, 128, False, 0.05, 0.0),
    (70, 5, 300, 130, True, 0.1, 0.0),
    (200, 2, 33, 7, True, 0.5, 0.0),
    (129, 4, 2048, 256, False, 0.03, 0.0),
    (96, 4, 700, 200, True, 0.08, 0.7),     # most inputs silent: the stages below them skipped
    (40, 2, 300, 64, False, 0.1, 1.0),      # every input silent: out = bias, dW = 0
]


@pytest.mark.gpu
@pytest.mark.parametrize('case', CASES, ids=[f'T{c[0]}B{c[1]}K{c[2]}M{c[3]}{"b" if c[4] else ""}q{c[6]}' for c in CASES])
def test_spike_linear_matches_linear(dev, case):
    from delrec.spike_linear import SpikeLinear, attach_bits
    T, B, K, M, bias, rate, quiet = case
    print(f'case {case}', flush=True)
    g = gen(11)
    y = (torch.rand(T, B, K, generator=g) < rate).float()
    y[:, :, torch.randperm(K, generator=g)[:int(quiet * K)]] = 0.0
    lin = SpikeLinear(K, M, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(M, K, generator=g) / K ** 0.5)
        if bias:
            lin.bias.copy_(torch.randn(M, generator=g))
    ref = torch.nn.functional.linear(y.double(), lin.weight.double(), None if not bias else lin.bias.double())
    lin = lin.to(dev)
    xg = attach_bits(y.to(dev).requires_grad_(True), pack_bits(y).to(dev))
    out = lin(xg)
    assert out.grad_fn is not None and 'SpikeLinear' in type(out.grad_fn).__name__, 'the HIP path was not taken'
    gout = torch.randn(T, B, M, generator=g)
    out.backward(gout.to(dev))
    torch.cuda.synchronize()
    # unscaled tolerances; an element whose terms cancel gets the fp32 accumulation budget of
    # its own terms (4 * 2^-20 * sqrt(sum of its squared terms), helpers.check_elementwise)
    y2, w64, g2 = y.reshape(-1, K), lin.weight.detach().cpu().double(), gout.reshape(-1, M)
    check_elementwise('out', out.detach().reshape(-1, M), ref.reshape(-1, M), 1e-5, 1e-6,
                      term_sq=gemm_term_sq(y2, w64.t()), eps=grad_eps(False))
    # the backward (dW on the spike bits, dx torch's GEMM at these sizes): against float64 autograd
    xr = y.double().requires_grad_(True)
    wr = lin.weight.detach().cpu().double().requires_grad_(True)
    torch.nn.functional.linear(xr, wr).backward(gout.double())
    check_elementwise('dx', xg.grad.reshape(-1, K), xr.grad.reshape(-1, K), 1e-4, 1e-5,
                      term_sq=gemm_term_sq(g2, w64), eps=grad_eps(False))
    check_elementwise('dW', lin.weight.grad, wr.grad, 1e-4, 1e-5, term_sq=gemm_term_sq(g2.t(), y2),
                      eps=grad_eps(False))


@pytest.mark.gpu
def test_recurrent_layer_output_feeds_the_spike_gemm(dev):
    """A hybrid layer's output carries its spike bits; the Linear after it reads them and
    matches the fp32 GEMM on the same spikes."""
    import bench
    w = bench.WORKLOADS['C3']
    m = bench.build(w, dev, T=40, B=8)
    from delrec.spike_linear import SpikeLinear
    with torch.no_grad():
        y = m.layers[0](m.x)
    from delrec.spike_linear import spike_bits
    bits = spike_bits(y)
    assert bits is not None and tuple(bits.shape) == (8, 2, w['N'])
    lin = SpikeLinear(w['N'], 96, bias=True).to(dev)
    with torch.no_grad():
        out = lin(y)
        ref = torch.nn.functional.linear(y.double(), lin.weight.double(), lin.bias.double())
    torch.cuda.synchronize()
    assert float(y.mean()) > 0
    N = w['N']
    check_elementwise('out', out.reshape(-1, 96), ref.reshape(-1, 96), 1e-5, 1e-6,
                      term_sq=gemm_term_sq(y.reshape(-1, N), lin.weight.detach().t()), eps=grad_eps(False))


@pytest.mark.gpu
@pytest.mark.parametrize('shape', [(40, 512, 2048, 2048), (33, 8, 4100, 4096)], ids=['c5_width', 'unsplit'])
def test_spike_linear_weight_gradient_at_the_c5_width(dev, shape):
    """dW = g^T y on the bits at the inter-layer width of C5 (K = M = 2048, 512 batch rows:
    128 tiles of 128 x 256, split four ways over the steps, the tiles of one output tile and
    split grouped on one XCD), and at a width whose 512 tiles run unsplit with K off the tile
    multiple, against float64."""
    from delrec.spike_linear import spike_linear_dw
    T, B, K, M = shape
    g = gen(12)
    y = (torch.rand(T, B, K, generator=g) < 0.03).float()
    gout = torch.randn(T, B, M, generator=g)
    dW = spike_linear_dw(gout.to(dev), pack_bits(y).to(dev), K)
    torch.cuda.synchronize()
    ref = gout.reshape(-1, M).double().t() @ y.reshape(-1, K).double()
    err = (dW.cpu().double() - ref).abs()
    print(f'  dW max abs err {float(err.max()):.3e}, |ref|max {float(ref.abs().max()):.3e}', flush=True)
    # fp32 accumulation of about 600 O(1) terms per entry: rtol 1e-5, atol 1e-5 unscaled; an
    # entry whose terms cancel gets the fp32 accumulation budget of its own terms
    check_elementwise('dW', dW, ref, 1e-5, 1e-5, term_sq=gemm_term_sq(gout.reshape(-1, M).t(), y.reshape(-1, K)),
                      eps=grad_eps(False))


@pytest.mark.gpu
def test_spike_linear_ignores_bits_of_a_modified_tensor(dev):
    """Bits attached to a spike train describe it only until it is modified in place: after
    that the Linear takes torch.nn.functional.linear on the tensor's current values."""
    from delrec.spike_linear import SpikeLinear, attach_bits, spike_bits
    T, B, K, M = 33, 2, 40, 24
    y = (torch.rand(T, B, K, generator=gen(13)) < 0.2).float()
    lin = SpikeLinear(K, M).to(dev)
    yg = attach_bits(y.to(dev), pack_bits(y).to(dev))
    assert 'SpikeLinear' in type(lin(yg.requires_grad_(True)).grad_fn).__name__
    with torch.no_grad():
        yg.mul_(2.0)
    assert spike_bits(yg) is None
    out = lin(yg)
    assert 'SpikeLinear' not in type(out.grad_fn).__name__
    torch.testing.assert_close(out.detach().cpu(), torch.nn.functional.linear(2.0 * y, lin.weight.detach().cpu(),
                                                                           lin.bias.detach().cpu()))


@pytest.mark.gpu
@pytest.mark.parametrize('M', [256, 130, 7])
def test_input_gradient_split_is_exact_bf16_rounding(dev, M):
    """``delrec_spike_linear_dx_split``: each row of g becomes [hi | lo | hi] with hi the bf16
    round-to-nearest-even of x and lo that of x - hi -- torch's own bf16 conversion, bit for
    bit (M a multiple of 4 takes the vector stores, 130 and 7 the element tail)."""
    from delrec import _lib
    rows = 1000
    print(f'rows={rows} M={M}', flush=True)
    g = (torch.randn(rows, M, generator=gen(5)) * torch.logspace(-30, 30, M, base=2.0)).to(dev)
    g[0, 0] = 0.0
    out = torch.empty(rows, 3 * M, device=dev, dtype=torch.bfloat16)
    _lib.spike_linear_dx_split(g, out, _lib.stream_of(g))
    torch.cuda.synchronize()
    hi = g.to(torch.bfloat16)
    lo = (g - hi.to(torch.float32)).to(torch.bfloat16)
    assert torch.equal(out[:, :M].view(torch.int16), hi.view(torch.int16))
    assert torch.equal(out[:, M:2 * M].view(torch.int16), lo.view(torch.int16))
    assert torch.equal(out[:, 2 * M:].view(torch.int16), hi.view(torch.int16))


@pytest.mark.gpu
def test_input_gradient_takes_the_bf16_split_gemm(dev, monkeypatch):
    """The Linear's input gradient as the split bf16 GEMM (torch's fp32-output bf16 mm is
    present on this device; forced here, the GEMM being below the size that takes it by
    itself) matches float64 at C5's width on 4 x 64 spike rows."""
    from delrec import _lib, spike_linear
    assert spike_linear._mm_out_dtype(dev), 'no fp32-output bf16 GEMM: the split path would not run'
    monkeypatch.setenv('DELREC_LINEAR_DX_SPLIT', '1')   # this GEMM is below the size the split takes
    calls = []
    real = _lib.spike_linear_dx_split
    monkeypatch.setattr(_lib, 'spike_linear_dx_split', lambda *a: (calls.append(1), real(*a))[1])
    T, B, K, M = 64, 4, 2048, 2048
    g = gen(17)
    y = (torch.rand(T, B, K, generator=g) < 0.05).float()
    lin = spike_linear.SpikeLinear(K, M, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(M, K, generator=g) / K ** 0.5)
    lin = lin.to(dev)
    xg = spike_linear.attach_bits(y.to(dev).requires_grad_(True), pack_bits(y).to(dev))
    gout = torch.randn(T, B, M, generator=g)
    lin(xg).backward(gout.to(dev))
    torch.cuda.synchronize()
    assert calls, 'the input gradient did not take the split GEMM'
    ref = gout.double().reshape(-1, M) @ lin.weight.detach().cpu().double()
    got = xg.grad.cpu().double().reshape(-1, K)
    err = float((got - ref).abs().max())
    print(f'  max |dx - float64| {err:.3e} (|dx| max {float(ref.abs().max()):.3e})', flush=True)
    # three bf16 products of the split operands: about 2^-16 per term
    check_elementwise('dx', got, ref, 1e-4, 1e-5, term_sq=gemm_term_sq(gout.reshape(-1, M), lin.weight.detach()),
                      eps=2.0 ** -16)
