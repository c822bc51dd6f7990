"""delrec_axonal_bwd_noalloc (library-owned scratch, no caller workspace) against
delrec_axonal_bwd (caller workspace) through the C ABI: two calls in a row on one GPU, the
second with smaller sizes, each compared with the workspace entry point's results on the
same saved forward state. Both run the same kernels, so the results must be identical."""

import ctypes

import pytest
import torch

from helpers import gen

# T, B, N, max delay, sigma: the first needs most of the 64 MiB scratch (the straight-line
# backward and its dW split partials), the second is smaller and takes the streamed kernels
CALLS = [(128, 96, 256, 30.0, 1.0), (24, 3, 300, 9.0, 0.5)]


def _forward(lib, T, B, N, dmax, sigma, dev, seed):
    from delrec import _lib
    from delrec.kernels._common import window_length_f32
    g = gen(seed)
    x = (torch.randn(T, B, N, generator=g) * 1.2 + 0.2).to(dev)
    W = (torch.randn(N, N, generator=g) * (1.5 / N ** 0.5)).to(dev)
    d = (torch.rand(N, generator=g) * dmax).to(dev)
    gy = torch.randn(T, B, N, generator=g).to(dev)
    L = max(window_length_f32(float(d.max()), 1.0 + sigma), 2)
    lif = _lib.make_lif(2.0, 1.0, 0.0, False, False, 1, 1.0, 2.0)
    y, u, z = (torch.empty(T, B, N, device=dev) for _ in range(3))
    bits = torch.empty(B, (T + 31) // 32, N, device=dev, dtype=torch.int32)
    ws = _lib.workspace(_lib.WS_AXONAL_FWD, T, B, N, L, 0, dev)
    fa = _lib.AxonalFwdArgs(T=T, B=B, N=N, L=L, x=_lib.ptr(x), W=_lib.ptr(W), w_bf16=0, bias=None,
                            d=_lib.ptr(d), s=None, s_uniform=1.0 + sigma, drop=None, taps=0, lif=lif,
                            y=_lib.ptr(y), u=_lib.ptr(u), rec=None, z=_lib.ptr(z), bits=_lib.ptr(bits),
                            workspace=_lib.ptr(ws), workspace_bytes=ws.numel())
    assert lib.delrec_axonal_fwd(ctypes.byref(fa), _lib.stream_of(x)) == 0
    return dict(T=T, B=B, N=N, L=L, sigma=sigma, W=W, d=d, gy=gy, u=u, z=z, bits=bits, lif=lif)


def _backward(lib, st, entry, with_workspace):
    from delrec import _lib
    T, B, N, L = st['T'], st['B'], st['N'], st['L']
    dev = st['u'].device
    dx = torch.full((T, B, N), float('nan'), device=dev)
    dW = torch.full((N, N), float('nan'), device=dev)
    db, dd = (torch.full((N,), float('nan'), device=dev) for _ in range(2))
    ws = _lib.workspace(_lib.WS_AXONAL_BWD, T, B, N, L, 0, dev) if with_workspace else None
    ba = _lib.AxonalBwdArgs(T=T, B=B, N=N, L=L, gy=_lib.ptr(st['gy']), u=_lib.ptr(st['u']),
                            bits=_lib.ptr(st['bits']), z=_lib.ptr(st['z']), W=_lib.ptr(st['W']), w_bf16=0,
                            d=_lib.ptr(st['d']), s=None, s_uniform=1.0 + st['sigma'], drop=None,
                            mode=_lib.DELREC_BWD_SOFT, lag=None, lif=st['lif'], dx=_lib.ptr(dx),
                            dW=_lib.ptr(dW), db=_lib.ptr(db), dd=_lib.ptr(dd), ds=None,
                            workspace=_lib.ptr(ws), workspace_bytes=0 if ws is None else ws.numel())
    status = getattr(lib, entry)(ctypes.byref(ba), _lib.stream_of(dx))
    assert status == 0, f'{entry}: status {status}'
    torch.cuda.synchronize()
    return {'dx': dx.cpu(), 'dW': dW.cpu(), 'db': db.cpu(), 'dd': dd.cpu()}


@pytest.mark.gpu
def test_axonal_bwd_noalloc_matches_workspace_entry(dev):
    from delrec import _lib
    lib = _lib.load()
    for k, (T, B, N, dmax, sigma) in enumerate(CALLS):
        print(f'call {k}: T={T} B={B} N={N} dmax={dmax} sigma={sigma}', flush=True)
        st = _forward(lib, T, B, N, dmax, sigma, dev, seed=40 + k)
        ref = _backward(lib, st, 'delrec_axonal_bwd', True)
        got = _backward(lib, st, 'delrec_axonal_bwd_noalloc', False)
        for name in ref:
            assert torch.isfinite(ref[name]).all(), f'{name}: workspace entry left NaN'
            assert torch.equal(got[name], ref[name]), (
                f'call {k} {name}: max abs diff {float((got[name] - ref[name]).abs().max()):.3e}')
        print(f'  identical: dx, dW, db, dd', flush=True)


@pytest.mark.gpu
def test_axonal_bwd_noalloc_rejects_sizes_beyond_scratch(dev):
    from delrec import _lib
    lib = _lib.load()
    # the straight-line backward at T=1024 B=128 N=256 needs 2 x 128 MiB of (T, B, N) buffers
    T, B, N, L = 1024, 128, 256, 20
    lif = _lib.make_lif(2.0, 1.0, 0.0, False, False, 1, 1.0, 2.0)
    dummy = torch.zeros(1, device=dev)
    p = _lib.ptr(dummy)
    ba = _lib.AxonalBwdArgs(T=T, B=B, N=N, L=L, gy=p, u=p, bits=p, z=p, W=p, w_bf16=0, d=p, s=None,
                            s_uniform=1.0, drop=None, mode=_lib.DELREC_BWD_SOFT, lag=None, lif=lif, dx=p,
                            dW=p, db=None, dd=None, ds=None, workspace=None, workspace_bytes=0)
    assert lib.delrec_axonal_bwd_noalloc(ctypes.byref(ba), _lib.stream_of(dummy)) == _lib.DELREC_ERR_SCRATCH
