"""Benchmark of the recurrent delayed-LIF layer: forward + BPTT backward throughput.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2|C3|C4] [--no-cpu]

One step is one forward + backward of the recurrent layer over one batch of synthetic
input, driven by a fixed upstream gradient captured once from the full model's loss
(projection -> recurrent layer -> readout -> time mean -> cross-entropy). Inputs, weights
and the upstream gradient are resident in HBM before the timed region. The metric is
neuron-timesteps per second, T * B * N / (seconds per step).

Workloads (synthetic data of the stated shape, random-init weights):
  C2  axonal, T=128 B=128 N=256, 9 analog inputs N(0,1) smoothed by a causal 5-tap mean,
      delays U[0,32], sigma=1, tau=10 (leak 0.9), threshold 1, fp32 Kaiming-uniform W,
      6-way readout                                           (default, N=1 headline)
  C3  hybrid, T=256 B=256 N=512, 700 Bernoulli(0.02) inputs, base U[0,40] + offsets
      {0..8}, sigma=0, bf16 W / fp32 state, 20-way readout
  C4  synaptic, T=250 B=256 N=1024, 700 Bernoulli(0.02) inputs, per-connection delays
      U[0,40], sigma=4, fp32, 35-way readout

Reported beside the GPU number: the roofline fraction of the dominant kernel (HIP-event
durations on the kernels' stream during the timed steps) and a CPU baseline, the oracle's
pure-PyTorch scan with autograd BPTT timed on the host cores over a bounded sample.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, 'snn-delays_amd'))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

PEAK_HBM = 8.0e12          # MI355X HBM3E, bytes/s
PEAK_FP32 = 157.3e12       # MI355X dense FP32 (vector and MFMA), flop/s
PEAK_BF16 = 2.5e15         # MI355X dense BF16 MFMA, flop/s

WORKLOADS = {
    'C2': dict(kind='axonal', T=128, B=128, N=256, C_in=9, classes=6, dmax=32.0, sigma=1.0, tau=10.0,
               inputs='analog_smoothed', gain=1.0, w_bf16=False, seed=1002,
               label='recurrent axonal-delay LIF, T128 B128 N256, delays U[0,32], sigma 1, fp32'),
    'C3': dict(kind='hybrid', T=256, B=256, N=512, C_in=700, classes=20, dmax=40.0, sigma=0.0, tau=2.0,
               inputs='bernoulli', p_in=0.02, gain=6.0, offset_max=8, w_bf16=True, seed=1003,
               label='recurrent hybrid-delay LIF, T256 B256 N512, base U[0,40] + offsets {0..8}, '
                     'sigma 0, bf16 W'),
    'C4': dict(kind='synaptic', T=250, B=256, N=1024, C_in=700, classes=35, dmax=40.0, sigma=4.0,
               tau=2.0, inputs='bernoulli', p_in=0.02, gain=6.0, w_bf16=False, seed=1004,
               label='recurrent synaptic-delay LIF, T250 B256 N1024, delays U[0,40], sigma 4, fp32'),
}


def make_config(w):
    from configs.perf_MEM import Config
    cfg = Config()
    cfg.tau = w['tau']
    cfg.sigma_init = w['sigma']
    cfg.init_rec_weights = 'kaiming_uniform'
    cfg.init_rec_delay = 'uniform'
    cfg.init_recdel_offset = 0.0
    cfg.max_rec_delay = w['dmax']
    cfg.hybrid_offset_scale = w.get('offset_max', 0)
    cfg.hybrid_base_centering = 'normal'
    return cfg


def build(w, device):
    """Input projection, recurrent layer, readout and the synthetic batch."""
    from delrec.delay_layers import axonal_recdel, synaptic_recdel
    from delrec.networks import _reparametrize_recurrent_delay
    torch.manual_seed(0)
    cfg = make_config(w)
    proj = torch.nn.Linear(w['C_in'], w['N'], bias=False)
    if w['kind'] == 'axonal':
        layer = axonal_recdel(cfg, w['N'])
    else:
        layer = synaptic_recdel(cfg, w['N'])
        if w['kind'] == 'hybrid':
            _reparametrize_recurrent_delay(layer, w['offset_max'], torch.Generator().manual_seed(123), cfg)
    if w['w_bf16']:
        layer.recurrent_weights = torch.nn.Parameter(layer.recurrent_weights.detach().bfloat16())
    readout = torch.nn.Linear(w['N'], w['classes'], bias=False)
    g = torch.Generator().manual_seed(w['seed'])
    T, B = w['T'], w['B']
    if w['inputs'] == 'analog_smoothed':
        raw = torch.randn(T, B, w['C_in'], generator=g)
        pad = torch.cat([torch.zeros(4, B, w['C_in']), raw], 0)
        inp = sum(pad[4 - k:4 - k + T] for k in range(5)) / 5.0
    else:
        inp = (torch.rand(T, B, w['C_in'], generator=g) < w['p_in']).float()
    labels = torch.randint(w['classes'], (B,), generator=g)
    proj, layer, readout = proj.to(device), layer.to(device), readout.to(device)
    with torch.no_grad():
        x = (proj(inp.to(device)) * w['gain']).contiguous()
    return layer, readout, x, labels.to(device), cfg


def upstream_gradient(layer, readout, x, labels):
    """dLoss/dy of the full model's loss, captured once."""
    y = layer(x)
    y_ = y.detach().requires_grad_(True)
    loss = torch.nn.functional.cross_entropy(readout(y_).mean(0), labels)
    (gy,) = torch.autograd.grad(loss, y_)
    return y.detach(), gy.contiguous()


def algorithmic_work(w):
    """Algorithmic bytes and flops per neuron-timestep of the whole fwd+BPTT and per kernel.

    Bytes: x read, y write, gy read, dx write in fp32 (16 B). Flops (useful MACs x2, no
    sparsity credit; k = non-zero triangle taps = 2(1 + sigma)): axonal / hybrid
    6N + 6k, synaptic 8kN. Forward scan kernel: the contraction and taps, 2N + 2k
    (axonal; 2kN synaptic).
    """
    N, sigma = w['N'], w['sigma']
    k = 2.0 * (1.0 + sigma)
    if w['kind'] == 'synaptic':
        return {'bytes': 16.0, 'flops': 8.0 * k * N, 'fwd_flops': 2.0 * k * N, 'fwd_bytes': 8.0}
    return {'bytes': 16.0, 'flops': 6.0 * N + 6.0 * k, 'fwd_flops': 2.0 * N + 2.0 * k, 'fwd_bytes': 8.0}


def cpu_baseline(w, budget_s=25.0):
    """The oracle (pure-PyTorch v2 scan, autograd BPTT, fp32) on the host cores, on a
    bounded sample: full B and N, the first T' steps, scaled to neuron-timesteps/s."""
    from oracle import neuron as oneuron, scans
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(cores)
    torch.manual_seed(0)
    T, B, N = w['T'], w['B'], w['N']
    lif = oneuron.LIFParams(tau=w['tau'])
    g = torch.Generator().manual_seed(7)
    W = (torch.rand(N, N, generator=g) * 2 - 1) / N ** 0.5
    if w['w_bf16']:
        W = W.bfloat16().float()
    if w['kind'] == 'axonal':
        d = torch.rand(N, generator=g) * w['dmax']
        fn = scans.axonal_v2
    elif w['kind'] == 'hybrid':
        d = (torch.rand(N, generator=g) * w['dmax'])[None, :] + torch.randint(
            w['offset_max'] + 1, (N, N), generator=g).float()
        fn = scans.synaptic_v2
    else:
        d = torch.rand(N, N, generator=g) * w['dmax']
        fn = scans.synaptic_v2

    def one(Tp):
        x = (torch.randn(Tp, B, N, generator=g) * 0.8).requires_grad_(True)
        Wl, dl = W.clone().requires_grad_(True), d.clone().requires_grad_(True)
        t0 = time.perf_counter()
        y, _ = fn(x, Wl, dl, lif, sigma=w['sigma'])
        y.sum().backward()
        return time.perf_counter() - t0

    Tp = min(T, 16)
    t_probe = one(Tp)
    # grow the sample while it fits the budget (1 warmup already done + 3 timed runs)
    while Tp < T and t_probe * 2 * 3 < budget_s:
        Tp = min(T, Tp * 2)
        t_probe = one(Tp)
    times = sorted(one(Tp) for _ in range(3))
    t_med = times[1]
    nts = Tp * B * N / t_med
    return {'value': nts, 'unit': 'neuron-timesteps/s', 'cores': cores, 'kind': 'port',
            'sample': f'oracle v2 scan + autograd BPTT, fp32, full B={B} N={N}, first {Tp} of '
                      f'T={T} steps, median of 3 (after 1 warmup), scaled per neuron-timestep',
            'seconds_per_sample': t_med}


def load_traffic(kernel, config):
    p = os.path.join(ROOT, 'profiles', f'traffic_{kernel}_{config}.json')
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get('bytes_per_launch')
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--config', default='C2', choices=sorted(WORKLOADS))
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline leg')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU; --gpus {args.gpus} is not supported by this build '
              f'(the layer shards over batch rows with one dW/dd all-reduce per step, not run here)',
              file=sys.stderr)
        sys.exit(2)
    w = WORKLOADS[args.config]
    dev = torch.device('cuda:0')
    from delrec import _lib
    _lib.load()
    layer, readout, x, labels, cfg = build(w, dev)
    T, B, N = w['T'], w['B'], w['N']
    y0, gy = upstream_gradient(layer, readout, x, labels)
    firing = float(y0.mean())
    xin = x.detach().requires_grad_(True)

    def step():
        layer.zero_grad(set_to_none=True)
        xin.grad = None
        y = layer(xin)
        y.backward(gy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    with _lib.timing() as rec:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    per_entry = {}
    for name, s, e in rec:
        per_entry.setdefault(name, []).append(s.elapsed_time(e))
    avg = {k: sum(v) / len(v) for k, v in per_entry.items()}
    nt = T * B * N
    value = nt / (ms * 1e-3)
    work = algorithmic_work(w)
    peak_c = PEAK_BF16 if (w['w_bf16'] and w['kind'] != 'synaptic') else PEAK_FP32
    t_bound = max(work['bytes'] * nt / PEAK_HBM, work['flops'] * nt / peak_c)

    fwd_entry = 'delrec_axonal_fwd' if w['kind'] == 'axonal' else 'delrec_syn_fwd'
    bwd_entry = 'delrec_axonal_bwd' if w['kind'] == 'axonal' else 'delrec_syn_bwd'
    dom = max(avg, key=avg.get) if avg else fwd_entry
    kernel = {'delrec_axonal_fwd': 'axonal_fwd_kernel', 'delrec_axonal_bwd': 'axonal_bwd(+dW gemm)',
              'delrec_syn_fwd': 'syn_fwd_kernel', 'delrec_syn_bwd': 'syn_bwd(+lag gemm)'}.get(dom, dom)
    if dom == fwd_entry:
        flops = work['fwd_flops'] * nt
    else:
        flops = (work['flops'] - work['fwd_flops']) * nt
    dur = avg.get(dom, ms) * 1e-3
    achieved = flops / dur
    traffic = load_traffic(kernel.split('(')[0], args.config)
    line = {
        'metric': 'neuron-timesteps/sec fwd+BPTT per recurrent layer',
        'value': value,
        'unit': 'neuron-timesteps/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': ms,
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16-weights/f32' if w['w_bf16'] else 'f32',
        'data': 'synthetic (seeded inputs of the stated shape, random-init weights)',
        'config': {'workload': f"{args.config}: {w['label']}", 'T': T, 'B': B, 'N': N,
                   'delay_kind': w['kind'], 'sigma': w['sigma'], 'firing_rate': firing},
        'roofline': {'bound': 'mfma', 'achieved': achieved / 1e12, 'peak': PEAK_FP32 / 1e12
                     if peak_c == PEAK_FP32 else peak_c / 1e12, 'unit': 'TFLOP/s',
                     'frac': achieved / peak_c, 'traffic': traffic, 'kernel': kernel,
                     'avg_launch_ms': avg.get(dom)},
        'layer_roofline': {'t_bound_ms': t_bound * 1e3, 'frac': t_bound / (ms * 1e-3),
                           'bytes_per_nt': work['bytes'], 'flops_per_nt': work['flops']},
        'entry_ms': avg,
    }
    if not args.no_cpu:
        line['cpu_baseline'] = cpu_baseline(w)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
