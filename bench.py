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
durations on the kernels' stream, recorded in a few extra steps after the timed ones so that
the events do not slow the timed steps) and a CPU baseline, the oracle's
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
    """Algorithmic bytes and flops per neuron-timestep, for the whole fwd+BPTT and for each
    time-scan kernel.

    Bytes: x read, y write, gy read, dx write in fp32 (16 B). Flops are useful MACs x 2
    with no sparsity credit; k = non-zero triangle taps = 2(1 + sigma). Axonal and hybrid
    (the hybrid's integer offsets only shift which step of z_j a connection reads):
    6N + 6k in total = forward scan 2N + 2k (contraction W z, taps of z) + backward scan
    2N + 4k (W^T gr, taps of the future gradient, delay-gradient taps) + dW GEMM 2N.
    Synaptic: 8kN in total = forward scan 2kN + backward scan 2kN + lag GEMM 4kN.
    """
    N, sigma = w['N'], w['sigma']
    k = 2.0 * (1.0 + sigma)
    if w['kind'] == 'synaptic':
        return {'bytes': 16.0, 'flops': 8.0 * k * N,
                'scan_flops': {'syn_fwd_scan': 2.0 * k * N, 'syn_bwd_scan': 2.0 * k * N}}
    return {'bytes': 16.0, 'flops': 6.0 * N + 6.0 * k,
            'scan_flops': {'axonal_fwd_scan': 2.0 * N + 2.0 * k, 'axonal_bwd_scan': 2.0 * N + 4.0 * k,
                           'syn_fwd_scan': 2.0 * N + 2.0 * k, 'syn_bwd_scan': 2.0 * N + 4.0 * k}}


# kernel symbol of each time-scan kind at each workload's shape (for the rocprof summaries)
SCAN_SYMBOL = {
    'C2': {'axonal_fwd_scan': 'axonal_fwd_wave_fast', 'axonal_bwd_scan': 'axonal_bwd_tiled_fast'},
    'C3': {'syn_fwd_scan': 'syn_fwd_scatter', 'syn_bwd_scan': 'syn_bwd_hyb'},
    # C4's scans are sequences of launches (per 8-step block one lagblock_kernel, per step one
    # lagstep_gemm_kernel + one LIF kernel): the scan time is the whole sequence's
    'C4': {'syn_fwd_scan': 'lagstep_fwd_sequence', 'syn_bwd_scan': 'lagstep_bwd_sequence'},
}


def cpu_baseline(layer, x, w, budget_s=25.0):
    """The oracle (pure-PyTorch v2 scan, autograd BPTT, fp32) on the host cores, on a
    bounded sample of the same workload: the layer's own weights and delays and the first
    T' steps of the same input at full B and N, scaled to neuron-timesteps/s."""
    from oracle import neuron as oneuron, scans
    from oracle.delays import hybrid_delays
    cores = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(cores)
    T, B, N = w['T'], w['B'], w['N']
    lif = oneuron.LIFParams(tau=w['tau'])
    W = layer.recurrent_weights.detach().float().cpu()
    if w['kind'] == 'axonal':
        d = layer.recurrent_delays.detach().cpu()
        fn = scans.axonal_v2
    elif w['kind'] == 'hybrid':
        par = layer.parametrizations.recurrent_delays
        d = hybrid_delays(par.original.detach().cpu(), par[0].offsets.detach().float().cpu())
        fn = scans.synaptic_v2
    else:
        d = layer.recurrent_delays.detach().cpu()
        fn = scans.synaptic_v2
    xc = x.detach().cpu()

    def one(Tp):
        xs = xc[:Tp].clone().requires_grad_(True)
        Wl, dl = W.clone().requires_grad_(True), d.clone().requires_grad_(True)
        t0 = time.perf_counter()
        y, _ = fn(xs, Wl, dl, lif, sigma=w['sigma'])
        y.sum().backward()
        return time.perf_counter() - t0

    Tp = min(T, 16)
    t_probe = one(Tp)
    # grow the sample while 3 timed runs stay within the budget (the probe is the warmup)
    while Tp < T and t_probe * 2 * 3 < budget_s:
        Tp = min(T, Tp * 2)
        t_probe = one(Tp)
    times = sorted(one(Tp) for _ in range(3))
    t_med = times[1]
    nts = Tp * B * N / t_med
    return {'value': nts, 'unit': 'neuron-timesteps/s', 'cores': cores, 'kind': 'port',
            'sample': f'oracle v2 scan + autograd BPTT, fp32, same weights/delays/input, full B={B} '
                      f'N={N}, first {Tp} of T={T} steps, median of 3 (after a warmup), scaled per '
                      f'neuron-timestep',
            'seconds_per_sample': t_med}


def calibrate_copy(mib):
    """A plain device copy of `mib` MiB, five times: the known-size kernel whose FETCH_SIZE /
    WRITE_SIZE readings scale the counters of the scan kernels to bytes."""
    n = mib * (1 << 20) // 4
    src = torch.rand(n, device='cuda:0')
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_bytes_read': n * 4, 'copy_bytes_written': n * 4, 'launches': 5}), flush=True)


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
    ap.add_argument('--calibrate-copy', type=int, metavar='MIB', default=0,
                    help='only run a plain device copy of MIB MiB (counter calibration)')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU; --gpus {args.gpus} is not supported by this build '
              f'(the layer shards over batch rows with one dW/dd all-reduce per step, not run here)',
              file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
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
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    # per scan kernel (HIP events on the kernels' stream) and per entry point (scan +
    # reductions + GEMMs), from a few extra steps outside the timed region: the event
    # pairs would otherwise add their own gaps to the timed steps
    n_extra = min(5, args.steps)
    with _lib.scan_timing(2 * n_extra + 8) as scans_t:
        for _ in range(n_extra):
            step()
        torch.cuda.synchronize()
    with _lib.timing() as rec:
        for _ in range(n_extra):
            step()
        torch.cuda.synchronize()
    per_entry, per_scan = {}, {}
    for name, s, e in rec:
        per_entry.setdefault(name, []).append(s.elapsed_time(e))
    for kind, dt in scans_t.launches:
        per_scan.setdefault(kind, []).append(dt)
    avg = {k: sum(v) / len(v) for k, v in per_entry.items()}
    scan_avg = {k: sum(v) / len(v) for k, v in per_scan.items()}
    nt = T * B * N
    value = nt / (ms * 1e-3)
    work = algorithmic_work(w)
    peak_c = PEAK_BF16 if (w['w_bf16'] and w['kind'] != 'synaptic') else PEAK_FP32
    t_bound = max(work['bytes'] * nt / PEAK_HBM, work['flops'] * nt / peak_c)

    # the dominant kernel: the time-scan kernel with the longest average launch
    dom = max(scan_avg, key=scan_avg.get)
    dur = scan_avg[dom] * 1e-3
    flops = work['scan_flops'][dom] * nt
    achieved = flops / dur
    kernel = SCAN_SYMBOL[args.config][dom]
    traffic = load_traffic(kernel, args.config)
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
        'roofline': {'bound': 'mfma', 'achieved': achieved / 1e12, 'peak': PEAK_FP32 / 1e12,
                     'unit': 'TFLOP/s', 'frac': achieved / PEAK_FP32, 'traffic': traffic,
                     'kernel': kernel, 'avg_launch_ms': scan_avg[dom],
                     'flops_per_launch': flops},
        'layer_roofline': {'t_bound_ms': t_bound * 1e3, 'frac': t_bound / (ms * 1e-3),
                           'bytes_per_nt': work['bytes'], 'flops_per_nt': work['flops']},
        'scan_ms': scan_avg,
    }
    if avg:
        line['entry_ms'] = avg
    if not args.no_cpu:
        line['cpu_baseline'] = cpu_baseline(layer, x, w)
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
