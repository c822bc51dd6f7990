"""Benchmark of the recurrent delayed-LIF layer: forward + BPTT backward throughput.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C1..C5] [--extra C1,C2,C3,C4]
                    [--no-cpu]

The headline is C5 (the largest configuration that fits one GPU); the other workloads are
reported under "extra", each with its own roofline and CPU baseline.

One step is one forward + backward of every recurrent layer of the workload over one
batch of synthetic input, each layer driven by its own fixed input and a fixed upstream
gradient captured once from the full model's loss (projection -> recurrent layer(s), with
the inter-layer Linear between stacked layers -> readout -> time mean -> cross-entropy).
Inputs, weights and upstream gradients are resident in HBM before the timed region. The
metric is neuron-timesteps per second, sum over layers of T * B * N / (seconds per step).

Workloads (synthetic data of the stated shape, random-init weights):
  C1  axonal, T=32 B=64 N=64: batch of 64 from 256 samples of 8 Bernoulli(0.1) input
      channels, delays U[0,16], sigma=0, orthogonal W (gain 0.5), leaky-integrator readout
      of 4 classes, fp32                         (the CPU-runnable memorisation config)
  C2  axonal, T=128 B=128 N=256, 9 analog inputs N(0,1) smoothed by a causal 5-tap mean,
      delays U[0,32], sigma=1, tau=10 (leak 0.9), threshold 1, fp32 Kaiming-uniform W,
      6-way readout
  C3  hybrid, T=256 B=256 N=512, 700 Bernoulli(0.02) inputs, base U[0,40] + offsets
      {0..8}, sigma=0, bf16 W / fp32 state, 20-way readout
  C4  synaptic, T=250 B=256 N=1024, 700 Bernoulli(0.02) inputs, per-connection delays
      U[0,40], sigma=4, fp32, 35-way readout, hidden firing about 5 %
  C5  two stacked hybrid layers, T=1024 B=512 N=2048 each with a Linear(2048 -> 2048)
      between them: 1 analog input U[0,1] per step, base U[0,60] + offsets {0..4}, sigma=0,
      bf16 W / fp32 accumulate, hidden firing 2-5 % in both layers, 10-way readout
      (default: the largest configuration that fits one GPU)

Reported beside the GPU number: the roofline of the dominant time scan (HIP-event
durations on the kernels' stream, recorded in a few extra steps after the timed ones so
that the events do not slow the timed steps), priced against the workload's binding
roofline (C2, C4: FP32; C3: HBM; C5: BF16 MFMA), and a CPU baseline, the oracle's
pure-PyTorch scan with autograd BPTT timed on the host cores over bounded samples.
"""

import argparse
import json
import os
import platform
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
    'C1': dict(kind='axonal', T=32, B=64, N=64, C_in=8, classes=4, dmax=16.0, sigma=0.0, tau=2.0,
               inputs='bernoulli_pool', p_in=0.1, pool=256, gain=3.0, w_init='orthogonal',
               w_gain=0.5, w_bf16=False, readout='li', seed=1001, bound='cpu',
               label='recurrent axonal-delay LIF, T32 B64 N64, delays U[0,16], sigma 0, fp32, LI readout'),
    'C2': dict(kind='axonal', T=128, B=128, N=256, C_in=9, classes=6, dmax=32.0, sigma=1.0, tau=10.0,
               inputs='analog_smoothed', gain=1.0, w_bf16=False, seed=1002, bound='fp32',
               label='recurrent axonal-delay LIF, T128 B128 N256, delays U[0,32], sigma 1, fp32'),
    'C3': dict(kind='hybrid', T=256, B=256, N=512, C_in=700, classes=20, dmax=40.0, sigma=0.0, tau=2.0,
               inputs='bernoulli', p_in=0.02, gain=6.0, offset_max=8, w_bf16=True, seed=1003, bound='hbm',
               label='recurrent hybrid-delay LIF, T256 B256 N512, base U[0,40] + offsets {0..8}, '
                     'sigma 0, bf16 W'),
    'C4': dict(kind='synaptic', T=250, B=256, N=1024, C_in=700, classes=35, dmax=40.0, sigma=4.0,
               tau=2.0, inputs='bernoulli', p_in=0.02, gain=7.0, w_bf16=False, seed=1004, bound='fp32',
               label='recurrent synaptic-delay LIF, T250 B256 N1024, delays U[0,40], sigma 4, fp32'),
    'C5': dict(kind='hybrid', layers=2, T=1024, B=512, N=2048, C_in=1, classes=10, dmax=60.0, sigma=0.0,
               tau=2.0, inputs='uniform', gain=1.0, gain2=5.0, offset_max=4, w_bf16=True, seed=1005,
               bound='bf16',
               label='two stacked recurrent hybrid-delay LIF layers, T1024 B512 N2048, base U[0,60] + '
                     'offsets {0..4}, sigma 0, bf16 W, Linear(2048->2048) between'),
}
DEFAULT_CONFIG = 'C5'


def make_config(w):
    from configs.perf_MEM import Config
    cfg = Config()
    cfg.tau = w['tau']
    cfg.sigma_init = w['sigma']
    cfg.init_rec_weights = w.get('w_init', 'kaiming_uniform')
    cfg.rec_delay_init_gain = w.get('w_gain', cfg.rec_delay_init_gain)
    cfg.init_rec_delay = 'uniform'
    cfg.init_recdel_offset = 0.0
    cfg.max_rec_delay = w['dmax']
    cfg.hybrid_offset_scale = w.get('offset_max', 0)
    cfg.hybrid_base_centering = 'normal'
    return cfg


class Model:
    """The workload's modules and synthetic batch: ``layers`` (recurrent), ``inter`` (the
    Linear between stacked layers), ``readout``, ``x`` (input of the first recurrent layer,
    already projected) and ``labels``."""


def build(w, device, T=None, B=None):
    """Input projection, recurrent layer(s), readout and the synthetic batch. ``T`` / ``B``
    shorten the batch (parity tests at the workload's N, delays, sigma and W dtype); the
    modules are the same."""
    from delrec.delay_layers import axonal_recdel, synaptic_recdel
    from delrec.networks import _reparametrize_recurrent_delay
    from delrec.spike_linear import SpikeLinear
    torch.manual_seed(0)
    cfg = make_config(w)
    N = w['N']
    proj = torch.nn.Linear(w['C_in'], N, bias=False)
    layers, inter = [], []
    offsets_gen = torch.Generator().manual_seed(123)      # one generator, layers in module order
    for k in range(w.get('layers', 1)):
        if k > 0:
            inter.append(SpikeLinear(N, N, bias=False))
        if w['kind'] == 'axonal':
            layer = axonal_recdel(cfg, N)
        else:
            layer = synaptic_recdel(cfg, N)
            if w['kind'] == 'hybrid':
                _reparametrize_recurrent_delay(layer, w['offset_max'], offsets_gen, cfg)
        if w['w_bf16']:
            layer.recurrent_weights = torch.nn.Parameter(layer.recurrent_weights.detach().bfloat16())
        layers.append(layer)
    readout = torch.nn.Linear(N, w['classes'], bias=False)
    g = torch.Generator().manual_seed(w['seed'])
    T = T or w['T']
    B = B or w['B']
    C = w['C_in']
    if w['inputs'] == 'analog_smoothed':
        raw = torch.randn(T, B, C, generator=g)
        pad = torch.cat([torch.zeros(4, B, C), raw], 0)
        inp = sum(pad[4 - k:4 - k + T] for k in range(5)) / 5.0
        labels = torch.randint(w['classes'], (B,), generator=g)
    elif w['inputs'] == 'bernoulli_pool':
        # a batch drawn from a fixed pool of seeded samples
        pool = (torch.rand(w['pool'], T, C, generator=g) < w['p_in']).float()
        pool_labels = torch.randint(w['classes'], (w['pool'],), generator=g)
        idx = torch.randperm(w['pool'], generator=torch.Generator().manual_seed(0))[:B]
        inp = pool[idx].transpose(0, 1).contiguous()
        labels = pool_labels[idx]
    elif w['inputs'] == 'uniform':
        inp = torch.rand(T, B, C, generator=g)
        labels = torch.randint(w['classes'], (B,), generator=g)
    else:
        inp = (torch.rand(T, B, C, generator=g) < w['p_in']).float()
        labels = torch.randint(w['classes'], (B,), generator=g)
    proj = proj.to(device)
    m = Model()
    m.w, m.cfg = w, cfg
    m.layers = [layer.to(device) for layer in layers]
    m.inter = [lin.to(device) for lin in inter]
    m.readout = readout.to(device)
    with torch.no_grad():
        m.x = (proj(inp.to(device)) * w['gain']).contiguous()
    m.labels = labels.to(device)
    return m


def loss_of(m, y):
    """Readout -> time mean -> cross-entropy (C1: a non-spiking leaky integrator, the
    membrane of a LIF with an unreachable threshold, then its time mean)."""
    logits = m.readout(y)
    if m.w.get('readout') == 'li':
        decay = 1.0 - 1.0 / m.w['tau']
        v = torch.zeros_like(logits[0])
        acc = torch.zeros_like(logits[0])
        for t in range(logits.shape[0]):
            v = v * decay + logits[t]
            acc = acc + v
        out = acc / logits.shape[0]
    else:
        out = logits.mean(0)
    return torch.nn.functional.cross_entropy(out, m.labels)


def layer_inputs(m):
    """Each recurrent layer's fixed input and the upstream gradient dLoss/dy of the full
    model at it (captured once), each layer's firing rate, and each layer's output (which
    carries its spike bits for the Linear that follows it)."""
    xs, ys = [], []
    x = m.x
    for k, layer in enumerate(m.layers):
        if k > 0:
            with torch.no_grad():
                x = (m.inter[k - 1](ys[-1]) * m.w['gain2']).contiguous()
        xs.append(x.detach())
        with torch.no_grad():
            ys.append(layer(x))
    # backward through the stack: gy of the last layer from the loss, then through each
    # layer and Linear in turn
    y_last = ys[-1].clone().requires_grad_(True)
    (g,) = torch.autograd.grad(loss_of(m, y_last), y_last)
    gys = [None] * len(m.layers)
    gys[-1] = g.contiguous()
    for k in range(len(m.layers) - 1, 0, -1):
        xk = xs[k].clone().requires_grad_(True)
        m.layers[k](xk).backward(gys[k])
        yprev = ys[k - 1].clone().requires_grad_(True)
        xin = m.inter[k - 1](yprev) * m.w['gain2']
        (gprev,) = torch.autograd.grad(xin, yprev, xk.grad)
        gys[k - 1] = gprev.contiguous()
        m.layers[k].zero_grad(set_to_none=True)
    firing = [float(y.mean()) for y in ys]
    return xs, gys, firing, ys


def inter_linear_ms(m, ys, reps=5):
    """The Linear between stacked layers on the first layer's spikes, forward and forward +
    backward: the binary-activation GEMMs on its spike bits (forward, and dW = g^T y; dx = g W
    the split bf16 GEMM) against torch's fp32 GEMMs on the fp32 spikes (same weights), average
    ms per call, and the largest differences between the two paths' outputs, weight gradients
    and input gradients (with the largest input gradient, for scale)."""
    from delrec.spike_linear import attach_bits, spike_bits
    lin, y = m.inter[0], ys[0]
    bits = spike_bits(y)
    T, B, _ = y.shape
    gout = torch.randn(T, B, lin.weight.shape[0], device=y.device, generator=torch.Generator(y.device).manual_seed(7))
    inputs = {'spike_bits_gemm': lambda: attach_bits(y.detach().requires_grad_(True), bits),
              'torch_fp32': lambda: y.detach().clone().requires_grad_(True)}
    out, res = {}, {}

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            r = fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps, r

    for name, make in inputs.items():
        x = make()
        with torch.no_grad():
            out[name], o = timed(lambda: lin(x))

        def fwd_bwd():
            lin.weight.grad = None
            xi = make()
            lin(xi).backward(gout)
            return lin.weight.grad, xi.grad

        out[name + '_fwd_bwd'], (dw, dx) = timed(fwd_bwd)
        res[name] = (o, dw.clone(), dx)
    out['max_abs_diff'] = float((res['spike_bits_gemm'][0] - res['torch_fp32'][0]).abs().max())
    out['max_abs_diff_dW'] = float((res['spike_bits_gemm'][1] - res['torch_fp32'][1]).abs().max())
    out['max_abs_diff_dx'] = float((res['spike_bits_gemm'][2] - res['torch_fp32'][2]).abs().max())
    out['max_abs_dx'] = float(res['torch_fp32'][2].abs().max())
    lin.weight.grad = None
    return out


def algorithmic_work(w):
    """Algorithmic bytes and flops per neuron-timestep of one layer, for the whole fwd+BPTT
    and for each time scan.

    Bytes: x read, y write (forward scan), gy read, dx write (backward scan), fp32: 16 B.
    Flops are useful MACs x 2 with no sparsity credit; k = non-zero triangle taps =
    2(1 + sigma). Axonal and hybrid (the hybrid's integer offsets only shift which step of
    z_j a connection reads): 6N + 6k in total = forward scan 2N + 2k (contraction W z, taps
    of z) + backward scan 2N + 4k (W^T gr, taps of the future gradient, delay-gradient taps)
    + dW GEMM 2N. Synaptic: 8kN in total = forward scan 2kN + backward scan 2kN + lag GEMM 4kN.
    """
    N, sigma = w['N'], w['sigma']
    k = 2.0 * (1.0 + sigma)
    scan_bytes = {'fwd': 8.0, 'bwd': 8.0}
    if w['kind'] == 'synaptic':
        return {'bytes': 16.0, 'flops': 8.0 * k * N, 'scan_bytes': scan_bytes,
                'scan_flops': {'fwd': 2.0 * k * N, 'bwd': 2.0 * k * N}}
    return {'bytes': 16.0, 'flops': 6.0 * N + 6.0 * k, 'scan_bytes': scan_bytes,
            'scan_flops': {'fwd': 2.0 * N + 2.0 * k, 'bwd': 2.0 * N + 4.0 * k}}


def peak_of(w):
    return {'fp32': PEAK_FP32, 'bf16': PEAK_BF16, 'hbm': PEAK_HBM}.get(w['bound'])


# kernel symbol of each time-scan kind at each workload's shape (for the rocprof summaries);
# a sequence is a scan run as per-step launches, timed as a whole
SCAN_SYMBOL = {
    'C1': {'axonal_fwd_scan': 'axonal_fwd_wave_fast', 'axonal_bwd_scan': 'axonal_bwd_tiled_fast'},
    'C2': {'axonal_fwd_scan': 'axonal_fwd_wave_fast', 'axonal_bwd_scan': 'axonal_bwd_tiled_fast'},
    'C3': {'syn_fwd_scan': 'hyb_fwd_arrive_kernel', 'syn_bwd_scan': 'syn_bwd_hyb_g'},
    'C4': {'syn_fwd_scan': 'lagstep_fwd_sequence', 'syn_bwd_scan': 'lagstep_bwd_sequence'},
    'C5': {'syn_fwd_scan': 'hyb_fwd_arrive_kernel', 'syn_bwd_scan': 'hybstep_bwd_sequence'},
}


def cpu_model():
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or 'unknown'


def cpu_baseline(layer, x, w, budget_s=60.0):
    """The oracle (pure-PyTorch v2 scan, autograd BPTT, fp32) on the host cores, on bounded
    samples of the same workload: the layer's own weights and delays and the first T' steps
    of the same input at full B and N, scaled to neuron-timesteps/s. The median of 3 samples
    (the reference profiler's protocol is a median of repeats) at the whole T where three
    passes fit the budget (C1-C3), else at T' = 32, 16 or 8 (C4, C5: the v2 scan's work per
    step does not depend on T); the same at T' / 2 checks that the time per step does not
    depend on T' (the scaling assumed), reported as the ratio of the two per-step times."""
    from oracle import neuron as oneuron, scans
    cores = max(1, len(os.sched_getaffinity(0)))
    threads = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        return _cpu_baseline(layer, x, w, budget_s, cores, oneuron, scans)
    finally:
        torch.set_num_threads(threads)


def cpu_inputs(layer, x, w):
    """Host copies of what the CPU baseline needs (the layer's weights and delays, its input
    -- the first 32 steps of runs longer than 256 --, its full length): taken right after the
    GPU measurement, so that the baseline can run after every GPU workload has been timed."""
    from oracle.delays import hybrid_delays
    W = layer.recurrent_weights.detach().float().cpu()
    if w['kind'] == 'hybrid':
        par = layer.parametrizations.recurrent_delays
        d = hybrid_delays(par.original.detach().cpu(), par[0].offsets.detach().float().cpu())
    else:
        d = layer.recurrent_delays.detach().cpu()
    T = x.shape[0]
    return {'W': W, 'd': d, 'x': x[:T if T <= 256 else 32].detach().cpu(), 'T': T}


def _cpu_baseline(layer, x, w, budget_s, cores, oneuron, scans):
    inp = layer if isinstance(layer, dict) else cpu_inputs(layer, x, w)
    W, d, xc, T = inp['W'], inp['d'], inp['x'], inp['T']
    B, N = xc.shape[1], xc.shape[2]
    lif = oneuron.LIFParams(tau=w['tau'])
    fn = scans.axonal_v2 if w['kind'] == 'axonal' else scans.synaptic_v2

    def one(Tp):
        xs = xc[:Tp].clone().requires_grad_(True)
        Wl, dl = W.clone().requires_grad_(True), d.clone().requires_grad_(True)
        t0 = time.perf_counter()
        y, _ = fn(xs, Wl, dl, lif, sigma=w['sigma'])
        y.sum().backward()
        return time.perf_counter() - t0

    tw = min(T, 8)
    per_step = one(tw) / tw                       # warmup, and the cost estimate
    # the median of 3 samples at T' and at T' / 2: T' = T where that fits the budget,
    # else the largest of 32, 16, 8 steps that does (one sample where none does)
    runs = 3
    Tl = min(T, xc.shape[0])
    while Tl > 8 and per_step * Tl * 1.5 * runs > budget_s:
        Tl = min(Tl, 32) if Tl > 32 else Tl // 2
    if per_step * Tl * 1.5 * runs > budget_s:
        runs = 1
    Ts = max(1, Tl // 2)

    def median(xs):
        xs = sorted(xs)
        return xs[len(xs) // 2]

    t_long = median([one(Tl) for _ in range(runs)])
    t_short = median([one(Ts) for _ in range(runs)])
    nts = Tl * B * N / t_long
    return {'value': nts, 'unit': 'neuron-timesteps/s', 'cores': cores, 'kind': 'port',
            'cpu_model': cpu_model(),
            'sample': f'oracle v2 scan + autograd BPTT, fp32, same weights/delays/input, full B={B} '
                      f'N={N}, first {Tl} of T={T} steps ({"median of 3" if runs == 3 else "1 sample"} '
                      f'after a warmup), scaled per '
                      f'neuron-timestep; one layer (stacked layers have the same shape)',
            'seconds_per_sample': t_long,
            'linearity': {'T_short': Ts, 'T_long': Tl, 's_per_step_short': t_short / Ts,
                          's_per_step_long': t_long / Tl, 'ratio': (t_long / Tl) / (t_short / Ts)}}


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


def measure_peaks():
    """Achievable peaks on this GPU, beside the datasheet figures: HBM bandwidth of a plain
    device copy (1 GiB read + 1 GiB written, torch's copy kernel) and the MFMA rate of a
    register-only loop of independent bf16 / fp32 matrix instructions on every CU
    (``delrec_peak_mfma``); each the median of 5 timed launches after a warmup, timed with
    events on the stream the work runs on (the reference profiler's protocol,
    experiments/profiling/profile_kernels.py:65-66,165-176, is a median of repeats)."""
    from delrec import _lib
    dev = torch.device('cuda:0')
    st = torch.cuda.current_stream()

    def median_ms(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(st)
            fn()
            b.record(st)
            b.synchronize()
            ts.append(a.elapsed_time(b))
        return sorted(ts)[len(ts) // 2]

    n = (1 << 30) // 4
    src = torch.rand(n, device=dev)
    dst = torch.empty_like(src)
    copy_ms = median_ms(lambda: dst.copy_(src))
    del src, dst
    out = {'copy_GBps': 2.0 * n * 4 / (copy_ms * 1e-3) / 1e9, 'copy_bytes': 2 * n * 4}
    sink = torch.empty(1024 * 1024, device=dev)
    for kind, name, iters in ((0, 'mfma_bf16_TFLOPs', 20000), (1, 'mfma_fp32_TFLOPs', 20000)):
        flops = [0.0]

        def run(kind=kind, iters=iters):
            flops[0] = _lib.peak_mfma(kind, iters, sink, st.cuda_stream)

        ms = median_ms(run)
        out[name] = flops[0] / (ms * 1e-3) / 1e12
    out['datasheet'] = {'hbm_GBps': PEAK_HBM / 1e9, 'bf16_TFLOPs': PEAK_BF16 / 1e12, 'fp32_TFLOPs': PEAK_FP32 / 1e12}
    return out


def with_measured(roof, peaks):
    """Add the measured peak of the roofline's bound and the fraction of it achieved."""
    if roof['unit'] == 'GB/s':
        meas = peaks['copy_GBps']
    else:
        meas = peaks['mfma_bf16_TFLOPs'] if roof['peak'] * 1e12 == PEAK_BF16 else peaks['mfma_fp32_TFLOPs']
    roof['peak_measured'] = meas
    roof['frac_of_measured'] = roof['achieved'] / meas


def load_traffic(kernel, config):
    p = os.path.join(ROOT, 'profiles', f'traffic_{kernel}_{config}.json')
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get('bytes_per_launch'), os.path.relpath(p, ROOT)
    return None, None


def measure(name, steps, warmup, with_cpu):
    """Time one workload; returns its JSON record."""
    from delrec import _lib
    w = WORKLOADS[name]
    dev = torch.device('cuda:0')
    m = build(w, dev)
    xs, gys, firing, ys_out = layer_inputs(m)
    inter_ms = inter_linear_ms(m, ys_out) if m.inter else None
    del ys_out
    T, B, N = xs[0].shape
    nl = len(m.layers)
    xins = [x.detach().clone().requires_grad_(True) for x in xs]

    def step():
        for layer, xin, gy in zip(m.layers, xins, gys):
            layer.zero_grad(set_to_none=True)
            xin.grad = None
            layer(xin).backward(gy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / steps
    # per scan kernel (HIP events on the kernels' stream) and per entry point (scan +
    # reductions + GEMMs), from a few extra steps outside the timed region: the event
    # pairs would otherwise add their own gaps to the timed steps
    n_extra = min(3, max(1, steps))
    with _lib.scan_timing(2 * n_extra * nl + 8) as scans_t:
        for _ in range(n_extra):
            step()
        torch.cuda.synchronize()
    with _lib.timing() as rec:
        for _ in range(n_extra):
            step()
        torch.cuda.synchronize()
    per_entry, per_scan = {}, {}
    for ename, s, e in rec:
        per_entry.setdefault(ename, []).append(s.elapsed_time(e))
    for kind, dt in scans_t.launches:
        per_scan.setdefault(kind, []).append(dt)
    avg = {k: sum(v) / len(v) for k, v in per_entry.items()}
    scan_avg = {k: sum(v) / len(v) for k, v in per_scan.items()}
    nt_layer = T * B * N
    value = nl * nt_layer / (ms * 1e-3)
    work = algorithmic_work(w)
    peak = peak_of(w)
    t_bound = None
    if w['bound'] != 'cpu':
        # compute priced at the peak of the weights' type: BF16 MFMA for bf16 W (C3, C5),
        # FP32 otherwise
        peak_c = PEAK_BF16 if w['w_bf16'] else PEAK_FP32
        t_bound = nl * max(work['bytes'] * nt_layer / PEAK_HBM, work['flops'] * nt_layer / peak_c)

    # the dominant kernel: the time scan with the longest average launch, priced against
    # the workload's binding roofline (algorithmic bytes for HBM, flops otherwise)
    dom = max(scan_avg, key=scan_avg.get)
    dur = scan_avg[dom] * 1e-3
    direction = 'fwd' if dom.endswith('fwd_scan') else 'bwd'
    kernel = SCAN_SYMBOL[name][dom]
    traffic, traffic_src = load_traffic(kernel, name)
    if w['bound'] == 'hbm':
        per_launch = work['scan_bytes'][direction] * nt_layer
        roof = {'bound': 'hbm', 'achieved': per_launch / dur / 1e9, 'peak': PEAK_HBM / 1e9, 'unit': 'GB/s',
                'frac': per_launch / dur / PEAK_HBM, 'bytes_per_launch': per_launch}
    else:
        per_launch = work['scan_flops'][direction] * nt_layer
        pk = PEAK_BF16 if w['bound'] == 'bf16' else PEAK_FP32
        roof = {'bound': 'mfma', 'achieved': per_launch / dur / 1e12, 'peak': pk / 1e12, 'unit': 'TFLOP/s',
                'frac': per_launch / dur / pk, 'flops_per_launch': per_launch}
    roof.update({'traffic': traffic, 'traffic_source': traffic_src, 'kernel': kernel,
                 'avg_launch_ms': scan_avg[dom]})
    line = {
        'workload': f"{name}: {w['label']}",
        'value': value,
        'ms_per_step': ms,
        'layers': nl,
        'T': T, 'B': B, 'N': N,
        'delay_kind': w['kind'], 'sigma': w['sigma'], 'firing_rate': firing,
        'roofline': roof,
        'layer_roofline': None if t_bound is None else {
            'bound': w['bound'], 't_bound_ms': t_bound * 1e3, 'frac': t_bound / (ms * 1e-3),
            'bytes_per_nt': work['bytes'], 'flops_per_nt': work['flops']},
        'scan_ms': scan_avg,
        'entry_ms': avg,
        'per_layer_value': nt_layer / (ms * 1e-3 / nl),
    }
    if inter_ms is not None:
        line['inter_linear_ms'] = inter_ms
    print(f'[bench] {name}: {ms:.2f} ms/step on the GPU', file=sys.stderr, flush=True)
    cpu_in = cpu_inputs(m.layers[0], xs[0], w) if with_cpu else None
    return line, cpu_in


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=10)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--config', default=None, choices=sorted(WORKLOADS),
                    help=f'the workload of the line (default {DEFAULT_CONFIG}, with the others as extras)')
    ap.add_argument('--extra', default=None,
                    help='comma-separated further workloads reported under "extra" (each with its own '
                         'roofline and CPU baseline); "" for none. Default: C1,C2,C3,C4 beside the '
                         'default workload, none beside an explicit --config')
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline leg')
    ap.add_argument('--calibrate-copy', type=int, metavar='MIB', default=0,
                    help='only run a plain device copy of MIB MiB (counter calibration)')
    args = ap.parse_args()
    if args.extra is None:
        args.extra = 'C1,C2,C3,C4' if args.config is None else ''
    if args.config is None:
        args.config = DEFAULT_CONFIG
    if args.gpus != 1:
        print(f'bench.py measures one GPU; --gpus {args.gpus} is not supported by this build '
              f'(the layer shards over batch rows with one dW/dd all-reduce per step, not run here)',
              file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return
    from delrec import _lib
    _lib.load()
    # every GPU measurement first, then the CPU baselines (whose worker threads would
    # otherwise compete with the host thread that feeds the GPU)
    rec, cpu_in = measure(args.config, args.steps, args.warmup, not args.no_cpu)
    w = WORKLOADS[args.config]
    line = {
        'metric': 'neuron-timesteps/sec fwd+BPTT per recurrent layer; % HBM GB/s or MFMA peak',
        'value': rec['value'],
        'unit': 'neuron-timesteps/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': rec['ms_per_step'],
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16-weights/f32' if w['w_bf16'] else 'f32',
        'data': 'synthetic (seeded inputs of the stated shape, random-init weights)',
        'config': {'workload': rec['workload'], 'layers': rec['layers'], 'T': rec['T'], 'B': rec['B'],
                   'N': rec['N'], 'delay_kind': rec['delay_kind'], 'sigma': rec['sigma'],
                   'firing_rate': rec['firing_rate']},
        'roofline': rec['roofline'],
        'layer_roofline': rec['layer_roofline'],
        'per_layer_value': rec['per_layer_value'],
        'scan_ms': rec['scan_ms'],
        'entry_ms': rec['entry_ms'],
    }
    if 'inter_linear_ms' in rec:
        line['inter_linear_ms'] = rec['inter_linear_ms']
    extra = [c for c in args.extra.split(',') if c]
    extra_cpu = {}
    if extra:
        line['extra'] = {}
        for c in extra:
            print(f'[bench] extra workload {c}', file=sys.stderr, flush=True)
            line['extra'][c], extra_cpu[c] = measure(c, args.steps, args.warmup, not args.no_cpu)
    # measured achievable peaks, and each dominant kernel's fraction of the measured one
    peaks = measure_peaks()
    line['peaks'] = peaks
    with_measured(line['roofline'], peaks)
    for c in extra:
        with_measured(line['extra'][c]['roofline'], peaks)
    if cpu_in is not None:
        print(f'[bench] CPU baseline {args.config}', file=sys.stderr, flush=True)
        line['cpu_baseline'] = cpu_baseline(cpu_in, None, w)
    for c in extra:
        if extra_cpu.get(c) is not None:
            print(f'[bench] CPU baseline {c}', file=sys.stderr, flush=True)
            line['extra'][c]['cpu_baseline'] = cpu_baseline(extra_cpu[c], None, WORKLOADS[c])
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
