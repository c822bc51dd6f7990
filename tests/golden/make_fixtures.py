"""Write the hand-derived fixtures of the parity tests (tests/golden/*.json).

Nothing here runs the oracle or the reference: every expected value is worked out from
the defining formulas by hand-written scalar Python.

known_answer_delay_grad.json
    The reference's known-answer inputs (tests/check_hybrid_kernel.py:143-152):
    d = [0, 1, 2, 0.25, 1.5] on every row, W = arange(1, 26) / 25, C[..., l] = l^2.
    dd[i,j] = W[i,j] * sum_l C_l * sign(l-1-d) * [|l-1-d| <= s] / s^2 with s = 1 + sigma.
single_spike.json
    One source spikes once at t = 0 and feeds one receiver through weight w: the
    recurrent input of the receiver at step t is w * h(t; d, s) with
    h(l; d, s) = max(0, s - |l - 1 - d|) / s^2 (the paper's Eq. 7: a spike of j at t
    reaches i at t + 1 + d, spread by the triangle).
"""

import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))


def sign(a):
    return (a > 0) - (a < 0)


def delay_grad_expected(sigma):
    s = 1.0 + sigma
    ds = [0.0, 1.0, 2.0, 0.25, 1.5]
    L = int(math.ceil(1.0 + max(ds) + s)) + 1
    out = []
    for i in range(5):
        row = []
        for j in range(5):
            w = (5 * i + j + 1) / 25.0
            acc = 0.0
            for l in range(1, L):
                a = l - 1.0 - ds[j]
                if abs(a) <= s:
                    acc += (l * l) * sign(a) / (s * s)
            row.append(w * acc)
        out.append(row)
    return {'sigma': sigma, 'L': L, 'd_row': ds, 'expected_dd': out}


def single_spike_expected(d, sigma, w, T):
    s = 1.0 + sigma
    rec = []
    for t in range(T):
        rec.append(w * max(0.0, s - abs(t - 1.0 - d)) / (s * s) if t >= 1 else 0.0)
    return {'d': d, 'sigma': sigma, 'w': w, 'T': T, 'expected_rec': rec}


def main():
    with open(os.path.join(HERE, 'known_answer_delay_grad.json'), 'w') as f:
        json.dump([delay_grad_expected(sg) for sg in (0.0, 0.5, 1.0)], f, indent=1)
    cases = [single_spike_expected(d, sg, 0.25, 12)
             for d, sg in ((3.0, 0.0), (2.3, 0.0), (2.3, 1.0), (0.0, 0.0), (4.5, 0.5), (1.75, 2.0))]
    with open(os.path.join(HERE, 'single_spike.json'), 'w') as f:
        json.dump(cases, f, indent=1)


if __name__ == '__main__':
    main()
