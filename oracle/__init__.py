"""CPU oracle for the delayed-LIF recurrent layer — TEST INFRASTRUCTURE ONLY.

This package is a from-scratch restatement, in plain PyTorch (fp32/fp64, autograd BPTT),
of the reference's pure-PyTorch scans and of the spikingjelly LIF neuron they call:

  * ``oracle.neuron``  LIF charge / fire / reset and the ATan / Triangle surrogates
                       (spikingjelly ``LIFNode`` semantics as called at
                       ``src/delrec/delay_layers_pytorch.py:179,310``; ``utils.Triangle``
                       at ``src/delrec/utils.py:23-41``).
  * ``oracle.delays``  the triangular delay kernel, its window length ``L`` and the
                       closed-form delay gradient (``triton_kernels/delays.py:13-63``,
                       ``triton_kernels/synaptic_hybrid.py:93-113``).
  * ``oracle.scans``   the dense sliding-window scans ``v2`` and the circular-buffer
                       scans ``v1`` for axonal and synaptic delays
                       (``delay_layers_pytorch.py:53-194, 220-325``).
  * ``oracle.model``   a reference forward of a whole ``SNN_*`` stack that swaps every
                       recurrent delay layer for the oracle scan.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this package, and only as the checker or the timed CPU baseline. The product
(``snn-delays_amd/delrec``) never imports it and has no CPU fallback.

Pinning status of each function is stated in its docstring. The pins -- closed forms,
the known-answer inputs of the reference's own tests, invariants and hand-derived golden
vectors (``tests/golden/make_fixtures.py``; no reference code is run) -- are in
``tests/test_oracle_*.py``.
Parity unpinned: only spikingjelly's fp32 operation order inside the ``v_reset != 0`` and
``decay_input`` charge forms (spikingjelly is not installed; the forms themselves are
pinned by their closed forms at zero recurrent weight).
"""

from . import neuron, delays, scans, model  # noqa: F401
