"""delrec-mi355x: DelRec's recurrent delayed-LIF layer on AMD MI355X (gfx950).

Forward and BPTT backward of the axonal, synaptic and hybrid delay layers run as
hand-written HIP kernels (``libdelrec_hip.so``, C ABI in ``include/delrec.h``) behind the
module / autograd API of the reference package ``delrec`` 1.0.0.
"""

__version__ = '0.1.0'
