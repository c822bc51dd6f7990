"""Surrogate-gradient ids (reference ``triton_kernels/surrogate.py``).

The ids are the reference's load-bearing contract, 0 = triangle(gamma), 1 = ATan(alpha),
and are the values ``delrec_lif.surrogate`` takes in the C ABI.
"""

_SURR_ID = {'triangle': 0, 'atan': 1}


def surrogate_id(surrogate_function, gamma=None):
    """``(id, gamma, alpha)`` for a config's ``surrogate_function``: the ``Triangle.apply``
    function, an ATan module (anything with ``surrogate_kind == 'atan'`` or a class name
    containing ``ATan``). Other surrogates are rejected rather than silently mapped."""
    from ..utils import Triangle
    g = 1.0 if gamma is None else float(gamma)
    is_triangle = (getattr(surrogate_function, '__self__', None) is Triangle
                   and getattr(surrogate_function, '__name__', '') == 'apply')
    if is_triangle or getattr(surrogate_function, 'surrogate_kind', None) == 'triangle':
        return _SURR_ID['triangle'], float(getattr(surrogate_function, 'gamma', g)), 2.0
    kind = getattr(surrogate_function, 'surrogate_kind', None)
    if kind == 'atan' or 'ATan' in type(surrogate_function).__name__:
        return _SURR_ID['atan'], g, float(getattr(surrogate_function, 'alpha', 2.0))
    raise ValueError(f'unsupported surrogate function {surrogate_function!r}: the HIP kernels '
                     f'implement Triangle (id 0) and ATan (id 1)')
