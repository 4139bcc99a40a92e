"""Float64 numpy oracle of tt-rl's learner-update path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (`tt-rl_amd/`) imports,
links or runs anything under this directory; only `tests/`,
`__graft_entry__.smoke()` and `bench.py`'s CPU-baseline leg use it, and only
as the checker (or, for the baseline, as the timed CPU restatement).

Each function restates the reference's arithmetic and cites the reference
file:line it follows.  How each part is pinned (known answers from the
reference's own tests, closed forms, brute force, finite differences and an
independent torch-CPU float64 autograd) is in tests/test_oracle_*.py.
"""

from contextlib import contextmanager

import numpy as np

_FLOAT = [np.float64]


def float_type():
    """The oracle's arithmetic type: float64 (the checker's), unless a
    `precision` block sets another."""
    return _FLOAT[0]


def fa(x):
    """np.asarray(x) in the oracle's arithmetic type."""
    return np.asarray(x, _FLOAT[0])


@contextmanager
def precision(dtype):
    """The oracle's arithmetic in `dtype` inside the block (bench.py's CPU
    baseline times it in float32, the GPU path's type, beside float64).
    Every parity check uses the float64 default."""
    old = _FLOAT[0]
    _FLOAT[0] = np.dtype(dtype).type
    try:
        yield
    finally:
        _FLOAT[0] = old
