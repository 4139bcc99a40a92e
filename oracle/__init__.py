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
