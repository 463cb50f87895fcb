"""CPU oracle for the nkilab kernel set -- TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference's NKI kernels (nkilab/kernels/*.py) and
host wrappers (nkilab/ops.py, nkilab/model.py), keeping their precision points
(fp32 accumulation per 128-deep K chunk, fp32 row statistics, reciprocal
multiplies, a negated running max, P rounded to bf16 before P.V, a single
round-to-nearest-even output cast).  Only tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg may import it, and only as the reference that
results are compared against; the product (nkilab) never calls it.

See nki_ref.py for the functions and how each one is pinned.
"""
from .nki_ref import *  # noqa: F401,F403
