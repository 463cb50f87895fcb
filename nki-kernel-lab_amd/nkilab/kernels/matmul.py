"""C[M, N] = lhsT.T @ rhs with the reference's tile constants and argument
layout (nkilab/kernels/matmul.py:19-82): lhsT is the left operand already
transposed ([K, M]), shapes are tile multiples, and the blocked kernel's
BM x BN fp32 accumulator tiles must fit 8 PSUM banks (checked by the C
library, ``nkl_check_blocks``, with the same error text)."""
from __future__ import annotations

import numpy as np

from .. import _lib, ops

TK = 128  # contraction tile
TM = 128  # output rows per tile
TN = 512  # output columns per tile (one fp32 PSUM bank of the reference)


def _lhs(lhsT):
    a = np.asarray(lhsT) if not hasattr(lhsT, "is_cuda") else lhsT
    return a.T


def matmul_naive(lhsT, rhs):
    """matmul.py:24-43: the variant that reloads both operands for every tile."""
    K, M = lhsT.shape
    N = rhs.shape[1]
    assert K % TK == 0 and M % TM == 0 and N % TN == 0
    return ops.matmul(_lhs(lhsT), rhs, variant="naive")


def matmul_blocked(lhsT, rhs, BM: int = 2, BN: int = 4):
    """matmul.py:46-82: the register-blocked variant; BM x BN output tiles per block."""
    K, M = lhsT.shape
    N = rhs.shape[1]
    _lib.call("nkl_check_blocks", int(BM), int(BN))  # "... PSUM ..." when BM * BN > 8
    assert K % TK == 0 and M % (TM * BM) == 0 and N % (TN * BN) == 0
    return ops.matmul(_lhs(lhsT), rhs, variant="blocked")
