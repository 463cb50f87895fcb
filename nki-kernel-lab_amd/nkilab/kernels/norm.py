"""Row kernels with the reference's names and row-tile constant
(nkilab/kernels/norm.py:14-136): x is [rows, cols]."""
from __future__ import annotations

from .. import ops

P = 128  # rows per tile in the reference's SBUF layout


def softmax_unfused(x):
    """norm.py:22-62: three passes through HBM."""
    return ops.softmax(x, fused=False)


def softmax_fused(x):
    """norm.py:65-89: one pass."""
    return ops.softmax(x, fused=True)


def rmsnorm_fused(x, weight, eps: float = 1e-6):
    """norm.py:92-118."""
    return ops.rmsnorm(x, weight, eps)


def swiglu_fused(gate, up):
    """norm.py:121-136."""
    return ops.swiglu(gate, up)
