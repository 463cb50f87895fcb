"""Causal attention kernels with the reference's names, tile constant and
argument layout (nkilab/kernels/attention.py:24-325): qT and kT are
[H, d, S] (q and k transposed per head), v is [H, S, d], S a multiple of
T, and the caller passes the softmax scale."""
from __future__ import annotations

import numpy as np

from .. import ops

T = 128  # query / key tile


def _run(variant, qT, kT, v, scale):
    H, d, S = qT.shape
    assert S % T == 0 and d <= 128
    tr = (lambda t: t.transpose(1, 2)) if hasattr(qT, "is_cuda") else (lambda t: np.asarray(t).transpose(0, 2, 1))
    return ops.attention(tr(qT), tr(kT), v, variant=variant, scale=scale)


def attention_naive(qT, kT, v, scale: float):
    """attention.py:35-89: scores and probabilities materialised in HBM."""
    return _run("naive", qT, kT, v, scale)


def flash_attention(qT, kT, v, scale: float):
    """attention.py:155-176."""
    return _run("flash", qT, kT, v, scale)


def flash_attention_kv_resident(qT, kT, v, scale: float):
    """attention.py:179-201."""
    return _run("flash_kv_resident", qT, kT, v, scale)


def flash_attention_balanced(qT, kT, v, scale: float):
    """attention.py:249-277."""
    return _run("flash_balanced", qT, kT, v, scale)


def flash_attention_pipelined(qT, kT, v, scale: float, ILP: int = 2):
    """attention.py:280-325 (ILP is the reference's interleave depth; the
    gfx950 kernel's pipelining is its own)."""
    return _run("flash_pipelined", qT, kT, v, scale)
