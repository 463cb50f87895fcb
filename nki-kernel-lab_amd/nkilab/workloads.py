"""Seeded synthetic inputs for the five benchmark workloads.

Every tensor is drawn as ``np.random.default_rng(seed).standard_normal(shape,
dtype=np.float32)`` (scaled where a distribution other than N(0, 1) is
named) and rounded to bfloat16 with torch (round-to-nearest-even), in the
draw order documented per function, so the GPU, the CPU oracle and the
PyTorch CPU reference all see the same values.
"""
from __future__ import annotations

import numpy as np
import torch

from .model import BlockConfig, DecoderBlock

MATMUL = dict(M=1024, N=1024, K=1024)
ROWS = dict(R=4096, D=2048, eps=1e-6)
ATTENTION = dict(H=8, S=2048, d=128)
LONG_A = dict(H=1, S=4096, d=128)
LONG_B = dict(H=32, S=16384, d=128)
DECODER = dict(S=2048, d_model=2048, n_heads=16, d_ff=5632, eps=1e-6)


def _normal(rng: np.random.Generator, shape, std: float = 1.0, mean: float = 0.0,
            dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    a = rng.standard_normal(shape, dtype=np.float32)
    if std != 1.0 or mean != 0.0:
        a = a * np.float32(std) + np.float32(mean)
    return torch.from_numpy(a).to(dtype)


def matmul_inputs(M=1024, N=1024, K=1024, seed=0, dtype=torch.bfloat16):
    """A [M, K] then B [K, N], N(0, 1)."""
    rng = np.random.default_rng(seed)
    return _normal(rng, (M, K), dtype=dtype), _normal(rng, (K, N), dtype=dtype)


def rows_inputs(R=4096, D=2048, seed=0, dtype=torch.bfloat16):
    """x [R, D] ~ N(0, 1); w [D] ~ N(1, 0.1); gate, up [R, D] ~ N(0, 1), in that order."""
    rng = np.random.default_rng(seed)
    x = _normal(rng, (R, D), dtype=dtype)
    w = _normal(rng, (D,), std=0.1, mean=1.0, dtype=dtype)
    gate = _normal(rng, (R, D), dtype=dtype)
    up = _normal(rng, (R, D), dtype=dtype)
    return x, w, gate, up


def attention_inputs(H=8, S=2048, d=128, seed=0, dtype=torch.bfloat16):
    """q, k, v [H, S, d] ~ N(0, 1), in that order."""
    rng = np.random.default_rng(seed)
    return tuple(_normal(rng, (H, S, d), dtype=dtype) for _ in range(3))


def decoder_inputs(S=2048, d_model=2048, n_heads=16, d_ff=5632, eps=1e-6, seed=0):
    """A DecoderBlock whose linear weights are bf16 values drawn from N(0, 0.02)
    (wqkv, wo, wg, wu, wd in that order, nn.Linear [out, in] layout) and whose
    norm weights are ones; then x [S, d_model] ~ N(0, 1) in fp32.  The block's
    parameters are fp32 tensors holding the bf16 values, so the fp32 eager
    block and the bf16 kernel path see identical weights."""
    cfg = BlockConfig(d_model=d_model, n_heads=n_heads, d_ff=d_ff, eps=eps)
    block = DecoderBlock(cfg).eval()
    rng = np.random.default_rng(seed)
    with torch.no_grad():
        for name in ("wqkv", "wo", "wg", "wu", "wd"):
            lin = getattr(block, name)
            lin.weight.copy_(_normal(rng, tuple(lin.weight.shape), std=0.02).float())
        block.norm1.weight.fill_(1.0)
        block.norm2.weight.fill_(1.0)
    x = _normal(rng, (S, d_model), dtype=torch.float32)
    return block, x


# Algorithmic work of the benchmark configurations (the roofline numerators).

def causal_flops(H: int, S: int, d: int) -> int:
    """Exact FLOPs of causal attention: 4 d per (query, key <= query) pair,
    4 H d S (S + 1) / 2 (two products of d multiply-adds per pair)."""
    return 4 * H * d * S * (S + 1) // 2


def decoder_flops(S=2048, d_model=2048, n_heads=16, d_ff=5632) -> int:
    """FLOPs of one decoder block forward: the five projections (2 M N K
    each) and causal attention."""
    hd = d_model // n_heads
    gemm = 2 * S * d_model * (3 * d_model) + 2 * S * d_model * d_model + 2 * (2 * S * d_model * d_ff) + \
        2 * S * d_ff * d_model
    return gemm + causal_flops(n_heads, S, hd)
