"""Writes the golden fixtures in this directory from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors and its kernels run only on the NKI
simulator, which cannot be installed here; these fixtures are inputs and
outputs of the oracle (oracle/nki_ref.py), which tests/test_oracle.py pins to
torch, closed forms and invariants.  The GPU tests compare the HIP kernels to
them.  bfloat16 tensors are stored as their fp32 values (exactly representable).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle as O  # noqa: E402


def _n(rng, shape, dtype, scale=1.0):
    x = (rng.standard_normal(shape) * scale).astype(np.float32)
    return O.bf16_round(x) if dtype == O.BF16 else x


def matmul_case():
    rng = np.random.default_rng(101)
    out = {}
    for tag, (M, K, N), dt in (("f32", (33, 70, 45), O.F32), ("f32b", (96, 128, 160), O.F32),
                                ("bf16", (128, 256, 160), O.BF16)):
        a, b = _n(rng, (M, K), dt), _n(rng, (K, N), dt)
        out.update({f"{tag}_a": a, f"{tag}_b": b, f"{tag}_c": O.ops_matmul(a, b, dtype=dt)})
    return out


def rows_case():
    rng = np.random.default_rng(202)
    out = {}
    for tag, (R, D), dt in (("f32", (5, 3), O.F32), ("f32b", (128, 64), O.F32), ("bf16", (64, 256), O.BF16),
                            ("bf16r", (9, 200), O.BF16)):
        x = _n(rng, (R, D), dt, scale=4.0)
        w = O.cast(rng.uniform(0.5, 1.5, D).astype(np.float32), dt)
        g, u = _n(rng, (R, D), dt), _n(rng, (R, D), dt)
        out.update({f"{tag}_x": x, f"{tag}_w": w, f"{tag}_g": g, f"{tag}_u": u,
                    f"{tag}_softmax": O.softmax_fused(x, dt), f"{tag}_softmax_unfused": O.softmax_unfused(x, dt),
                    f"{tag}_rmsnorm": O.rmsnorm_fused(x, w, 1e-6, dt), f"{tag}_swiglu": O.swiglu_fused(g, u, dt)})
    return out


def attention_case():
    rng = np.random.default_rng(303)
    out = {}
    for tag, (H, S, d), dt in (("f32", (2, 200, 32), O.F32), ("bf16", (2, 256, 64), O.BF16),
                                ("bf16r", (1, 131, 128), O.BF16)):
        q, k, v = (_n(rng, (H, S, d), dt) for _ in range(3))
        out.update({f"{tag}_q": q, f"{tag}_k": k, f"{tag}_v": v,
                    f"{tag}_flash": O.ops_attention(q, k, v, "flash_pipelined", dt),
                    f"{tag}_naive": O.ops_attention(q, k, v, "naive", dt)})
    return out


def decoder_case():
    rng = np.random.default_rng(404)
    d, H, f, S = 64, 4, 128, 40
    params = {"wqkv": _n(rng, (3 * d, d), O.F32, 0.1), "wo": _n(rng, (d, d), O.F32, 0.1),
              "wg": _n(rng, (f, d), O.F32, 0.1), "wu": _n(rng, (f, d), O.F32, 0.1),
              "wd": _n(rng, (d, f), O.F32, 0.1),
              "norm1": rng.uniform(0.5, 1.5, d).astype(np.float32),
              "norm2": rng.uniform(0.5, 1.5, d).astype(np.float32)}
    x = _n(rng, (S, d), O.F32)
    y = O.nki_forward_ref(params, x, H, 1e-6, "flash_pipelined", O.F32)
    return {**params, "x": x, "y": y, "n_heads": np.array(H)}


CASES = {"matmul": matmul_case, "rows": rows_case, "attention": attention_case, "decoder": decoder_case}


def main():
    for name, build in CASES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **build())
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
