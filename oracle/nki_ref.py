"""NumPy restatement of the reference's NKI kernel set -- the ORACLE.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg, as the reference that results are compared
against; never by the nkilab product.

Conventions.  Arrays are np.float32.  A bfloat16 tensor is an np.float32 array
whose values are all bf16-representable, tagged by a ``dtype`` argument
("float32" or "bfloat16"); rounding to bfloat16 is ``bf16_round``
(round-to-nearest-even, the rounding of torch's ``.to(torch.bfloat16)``).
Every function cites the reference lines it restates (paths relative to the
reference repository).

How each function is pinned (tests/test_oracle.py):
  bf16_round           torch .to(bfloat16) on random, tie, subnormal, inf, nan inputs
  choose_blocks        brute force over 8 x 16 grids (ref tests/test_matmul.py:40-45)
  matmul_*/ops_matmul  float64 A @ B: rel < 1e-5 fp32 at the reference test shapes
                       (tests/test_matmul.py:15-20); bf16 output equals bf16_round of
                       the float64 product except at rounding ties; Hypothesis shapes
  softmax_*            torch.softmax (rtol 1e-5, atol 1e-6), rows sum to 1, finite at
                       1e4 logits (tests/test_norm.py:14-38)
  rmsnorm_fused        torch closed form, rel < 1e-5 (tests/test_norm.py:41-47)
  swiglu_fused         F.silu(g) * u, rel < 1e-5 (tests/test_norm.py:58-62)
  attention (all)      torch SDPA(is_causal=True), atol 2e-5 fp32; bf16 rel < 3e-2;
                       row 0 == v[0]; flash_balanced == flash_pipelined bitwise;
                       QK^T tile count n(n+1)/2 vs n^2 (tests/test_attention.py,
                       tests/test_profiler.py:51-61)
  nki_forward_ref      torch DecoderBlock, atol 1e-5 fp32 (tests/test_model.py:8-17)
  rope                 (not in the reference) identity at position 0; each (i, i + d/2)
                       pair keeps its norm; <rope(q, m), rope(k, n)> depends on m - n
                       only; equals an independent torch float64 rotate-half formula
  GQA in ops_attention (not in the reference) SDPA on K/V heads repeated H / Hkv times

Parity unpinned at the bit level (no reference test or fixture fixes them, and
the NKI simulator is not installable here): the simulator's exp / rsqrt /
reciprocal / silu accuracy; whether an activation's fused row reduction sums
the fp32 results or the dtype-cast ones (fp32 here); whether scale*x + bias is
fused; the PSUM accumulation order inside one 128-deep K chunk.  All of these
sit below the tolerances above.
"""
from __future__ import annotations

import math

import numpy as np

F32, BF16 = "float32", "bfloat16"

TK, TM, TN = 128, 128, 512      # kernels/matmul.py:19-21
P = 128                         # kernels/norm.py:14
T = 128                         # kernels/attention.py:24
NEG_INF = np.float32(-3.0e38)   # kernels/attention.py:25

__all__ = [
    "F32", "BF16", "TK", "TM", "TN", "T", "NEG_INF", "bf16_round", "cast", "choose_blocks",
    "matmul_naive", "matmul_blocked", "ops_matmul", "softmax_fused", "softmax_unfused",
    "rmsnorm_fused", "swiglu_fused", "attention_naive", "flash_attention",
    "flash_attention_kv_resident", "flash_attention_balanced", "flash_attention_pipelined",
    "ATTENTION_VARIANTS", "ops_attention", "nki_forward_ref", "rel_err", "causal_flops", "rope",
]


# ---------------------------------------------------------------- dtypes --

def bf16_round(x) -> np.ndarray:
    """fp32 -> nearest bf16 value (ties to even), returned as fp32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out)
    return out


def cast(x, dtype: str) -> np.ndarray:
    """Output cast of an NKI tile copy: fp32 passes through, bf16 rounds once."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == BF16:
        return bf16_round(x)
    if dtype != F32:
        raise ValueError(f"dtype {dtype!r}")
    return x


def rel_err(a, b) -> float:
    """max|a - b| / max|b| in float64 (the reference's tests/conftest.py:15-18)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-12))


# ---------------------------------------------------------------- matmul --

def choose_blocks(m_tiles: int, n_tiles: int) -> tuple[int, int]:
    """ops.py:27-35: the BM x BN block with BM*BN <= 8 dividing the tile grid that
    has the most tiles, ties going to the larger BN."""
    best = (1, 1)
    for bm in (1, 2, 4):
        for bn in (1, 2, 4, 8):
            if bm * bn > 8 or m_tiles % bm or n_tiles % bn:
                continue
            if (bm * bn, bn) > (best[0] * best[1], best[1]):
                best = (bm, bn)
    return best


def _matmul_k_chunks(lhsT: np.ndarray, rhs: np.ndarray) -> np.ndarray:
    """fp32 accumulator += lhsT[k].T @ rhs[k] over 128-deep K chunks in order
    (the PSUM accumulate=(k > 0) chain, matmul.py:34-39 and :64-75)."""
    K = lhsT.shape[0]
    acc = np.zeros((lhsT.shape[1], rhs.shape[1]), np.float32)
    for k in range(K // TK):
        a = np.asarray(lhsT[k * TK:(k + 1) * TK], np.float32)
        b = np.asarray(rhs[k * TK:(k + 1) * TK], np.float32)
        acc += a.T @ b
    return acc


def matmul_naive(lhsT, rhs, dtype: str = F32) -> np.ndarray:
    """matmul.py:24-43: C = lhsT.T @ rhs, one cast of the fp32 accumulator."""
    K, M = lhsT.shape
    N = rhs.shape[1]
    assert K % TK == 0 and M % TM == 0 and N % TN == 0
    return cast(_matmul_k_chunks(lhsT, rhs), dtype)


def matmul_blocked(lhsT, rhs, BM: int = 2, BN: int = 4, dtype: str = F32) -> np.ndarray:
    """matmul.py:46-82.  Blocking changes only which accumulators are live at once;
    every output tile sums the same K chunks in the same order as the naive kernel."""
    K, M = lhsT.shape
    N = rhs.shape[1]
    assert K % TK == 0 and M % (TM * BM) == 0 and N % (TN * BN) == 0
    assert BM * BN <= 8, "BM*BN fp32 [128,512] accumulators must fit 8 PSUM banks"
    return cast(_matmul_k_chunks(lhsT, rhs), dtype)


def _pad_to(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.zeros((rows, cols), np.float32)
    out[: x.shape[0], : x.shape[1]] = x
    return out


def ops_matmul(a, b, variant: str = "blocked", dtype: str = F32) -> np.ndarray:
    """ops.py:38-52: pad to (128, 128, 512) multiples, lhsT = A^T, run, crop."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, (a.shape, b.shape)
    Mp, Kp, Np = (math.ceil(M / TM) * TM, math.ceil(K / TK) * TK, math.ceil(N / TN) * TN)
    lhsT = _pad_to(a, Mp, Kp).T.copy()
    rhs = _pad_to(b, Kp, Np)
    if variant == "naive":
        c = matmul_naive(lhsT, rhs, dtype)
    else:
        bm, bn = choose_blocks(Mp // TM, Np // TN)
        c = matmul_blocked(lhsT, rhs, bm, bn, dtype)
    return c[:M, :N]


# -------------------------------------------------------------- row ops --

def softmax_fused(x, dtype: str = F32) -> np.ndarray:
    """norm.py:65-89: neg_max = -max(x); e = exp(x + neg_max) with the row sum;
    rinv = 1/sum; y = e * rinv, cast once."""
    x = np.asarray(x, np.float32)
    neg_max = -x.max(axis=1, keepdims=True)
    e = np.exp(x + neg_max)
    ssum = e.sum(axis=1, keepdims=True, dtype=np.float32)
    rinv = np.float32(1.0) / ssum
    return cast(e * rinv, dtype)


def softmax_unfused(x, dtype: str = F32) -> np.ndarray:
    """norm.py:22-62: m = max(x); e = exp(x - m) (fp32, via HBM); s = sum(e); y = e / s."""
    x = np.asarray(x, np.float32)
    m = x.max(axis=1, keepdims=True)
    e = np.exp(x - m)
    s = e.sum(axis=1, keepdims=True, dtype=np.float32)
    return cast(e / s, dtype)


def rmsnorm_fused(x, weight, eps: float = 1e-6, dtype: str = F32) -> np.ndarray:
    """norm.py:92-118: ssq = sum(x^2); ms = ssq * (1/D) + eps; rstd = rsqrt(ms);
    xn = x * rstd (fp32); y = xn * w, cast once."""
    x = np.asarray(x, np.float32)
    w = np.asarray(weight, np.float32).reshape(1, -1)
    D = x.shape[1]
    ssq = (x * x).sum(axis=1, keepdims=True, dtype=np.float32)
    ms = ssq * np.float32(1.0 / D) + np.float32(eps)
    rstd = np.float32(1.0) / np.sqrt(ms)
    xn = x * rstd
    return cast(xn * w, dtype)


def swiglu_fused(gate, up, dtype: str = F32) -> np.ndarray:
    """norm.py:121-136: a = silu(g) in fp32; y = a * u, cast once."""
    g = np.asarray(gate, np.float32)
    u = np.asarray(up, np.float32)
    with np.errstate(over="ignore"):
        a = g / (np.float32(1.0) + np.exp(-g))
    return cast(a * u, dtype)


# ------------------------------------------------------------ attention --

def causal_flops(H: int, S: int, d: int) -> int:
    """Exact FLOPs of causal attention: 4*d per (query, key <= query) pair."""
    return 4 * H * d * S * (S + 1) // 2


def _mask_tile(s: np.ndarray, q0: int, k0: int) -> np.ndarray:
    """attention.py:28-32: keep s where (q0 + p) - (k0 + c) >= 0, else NEG_INF."""
    p = np.arange(s.shape[0])[:, None]
    c = np.arange(s.shape[1])[None, :]
    return np.where((q0 + p) - (k0 + c) >= 0, s, NEG_INF).astype(np.float32)


def _qk(q_tile_T: np.ndarray, k_tile_T: np.ndarray, stats: dict | None) -> np.ndarray:
    """nc_matmul(stationary=q [d, T], moving=k [d, T]) = q.T @ k, fp32."""
    if stats is not None:
        stats["qk_tiles"] = stats.get("qk_tiles", 0) + 1
    return q_tile_T.T @ k_tile_T


def _flash_update(s, vt, scale, m_run, l_run, o_run, diag, q0, k0, vdtype):
    """attention.py:92-134 (flash_attention, flash_attention_kv_resident)."""
    s_src = _mask_tile(s, q0, k0) if diag else s
    tmax = s_src.max(axis=1, keepdims=True)
    m_new = np.maximum(m_run, tmax * np.float32(scale))
    neg_m = m_new * np.float32(-1.0)
    e = np.exp(s_src * np.float32(scale) + neg_m)
    p = cast(e, vdtype)
    rsum = e.sum(axis=1, keepdims=True, dtype=np.float32)
    corr = np.exp(m_run + neg_m)
    l_new = l_run * corr + rsum
    o_new = o_run * corr + p @ vt
    return m_new, l_new, o_new


def _flash_update_balanced(s, vt, scale, nm_run, l_run, o_run, diag, q0, k0, vdtype):
    """attention.py:204-246: the running max is kept negated, nm = -m."""
    s_src = _mask_tile(s, q0, k0) if diag else s
    tmax = s_src.max(axis=1, keepdims=True)
    nm_new = np.minimum(tmax * np.float32(-scale), nm_run)
    e = np.exp(s_src * np.float32(scale) + nm_new)
    p = cast(e, vdtype)
    rsum = e.sum(axis=1, keepdims=True, dtype=np.float32)
    corr = np.exp(nm_run * np.float32(-1.0) + nm_new)
    l_new = l_run * corr + rsum
    o_new = o_run * corr + p @ vt
    return nm_new, l_new, o_new


def _flash_finish(o_run, l_run, vdtype):
    """attention.py:137-142: o * (1 / l), cast once."""
    return cast(o_run * (np.float32(1.0) / l_run), vdtype)


def _check(qT, kT, v):
    H, d, S = qT.shape
    assert S % T == 0 and d <= 128
    return H, d, S


def flash_attention(qT, kT, v, scale: float, dtype: str = F32, stats: dict | None = None) -> np.ndarray:
    """attention.py:155-176: per query tile, key tiles 0..i (later ones skipped)."""
    H, d, S = _check(qT, kT, v)
    nt = S // T
    out = np.zeros((H, S, d), np.float32)
    for h in range(H):
        for i in range(nt):
            m, l, o = np.full((T, 1), NEG_INF), np.zeros((T, 1), np.float32), np.zeros((T, d), np.float32)
            for j in range(i + 1):
                s = _qk(qT[h][:, i * T:(i + 1) * T], kT[h][:, j * T:(j + 1) * T], stats)
                m, l, o = _flash_update(s, v[h][j * T:(j + 1) * T], scale, m, l, o, j == i, i * T, j * T, dtype)
            out[h, i * T:(i + 1) * T] = _flash_finish(o, l, dtype)
    return out


def flash_attention_kv_resident(qT, kT, v, scale: float, dtype: str = F32, stats: dict | None = None):
    """attention.py:179-201: same arithmetic as flash_attention (K/V residency only
    changes where the tiles are read from)."""
    return flash_attention(qT, kT, v, scale, dtype, stats)


def flash_attention_balanced(qT, kT, v, scale: float, dtype: str = F32, stats: dict | None = None):
    """attention.py:249-277: the negated-max update, one query tile at a time."""
    H, d, S = _check(qT, kT, v)
    nt = S // T
    out = np.zeros((H, S, d), np.float32)
    for h in range(H):
        for i in range(nt):
            nm, l, o = np.full((T, 1), -NEG_INF), np.zeros((T, 1), np.float32), np.zeros((T, d), np.float32)
            for j in range(i + 1):
                s = _qk(qT[h][:, i * T:(i + 1) * T], kT[h][:, j * T:(j + 1) * T], stats)
                nm, l, o = _flash_update_balanced(s, v[h][j * T:(j + 1) * T], scale, nm, l, o, j == i, i * T,
                                                  j * T, dtype)
            out[h, i * T:(i + 1) * T] = _flash_finish(o, l, dtype)
    return out


def flash_attention_pipelined(qT, kT, v, scale: float, ILP: int = 2, dtype: str = F32,
                              stats: dict | None = None) -> np.ndarray:
    """attention.py:280-325: ILP query tiles advanced step by step in program order."""
    H, d, S = _check(qT, kT, v)
    nt = S // T
    out = np.zeros((H, S, d), np.float32)
    for h in range(H):
        for g0 in range(0, nt, ILP):
            tiles = list(range(g0, min(g0 + ILP, nt)))
            state = {i: [np.full((T, 1), -NEG_INF), np.zeros((T, 1), np.float32), np.zeros((T, d), np.float32)]
                     for i in tiles}
            for j in range(tiles[-1] + 1):
                for i in tiles:
                    if j > i:
                        continue
                    s = _qk(qT[h][:, i * T:(i + 1) * T], kT[h][:, j * T:(j + 1) * T], stats)
                    state[i] = list(_flash_update_balanced(s, v[h][j * T:(j + 1) * T], scale, *state[i],
                                                           j == i, i * T, j * T, dtype))
            for i in tiles:
                _, l, o = state[i]
                out[h, i * T:(i + 1) * T] = _flash_finish(o, l, dtype)
    return out


def attention_naive(qT, kT, v, scale: float, dtype: str = F32, stats: dict | None = None) -> np.ndarray:
    """attention.py:35-89: scaled, masked fp32 scores for all nt x nt tiles; a row
    softmax writes P in the input dtype; O = P V accumulated over key tiles."""
    H, d, S = _check(qT, kT, v)
    nt = S // T
    out = np.zeros((H, S, d), np.float32)
    for h in range(H):
        scores = np.zeros((S, S), np.float32)
        for i in range(nt):
            for j in range(nt):
                s = _qk(qT[h][:, i * T:(i + 1) * T], kT[h][:, j * T:(j + 1) * T], stats) * np.float32(scale)
                scores[i * T:(i + 1) * T, j * T:(j + 1) * T] = _mask_tile(s, i * T, j * T)
        nmax = -scores.max(axis=1, keepdims=True)
        e = np.exp(scores + nmax)
        rinv = np.float32(1.0) / e.sum(axis=1, keepdims=True, dtype=np.float32)
        probs = cast(e * rinv, dtype)
        for i in range(nt):
            acc = np.zeros((T, d), np.float32)
            for j in range(nt):
                acc += probs[i * T:(i + 1) * T, j * T:(j + 1) * T] @ v[h][j * T:(j + 1) * T]
            out[h, i * T:(i + 1) * T] = cast(acc, dtype)
    return out


ATTENTION_VARIANTS = {
    "naive": attention_naive,
    "flash": flash_attention,
    "flash_kv_resident": flash_attention_kv_resident,
    "flash_balanced": flash_attention_balanced,
    "flash_pipelined": flash_attention_pipelined,
}


def ops_attention(q, k, v, variant: str = "flash_pipelined", dtype: str = F32,
                  stats: dict | None = None) -> np.ndarray:
    """ops.py:77-91: pad S to a multiple of 128 at the end, qT/kT = [H, d, S],
    scale = 1/sqrt(d), run, crop.  k and v with Hkv < H heads (grouped-query
    attention, which the reference lacks) serve query heads h with K/V head
    h // (H / Hkv): they are repeated to H heads first."""
    fn = ATTENTION_VARIANTS[variant]
    q, k, v = (np.asarray(t, np.float32) for t in (q, k, v))
    H, S, d = q.shape
    if k.shape[0] != H:
        k, v = (np.repeat(t, H // t.shape[0], axis=0) for t in (k, v))
    Sp = math.ceil(S / T) * T
    if Sp != S:
        pad = ((0, 0), (0, Sp - S), (0, 0))
        q, k, v = (np.pad(t, pad) for t in (q, k, v))
    qT = np.ascontiguousarray(q.transpose(0, 2, 1))
    kT = np.ascontiguousarray(k.transpose(0, 2, 1))
    o = fn(qT, kT, np.ascontiguousarray(v), 1.0 / math.sqrt(d), dtype=dtype, stats=stats)
    return o[:, :S, :]


# ------------------------------------------------------------------ RoPE --

def rope(x, pos0: int = 0, base: float = 10000.0, dtype: str = F32) -> np.ndarray:
    """Rotary position embedding, rotate-half layout: RoFormer (Su et al., 2021)
    as GPT-NeoX and Llama apply it.  Not in the reference (README.md:89 lists it
    as not done).  x [H, S, d], d even: elements i < d/2 and i + d/2 of row s
    rotate by (pos0 + s) * base^(-2 i / d), computed in float64; one rounding."""
    x = np.asarray(x, np.float32)
    H, S, d = x.shape
    half = d // 2
    inv = base ** (-2.0 * np.arange(half, dtype=np.float64) / d)
    a = (pos0 + np.arange(S, dtype=np.float64))[:, None] * inv[None, :]
    c, s = np.cos(a), np.sin(a)
    x1, x2 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    y = np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)
    return cast(y.astype(np.float32), dtype)


# -------------------------------------------------------------- decoder --

def nki_forward_ref(params: dict, x, n_heads: int, eps: float = 1e-6, attention_variant: str = "flash_pipelined",
                    dtype: str = F32, n_kv_heads: int | None = None, rope_base: float | None = None) -> np.ndarray:
    """model.py:70-89 on the oracle kernels.  params: numpy arrays 'wqkv', 'wo', 'wg',
    'wu', 'wd' in nn.Linear layout [out, in], and 'norm1', 'norm2' [d].  Options the
    reference lacks: n_kv_heads < n_heads (grouped-query attention; wqkv then
    projects to d + 2 n_kv_heads head_dim) and rope_base (RoPE on q and k)."""
    x = np.asarray(x, np.float32)
    S, d = x.shape
    hd = d // n_heads
    hkv = n_kv_heads or n_heads
    kvd = hkv * hd
    w = lambda name: cast(np.asarray(params[name], np.float32).T.copy(), dtype)  # noqa: E731  [in, out]
    g = lambda name: cast(params[name], dtype)  # noqa: E731
    h = rmsnorm_fused(x, g("norm1"), eps, dtype)
    qkv = ops_matmul(h, w("wqkv"), dtype=dtype)
    q = qkv[:, :d].reshape(S, n_heads, hd).transpose(1, 0, 2)
    k = qkv[:, d:d + kvd].reshape(S, hkv, hd).transpose(1, 0, 2)
    v = qkv[:, d + kvd:d + 2 * kvd].reshape(S, hkv, hd).transpose(1, 0, 2)
    if rope_base is not None:
        q, k = rope(q, 0, rope_base, dtype), rope(k, 0, rope_base, dtype)
    a = ops_attention(q, k, v, attention_variant, dtype)
    x = cast(x + ops_matmul(a.transpose(1, 0, 2).reshape(S, d), w("wo"), dtype=dtype), dtype)
    h = rmsnorm_fused(x, g("norm2"), eps, dtype)
    act = swiglu_fused(ops_matmul(h, w("wg"), dtype=dtype), ops_matmul(h, w("wu"), dtype=dtype), dtype)
    return cast(x + ops_matmul(act, w("wd"), dtype=dtype), dtype)
