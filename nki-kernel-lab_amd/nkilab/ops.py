"""Host-side wrappers: layout, padding and tile choice around the HIP kernels.

Drop-in for the reference's nkilab/ops.py: same names, signatures, argument
meaning, output dtype (= input dtype) and errors.  Every op takes NumPy arrays
(float32, or ml_dtypes.bfloat16 when installed) or torch tensors.  NumPy in
gives NumPy out, synchronously, as in the reference; torch GPU tensors stay on
the GPU and the call is asynchronous on torch's current HIP stream.

Where the reference calls ``nki.simulate(kernel)(...)`` (ops.py:48-90), these
wrappers call the C ABI of libnkilab_hip.so (include/nkilab_hip.h).  There is
no CPU fallback: without the library or a GPU the ops raise.

The ``*_into`` functions are the GPU-tensor layer underneath: they write into
a caller-provided output, accept strided views and never copy weights, and are
what nkilab.model uses.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._tensors import dtype_code, from_device, ptr, stream_handle, to_device, workspace

# Reference tile sizes (nkilab/kernels/matmul.py:19-21, attention.py:24).  They
# define choose_blocks' grid and _pad_to's semantics; the HIP kernels handle
# ragged shapes themselves and never need host padding.
TK, TM, TN = 128, 128, 512
T = 128


def _pad_to(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Zero-pad a 2-D array at the end of both axes (ops.py:19-24)."""
    if x.shape == (rows, cols):
        return np.ascontiguousarray(x)
    out = np.zeros((rows, cols), dtype=x.dtype)
    out[: x.shape[0], : x.shape[1]] = x
    return out


def choose_blocks(m_tiles: int, n_tiles: int) -> tuple[int, int]:
    """Largest BM x BN accumulator block with BM*BN <= 8 that divides the tile grid;
    among equal-size blocks the one with the larger BN (ops.py:27-35)."""
    cands = [(bm, bn) for bm in (1, 2, 4) for bn in (1, 2, 4, 8)
             if bm * bn <= 8 and m_tiles % bm == 0 and n_tiles % bn == 0]
    return max(cands, key=lambda c: (c[0] * c[1], c[1]))


# ------------------------------------------------------------------ GEMM --

_MATMUL_VARIANTS = {"blocked": _lib.GEMM_BLOCKED, "naive": _lib.GEMM_NAIVE}


def _row_major(t: torch.Tensor, cols: int) -> tuple[torch.Tensor, int]:
    """(tensor, leading dim) with unit column stride."""
    if t.dim() == 2 and (t.stride(1) == 1 or t.shape[1] == 1) and t.stride(0) >= cols and t.shape[0] > 0:
        return t, t.stride(0)
    t = t.contiguous()
    return t, max(cols, 1)


def _gemm(a: torch.Tensor, bmat: torch.Tensor, ldb: int, b_trans: bool, c: torch.Tensor,
          residual: torch.Tensor | None, variant: str) -> torch.Tensor:
    # The C ABI takes bare pointers and sizes: every shape is checked here, so
    # that a mismatch raises instead of reading or writing past a buffer.
    if a.dim() != 2 or bmat.dim() != 2 or c.dim() != 2:
        raise ValueError(f"gemm: 2-D operands expected, got {tuple(a.shape)}, {tuple(bmat.shape)}, {tuple(c.shape)}")
    M, K = a.shape
    N = c.shape[1]
    if c.shape[0] != M:
        raise ValueError(f"gemm: output {tuple(c.shape)} does not have the {M} rows of a {tuple(a.shape)}")
    want_b = (N, K) if b_trans else (K, N)
    if tuple(bmat.shape) != want_b:
        raise ValueError(f"gemm: b {tuple(bmat.shape)} does not match [{'N, K' if b_trans else 'K, N'}] = {want_b}")
    if residual is not None and tuple(residual.shape) != (M, N):
        raise ValueError(f"gemm: residual {tuple(residual.shape)} does not match the output [{M}, {N}]")
    if a.dtype != bmat.dtype:
        raise TypeError(f"gemm: a and b must share a dtype, got {a.dtype} and {bmat.dtype}")
    a, lda = _row_major(a, K)
    if c.dim() != 2 or (c.stride(1) != 1 and N > 1) or (M > 1 and c.stride(0) < N):
        raise ValueError("gemm: the output must be a row-major [M, N] tensor")
    ldc = c.stride(0) if M > 1 else max(N, 1)
    ldr = 0
    if residual is not None:
        residual, ldr = _row_major(residual, N)
    if M == 0 or N == 0:
        return c
    if K == 0:
        c.copy_(residual if residual is not None else torch.zeros_like(c))
        return c
    _lib.call("nkl_gemm", ptr(a), ptr(bmat), ptr(c), ptr(residual), M, N, K, lda, ldb, ldc, ldr,
              int(b_trans), 1, 0, 0, 0, 0, dtype_code(a.dtype), dtype_code(c.dtype),
              _MATMUL_VARIANTS[variant], stream_handle())
    return c


def gemm_into(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, residual: torch.Tensor | None = None,
              variant: str = "blocked") -> torch.Tensor:
    """c = a @ b (+ residual) on the GPU; a: [M, K], b: [K, N], c: [M, N].
    A b stored column-major (e.g. ``w.t()`` of a row-major [N, K] weight) is
    read in place by the B^T kernel; no transpose copy is made."""
    K, N = b.shape
    if N > 1 and K > 1 and b.stride(0) == 1 and b.stride(1) >= K:
        return _gemm(a, b.t(), b.stride(1), True, c, residual, variant)
    bm, ldb = _row_major(b, N)
    return _gemm(a, bm, ldb, False, c, residual, variant)


def linear_into(a: torch.Tensor, w: torch.Tensor, c: torch.Tensor, residual: torch.Tensor | None = None,
                variant: str = "blocked") -> torch.Tensor:
    """c = a @ w^T (+ residual) for an nn.Linear-layout weight w: [N, K]."""
    K = a.shape[1]
    wm, ldw = _row_major(w, K)
    return _gemm(a, wm, ldw, True, c, residual, variant)


GATE_UP_GROUP = 32  # rows of Wg, then of Wu, per group of the packed gate/up weight


def pack_gate_up(wg: torch.Tensor, wu: torch.Tensor) -> torch.Tensor:
    """The [2N, K] weight ``gemm_swiglu_into`` takes: the rows of Wg and Wu
    ([N, K] each, nn.Linear layout) interleaved in groups of 32."""
    if wg.shape != wu.shape or wg.dim() != 2:
        raise ValueError(f"pack_gate_up: Wg {tuple(wg.shape)} and Wu {tuple(wu.shape)} must be equal 2-D shapes")
    N, K = wg.shape
    if N % GATE_UP_GROUP:
        raise ValueError(f"pack_gate_up: N={N} must be a multiple of {GATE_UP_GROUP}")
    g = wg.reshape(N // GATE_UP_GROUP, GATE_UP_GROUP, K)
    u = wu.reshape(N // GATE_UP_GROUP, GATE_UP_GROUP, K)
    return torch.stack((g, u), dim=1).reshape(2 * N, K).contiguous()


def gemm_swiglu_into(a: torch.Tensor, w_gu: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """c = silu(a @ Wg^T) * (a @ Wu^T) in one GEMM (model.py:88's gate, up and
    SwiGLU), for bf16 (or fp16) a [M, K], the packed weight w_gu =
    pack_gate_up(Wg, Wu) [2N, K] and c [M, N], all of one dtype.  Equal to two
    linear_into calls in that dtype and a SwiGLU in that dtype."""
    M, K = a.shape
    N = c.shape[1]
    if c.shape[0] != M:
        raise ValueError(f"gemm_swiglu_into: output {tuple(c.shape)} does not have the {M} rows of a")
    if w_gu.shape != (2 * N, K):
        raise ValueError(f"gemm_swiglu_into: packed weight {tuple(w_gu.shape)} does not match [2*{N}, {K}]")
    if not (a.dtype == w_gu.dtype == c.dtype) or a.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("gemm_swiglu_into: bf16 or fp16 operands, all of one dtype")
    a, lda = _row_major(a, K)
    wm, ldw = _row_major(w_gu, K)
    if c.dim() != 2 or (c.stride(1) != 1 and N > 1) or (M > 1 and c.stride(0) < N):
        raise ValueError("gemm_swiglu_into: the output must be a row-major [M, N] tensor")
    ldc = c.stride(0) if M > 1 else max(N, 1)
    _lib.call("nkl_gemm_swiglu", ptr(a), ptr(wm), ptr(c), M, N, K, lda, ldw, ldc, dtype_code(a.dtype),
              stream_handle())
    return c


def matmul(a, b, variant: str = "blocked"):
    """C = A @ B for any shapes (ops.py:38-52).  bf16 inputs accumulate in fp32 and
    C is rounded once; the output dtype is the input dtype."""
    M, K = a.shape
    K2, N = b.shape
    assert K == K2, (a.shape, b.shape)
    if variant not in _MATMUL_VARIANTS:
        raise ValueError(f"unknown matmul variant {variant!r}; expected one of {sorted(_MATMUL_VARIANTS)}")
    ta, kind = to_device(a)
    tb, _ = to_device(b)
    if ta.dtype != tb.dtype:
        raise TypeError(f"matmul operands must share a dtype, got {ta.dtype} and {tb.dtype}")
    c = torch.empty((M, N), dtype=ta.dtype, device=ta.device)
    gemm_into(ta, tb, c, variant=variant)
    return from_device(c, kind)


def split_bf16_into(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """y[:, :K] = bf16(x), y[:, K:] = bf16(x - y[:, :K]) for an fp32 x [M, K] and a
    bf16 y [M, 2K]: the hi/lo pair a bf16 GEMM against ``stack_k(w)``
    multiplies with fp32 accuracy."""
    if x.dim() != 2 or y.dim() != 2 or y.shape != (x.shape[0], 2 * x.shape[1]):
        raise ValueError(f"split_bf16_into: y {tuple(y.shape)} must be [M, 2K] for x {tuple(x.shape)}")
    if x.dtype != torch.float32 or y.dtype != torch.bfloat16:
        raise TypeError("split_bf16_into: fp32 x and bf16 y expected")
    M, K = x.shape
    x2, _, _, ldx = _as_rows(x)
    if y.stride(1) != 1:
        raise ValueError("split_bf16_into: y must have unit column stride")
    _lib.call("nkl_split_bf16", ptr(x2), ptr(y), M, K, ldx, y.stride(0) if M > 1 else 2 * K, stream_handle())
    return y


def stack_k(w: torch.Tensor) -> torch.Tensor:
    """[w | w] along K for an nn.Linear weight w [N, K] (bf16): the B operand
    that pairs with split_bf16_into's [hi | lo] activations."""
    return torch.cat((w, w), dim=1).contiguous()


# ---------------------------------------------------------------- RoPE --

def rope_into(x: torch.Tensor, y: torch.Tensor, base: float = 10000.0, pos0: int = 0) -> torch.Tensor:
    """Rotary position embedding (rotate-half layout) of x [H, S, d] into y
    (which may be x): elements i and i + d/2 of row s rotate by
    (pos0 + s) * base^(-2 i / d).  Any strides along H and S; d contiguous."""
    if x.dim() != 3 or y.shape != x.shape or x.dtype != y.dtype:
        raise ValueError(f"rope_into: x {tuple(x.shape)} and y {tuple(y.shape)} must be equal [H, S, d] tensors")
    H, S, d = x.shape
    for t in (x, y):
        if t.stride(2) != 1 and d > 1:
            raise ValueError("rope_into: the head dim must be contiguous")
    _lib.call("nkl_rope", ptr(x), ptr(y), H, S, d, x.stride(0), x.stride(1), y.stride(0), y.stride(1), int(pos0),
              float(base), dtype_code(x.dtype), stream_handle())
    return y


def rope(x, base: float = 10000.0, pos0: int = 0):
    """RoPE of x [H, S, d] (NumPy or torch); returns a new array of x's kind."""
    tx, kind = to_device(x)
    y = torch.empty_like(tx)
    return from_device(rope_into(tx, y, base, pos0), kind)


# ------------------------------------------------------------- row ops --

def _as_rows(t: torch.Tensor) -> tuple[torch.Tensor, int, int, int]:
    """View t as [rows, cols] with unit column stride: (t2d, rows, cols, ld)."""
    cols = t.shape[-1] if t.dim() > 0 else 1
    t2 = t.reshape(-1, cols) if t.dim() != 2 else t
    if t2.dim() != 2 or (t2.stride(1) != 1 and cols > 1) or t2.stride(0) < cols:
        t2 = t2.contiguous()
    ld = t2.stride(0) if t2.shape[0] > 1 else max(cols, 1)
    return t2, t2.shape[0], cols, max(ld, cols)


def softmax_into(x: torch.Tensor, y: torch.Tensor, fused: bool = True) -> torch.Tensor:
    if y.shape != x.shape or y.dtype != x.dtype:
        raise ValueError(f"softmax_into: y {tuple(y.shape)} {y.dtype} must match x {tuple(x.shape)} {x.dtype}")
    x2, R, D, ldx = _as_rows(x)
    y2, _, _, ldy = _as_rows(y)
    dt = dtype_code(x2.dtype)
    if fused:
        _lib.call("nkl_softmax", ptr(x2), ptr(y2), R, D, ldx, ldy, dt, stream_handle())
    else:
        nbytes = _lib.lib().nkl_softmax_unfused_workspace_bytes(R, D)
        ws = workspace(nbytes, x2.device)
        _lib.call("nkl_softmax_unfused", ptr(x2), ptr(y2), ptr(ws), nbytes, R, D, ldx, ldy, dt, stream_handle())
    if y2.data_ptr() != y.data_ptr():
        y.copy_(y2.view_as(y))
    return y


def softmax(x, fused: bool = True):
    """Row softmax over the last dim (ops.py:55-57).  fused=True: one HBM pass
    (norm.py:65); fused=False: three passes through HBM (norm.py:22)."""
    t, kind = to_device(x)
    y = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    return from_device(softmax_into(t, y, fused=fused), kind)


def rmsnorm_into(x: torch.Tensor, weight: torch.Tensor, y: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * weight.  The normalised row stays in
    fp32 and is multiplied by the weight in the weight's own dtype (fp32 or
    bf16, independent of x's), then rounded once to y's dtype (x's, or bf16
    for an fp32 x)."""
    if y.shape != x.shape:
        raise ValueError(f"rmsnorm_into: y {tuple(y.shape)} must match x {tuple(x.shape)}")
    x2, R, D, ldx = _as_rows(x)
    if weight.numel() != D:
        raise ValueError(f"rmsnorm_into: weight has {weight.numel()} elements, x rows have {D}")
    if y.stride(-1) != 1 or not y.is_contiguous():
        raise ValueError("rmsnorm_into: output must be contiguous")
    y2 = y.view(R, D)
    w = weight.contiguous()
    _lib.call("nkl_rmsnorm_ex", ptr(x2), ptr(w), ptr(y2), R, D, ldx, D, float(eps), dtype_code(x2.dtype),
              dtype_code(w.dtype), dtype_code(y2.dtype), stream_handle())
    return y


def rmsnorm(x, weight, eps: float = 1e-6):
    """y = x * rsqrt(mean(x^2, -1) + eps) * weight (ops.py:60-61)."""
    t, kind = to_device(x)
    w, _ = to_device(weight)
    y = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    return from_device(rmsnorm_into(t, w, y, eps), kind)


def swiglu_into(gate: torch.Tensor, up: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    if up.shape != gate.shape or y.shape != gate.shape:
        raise ValueError(f"swiglu_into: gate {tuple(gate.shape)}, up {tuple(up.shape)} and y {tuple(y.shape)} "
                         "must have one shape")
    if not (gate.dtype == up.dtype == y.dtype):
        raise TypeError(f"swiglu_into: gate, up and y must share a dtype, got {gate.dtype}, {up.dtype}, {y.dtype}")
    g, u = gate.contiguous(), up.contiguous()
    if not y.is_contiguous():
        raise ValueError("swiglu_into: output must be contiguous")
    _lib.call("nkl_swiglu", ptr(g), ptr(u), ptr(y), g.numel(), dtype_code(g.dtype), stream_handle())
    return y


def swiglu(gate, up):
    """y = silu(gate) * up (ops.py:64-65)."""
    g, kind = to_device(gate)
    u, _ = to_device(up)
    if g.shape != u.shape:
        raise ValueError(f"swiglu: gate {tuple(g.shape)} and up {tuple(u.shape)} differ in shape")
    if g.dtype != u.dtype:
        raise TypeError(f"swiglu: gate and up must share a dtype, got {g.dtype} and {u.dtype}")
    y = torch.empty(g.shape, dtype=g.dtype, device=g.device)
    return from_device(swiglu_into(g, u, y), kind)


# ------------------------------------------------------------ attention --

@dataclass(frozen=True)
class AttentionVariant:
    """One entry of ATTENTION_VARIANTS: which HIP path serves a reference variant."""
    name: str
    path: str          # "flash" (nkl_flash_attn_causal) or "naive" (nkl_attention_naive)
    reference: str     # the reference kernel it stands for


# The reference's four flash kernels differ only in Trainium engine scheduling
# and are numerically the same online-softmax recurrence; on gfx950 one flash
# kernel serves all four (so they agree bitwise).  "naive" keeps the unfused
# three-pass structure with scores and probabilities in HBM.
ATTENTION_VARIANTS = {
    "naive": AttentionVariant("naive", "naive", "attention.py:35 attention_naive"),
    "flash": AttentionVariant("flash", "flash", "attention.py:155 flash_attention"),
    "flash_kv_resident": AttentionVariant("flash_kv_resident", "flash", "attention.py:179 flash_attention_kv_resident"),
    "flash_balanced": AttentionVariant("flash_balanced", "flash", "attention.py:249 flash_attention_balanced"),
    "flash_pipelined": AttentionVariant("flash_pipelined", "flash", "attention.py:280 flash_attention_pipelined"),
}


# Flash-attention scratch, one pair per (device, stream): a partial-state
# workspace (no initialisation needed) and an arrival-counter array zeroed
# once, which the kernel leaves at zero after every call.  Calls on one stream
# run one after another, so they can share both.  Each is grown when a call
# needs more (the counters are then re-zeroed).  Buffers a call has used are
# never freed: a captured HIP graph may still replay launches that point at
# them, so outgrown ones are kept for the life of the process.
_FLASH_SCRATCH: dict = {}
_FLASH_RETIRED: list = []


def _flash_scratch(ws_bytes: int, counter_bytes: int, dev: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
    key = (dev, stream_handle())
    ws, cnt = _FLASH_SCRATCH.get(key, (None, None))
    if ws is None or ws.numel() < ws_bytes:
        if ws is not None:
            _FLASH_RETIRED.append(ws)
        ws = torch.empty(max(ws_bytes, 1 << 20), dtype=torch.uint8, device=dev)
    if cnt is None or cnt.numel() * 4 < counter_bytes:
        if cnt is not None:
            _FLASH_RETIRED.append(cnt)
        cnt = torch.zeros(max(counter_bytes // 4, 4096), dtype=torch.int32, device=dev)
    _FLASH_SCRATCH[key] = (ws, cnt)
    return ws, cnt


# The attention entry points' stride limits (elements): between heads, and
# between rows (32-bit byte offsets within a block of up to 256 rows).
ATTN_MAX_HEAD_STRIDE, ATTN_MAX_ROW_STRIDE = 1 << 24, 1 << 21


def _attn_strides_ok(t: torch.Tensor, E: int) -> bool:
    return (t.stride(2) == 1 and t.data_ptr() % 16 == 0 and t.stride(0) % E == 0 and t.stride(1) % E == 0
            and 0 <= t.stride(0) <= ATTN_MAX_HEAD_STRIDE and 0 <= t.stride(1) <= ATTN_MAX_ROW_STRIDE)


def _attn_operand(t: torch.Tensor, E: int) -> torch.Tensor:
    return t if _attn_strides_ok(t, E) else t.contiguous()


def attention_into(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
                   variant: str = "flash_pipelined", scale: float | None = None) -> torch.Tensor:
    """Causal attention into o; q, o: [H, S, d] and k, v: [Hkv, S, d] GPU tensors
    (Hkv = H, or a divisor of H for grouped-query attention: query head h reads
    K/V head h // (H / Hkv)), any strides along heads and S (d contiguous).
    d must be a multiple of 8 (bf16) / 4 (fp32)."""
    spec = ATTENTION_VARIANTS[variant]
    H, S, d = q.shape
    Hkv = k.shape[0]
    if k.shape != v.shape or k.shape[1:] != q.shape[1:] or Hkv < 1 or H % Hkv:
        raise ValueError(f"attention_into: k, v {tuple(k.shape)}, {tuple(v.shape)} must be [Hkv, S, d] with Hkv "
                         f"dividing the {H} query heads of q {tuple(q.shape)}")
    if o.shape != q.shape or o.dtype != q.dtype or not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"attention_into: o {tuple(o.shape)} {o.dtype} must match q {tuple(q.shape)} {q.dtype}, "
                         "and k, v share q's dtype")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    E = 8 if q.element_size() == 2 else 4
    q, k, v = (_attn_operand(t, E) for t in (q, k, v))
    o_ok = _attn_strides_ok(o, E)
    out = o if o_ok else torch.empty((H, S, d), dtype=o.dtype, device=o.device)
    strides = (q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
               out.stride(0), out.stride(1))
    dt = dtype_code(q.dtype)
    gqa = Hkv != H
    if spec.path == "flash":
        nbytes = _lib.lib().nkl_flash_attn_causal_workspace_bytes(H, S, d, dt)
        if gqa:
            ws = cnt = None
            if nbytes:
                ws, cnt = _flash_scratch(nbytes, _lib.lib().nkl_flash_attn_causal_counter_bytes(H, S, dt), q.device)
            _lib.call("nkl_flash_attn_causal_gqa", ptr(q), ptr(k), ptr(v), ptr(out), ptr(ws),
                      ws.numel() if ws is not None else 0, ptr(cnt), cnt.numel() * 4 if cnt is not None else 0,
                      H, Hkv, S, d, *strides, float(scale), dt, stream_handle())
        elif nbytes:
            ws, cnt = _flash_scratch(nbytes, _lib.lib().nkl_flash_attn_causal_counter_bytes(H, S, dt), q.device)
            _lib.call("nkl_flash_attn_causal_ws", ptr(q), ptr(k), ptr(v), ptr(out), ptr(ws), ws.numel(), ptr(cnt),
                      cnt.numel() * 4, H, S, d, *strides, float(scale), dt, stream_handle())
        else:
            _lib.call("nkl_flash_attn_causal", ptr(q), ptr(k), ptr(v), ptr(out), H, S, d, *strides, float(scale), dt,
                      stream_handle())
    else:
        nbytes = _lib.lib().nkl_attention_naive_workspace_bytes(H, S, dt)
        ws = workspace(nbytes, q.device)
        if gqa:
            _lib.call("nkl_attention_naive_gqa", ptr(q), ptr(k), ptr(v), ptr(out), ptr(ws), nbytes, H, Hkv, S, d,
                      *strides, float(scale), dt, stream_handle())
        else:
            _lib.call("nkl_attention_naive", ptr(q), ptr(k), ptr(v), ptr(out), ptr(ws), nbytes, H, S, d, *strides,
                      float(scale), dt, stream_handle())
    if out is not o:
        o.copy_(out)
    return o


def attention(q, k, v, variant: str = "flash_pipelined", scale: float | None = None):
    """Causal attention. q, k, v: [H, S, d] (ops.py:77-91); scale 1/sqrt(d)
    unless given (the kernel-level entry points of nkilab.kernels.attention
    pass theirs).
    k and v may also have fewer heads Hkv dividing H (grouped-query attention:
    query head h uses K/V head h // (H / Hkv)), which the reference lacks.

    The reference pads S to a multiple of 128 and transposes q and k on the
    host; the HIP kernels take [H, S, d] as is and bound-check ragged S, so
    neither copy is made.  A head dim that is not a multiple of the 16-byte
    vector width is zero-padded here (zeros change no dot product) and cropped.
    """
    spec = ATTENTION_VARIANTS[variant]  # KeyError for unknown names, as in the reference
    tq, kind = to_device(q)
    tk, _ = to_device(k)
    tv, _ = to_device(v)
    if not (tq.dtype == tk.dtype == tv.dtype):
        raise TypeError("attention: q, k and v must share a dtype")
    if (tq.dim() != 3 or tk.shape != tv.shape or tk.dim() != 3 or tk.shape[1:] != tq.shape[1:]
            or tk.shape[0] < 1 or tq.shape[0] % tk.shape[0]):
        raise ValueError(f"attention: q must be [H, S, d] and k, v [Hkv, S, d] with Hkv dividing H, got "
                         f"{tuple(tq.shape)}, {tuple(tk.shape)}, {tuple(tv.shape)}")
    H, S, d = tq.shape
    assert d <= 128, "head dim must be <= 128"
    E = 8 if tq.element_size() == 2 else 4
    dp = -(-d // E) * E
    if dp != d:
        tq, tk, tv = (torch.nn.functional.pad(t, (0, dp - d)) for t in (tq, tk, tv))
    o = torch.empty((H, S, dp), dtype=tq.dtype, device=tq.device)
    attention_into(tq, tk, tv, o, variant=spec.name, scale=1.0 / math.sqrt(d) if scale is None else float(scale))
    if dp != d:
        o = o[:, :, :d].contiguous()
    return from_device(o, kind)
