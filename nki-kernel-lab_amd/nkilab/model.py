"""A Llama-style decoder block run two ways: PyTorch eager and the HIP kernels.

    x = x + Wo . causal_attention(split_heads(RMSNorm(x) . Wqkv))
    x = x + Wd . (silu(RMSNorm(x) . Wg) * (RMSNorm(x) . Wu))

Drop-in for the reference's nkilab/model.py: BlockConfig, RMSNorm and
DecoderBlock keep the reference's fields, attribute names and eager math
(model.py:22-67, no rotary embeddings), because callers reach into them
(``block.norm1.weight``, ``block.wqkv``...).  ``nki_forward`` (model.py:70-89)
runs every heavy op -- 2 RMSNorm, 5 GEMM, 1 attention, 1 SwiGLU -- on the
gfx950 kernels.

Differences from the reference's host glue, none of which changes the math:
  * weights are used in nn.Linear's own [out, in] layout by the B^T GEMM
    instead of being transposed and copied on every call (model.py:76-77);
    device copies are cached per parameter version;
  * the head split and merge are strided views fed to the attention kernel,
    not copies (model.py:84-86);
  * the residual adds run in the out-projection / down-projection GEMM
    epilogues (model.py:86, :89);
  * in bf16 the gate and up projections and the SwiGLU between them
    (model.py:88) are one GEMM over the two weights interleaved in groups of
    32 rows, with SwiGLU in its epilogue (the same values as the three calls);
  * ``BlockConfig(n_kv_heads=..., rope_base=...)`` adds grouped-query
    attention and rotary embeddings, which the reference lacks (README.md:89);
    both default off, giving the reference's block;
  * ``compute_dtype="bfloat16"`` runs the block in bf16 with an fp32 residual
    stream (the GEMMs that feed the residual emit fp32).  The default keeps
    the reference's behaviour: everything in x's dtype.
  * ``compute_dtype="float16"`` runs the same kernels with fp16 activations
    and weights (fp32 x and residual stream): 11 significant bits per
    rounding instead of bf16's 8, which keeps the block within 1e-3 of the
    fp32 block at the bf16 path's cost (the activations must stay inside
    fp16's range, |v| < 65504).
  * ``compute_dtype="split"`` keeps fp32 activations and the fp32 residual
    but runs the projections on bf16 MFMA: every GEMM operand is an fp32
    activation carried as a bf16 hi/lo pair (K doubled) against the bf16
    weight stacked twice along K, which accumulates to fp32 accuracy; the
    attention runs in fp32.  It needs bf16-valued weights (others take the
    fp32 GEMM) and meets the 1e-3 bound against the fp32 block that no bf16
    rounding of an activation does.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from ._tensors import from_device, to_device


@dataclass
class BlockConfig:
    d_model: int = 256
    n_heads: int = 4
    d_ff: int = 1024
    eps: float = 1e-6
    # Options the reference lacks (README.md:89); the defaults keep its block.
    n_kv_heads: int | None = None   # grouped-query attention: K/V heads (dividing n_heads)
    rope_base: float | None = None  # rotary embedding of q and k (rotate-half layout)

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def kv_heads(self) -> int:
        return self.n_kv_heads or self.n_heads


def rope_reference(x: torch.Tensor, base: float, pos0: int = 0) -> torch.Tensor:
    """RoPE of x [..., S, d] in PyTorch (rotate-half layout, fp32 angles): the
    eager block's rotary embedding."""
    S, d = x.shape[-2], x.shape[-1]
    half = d // 2
    inv = base ** (-2.0 * torch.arange(half, dtype=torch.float64, device=x.device) / d)
    a = ((pos0 + torch.arange(S, dtype=torch.float64, device=x.device))[:, None] * inv[None, :]).float()
    c, s = torch.cos(a), torch.sin(a)
    x1, x2 = x[..., :half].float(), x[..., half:].float()
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1).to(x.dtype)


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2, -1) + eps) * weight, weight initialised to ones."""

    def __init__(self, d: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x):
        inv_rms = torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return x * inv_rms * self.weight


class DecoderBlock(nn.Module):
    """Pre-norm decoder block in PyTorch eager: the oracle nki_forward is held to."""

    def __init__(self, cfg: BlockConfig):
        super().__init__()
        self.cfg = cfg
        d, f = cfg.d_model, cfg.d_ff
        self.norm1 = RMSNorm(d, cfg.eps)
        self.norm2 = RMSNorm(d, cfg.eps)
        if cfg.n_heads % cfg.kv_heads:
            raise ValueError(f"BlockConfig: n_kv_heads={cfg.n_kv_heads} must divide n_heads={cfg.n_heads}")
        self.wqkv = nn.Linear(d, d + 2 * cfg.kv_heads * cfg.head_dim, bias=False)
        self.wo = nn.Linear(d, d, bias=False)
        self.wg = nn.Linear(d, f, bias=False)
        self.wu = nn.Linear(d, f, bias=False)
        self.wd = nn.Linear(f, d, bias=False)
        # Norm weights away from 1 so that a dropped weight multiply is visible.
        with torch.no_grad():
            for norm in (self.norm1, self.norm2):
                norm.weight.uniform_(0.5, 1.5)

    def forward(self, x):  # x: [S, d_model]
        S, d = x.shape
        H, hd, Hkv = self.cfg.n_heads, self.cfg.head_dim, self.cfg.kv_heads
        qkv = self.wqkv(self.norm1(x))
        q = qkv[:, :d].reshape(S, H, hd).transpose(0, 1)  # [H, S, hd]
        k, v = (t.reshape(S, Hkv, hd).transpose(0, 1) for t in qkv[:, d:].chunk(2, dim=-1))
        if self.cfg.rope_base is not None:
            q, k = rope_reference(q, self.cfg.rope_base), rope_reference(k, self.cfg.rope_base)
        if Hkv != H:
            k, v = (t.repeat_interleave(H // Hkv, dim=0) for t in (k, v))
        attn = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + self.wo(attn.transpose(0, 1).reshape(S, d))
        h = self.norm2(x)
        return x + self.wd(F.silu(self.wg(h)) * self.wu(h))


_DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16,
           torch.float32: torch.float32, torch.bfloat16: torch.bfloat16, torch.float16: torch.float16}
SPLIT = "split"


def _device_param(block: nn.Module, name: str, p: torch.Tensor, dtype: torch.dtype, dev: torch.device):
    """Device copy of a parameter in `dtype`, cached until the parameter changes."""
    cache = block.__dict__.setdefault("_nkl_param_cache", {})
    key = (name, dtype, dev)
    stamp = (p.data_ptr(), p._version)
    hit = cache.get(key)
    if hit is not None and hit[0] == stamp:
        return hit[1]
    t = p.detach().to(device=dev, dtype=dtype).contiguous()
    cache[key] = (stamp, t)
    return t


def _packed_gate_up(block: DecoderBlock, dev: torch.device, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """pack_gate_up(Wg, Wu) in `dtype` (bf16 or fp16) on dev, rebuilt when
    either weight changes."""
    cache = block.__dict__.setdefault("_nkl_param_cache", {})
    key = ("gate_up", dtype, dev)
    stamp = tuple((p.data_ptr(), p._version) for p in (block.wg.weight, block.wu.weight))
    hit = cache.get(key)
    if hit is not None and hit[0] == stamp:
        return hit[1]
    wg = block.wg.weight.detach().to(device=dev, dtype=dtype)
    wu = block.wu.weight.detach().to(device=dev, dtype=dtype)
    t = ops.pack_gate_up(wg, wu)
    cache[key] = (stamp, t)
    return t


def _stacked_weight(block: nn.Module, name: str, dev: torch.device) -> torch.Tensor | None:
    """ops.stack_k of a weight in bf16 on dev when the weight's values are bf16
    numbers (None otherwise), cached until the parameter changes."""
    cache = block.__dict__.setdefault("_nkl_param_cache", {})
    p = getattr(block, name).weight
    key = (name, SPLIT, dev)
    stamp = (p.data_ptr(), p._version)
    hit = cache.get(key)
    if hit is not None and hit[0] == stamp:
        return hit[1]
    wf = p.detach().to(device=dev, dtype=torch.float32)
    wb = wf.to(torch.bfloat16)
    t = ops.stack_k(wb) if torch.equal(wb.float(), wf) else None
    cache[key] = (stamp, t)
    return t


def _split_forward(block: DecoderBlock, xt: torch.Tensor, attention_variant: str) -> torch.Tensor:
    """The block with fp32 activations and bf16-MFMA projections over hi/lo
    operand pairs (compute_dtype="split")."""
    cfg = block.cfg
    dev = xt.device
    S, d = xt.shape
    H, hd, Hkv = cfg.n_heads, cfg.head_dim, cfg.kv_heads
    kvd = Hkv * hd
    f32, bf = torch.float32, torch.bfloat16

    def linear(a: torch.Tensor, name: str, out: torch.Tensor, residual=None):
        w2 = _stacked_weight(block, name, dev)
        if w2 is None:  # weights that are not bf16 numbers: the fp32 GEMM
            return ops.linear_into(a, _device_param(block, name, getattr(block, name).weight, f32, dev), out, residual)
        a2 = torch.empty((a.shape[0], 2 * a.shape[1]), dtype=bf, device=dev)
        ops.split_bf16_into(a, a2)
        return ops.linear_into(a2, w2, out, residual)

    g1 = _device_param(block, "norm1", block.norm1.weight, f32, dev)
    g2 = _device_param(block, "norm2", block.norm2.weight, f32, dev)
    h = torch.empty((S, d), dtype=f32, device=dev)
    ops.rmsnorm_into(xt, g1, h, cfg.eps)
    qkv = torch.empty((S, d + 2 * kvd), dtype=f32, device=dev)
    linear(h, "wqkv", qkv)
    q = qkv[:, :d].view(S, H, hd).transpose(0, 1)
    k = qkv[:, d:d + kvd].view(S, Hkv, hd).transpose(0, 1)
    v = qkv[:, d + kvd:].view(S, Hkv, hd).transpose(0, 1)
    if cfg.rope_base is not None:
        ops.rope_into(q, q, cfg.rope_base)
        ops.rope_into(k, k, cfg.rope_base)
    a = torch.empty((S, d), dtype=f32, device=dev)
    ops.attention_into(q, k, v, a.view(S, H, hd).transpose(0, 1), variant=attention_variant)
    x1 = torch.empty((S, d), dtype=f32, device=dev)
    linear(a, "wo", x1, residual=xt)
    h2 = torch.empty((S, d), dtype=f32, device=dev)
    ops.rmsnorm_into(x1, g2, h2, cfg.eps)
    gate = torch.empty((S, cfg.d_ff), dtype=f32, device=dev)
    up = torch.empty((S, cfg.d_ff), dtype=f32, device=dev)
    linear(h2, "wg", gate)
    linear(h2, "wu", up)
    act = torch.empty((S, cfg.d_ff), dtype=f32, device=dev)
    ops.swiglu_into(gate, up, act)
    out = torch.empty((S, d), dtype=f32, device=dev)
    linear(act, "wd", out, residual=x1)
    return out


def nki_forward(block: DecoderBlock, x, attention_variant: str = "flash_pipelined", compute_dtype=None):
    """The same block with every heavy op on the HIP kernels (model.py:70-89).

    x: [S, d_model] as NumPy or torch (CPU or GPU); returns the same kind.
    compute_dtype: None (= x's dtype, the reference's behaviour), "bfloat16"
    for bf16 GEMM/attention operands with the residual stream kept in x's
    dtype, "float16" (fp32 x only) for fp16 operands (within 1e-3 of the fp32
    block at bf16 cost), or "split" (fp32 x only) for fp32 activations with
    the projections on bf16 MFMA over hi/lo operand pairs.
    """
    cfg = block.cfg
    xt, kind = to_device(x)
    if compute_dtype == SPLIT:
        if xt.dtype != torch.float32:
            raise ValueError("nki_forward: compute_dtype='split' needs an fp32 x")
        return from_device(_split_forward(block, xt, attention_variant), kind)
    dev = xt.device
    S, d = xt.shape
    H, hd = cfg.n_heads, cfg.head_dim
    rdt = xt.dtype
    cdt = rdt if compute_dtype is None else _DTYPES[compute_dtype]
    if cdt == torch.float32 and rdt == torch.bfloat16:
        raise ValueError("nki_forward: fp32 compute on a bf16 residual stream is not supported")
    if cdt == torch.float16 and rdt != torch.float32:
        raise ValueError("nki_forward: compute_dtype='float16' needs an fp32 x")
    W = {n: _device_param(block, n, getattr(block, n).weight, cdt, dev) for n in ("wqkv", "wo", "wg", "wu", "wd")}
    g1 = _device_param(block, "norm1", block.norm1.weight, rdt, dev)
    g2 = _device_param(block, "norm2", block.norm2.weight, rdt, dev)

    h = torch.empty((S, d), dtype=cdt, device=dev)
    ops.rmsnorm_into(xt, g1, h, cfg.eps)
    Hkv = cfg.kv_heads
    kvd = Hkv * hd
    qkv = torch.empty((S, d + 2 * kvd), dtype=cdt, device=dev)
    ops.linear_into(h, W["wqkv"], qkv)
    q = qkv[:, :d].view(S, H, hd).transpose(0, 1)
    k = qkv[:, d:d + kvd].view(S, Hkv, hd).transpose(0, 1)
    v = qkv[:, d + kvd:].view(S, Hkv, hd).transpose(0, 1)
    if cfg.rope_base is not None:  # in place on the q and k columns of qkv
        ops.rope_into(q, q, cfg.rope_base)
        ops.rope_into(k, k, cfg.rope_base)
    a = torch.empty((S, d), dtype=cdt, device=dev)
    ops.attention_into(q, k, v, a.view(S, H, hd).transpose(0, 1), variant=attention_variant)
    x1 = torch.empty((S, d), dtype=rdt, device=dev)
    ops.linear_into(a, W["wo"], x1, residual=xt)
    h2 = torch.empty((S, d), dtype=cdt, device=dev)
    ops.rmsnorm_into(x1, g2, h2, cfg.eps)
    act = torch.empty((S, cfg.d_ff), dtype=cdt, device=dev)
    if cdt in (torch.bfloat16, torch.float16) and cfg.d_ff % ops.GATE_UP_GROUP == 0 and d % 8 == 0:
        # gate, up and SwiGLU in one GEMM over the packed weight (same values)
        ops.gemm_swiglu_into(h2, _packed_gate_up(block, dev, cdt), act)
    else:
        gate = torch.empty((S, cfg.d_ff), dtype=cdt, device=dev)
        up = torch.empty((S, cfg.d_ff), dtype=cdt, device=dev)
        ops.linear_into(h2, W["wg"], gate)
        ops.linear_into(h2, W["wu"], up)
        ops.swiglu_into(gate, up, act)
    out = torch.empty((S, d), dtype=rdt, device=dev)
    ops.linear_into(act, W["wd"], out, residual=x1)
    return from_device(out, kind)
