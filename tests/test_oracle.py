"""Pins the CPU oracle (oracle/nki_ref.py) before anything is checked against it.

Each check is independent of the oracle's own formulas: a library routine
(torch), a closed form evaluated in float64, an invariant, or brute force --
chosen so that a dropped term, a wrong sign or index, a missing mask or a
transposed operand fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

import oracle as O
from conftest import load_golden, rel_err

ATTN_SHAPES = [(1, 128, 64), (2, 512, 64), (2, 200, 32), (1, 384, 128)]


def _sdpa(q, k, v):
    return torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(np.asarray(t, np.float32)) for t in (q, k, v)), is_causal=True).numpy()


# ------------------------------------------------------------- bf16 cast --

def test_bf16_round_matches_torch(rng):
    x = np.concatenate([
        (rng.standard_normal(200_000) * 10.0 ** rng.integers(-40, 38, 200_000)).astype(np.float32),
        # exact ties: bf16 value + half an ulp, both parities of the kept bit
        (np.arange(1, 20001, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, 1e-39, np.nan], np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    out = O.bf16_round(x)
    assert np.array_equal(np.isnan(out), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(out[ok].view(np.uint32), ref[ok].view(np.uint32))


# ---------------------------------------------------------------- matmul --

@pytest.mark.parametrize("variant", ["naive", "blocked"])
@pytest.mark.parametrize("M,K,N", [(128, 128, 512), (256, 384, 1024), (200, 300, 130), (1, 7, 3)])
def test_matmul_fp32_matches_float64(rng, variant, M, K, N):
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_err(O.ops_matmul(a, b, variant), ref) < 1e-5
    if M > 1 and N > 1:  # a transposed operand or a dropped K chunk is far outside 1e-5
        assert rel_err(O.ops_matmul(a, b, variant)[:, ::-1], ref) > 1e-2


def test_matmul_bf16_is_one_rounding_of_the_exact_product(rng):
    a = O.bf16_round(rng.standard_normal((256, 1024)).astype(np.float32))
    b = O.bf16_round(rng.standard_normal((1024, 512)).astype(np.float32))
    exact = a.astype(np.float64) @ b.astype(np.float64)
    out = O.ops_matmul(a, b, dtype=O.BF16)
    assert rel_err(out, exact) < 1e-2
    once = O.bf16_round(exact.astype(np.float32))
    # fp32 accumulation can only move a value across a rounding boundary it sits next to
    assert (out != once).mean() < 1e-3


def test_blocked_rejects_psum_overflow():
    with pytest.raises(AssertionError, match="PSUM"):
        O.matmul_blocked(np.zeros((128, 384), np.float32), np.zeros((128, 1536), np.float32), BM=3, BN=3)


def test_choose_blocks_brute_force():
    for mt in range(1, 9):
        for nt in range(1, 17):
            valid = [(bm, bn) for bm in range(1, 9) for bn in range(1, 9)
                     if bm * bn <= 8 and mt % bm == 0 and nt % bn == 0 and bm in (1, 2, 4) and bn in (1, 2, 4, 8)]
            bm, bn = O.choose_blocks(mt, nt)
            assert (bm, bn) in valid
            assert bm * bn == max(x * y for x, y in valid)
            assert bn == max(y for x, y in valid if x * y == bm * bn)
    assert O.choose_blocks(4, 4) in {(2, 4), (4, 2)}
    assert O.choose_blocks(8, 2) == (4, 2)


@settings(max_examples=12, deadline=None)
@given(M=st.integers(1, 300), K=st.integers(1, 300), N=st.integers(1, 700))
def test_matmul_property_any_shape(M, K, N):
    r = np.random.default_rng(M * 1000003 + K * 1009 + N)
    a = r.uniform(-1, 1, (M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    out = O.ops_matmul(a, b)
    assert out.shape == (M, N)
    np.testing.assert_allclose(out, a.astype(np.float64) @ b, rtol=1e-4, atol=1e-4)


# --------------------------------------------------------------- row ops --

@pytest.mark.parametrize("fn", [O.softmax_fused, O.softmax_unfused])
@pytest.mark.parametrize("R,D", [(128, 64), (1000, 2048), (5, 3)])
def test_softmax_matches_torch(rng, fn, R, D):
    x = (rng.standard_normal((R, D)) * 4).astype(np.float32)
    ref = torch.softmax(torch.from_numpy(x).double(), -1).numpy()
    np.testing.assert_allclose(fn(x), ref, rtol=1e-5, atol=1e-6)


def test_softmax_is_stable_for_large_logits(rng):
    x = (rng.standard_normal((256, 512)) * 1e4).astype(np.float32)
    out = O.softmax_fused(x)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out.sum(-1), 1.0, atol=1e-5)


@settings(max_examples=10, deadline=None)
@given(R=st.integers(1, 400), D=st.integers(1, 1024), s=st.floats(0.1, 50))
def test_softmax_rows_sum_to_one(R, D, s):
    x = (np.random.default_rng(R * 7 + D).standard_normal((R, D)) * s).astype(np.float32)
    out = O.softmax_fused(x)
    np.testing.assert_allclose(out.sum(-1), 1.0, atol=1e-5)
    assert (out >= 0).all()


@pytest.mark.parametrize("R,D", [(128, 256), (300, 1024), (7, 33)])
def test_rmsnorm_matches_closed_form(rng, R, D):
    x = rng.standard_normal((R, D)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert rel_err(O.rmsnorm_fused(x, w), ref) < 1e-5


def test_rmsnorm_bf16(rng):
    x = O.bf16_round(rng.standard_normal((256, 512)).astype(np.float32))
    w = np.ones(512, np.float32)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    assert rel_err(O.rmsnorm_fused(x, w, dtype=O.BF16), ref) < 1e-2


def test_swiglu_matches_torch(rng):
    g = rng.standard_normal((300, 1024)).astype(np.float32)
    u = rng.standard_normal((300, 1024)).astype(np.float32)
    ref = (torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
    assert rel_err(O.swiglu_fused(g, u), ref) < 1e-5
    assert np.isfinite(O.swiglu_fused(np.array([[-1e4, 1e4]], np.float32), np.ones((1, 2), np.float32))).all()


# ------------------------------------------------------------- attention --

@pytest.mark.parametrize("variant", list(O.ATTENTION_VARIANTS))
@pytest.mark.parametrize("H,S,d", ATTN_SHAPES)
def test_attention_matches_torch_sdpa(rng, variant, H, S, d):
    q, k, v = (rng.standard_normal((H, S, d)).astype(np.float32) for _ in range(3))
    out = O.ops_attention(q, k, v, variant)
    assert out.shape == (H, S, d)
    np.testing.assert_allclose(out, _sdpa(q, k, v), atol=2e-5)


def test_attention_oracle_catches_planted_mistakes(rng):
    """The SDPA check separates the right recurrence from near misses."""
    q, k, v = (rng.standard_normal((1, 256, 64)).astype(np.float32) for _ in range(3))
    ref = _sdpa(q, k, v)
    # no causal mask
    nomask = torch.nn.functional.scaled_dot_product_attention(*map(torch.from_numpy, (q, k, v))).numpy()
    assert np.abs(nomask - ref).max() > 1e-2
    # wrong scale
    sc = torch.nn.functional.scaled_dot_product_attention(*map(torch.from_numpy, (q, k, v)), is_causal=True,
                                                          scale=1.0 / 64).numpy()
    assert np.abs(sc - ref).max() > 1e-2
    assert np.abs(O.ops_attention(q, k, v) - ref).max() < 2e-5


@pytest.mark.parametrize("variant", ["naive", "flash_pipelined"])
def test_attention_bf16(rng, variant):
    q, k, v = (O.bf16_round(rng.standard_normal((2, 256, 64)).astype(np.float32)) for _ in range(3))
    assert rel_err(O.ops_attention(q, k, v, variant, O.BF16), _sdpa(q, k, v)) < 3e-2


def test_first_token_attends_only_to_itself(rng):
    q, k, v = (rng.standard_normal((1, 256, 64)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(O.ops_attention(q, k, v)[0, 0], v[0, 0], atol=1e-6)


def test_flash_family_agrees_bitwise(rng):
    q, k, v = (rng.standard_normal((2, 512, 64)).astype(np.float32) for _ in range(3))
    a = O.ops_attention(q, k, v, "flash_balanced")
    b = O.ops_attention(q, k, v, "flash_pipelined")
    assert np.array_equal(a, b)


def test_flash_skips_masked_tiles():
    q = np.zeros((1, 512, 64), np.float32)
    nt = 4
    sn, sf = {}, {}
    O.ops_attention(q, q, q, "naive", stats=sn)
    O.ops_attention(q, q, q, "flash", stats=sf)
    assert sn["qk_tiles"] == nt * nt
    assert sf["qk_tiles"] == nt * (nt + 1) // 2


def test_causal_flop_count():
    assert O.causal_flops(8, 2048, 128) == 8_594_128_896
    # brute force on a small case: 4 d FLOPs per unmasked (query, key) pair
    H, S, d = 2, 37, 16
    pairs = sum(1 for i in range(S) for j in range(S) if j <= i)
    assert O.causal_flops(H, S, d) == 4 * H * d * pairs


# --------------------------------------------------------------- decoder --

@pytest.mark.parametrize("S", [128, 300])
@pytest.mark.parametrize("variant", ["naive", "flash_pipelined"])
def test_decoder_oracle_matches_pytorch_block(S, variant):
    from nkilab.model import BlockConfig, DecoderBlock

    torch.manual_seed(0)
    block = DecoderBlock(BlockConfig()).eval()
    x = torch.randn(S, block.cfg.d_model)
    with torch.no_grad():
        ref = block(x).numpy()
    params = {n: getattr(block, n).weight.detach().numpy() for n in ("wqkv", "wo", "wg", "wu", "wd", "norm1", "norm2")}
    out = O.nki_forward_ref(params, x.numpy(), block.cfg.n_heads, block.cfg.eps, variant)
    np.testing.assert_allclose(out, ref, atol=1e-5)


# -------------------------------------------------------- golden vectors --

def test_oracle_reproduces_committed_golden_vectors():
    """The fixtures in tests/golden were written by tests/golden/make_golden.py;
    the oracle must still produce them bit for bit."""
    import importlib.util
    import os

    here = os.path.join(os.path.dirname(__file__), "golden", "make_golden.py")
    spec = importlib.util.spec_from_file_location("make_golden", here)
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    for name, build in mg.CASES.items():
        fresh = build()
        stored = load_golden(name)
        assert set(fresh) == set(stored), name
        for key in fresh:
            assert np.array_equal(fresh[key], stored[key]), f"{name}:{key}"


def test_exact_scale_is_reciprocal_sqrt():
    assert math.isclose(1.0 / math.sqrt(128), 0.08838834764831845)


# ------------------------------------------------- RoPE and GQA (not in the reference) --

def _torch_rope_rotate_half(x, pos0, base):
    """An independent float64 statement in the form Hugging Face's Llama uses:
    emb = cat(freqs, freqs); x * cos(emb) + rotate_half(x) * sin(emb)."""
    x = torch.from_numpy(np.asarray(x, np.float64))
    S, d = x.shape[-2], x.shape[-1]
    inv = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    freqs = torch.outer(torch.arange(pos0, pos0 + S, dtype=torch.float64), inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    x1, x2 = x[..., :d // 2], x[..., d // 2:]
    rot = torch.cat((-x2, x1), dim=-1)
    return (x * emb.cos() + rot * emb.sin()).numpy()


@pytest.mark.parametrize("H,S,d,pos0,base", [(2, 7, 8, 0, 10000.0), (1, 33, 128, 100, 10000.0),
                                             (3, 5, 64, 4090, 500000.0)])
def test_rope_matches_rotate_half_form(rng, H, S, d, pos0, base):
    x = rng.standard_normal((H, S, d)).astype(np.float32)
    np.testing.assert_allclose(O.rope(x, pos0, base), _torch_rope_rotate_half(x, pos0, base), rtol=1e-5, atol=1e-5)


def test_rope_properties(rng):
    """Identity at position 0; every (i, i + d/2) pair keeps its norm; the dot
    product of a rotated query and key depends only on their distance; and a
    planted sign mistake in the oracle's rotation is caught by the
    rotate-half comparison."""
    d = 64
    x = rng.standard_normal((1, 1, d)).astype(np.float32)
    np.testing.assert_array_equal(O.rope(x, 0), x)
    x2 = rng.standard_normal((2, 50, d)).astype(np.float32)
    r2 = O.rope(x2, 17)
    n_in = x2[..., :d // 2].astype(np.float64) ** 2 + x2[..., d // 2:].astype(np.float64) ** 2
    n_out = r2[..., :d // 2].astype(np.float64) ** 2 + r2[..., d // 2:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5)
    q, k = (rng.standard_normal((1, 1, d)).astype(np.float32) for _ in range(2))
    dots = [float(np.sum(O.rope(q, m).astype(np.float64) * O.rope(k, m - 5))) for m in (5, 40, 300)]
    np.testing.assert_allclose(dots, dots[0], rtol=1e-5)
    # the oracle's rotation with the sine's sign flipped (a plausible slip):
    # still norm-preserving, but the rotate-half comparison rejects it
    half = d // 2
    a = (17 + np.arange(50, dtype=np.float64))[:, None] * 10000.0 ** (-2.0 * np.arange(half) / d)
    c, sn = np.cos(a), np.sin(a)
    lo, hi = x2[..., :half].astype(np.float64), x2[..., half:].astype(np.float64)
    flipped = np.concatenate([lo * c + hi * sn, hi * c - lo * sn], axis=-1)
    ref = _torch_rope_rotate_half(x2, 17, 10000.0)
    assert not np.allclose(flipped, ref, atol=1e-3)
    np.testing.assert_allclose(r2, ref, atol=1e-5)


@pytest.mark.parametrize("H,Hkv", [(4, 2), (4, 1), (6, 3)])
def test_gqa_attention_repeats_kv_heads(rng, H, Hkv):
    S, d = 150, 32
    q = rng.standard_normal((H, S, d)).astype(np.float32)
    k, v = (rng.standard_normal((Hkv, S, d)).astype(np.float32) for _ in range(2))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), *(torch.from_numpy(t).repeat_interleave(H // Hkv, dim=0) for t in (k, v)),
        is_causal=True).numpy()
    for variant in ("naive", "flash_pipelined"):
        np.testing.assert_allclose(O.ops_attention(q, k, v, variant), ref, atol=2e-5)


@pytest.mark.parametrize("n_kv_heads,rope_base", [(2, None), (None, 10000.0), (1, 500000.0)])
def test_decoder_oracle_gqa_rope_matches_pytorch_block(n_kv_heads, rope_base):
    from nkilab.model import BlockConfig, DecoderBlock

    torch.manual_seed(0)
    block = DecoderBlock(BlockConfig(n_kv_heads=n_kv_heads, rope_base=rope_base)).eval()
    assert block.wqkv.weight.shape[0] == 256 + 2 * (n_kv_heads or 4) * 64
    x = torch.randn(130, 256)
    with torch.no_grad():
        ref = block(x).numpy()
    params = {n: getattr(block, n).weight.detach().numpy() for n in ("wqkv", "wo", "wg", "wu", "wd", "norm1", "norm2")}
    out = O.nki_forward_ref(params, x.numpy(), 4, 1e-6, "flash_pipelined", n_kv_heads=n_kv_heads,
                            rope_base=rope_base)
    np.testing.assert_allclose(out, ref, atol=1e-5)


def test_float16_policy_error_budget_on_cpu():
    """The benchmark decoder block (seq 2048, hidden 2048, FFN 5632) with its
    rounding points -- RMSNorm outputs, QKV, P, the attention output, gate/up,
    the SwiGLU output -- emulated on the CPU in fp32: at fp16 (weights too)
    the block stays within 1e-3 of the fp32 block (2.8e-4), at bf16 it does not
    (2.6e-3: each bf16 rounding point alone costs ~1e-3; fp16 keeps 3 more
    significand bits)."""
    import torch

    from nkilab import workloads

    torch.set_num_threads(min(8, torch.get_num_threads()))
    block, x = workloads.decoder_inputs()
    S, d = x.shape
    H = block.cfg.n_heads
    hd = d // H
    with torch.no_grad():
        ref = block(x)
        W = {n: getattr(block, n).weight.detach() for n in ("wqkv", "wo", "wg", "wu", "wd")}
        mask = torch.triu(torch.ones(S, S, dtype=torch.bool), 1)

        def run(dt):
            R = lambda t: t.to(dt).float()  # noqa: E731
            Wd = {n: R(w) for n, w in W.items()}
            h = R(block.norm1(x))
            qkv = R(h @ Wd["wqkv"].T)
            q, k, v = (qkv[:, i * d:(i + 1) * d].reshape(S, H, hd).transpose(0, 1) for i in range(3))
            s = ((q @ k.transpose(1, 2)) / hd ** 0.5).masked_fill(mask, float("-inf"))
            e = torch.exp(s - s.amax(-1, keepdim=True))
            a = R(((R(e) @ v) / e.sum(-1, keepdim=True)).transpose(0, 1).reshape(S, d))
            x1 = x + a @ Wd["wo"].T
            h2 = R(block.norm2(x1))
            g, u = R(h2 @ Wd["wg"].T), R(h2 @ Wd["wu"].T)
            return x1 + R(torch.nn.functional.silu(g) * u) @ Wd["wd"].T

        err = {n: float((run(dt) - ref).abs().max() / ref.abs().max())
               for n, dt in (("fp16", torch.float16), ("bf16", torch.bfloat16))}
    assert err["fp16"] < 5e-4 and err["bf16"] > 1e-3, err
