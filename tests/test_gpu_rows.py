"""Row kernels on the GPU (softmax, RMSNorm, SwiGLU) against the oracle, torch and
the golden fixtures.  Tolerances follow the reference's tests
(tests/test_norm.py) for fp32; bf16 results must sit within one bf16 ulp of the
oracle's correctly rounded value."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import assert_within_bf16_ulps, load_golden, rel_err

pytestmark = pytest.mark.gpu


def _bf(t):
    return torch.from_numpy(np.asarray(t, np.float32)).to(torch.bfloat16).cuda()


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("R,D", [(128, 64), (1000, 2048), (5, 3), (3, 5000), (2, 20000)])
def test_softmax_matches_torch(rng, fused, R, D):
    from nkilab import ops

    x = (rng.standard_normal((R, D)) * 4).astype(np.float32)
    out = ops.softmax(x, fused=fused)
    assert out.dtype == np.float32 and out.shape == (R, D)
    ref = torch.softmax(torch.from_numpy(x), -1).numpy()
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, O.softmax_fused(x) if fused else O.softmax_unfused(x), rtol=1e-5, atol=1e-6)


def test_softmax_is_stable_for_large_logits(rng):
    from nkilab import ops

    x = (rng.standard_normal((256, 512)) * 1e4).astype(np.float32)
    out = ops.softmax(x)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out.sum(-1), 1.0, atol=1e-5)


@pytest.mark.parametrize("R,D,s", [(1, 1, 1.0), (400, 1023, 50.0), (37, 129, 0.1), (64, 777, 3.0)])
def test_softmax_rows_sum_to_one(R, D, s):
    from nkilab import ops

    x = (np.random.default_rng(R * 7 + D).standard_normal((R, D)) * s).astype(np.float32)
    out = ops.softmax(x)
    np.testing.assert_allclose(out.sum(-1), 1.0, atol=1e-5)
    assert (out >= 0).all()


@pytest.mark.parametrize("R,D", [(128, 256), (300, 1024), (7, 33)])
def test_rmsnorm_matches_torch(rng, R, D):
    from nkilab import ops

    x = rng.standard_normal((R, D)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    xt = torch.from_numpy(x)
    ref = (xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-6) * torch.from_numpy(w)).numpy()
    assert rel_err(ops.rmsnorm(x, w), ref) < 1e-5


def test_rmsnorm_bf16(rng):
    from nkilab import ops

    x = _bf(rng.standard_normal((256, 512)))
    w = torch.ones(512, dtype=torch.bfloat16, device="cuda")
    xf = _np(x).astype(np.float64)
    ref = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6)
    out = ops.rmsnorm(x, w)
    assert out.dtype == torch.bfloat16 and out.is_cuda
    assert rel_err(_np(out), ref) < 1e-2


@pytest.mark.parametrize("R,D", [(64, 2048), (33, 520), (5, 77)])
def test_rmsnorm_bf16_activations_fp32_weight(rng, R, D):
    """bf16 x with an fp32 weight: the fp32 normalised row is multiplied by the
    fp32 weight and rounded once (norm.py:116), as the oracle does -- not by a
    weight first rounded to bf16."""
    from nkilab import ops

    x = _bf(rng.standard_normal((R, D)))
    w = torch.from_numpy(rng.uniform(0.5, 1.5, D).astype(np.float32)).cuda()
    out = ops.rmsnorm(x, w)
    assert out.dtype == torch.bfloat16
    ref = O.rmsnorm_fused(_np(x), w.cpu().numpy(), 1e-6, O.BF16)
    assert_within_bf16_ulps(_np(out), ref, 1.0, 1e-6)
    # rounding the weight to bf16 first gives a different result on some elements
    coarse = O.rmsnorm_fused(_np(x), O.bf16_round(w.cpu().numpy()), 1e-6, O.BF16)
    assert np.abs(ref - coarse).max() > 0


def test_swiglu_matches_torch(rng):
    from nkilab import ops

    g = rng.standard_normal((300, 1024)).astype(np.float32)
    u = rng.standard_normal((300, 1024)).astype(np.float32)
    ref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    assert rel_err(ops.swiglu(g, u), ref) < 1e-5
    odd = rng.standard_normal(1001).astype(np.float32)  # not a multiple of the vector width
    np.testing.assert_allclose(ops.swiglu(odd, odd), O.swiglu_fused(odd, odd), rtol=1e-5, atol=1e-6)


def test_row_kernels_match_golden_vectors():
    from nkilab import ops

    gd = load_golden("rows")
    for tag, dt in (("f32", O.F32), ("f32b", O.F32), ("bf16", O.BF16), ("bf16r", O.BF16)):
        to = (lambda a: torch.from_numpy(a).cuda()) if dt == O.F32 else _bf
        x, w, g, u = (to(gd[f"{tag}_{k}"]) for k in ("x", "w", "g", "u"))
        got = {"softmax": ops.softmax(x), "softmax_unfused": ops.softmax(x, fused=False),
               "rmsnorm": ops.rmsnorm(x, w), "swiglu": ops.swiglu(g, u)}
        for k, v in got.items():
            ref = gd[f"{tag}_{k}"]
            if dt == O.F32:
                np.testing.assert_allclose(_np(v), ref, rtol=2e-5, atol=1e-6, err_msg=f"{tag}_{k}")
            else:
                assert_within_bf16_ulps(_np(v), ref, 1.0, 1e-6)


# --------------------------------------------- the 4096 x 2048 bf16 config --

@pytest.fixture(scope="module")
def rows_config():
    from nkilab import workloads

    x, w, gate, up = workloads.rows_inputs()
    return tuple(t.cuda() for t in (x, w, gate, up))


def test_softmax_config(rows_config):
    from nkilab import ops

    x = rows_config[0]
    out = _np(ops.softmax(x))
    xf = _np(x)
    assert np.abs(out - torch.softmax(torch.from_numpy(xf), -1).numpy()).max() <= 1e-2
    assert_within_bf16_ulps(out, O.softmax_fused(xf, O.BF16), 1.0, 1e-7)
    np.testing.assert_allclose(out.astype(np.float64).sum(-1), 1.0, atol=1e-2)


def test_rmsnorm_config(rows_config):
    from nkilab import ops

    x, w = rows_config[0], rows_config[1]
    out = _np(ops.rmsnorm(x, w, 1e-6))
    xf, wf = _np(x).astype(np.float64), _np(w).astype(np.float64)
    exact = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-6) * wf
    assert rel_err(out, exact) < 1e-2
    assert_within_bf16_ulps(out, O.rmsnorm_fused(_np(x), _np(w), 1e-6, O.BF16), 1.0, 1e-6)


def test_swiglu_config(rows_config):
    from nkilab import ops

    g, u = rows_config[2], rows_config[3]
    out = _np(ops.swiglu(g, u))
    gf, uf = _np(g).astype(np.float64), _np(u).astype(np.float64)
    assert rel_err(out, gf / (1 + np.exp(-gf)) * uf) < 1e-2
    assert_within_bf16_ulps(out, O.swiglu_fused(_np(g), _np(u), O.BF16), 1.0, 1e-6)


def test_rmsnorm_fp32_input_to_bf16_output(rng):
    """The decoder's mixed path: an fp32 residual stream normalised into bf16."""
    from nkilab import ops

    x = torch.from_numpy(rng.standard_normal((64, 2048)).astype(np.float32)).cuda()
    w = torch.from_numpy(rng.uniform(0.5, 1.5, 2048).astype(np.float32)).cuda()
    y = torch.empty((64, 2048), dtype=torch.bfloat16, device="cuda")
    ops.rmsnorm_into(x, w, y, 1e-6)
    assert_within_bf16_ulps(_np(y), O.rmsnorm_fused(_np(x), _np(w), 1e-6, O.BF16), 1.0, 1e-6)


def test_strided_rows_and_async_tensors(rng):
    from nkilab import ops

    base = torch.from_numpy(rng.standard_normal((64, 300)).astype(np.float32)).cuda()
    x = base[:, :256]  # ld 300 > cols 256
    out = ops.softmax(x)
    assert out.is_cuda
    np.testing.assert_allclose(_np(out), torch.softmax(x.cpu(), -1).numpy(), rtol=1e-5, atol=1e-6)


# -------------------------------------------------- RoPE (not in the reference) --

@pytest.mark.parametrize("dt", ["float32", "bfloat16"])
@pytest.mark.parametrize("H,S,d,pos0,base", [(2, 300, 128, 0, 10000.0), (4, 65, 64, 1000, 500000.0),
                                             (1, 7, 8, 5, 10000.0), (8, 2048, 128, 0, 10000.0)])
def test_rope_matches_oracle(rng, dt, H, S, d, pos0, base):
    """The RoPE kernel against the oracle (float64 angles).  fp32 outputs are
    within the fp32 angle error (relative 2e-7 of the angle, times the pair's
    norm); bf16 outputs within one bf16 step of the oracle's value plus that."""
    import torch

    import oracle as O
    from nkilab import ops

    x = rng.standard_normal((H, S, d)).astype(np.float32)
    tdt = getattr(torch, dt)
    xt = torch.from_numpy(x).to(tdt).cuda()
    out = ops.rope_into(xt, torch.empty_like(xt), base, pos0).float().cpu().numpy()
    ref = O.rope(xt.float().cpu().numpy(), pos0, base, O.F32)
    # fp32 angles: relative error ~2e-7 of (pos0 + s) rad, times the pair's norm
    angle_floor = 1e-5 + 4e-7 * (pos0 + S) * np.abs(x).max()
    if dt == "float32":
        assert np.abs(out - ref).max() <= angle_floor
    else:
        assert_within_bf16_ulps(out, ref, 1, floor=angle_floor)


def test_rope_in_place_on_strided_views(rng):
    """In place on the q columns of a packed [S, 3 d] qkv buffer (the decoder's
    layout), leaving the other columns untouched."""
    import torch

    import oracle as O
    from nkilab import ops

    S, H, hd = 200, 4, 64
    qkv = torch.from_numpy(rng.standard_normal((S, 3 * H * hd)).astype(np.float32)).cuda()
    before = qkv.clone()
    q = qkv[:, :H * hd].view(S, H, hd).transpose(0, 1)
    ops.rope_into(q, q, 10000.0)
    ref = O.rope(before[:, :H * hd].view(S, H, hd).transpose(0, 1).cpu().numpy(), 0, 10000.0)
    assert np.abs(q.cpu().numpy() - ref).max() < 1e-4
    assert torch.equal(qkv[:, H * hd:], before[:, H * hd:])


@pytest.mark.parametrize("nbytes", [16, 4096 * 2048 * 2, 16 * 1000 + 16 * 257, 16 * 1024 * 4 + 16])
def test_stream_copy_is_exact(nbytes):
    """The HBM-ceiling copy (measurement entry point): y == x byte for byte,
    including sizes that leave a partial last workgroup; bytes past the end
    stay untouched."""
    from nkilab import _lib
    from nkilab._tensors import stream_handle

    x = torch.randint(0, 256, (nbytes + 64,), dtype=torch.uint8, device="cuda")
    y = torch.full((nbytes + 64,), 7, dtype=torch.uint8, device="cuda")
    _lib.call("nkl_stream_copy", x.data_ptr(), y.data_ptr(), nbytes, stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(y[:nbytes], x[:nbytes])
    assert bool((y[nbytes:] == 7).all())
