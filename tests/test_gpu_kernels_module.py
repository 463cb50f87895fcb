"""nkilab.kernels (the reference's kernel-level modules: pre-transposed
operands, tile-multiple shapes, explicit softmax scale) against nkilab.ops on
the same inputs."""
import math

import numpy as np
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", [np.float32, "bf16"])
def test_matmul_kernels_take_lhsT(rng, dt):
    from nkilab import ops
    from nkilab.kernels import matmul as mm

    a = rng.standard_normal((256, 384)).astype(np.float32)
    b = rng.standard_normal((384, 1024)).astype(np.float32)
    if dt == "bf16":
        a, b = (torch.from_numpy(t).to(torch.bfloat16).cuda() for t in (a, b))
        lhsT = a.t().contiguous()
    else:
        lhsT = np.ascontiguousarray(a.T)
    for fn, variant, kw in ((mm.matmul_naive, "naive", {}), (mm.matmul_blocked, "blocked", {"BM": 2, "BN": 2})):
        out = fn(lhsT, b, **kw)
        ref = ops.matmul(a, b, variant=variant)
        if dt == "bf16":
            exact = a.double().cpu() @ b.double().cpu()
            assert rel_err(out.float().cpu().numpy(), exact.numpy()) < 4e-3
            assert rel_err(out.float().cpu().numpy(), ref.float().cpu().numpy()) < 4e-3
        else:
            np.testing.assert_array_equal(out, ref)
            assert rel_err(out, a.astype(np.float64) @ b) < 1e-5
    with pytest.raises(AssertionError):
        mm.matmul_blocked(np.zeros((128, 128), np.float32), np.zeros((128, 512), np.float32), BM=2, BN=1)


def test_norm_kernels_equal_ops(rng):
    from nkilab import ops
    from nkilab.kernels import norm

    x = torch.from_numpy(rng.standard_normal((256, 512)).astype(np.float32)).to(torch.bfloat16).cuda()
    w = torch.from_numpy((1 + 0.1 * rng.standard_normal(512)).astype(np.float32)).to(torch.bfloat16).cuda()
    assert torch.equal(norm.softmax_fused(x), ops.softmax(x))
    assert torch.equal(norm.softmax_unfused(x), ops.softmax(x, fused=False))
    assert torch.equal(norm.rmsnorm_fused(x, w, 1e-6), ops.rmsnorm(x, w, 1e-6))
    assert torch.equal(norm.swiglu_fused(x, x), ops.swiglu(x, x))


def test_attention_kernels_take_qT_kT_and_a_scale(rng):
    from nkilab import ops
    from nkilab.kernels import attention as attn

    H, S, d = 2, 256, 64
    q, k, v = (torch.from_numpy(rng.standard_normal((H, S, d)).astype(np.float32)).to(torch.bfloat16).cuda()
               for _ in range(3))
    qT, kT = q.transpose(1, 2).contiguous(), k.transpose(1, 2).contiguous()
    for fn, variant in ((attn.attention_naive, "naive"), (attn.flash_attention, "flash"),
                        (attn.flash_attention_kv_resident, "flash_kv_resident"),
                        (attn.flash_attention_balanced, "flash_balanced"),
                        (attn.flash_attention_pipelined, "flash_pipelined")):
        assert torch.equal(fn(qT, kT, v, 1.0 / math.sqrt(d)), ops.attention(q, k, v, variant=variant)), variant
    # the caller's scale is the one applied: fp32 causal attention at half the usual scale
    scale = 0.5 / math.sqrt(d)
    qf, kf, vf = (t.float().cpu() for t in (q, k, v))
    s = (qf @ kf.transpose(1, 2)) * scale
    s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    ref = torch.softmax(s, -1) @ vf
    for fn in (attn.attention_naive, attn.flash_attention, attn.flash_attention_pipelined):
        out = fn(qT, kT, v, scale).float().cpu()
        assert rel_err(out.numpy(), ref.numpy()) < 3e-3
    with pytest.raises(AssertionError):
        attn.flash_attention(qT[:, :, :100], kT[:, :, :100], v[:, :100], 0.1)
