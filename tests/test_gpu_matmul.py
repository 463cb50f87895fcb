"""GEMM kernels on the GPU against float64 products, the oracle and the golden
fixtures (the reference's tests/test_matmul.py, plus the 1024^3 bf16 config)."""
import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

import oracle as O
from conftest import assert_within_bf16_ulps, load_golden, rel_err

pytestmark = pytest.mark.gpu


def _bf(t):
    return torch.from_numpy(np.asarray(t, np.float32)).to(torch.bfloat16).cuda()


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("variant", ["naive", "blocked"])
@pytest.mark.parametrize("M,K,N", [(128, 128, 512), (256, 384, 1024), (200, 300, 130), (1, 7, 3)])
def test_matmul_fp32(rng, variant, M, K, N):
    from nkilab import ops

    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    assert rel_err(ops.matmul(a, b, variant=variant), a.astype(np.float64) @ b) < 1e-5


@pytest.mark.parametrize("variant", ["naive", "blocked"])
def test_matmul_bf16_accumulates_in_fp32(rng, variant):
    from nkilab import ops

    a = _bf(rng.standard_normal((256, 1024)))
    b = _bf(rng.standard_normal((1024, 1024)))
    ref = _np(a).astype(np.float64) @ _np(b)
    out = ops.matmul(a, b, variant=variant)
    assert out.dtype == torch.bfloat16
    assert rel_err(_np(out), ref) < 1e-2  # only the final bf16 rounding of C
    assert_within_bf16_ulps(_np(out), O.bf16_round(ref.astype(np.float32)), 1.0, 1e-3)


def test_matmul_1024_cubed_bf16_config():
    """M = N = K = 1024, A and B ~ N(0, 1) bf16 from seed 0: max relative error
    <= 3e-3 against the exact product (the bf16 rounding floor of this input is
    2.965e-3)."""
    from nkilab import ops, workloads

    a, b = (t.cuda() for t in workloads.matmul_inputs())
    out = _np(ops.matmul(a, b))
    exact = _np(a).astype(np.float64) @ _np(b).astype(np.float64)
    floor = rel_err(O.bf16_round(exact.astype(np.float32)), exact)
    err = rel_err(out, exact)
    assert err <= 3e-3, (err, floor)
    assert err <= floor * 1.01 + 1e-6, (err, floor)
    assert_within_bf16_ulps(out, O.bf16_round(exact.astype(np.float32)), 1.0, 1e-3)


def test_matmul_matches_golden_vectors():
    from nkilab import ops

    gd = load_golden("matmul")
    for tag, dt in (("f32", O.F32), ("f32b", O.F32), ("bf16", O.BF16)):
        to = (lambda x: torch.from_numpy(x).cuda()) if dt == O.F32 else _bf
        out = _np(ops.matmul(to(gd[f"{tag}_a"]), to(gd[f"{tag}_b"])))
        ref = gd[f"{tag}_c"]
        if dt == O.F32:
            assert rel_err(out, ref) < 1e-5
        else:
            assert_within_bf16_ulps(out, ref, 1.0, 1e-3)


@settings(max_examples=12, deadline=None)
@given(M=st.integers(1, 300), K=st.integers(1, 300), N=st.integers(1, 700))
def test_matmul_property_any_shape(M, K, N):
    from nkilab import ops

    r = np.random.default_rng(M * 1000003 + K * 1009 + N)
    a = r.uniform(-1, 1, (M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    out = ops.matmul(a, b)
    assert out.shape == (M, N)
    np.testing.assert_allclose(out, a.astype(np.float64) @ b, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_linear_layout_and_residual_epilogue(rng, dt):
    """C = A . W^T + R with W in nn.Linear [out, in] layout (the B^T kernel), and the
    bf16 -> fp32 output used for the decoder's residual stream."""
    from nkilab import ops

    M, K, N = 192, 320, 256
    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(dt).cuda()
    w = torch.from_numpy(rng.standard_normal((N, K)).astype(np.float32)).to(dt).cuda()
    res = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
    c = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ops.linear_into(a, w, c, residual=res)
    ref = _np(a).astype(np.float64) @ _np(w).astype(np.float64).T + _np(res)
    assert rel_err(_np(c), ref) < 1e-5
    # the same product through gemm_into with b = w.t() (a column-major view)
    c2 = torch.empty((M, N), dtype=dt, device="cuda")
    ops.gemm_into(a, w.t(), c2)
    tol = 1e-5 if dt == torch.float32 else 1e-2
    assert rel_err(_np(c2), ref - _np(res)) < tol


def test_nonaligned_leading_dimensions(rng):
    from nkilab import ops

    base_a = torch.from_numpy(rng.standard_normal((100, 77)).astype(np.float32)).cuda()
    base_b = torch.from_numpy(rng.standard_normal((61, 90)).astype(np.float32)).cuda()
    a, b = base_a[:, :61], base_b[:, :45]  # lda 77, ldb 90, K 61: the general-stride kernel
    c = ops.matmul(a, b)
    ref = _np(a).astype(np.float64) @ _np(b)
    assert rel_err(_np(c), ref) < 1e-5


@pytest.mark.parametrize("M,K,N,out_dt,res", [(192, 320, 256, torch.bfloat16, False), (130, 64, 72, torch.bfloat16, True),
                                               (257, 128, 40, torch.float32, True), (1000, 256, 1536, torch.float32, True),
                                               (64, 96, 132, torch.float32, False)])
def test_staged_epilogue_matches_element_epilogue(rng, M, K, N, out_dt, res):
    """bf16 GEMMs whose outputs take the 16-byte staged epilogue (aligned rows)
    against the same product written into a view whose rows are not 16-byte
    aligned (the element epilogue): identical values, residual included."""
    from nkilab import ops

    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    w = torch.from_numpy(rng.standard_normal((N, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    r = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(out_dt).cuda() if res else None
    c = torch.empty((M, N), dtype=out_dt, device="cuda")
    ops.linear_into(a, w, c, residual=r)
    big = torch.empty((M, N + 1), dtype=out_dt, device="cuda")
    c_odd = big[:, 1:]  # data pointer off by one element, ld N + 1
    ops.linear_into(a, w, c_odd, residual=r)
    assert torch.equal(c, c_odd)
    ref = _np(a).astype(np.float64) @ _np(w).astype(np.float64).T + (_np(r) if res else 0)
    assert rel_err(_np(c), ref) < (1e-5 if out_dt == torch.float32 else 1e-2)


# Shapes the tile choice sends to 256x192, 256x256, 256x128 and 128x128 (in
# that order; rounds of 256 workgroups x measured cost per K-step), each with
# partial tiles at both edges of C; then long K-loops (hundreds of stage
# hand-overs) on 128x128, 256x128 and 64x128.
@pytest.mark.parametrize("M,K,N", [(2000, 136, 6104), (4000, 136, 4000), (2040, 136, 4088), (2000, 200, 2000),
                                   (2000, 5632, 2000), (2040, 2056, 4088), (1000, 3000, 1000)])
@pytest.mark.parametrize("layout", ["nt", "nn"])
def test_large_tile_gemms_with_ragged_edges(rng, M, K, N, layout):
    """bf16 GEMMs on the large tiles against a float64 product; the staged
    epilogue (aligned C) and the element epilogue (C one element off) agree
    exactly, residual included."""
    from nkilab import ops

    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    b = torch.from_numpy(rng.standard_normal((N, K) if layout == "nt" else (K, N)).astype(np.float32))
    b = b.to(torch.bfloat16).cuda()
    r = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(torch.bfloat16).cuda()
    run = (lambda c: ops.linear_into(a, b, c, residual=r)) if layout == "nt" else \
        (lambda c: ops.gemm_into(a, b, c, residual=r))
    c = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    run(c)
    big = torch.empty((M, N + 1), dtype=torch.bfloat16, device="cuda")
    run(big[:, 1:])
    assert torch.equal(c, big[:, 1:])
    bt = b.double().cpu() if layout == "nn" else b.double().cpu().t()
    ref = (a.double().cpu() @ bt + r.double().cpu()).numpy()
    assert rel_err(_np(c), ref) < 1e-2
    # one rounding of the fp32 sum: within one bf16 ulp of the exact value, plus
    # the fp32 accumulation error (~K * 2^-24 * |terms|) where C is near zero
    assert_within_bf16_ulps(_np(c), ref, 1, floor=2e-3)


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 11264), (3000, 1024, 7000), (2000, 512, 11000)])
@pytest.mark.parametrize("layout", ["nt", "nn"])
@pytest.mark.parametrize("out_dt", [torch.bfloat16, torch.float32])
def test_column_split_matches_column_slices(rng, M, K, N, layout, out_dt):
    """Shapes whose 256-row tiles leave a partial last round run as two
    launches over column ranges (2048 x 11264: 256 x 256 tiles over the first
    8192 columns, 256 x 128 over the rest).  Every column equals, bit for
    bit, what a GEMM over a slice of the columns computes, residual included,
    and is within one bf16 ulp of the float64 product."""
    from nkilab import ops

    a = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    b = torch.from_numpy(rng.standard_normal((N, K) if layout == "nt" else (K, N)).astype(np.float32))
    b = b.to(torch.bfloat16).cuda()
    r = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(out_dt).cuda()

    def run(bm, c, res):
        return ops.linear_into(a, bm, c, residual=res) if layout == "nt" else ops.gemm_into(a, bm, c, residual=res)

    c = torch.empty((M, N), dtype=out_dt, device="cuda")
    run(b, c, r)
    # slices of 2048 columns: their GEMMs take one-K-group tiles too, or the
    # element kernel for a [K, N] slice that is not 16-byte aligned, both
    # summing K in the same order (fewer columns would give the small
    # two-K-group tiles another sum order)
    for lo, hi in [(0, 2048), (N // 2 - 1088, N // 2 + 960), (N - 2048, N)]:
        bs = b[lo:hi] if layout == "nt" else b[:, lo:hi]
        cs = torch.empty((M, hi - lo), dtype=out_dt, device="cuda")
        run(bs, cs, r[:, lo:hi])
        assert torch.equal(c[:, lo:hi], cs), (lo, hi)
        bt = bs.double().cpu() if layout == "nn" else bs.double().cpu().t()
        ref = (a[:512].double().cpu() @ bt + r[:512, lo:hi].double().cpu()).numpy()  # first 512 rows
        if out_dt == torch.bfloat16:
            assert_within_bf16_ulps(_np(cs[:512]), ref, 1, floor=2e-3)
        else:
            assert rel_err(_np(cs[:512]), ref) < 1e-5


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 5632), (300, 256, 96), (64, 128, 32), (1, 64, 64), (513, 384, 704)])
def test_gemm_swiglu_equals_gate_up_then_swiglu(rng, M, K, N):
    """The fused gate/up GEMM with SwiGLU in its epilogue is bit-identical to
    two bf16 linear layers followed by the SwiGLU kernel (model.py:88), and
    within bf16 tolerance of the float64 product."""
    from nkilab import ops

    h = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    wg = torch.from_numpy((0.05 * rng.standard_normal((N, K))).astype(np.float32)).to(torch.bfloat16).cuda()
    wu = torch.from_numpy((0.05 * rng.standard_normal((N, K))).astype(np.float32)).to(torch.bfloat16).cuda()
    fused = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ops.gemm_swiglu_into(h, ops.pack_gate_up(wg, wu), fused)
    gate, up, act = (torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for _ in range(3))
    ops.linear_into(h, wg, gate)
    ops.linear_into(h, wu, up)
    ops.swiglu_into(gate, up, act)
    assert torch.equal(fused, act)
    g64 = _np(h).astype(np.float64) @ _np(wg).astype(np.float64).T
    u64 = _np(h).astype(np.float64) @ _np(wu).astype(np.float64).T
    ref = g64 / (1 + np.exp(-g64)) * u64
    assert rel_err(_np(fused), ref) < 2e-2


def test_gemm_swiglu_rejects_bad_shapes():
    from nkilab import ops

    h = torch.zeros((16, 64), dtype=torch.bfloat16, device="cuda")
    w = torch.zeros((2 * 48, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="multiple of 32"):
        ops.gemm_swiglu_into(h, w, torch.empty((16, 48), dtype=torch.bfloat16, device="cuda"))


@pytest.mark.parametrize("layout", ["nt", "nn"])
def test_batched_gemm_on_large_tiles(rng, layout):
    """Three independent products in one launch (blockIdx.z over the batch,
    per-batch strides), a shape the tile choice sends to 256x128 and with
    partial tiles at both edges: each batch entry against its own float64
    product, residual included."""
    from nkilab import _lib
    from nkilab._tensors import stream_handle

    B, M, N, K = 3, 1500, 1600, 136
    a = torch.from_numpy(rng.standard_normal((B, M, K)).astype(np.float32)).to(torch.bfloat16).cuda()
    bsh = (B, N, K) if layout == "nt" else (B, K, N)
    b = torch.from_numpy(rng.standard_normal(bsh).astype(np.float32)).to(torch.bfloat16).cuda()
    r = torch.from_numpy(rng.standard_normal((B, M, N)).astype(np.float32)).to(torch.bfloat16).cuda()
    c = torch.empty((B, M, N), dtype=torch.bfloat16, device="cuda")
    ldb = K if layout == "nt" else N
    _lib.call("nkl_gemm", a.data_ptr(), b.data_ptr(), c.data_ptr(), r.data_ptr(), M, N, K, K, ldb, N, N,
              1 if layout == "nt" else 0, B, M * K, bsh[1] * bsh[2], M * N, M * N, 1, 1, 0, stream_handle())
    torch.cuda.synchronize()
    for i in range(B):
        bt = b[i].double().cpu() if layout == "nn" else b[i].double().cpu().t()
        ref = (a[i].double().cpu() @ bt + r[i].double().cpu()).numpy()
        assert_within_bf16_ulps(_np(c[i]), ref, 1, floor=2e-3)
