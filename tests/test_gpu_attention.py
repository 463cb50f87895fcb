"""Causal attention on the GPU against torch SDPA, the oracle and the golden fixtures
(the reference's tests/test_attention.py, plus the 8 x 2048 x 128 bf16 and
long-context configs)."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from conftest import load_golden, rel_err

pytestmark = pytest.mark.gpu

VARIANTS = ["naive", "flash", "flash_kv_resident", "flash_balanced", "flash_pipelined"]

# bf16 outputs on random N(0, 1) inputs, against fp32 SDPA or the oracle: the
# reference's own algorithm in bf16 arithmetic (the oracle) is up to 3.1e-3
# from fp32 SDPA on such inputs (30 seeded cases of the shapes below), from the
# bf16 rounding of P and of O itself (2^-9 of an element).  The benchmark
# configurations are held to 3e-3.
BF16_TOL = 4e-3


def _bf(t):
    return torch.from_numpy(np.asarray(t, np.float32)).to(torch.bfloat16).cuda()


def _np(t):
    return t.float().cpu().numpy()


def _sdpa_cpu(q, k, v):
    """fp32 SDPA on the CPU (the reference oracle of tests/test_attention.py:14-16)."""
    return torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(np.asarray(t, np.float32)) for t in (q, k, v)), is_causal=True).numpy()


# The oracle's flash attention in bf16 arithmetic (the reference's algorithm:
# 128-query x 128-key tiles, P rounded to bf16 before P V) on the same bf16
# inputs, kept for the last few input sets (the parametrised tests repeat them).
# The benchmark configurations are held to 3e-3 of it.  On random shapes the
# kernels' 32-key tiles and lazily raised max round P to bf16 at other scales
# than the oracle's 128-key tiles, and the two bf16 outputs differ by up to
# 3.4e-3 (80 seeded random shapes, H 1-4, S 1-700, d 64/96/128: one above
# 3e-3, at 1 x 437 x 96; 1 x 225 x 128 gives 3.07e-3), as the oracle itself
# is up to 3.1e-3 from fp32 SDPA: random shapes are held to 4e-3.
ORACLE_TOL = 3e-3
ORACLE_TOL_RANDOM = 4e-3
_oracle_cache: dict = {}


def _oracle_bf16(qn, kn, vn, variant="flash_pipelined"):
    key = tuple(hash(t.tobytes()) for t in (qn, kn, vn)) + (qn.shape, variant)
    if key not in _oracle_cache:
        if len(_oracle_cache) >= 8:
            _oracle_cache.pop(next(iter(_oracle_cache)))
        _oracle_cache[key] = O.ops_attention(qn, kn, vn, variant, O.BF16)
    return _oracle_cache[key]


def assert_bf16_attention(out, q, k, v, ctx=(), variant="flash_pipelined"):
    """A bf16 attention output on random inputs against fp32 SDPA (BF16_TOL)
    and against the oracle's same variant (ORACLE_TOL_RANDOM) on the same bf16
    inputs; k and v with as many heads as q."""
    qn, kn, vn = (_np(t) for t in (q, k, v))
    err = rel_err(out, _sdpa_cpu(qn, kn, vn))
    assert err <= BF16_TOL, (ctx, "sdpa", err)
    err = rel_err(out, _oracle_bf16(qn, kn, vn, variant))
    assert err <= ORACLE_TOL_RANDOM, (ctx, "oracle", err)


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("H,S,d", [(1, 128, 64), (2, 512, 64), (2, 200, 32), (1, 384, 128), (3, 77, 128),
                                   (1, 1, 64), (2, 65, 48)])
def test_attention_matches_torch(rng, variant, H, S, d):
    from nkilab import ops

    q, k, v = (rng.standard_normal((H, S, d)).astype(np.float32) for _ in range(3))
    out = ops.attention(q, k, v, variant=variant)
    assert out.shape == (H, S, d) and out.dtype == np.float32
    np.testing.assert_allclose(out, _sdpa_cpu(q, k, v), atol=2e-5)


@pytest.mark.parametrize("variant", ["naive", "flash_pipelined"])
def test_attention_bf16(rng, variant):
    from nkilab import ops

    q, k, v = (_bf(rng.standard_normal((2, 256, 64))) for _ in range(3))
    out = ops.attention(q, k, v, variant=variant)
    assert out.dtype == torch.bfloat16
    assert_bf16_attention(_np(out), q, k, v, variant, variant)


def test_first_token_attends_only_to_itself(rng):
    from nkilab import ops

    q, k, v = (rng.standard_normal((1, 256, 64)).astype(np.float32) for _ in range(3))
    out = ops.attention(q, k, v)
    np.testing.assert_allclose(out[0, 0], v[0, 0], atol=1e-6)


def test_variants_agree_bitwise_on_flash_family(rng):
    from nkilab import ops

    q, k, v = (rng.standard_normal((2, 512, 64)).astype(np.float32) for _ in range(3))
    outs = [ops.attention(q, k, v, variant=n) for n in ("flash_balanced", "flash_pipelined")]
    np.testing.assert_array_equal(outs[0], outs[1])


def test_attention_matches_golden_vectors():
    from nkilab import ops

    gd = load_golden("attention")
    for tag, dt in (("f32", O.F32), ("bf16", O.BF16), ("bf16r", O.BF16)):
        to = (lambda x: torch.from_numpy(x).cuda()) if dt == O.F32 else _bf
        q, k, v = (to(gd[f"{tag}_{n}"]) for n in "qkv")
        for var, key in (("flash_pipelined", "flash"), ("naive", "naive")):
            out = _np(ops.attention(q, k, v, variant=var))
            ref = gd[f"{tag}_{key}"]
            if dt == O.F32:
                np.testing.assert_allclose(out, ref, atol=2e-5, err_msg=f"{tag} {var}")
            else:
                # P is rounded to bf16 relative to a running max that depends on the
                # key tiling, so bf16 results agree to the bf16 tolerance, not bitwise.
                assert rel_err(out, ref) <= BF16_TOL, (tag, var)


def test_strided_heads_layout(rng):
    """q/k/v as head-split views of a fused [S, 3 * d] projection, output written
    straight into the merged [S, d] layout: what nkilab.model does."""
    from nkilab import ops

    S, H, hd = 300, 4, 64
    d = H * hd
    qkv = torch.from_numpy(rng.standard_normal((S, 3 * d)).astype(np.float32)).to(torch.bfloat16).cuda()
    q, k, v = (qkv[:, i * d:(i + 1) * d].view(S, H, hd).transpose(0, 1) for i in range(3))
    merged = torch.empty((S, d), dtype=torch.bfloat16, device="cuda")
    ops.attention_into(q, k, v, merged.view(S, H, hd).transpose(0, 1))
    got = _np(merged).reshape(S, H, hd).transpose(1, 0, 2)
    assert_bf16_attention(got, *(t.contiguous() for t in (q, k, v)))


@pytest.mark.parametrize("kernel", [None, "teams", "w64x4", "fwd", "ks"])
@pytest.mark.parametrize("d", [64, 96, 128])
def test_largest_row_stride(rng, flash_cfg, kernel, d):
    """q, k and v with a row stride of 2^21 elements, the largest the entry
    points take, in a buffer of NaNs: the kernels' 32-bit offsets across a
    block of up to 256 rows stay exact, and the chunks past d (the head-dim
    padding, read from outside the buffer) stay zero rather than NaN."""
    from nkilab import ops

    H, S, RS = 1, 300, 1 << 21
    if kernel:
        flash_cfg(kernel=kernel)
    buf = torch.full((S, RS), float("nan"), dtype=torch.bfloat16, device="cuda")  # 1.2 GiB
    views = []
    for i in range(3):
        src = _bf(rng.standard_normal((S, d)))
        buf[:, 256 * i:256 * i + d] = src
        views.append(torch.as_strided(buf, (H, S, d), (0, RS, 1), 256 * i))
    out = _np(ops.attention(*views))
    assert np.isfinite(out).all()
    assert_bf16_attention(out, *(t.contiguous() for t in views), ctx=(kernel, d))
    del buf, views


def test_strides_beyond_the_entry_limits_are_copied(rng):
    """ops.attention takes any strides: operands past the entry points' row
    stride limit go through a contiguous copy, and so does the output."""
    from nkilab import ops

    H, S, d, RS = 2, 40, 64, (1 << 21) + 256
    buf = _bf(rng.standard_normal((S, RS // 64, 64))).view(S, RS)
    q, k, v = (torch.as_strided(buf, (H, S, d), (d, RS, 1), 2 * d * i) for i in range(3))
    obuf = torch.zeros((S, RS), dtype=torch.bfloat16, device="cuda")
    o = torch.as_strided(obuf, (H, S, d), (d, RS, 1))
    ops.attention_into(q, k, v, o)
    assert_bf16_attention(_np(o), *(t.contiguous() for t in (q, k, v)))


def test_flash_scratch_reused_across_shapes(rng):
    """One stream's scratch serves calls of different shapes in turn: a large call's
    partial states must not disturb a later small call's arrival counters."""
    from nkilab import ops

    for H, S, d in [(8, 2048, 128), (1, 131, 128), (2, 96, 64), (4, 1000, 64), (1, 33, 32), (8, 2048, 128)]:
        q, k, v = (_bf(rng.standard_normal((H, S, d))) for _ in range(3))
        out = _np(ops.attention(q, k, v))
        assert_bf16_attention(out, q, k, v, (H, S, d))


SCHEDULES = [(qb, s) for qb in ("64", "128") for s in ("balanced", "pairs", "block")]


@pytest.mark.parametrize("kernel", ["teams", "teams4"])
@pytest.mark.parametrize("qb,schedule", SCHEDULES)
@pytest.mark.parametrize("H,S,d", [(1, 1, 64), (2, 65, 32), (3, 77, 128), (1, 300, 128), (4, 1000, 64),
                                   (2, 1537, 128), (5, 640, 96), (1, 129, 128), (1, 192, 128)])
def test_flash_bf16_schedules(rng, flash_cfg, kernel, qb, schedule, H, S, d):
    """Every configuration of the bf16 teams kernel -- 8 or 4 wavefronts; 64-
    or 128-query blocks; split blocks merged by the last workgroup, one
    workgroup per pair of blocks, or one per block -- on ragged S and several
    head dims."""
    from nkilab import ops

    flash_cfg(kernel=kernel, schedule=schedule, qb=qb)
    q, k, v = (_bf(rng.standard_normal((H, S, d))) for _ in range(3))
    out = _np(ops.attention(q, k, v))
    assert_bf16_attention(out, q, k, v, (schedule, H, S, d))
    np.testing.assert_allclose(out[:, 0], _np(v)[:, 0], rtol=2 ** -8, atol=0)  # query 0 sees only key 0


@pytest.mark.parametrize("kernel", ["w1", "w1o2", "w64", "w64x4", "fwd", "pp", "ks"])
@pytest.mark.parametrize("schedule", ["balanced", "pairs", "block"])
@pytest.mark.parametrize("H,S,d", [(1, 1, 128), (3, 77, 128), (1, 300, 128), (2, 1537, 128), (5, 640, 96),
                                   (1, 129, 128), (2, 4096, 128), (4, 257, 72)])
def test_flash_bf16_one_wave_per_simd_kernel(rng, flash_cfg, kernel, schedule, H, S, d):
    """The one-wavefront-per-SIMD kernels (LDS-DMA staging, swizzled rows) under
    each schedule: 32 queries x 4 wavefronts, 64 x 2 and 64 x 4."""
    from nkilab import ops

    flash_cfg(kernel=kernel, schedule=schedule)
    q, k, v = (_bf(rng.standard_normal((H, S, d))) for _ in range(3))
    out = _np(ops.attention(q, k, v))
    assert_bf16_attention(out, q, k, v, (kernel, schedule, H, S, d))
    np.testing.assert_allclose(out[:, 0], _np(v)[:, 0], rtol=2 ** -8, atol=0)


@pytest.mark.parametrize("H,Hkv,S,d", [(1, 1, 1, 128), (1, 1, 128, 128), (1, 1, 256, 128), (3, 3, 77, 128),
                                       (2, 2, 200, 96), (4, 4, 129, 72), (8, 8, 256, 128), (8, 2, 250, 128),
                                       (2, 1, 33, 128), (1, 1, 224, 120), (1, 1, 225, 128), (5, 5, 31, 80)])
@pytest.mark.parametrize("explicit", [False, True])
def test_flash_short_sequence_kernel(rng, flash_cfg, H, Hkv, S, d, explicit):
    """The one-pass kernel for S <= 256 (every key row of a 128-query block
    staged in LDS at once, one workgroup per block), the default up to 224
    positions for 64 < d <= 128, and forced by name: against fp32 SDPA and the
    oracle, grouped-query heads included, query 0 seeing only key 0, and
    repeated calls bitwise equal."""
    from nkilab import _lib, ops

    if explicit:
        flash_cfg(kernel="tiny")
    grid, units, split, parts, polls = _lib.flash_plan_check(H, S, d)
    assert split == 0 and polls == -1  # one workgroup per block, no scratch
    q = _bf(rng.standard_normal((H, S, d)))
    k, v = (_bf(rng.standard_normal((Hkv, S, d))) for _ in range(2))
    out = ops.attention(q, k, v)
    kr, vr = (t.repeat_interleave(H // Hkv, dim=0) for t in (k, v))
    assert_bf16_attention(_np(out), q, kr, vr, (H, Hkv, S, d, explicit))
    np.testing.assert_allclose(_np(out)[:, 0], _np(vr)[:, 0], rtol=2 ** -8, atol=0)
    assert torch.equal(ops.attention(q, k, v), out)


def test_flash_short_sequence_kernel_largest_row_stride(rng, flash_cfg):
    """The one-pass kernel's 32-bit copy offsets at the largest row stride the
    entry points take (2^21 elements) over all 256 rows, in a buffer of NaNs:
    exact, and the head-dim chunks past d (read from outside the buffer) stay
    zero rather than NaN."""
    from nkilab import ops

    flash_cfg(kernel="tiny")
    H, S, RS, d = 1, 256, 1 << 21, 96
    buf = torch.full((S, RS), float("nan"), dtype=torch.bfloat16, device="cuda")  # 1 GiB
    views = []
    for i in range(3):
        src = _bf(rng.standard_normal((S, d)))
        buf[:, 256 * i:256 * i + d] = src
        views.append(torch.as_strided(buf, (H, S, d), (0, RS, 1), 256 * i))
    out = _np(ops.attention(*views))
    assert np.isfinite(out).all()
    assert_bf16_attention(out, *(t.contiguous() for t in views), ctx=("tiny", d))
    del buf, views


def test_flash_short_sequence_kernel_falls_back_past_its_range(rng, flash_cfg):
    """Forced where it does not apply (S > 256, d <= 64), the one-pass kernel
    gives way to the teams kernel: the same results as the default."""
    from nkilab import ops

    for H, S, d in ((2, 300, 128), (2, 200, 64)):
        q, k, v = (_bf(rng.standard_normal((H, S, d))) for _ in range(3))
        flash_cfg(kernel="tiny")
        out = ops.attention(q, k, v)
        assert_bf16_attention(_np(out), q, k, v, (H, S, d))


@pytest.mark.parametrize("kernel", ["w1", "w1o2", "w64", "w64x4", "teams4", "fwd", "pp", "ks"])
def test_flash_bf16_one_wave_per_simd_config(flash_cfg, kernel):
    """8 x 2048 x 128 through each one-wavefront-per-SIMD kernel (balanced):
    within 3e-3 of fp32 SDPA."""
    from nkilab import ops, workloads

    flash_cfg(kernel=kernel, schedule="balanced")
    q, k, v = (t.cuda() for t in workloads.attention_inputs())
    out = _np(ops.attention(q, k, v))
    assert rel_err(out, _sdpa_cpu(*(_np(t) for t in (q, k, v)))) <= 3e-3


@pytest.mark.parametrize("qb,schedule", SCHEDULES)
def test_flash_bf16_schedules_agree_on_config(flash_cfg, qb, schedule):
    """8 x 2048 x 128 under each configuration: within 3e-3 of fp32 SDPA."""
    from nkilab import ops, workloads

    flash_cfg(schedule=schedule, qb=qb)
    q, k, v = (t.cuda() for t in workloads.attention_inputs())
    out = _np(ops.attention(q, k, v))
    assert rel_err(out, _sdpa_cpu(*(_np(t) for t in (q, k, v)))) <= 3e-3


@pytest.mark.parametrize("kernel,qb", [("teams", "64"), ("teams", "128"), ("teams4", "64"), ("w1o2", "128"),
                                       ("fwd", "128"), ("pp", "128"), ("ks", "64")])
@pytest.mark.parametrize("cpb", ["0", "3", "15", "1000"])
@pytest.mark.parametrize("H,S,d", [(8, 2048, 128), (3, 1537, 128), (5, 300, 64), (16, 640, 96)])
def test_flash_bf16_balanced_block_start_cost(rng, flash_cfg, kernel, qb, cpb, H, S, d):
    """The balanced split with block start costs from none to more than a
    range holds (the planner lowers it until every range keeps a unit): every
    unit is computed once and every split block merged once, whatever the
    ranges; two calls in a row agree bitwise (the parts of a split block are
    folded in a fixed order, whichever workgroup arrives last)."""
    from nkilab import ops

    flash_cfg(kernel=kernel, schedule="balanced", qb=qb, cpb=cpb)
    q, k, v = (_bf(rng.standard_normal((H, S, d))) for _ in range(3))
    out = _np(ops.attention(q, k, v))
    assert_bf16_attention(out, q, k, v, (kernel, qb, cpb, H, S, d))
    np.testing.assert_allclose(out[:, 0], _np(v)[:, 0], rtol=2 ** -8, atol=0)
    for _ in range(3):
        np.testing.assert_array_equal(_np(ops.attention(q, k, v)), out)


# (H, S, most parts of a split block): the 128-query teams form folds blocks of
# up to six parts as the parts arrive (a bit per part in the block's counter;
# 3 x 1537 at a poll budget of 0, where the holder folds what is in and hands
# the rest over) and counts the arrivals of blocks of more parts.
@pytest.mark.parametrize("H,S,parts", [(8, 2048, 4), (6, 2048, 5), (3, 1537, 6), (2, 4096, 8), (1, 6144, 11)])
def test_teams_128_merge_protocols(flash_cfg, H, S, parts):
    """The teams kernel with 128-query blocks over balanced ranges, on shapes
    that take each merge protocol: within 4e-3 of fp32 SDPA (the bound of the
    random-shape tests), repeated calls bitwise equal, and a poll budget of 0
    (every holder gives up at once) gives the same bits."""
    from nkilab import _lib, ops, workloads

    flash_cfg(kernel="teams", schedule="balanced", qb=128)
    assert _lib.flash_plan_check(H, S, 128)[3] == parts
    q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, 128))
    want = ops.attention(q, k, v)
    torch.cuda.synchronize()
    assert rel_err(_np(want), _sdpa_cpu(*(_np(t) for t in (q, k, v)))) <= 4e-3
    for _ in range(2):
        assert torch.equal(ops.attention(q, k, v), want), (H, S)
    _lib.flash_configure_polls(0)
    try:
        for _ in range(2):
            assert torch.equal(ops.attention(q, k, v), want), (H, S, "polls 0")
    finally:
        _lib.flash_configure_polls()


@pytest.mark.parametrize("kernel", [None, "teams", "teams4", "w1o2", "w64x4", "fwd", "ks"])
@pytest.mark.parametrize("H,S,d", [(8, 2048, 128), (3, 1537, 128), (1, 4096, 128), (5, 300, 64)])
def test_balanced_merge_without_polling_gives_the_same_bits(flash_cfg, kernel, H, S, d):
    """With a poll budget of 0 the workgroup holding a split block's last part
    never waits for the others: every part stores its state and the last to
    arrive merges.  The parts are folded in one fixed order either way, so the
    output has the same bits as with the default budget."""
    from nkilab import _lib, ops, workloads

    flash_cfg(kernel=kernel, schedule="balanced")
    q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, d))
    want = ops.attention(q, k, v)
    _lib.flash_configure_polls(0)
    for _ in range(3):
        assert torch.equal(ops.attention(q, k, v), want), (kernel, H, S, d)
    _lib.flash_configure_polls()
    assert torch.equal(ops.attention(q, k, v), want)


@pytest.mark.parametrize("H,S", [(8, 2048), (1, 4096), (8, 8192), (3, 1537)])
def test_default_attention_is_bitwise_reproducible(H, S):
    """The automatic choice (teams kernel over balanced ranges with 64- or
    128-query blocks, or the two-wavefront-per-SIMD kernel over balanced
    ranges at 8 x 8192): repeated calls give identical bits."""
    from nkilab import ops, workloads

    q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, 128))
    first = ops.attention(q, k, v)
    for _ in range(4):
        assert torch.equal(ops.attention(q, k, v), first), (H, S)


# ------------------------------------------------ benchmark configurations --

def test_causal_attention_8x2048x128_bf16_config():
    """8 heads, S = 2048, d = 128, bf16 from seed 0: max relative error <= 3e-3
    against fp32 SDPA of the same bf16 inputs."""
    from nkilab import ops, workloads

    q, k, v = (t.cuda() for t in workloads.attention_inputs())
    out = _np(ops.attention(q, k, v))
    qn, kn, vn = (_np(t) for t in (q, k, v))
    ref = _sdpa_cpu(qn, kn, vn)
    err = rel_err(out, ref)
    assert err <= 3e-3, err
    orc = O.ops_attention(qn, kn, vn, "flash_pipelined", O.BF16)
    assert rel_err(out, orc) <= 3e-3


def test_long_context_1x4096_bf16():
    from nkilab import ops, workloads

    q, k, v = (t.cuda() for t in workloads.attention_inputs(1, 4096, 128))
    out = _np(ops.attention(q, k, v))
    ref = _sdpa_cpu(*(_np(t) for t in (q, k, v)))
    assert rel_err(out, ref) <= 3e-3
    assert rel_err(out, _oracle_bf16(*(_np(t) for t in (q, k, v)))) <= ORACLE_TOL


def _rows_reference(qn, kn, vn, h, rows, scale):
    """Exact causal attention for a few query rows of one head, float64."""
    out = []
    for i in rows:
        s = (kn[h, :i + 1].astype(np.float64) @ qn[h, i].astype(np.float64)) * scale
        p = np.exp(s - s.max())
        out.append((p / p.sum()) @ vn[h, :i + 1].astype(np.float64))
    return np.stack(out)


def test_long_context_32x16384_bf16_sampled():
    """32 heads x 16384: the full CPU reference is out of reach, so a sample of heads
    and query rows (first, last, tile edges, random) is checked exactly, and every
    output row is checked for the convex-combination bound min(v) <= o <= max(v)."""
    from nkilab import ops, workloads

    H, S, d = 32, 16384, 128
    q, k, v = (t.cuda() for t in workloads.attention_inputs(H, S, d))
    out = ops.attention(q, k, v)
    torch.cuda.synchronize()
    # every row is a convex combination of the value rows it attends to
    vmax = torch.cummax(v.float(), dim=1).values
    vmin = torch.cummin(v.float(), dim=1).values
    of = out.float()
    slack = 1e-2 * v.float().abs().amax()
    assert bool((of <= vmax + slack).all()) and bool((of >= vmin - slack).all())
    assert bool(torch.isfinite(of).all())
    qn, kn, vn = (_np(t[[0, 13, 31]]) for t in (q, k, v))
    on = _np(out[[0, 13, 31]])
    rng = np.random.default_rng(5)
    rows = sorted({0, 1, 63, 64, 127, 128, 8191, 8192, S - 1, *rng.integers(0, S, 12).tolist()})
    for hi in range(3):
        ref = _rows_reference(qn, kn, vn, hi, rows, 1.0 / math.sqrt(d))
        assert rel_err(on[hi, rows], ref) <= 3e-3


# ------------------------------------ grouped-query attention (not in the reference) --

@pytest.mark.parametrize("variant", ["naive", "flash_pipelined"])
@pytest.mark.parametrize("H,Hkv,S,d", [(8, 2, 300, 128), (4, 1, 129, 64), (6, 3, 77, 32), (16, 4, 1024, 128)])
def test_gqa_attention_matches_sdpa_on_repeated_kv(rng, variant, H, Hkv, S, d):
    """K/V with Hkv heads serve H query heads (head h uses K/V head h // (H / Hkv)),
    fp32 and bf16, against SDPA on K/V repeated to H heads and against the oracle."""
    from nkilab import ops

    q = rng.standard_normal((H, S, d)).astype(np.float32)
    k, v = (rng.standard_normal((Hkv, S, d)).astype(np.float32) for _ in range(2))
    rep = lambda t: np.repeat(t, H // Hkv, axis=0)  # noqa: E731
    ref = _sdpa_cpu(q, rep(k), rep(v))
    out = ops.attention(q, k, v, variant=variant)
    assert rel_err(out, ref) < 1e-5, ("fp32", variant)
    qb, kb, vb = (_bf(t) for t in (q, k, v))
    outb = _np(ops.attention(qb, kb, vb, variant=variant))
    refb = _sdpa_cpu(_np(qb), rep(_np(kb)), rep(_np(vb)))
    assert rel_err(outb, refb) <= BF16_TOL, ("bf16", variant)
    assert rel_err(outb, O.ops_attention(_np(qb), _np(kb), _np(vb), variant, O.BF16)) <= ORACLE_TOL_RANDOM


@pytest.mark.parametrize("kernel,qb,schedule", [("teams", "128", "balanced"), ("teams", "64", "balanced"),
                                                ("teams", "128", "pairs"), ("teams", "128", "block"),
                                                ("w64", "128", "balanced"), ("teams4", "64", "balanced"),
                                                ("fwd", "128", "balanced"), ("fwd", "128", "pairs"),
                                                ("pp", "128", "balanced"), ("pp", "128", "pairs"),
                                                ("ks", "64", "balanced"), ("ks", "64", "pairs")])
def test_gqa_bf16_every_kernel_and_schedule(rng, flash_cfg, kernel, qb, schedule):
    from nkilab import ops

    flash_cfg(kernel=kernel, schedule=schedule, qb=qb)
    H, Hkv, S, d = 8, 2, 1537, 128
    q = _bf(rng.standard_normal((H, S, d)))
    k, v = (_bf(rng.standard_normal((Hkv, S, d))) for _ in range(2))
    out = _np(ops.attention(q, k, v))
    kr, vr = (t.repeat_interleave(H // Hkv, dim=0) for t in (k, v))
    assert_bf16_attention(out, q, kr, vr, (kernel, qb, schedule))
