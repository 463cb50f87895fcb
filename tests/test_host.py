"""CPU-only checks of the host layer and of the C ABI's shape (no kernel launches)."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "nkilab_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nkl_\w+)\s*\(", text)))


def test_header_declares_the_abi():
    syms = _declared_symbols()
    for name in ("nkl_gemm", "nkl_softmax", "nkl_softmax_unfused", "nkl_rmsnorm", "nkl_swiglu",
                 "nkl_flash_attn_causal", "nkl_attention_naive", "nkl_last_error_string", "nkl_abi_version"):
        assert name in syms


def test_library_loads_and_exports_every_declared_symbol():
    from nkilab import _lib

    L = _lib.lib()  # dlopen only: no HIP call is made
    for name in _declared_symbols():
        assert hasattr(L, name), name
    assert set(_declared_symbols()) == set(_lib.SIGNATURES)
    assert L.nkl_abi_version() == _lib.ABI_VERSION


def test_abi_rejects_bad_arguments_before_launching():
    from nkilab import _lib

    L = _lib.lib()
    assert L.nkl_gemm(None, None, None, None, -1, 4, 4, 4, 4, 4, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0, None) == -1
    assert b"negative" in L.nkl_last_error_string()
    assert L.nkl_gemm(None, None, None, None, 4, 4, 4, 4, 4, 4, 0, 0, 1, 0, 0, 0, 0, 0, 0, 7, None) == -1
    assert L.nkl_gemm(None, None, None, None, 4, 4, 4, 4, 4, 4, 0, 0, 1, 0, 0, 0, 0, 5, 5, 0, None) in (-1, -2)
    assert L.nkl_softmax(None, None, 0, 16, 16, 16, 1, None) == 0  # empty: nothing to do
    assert L.nkl_softmax(None, None, 4, 16, 8, 16, 1, None) == -1  # ld < cols
    assert L.nkl_swiglu(None, None, None, -3, 0, None) == -1
    assert L.nkl_stream_copy(None, None, 0, None) == 0  # empty: nothing to do
    assert L.nkl_stream_copy(None, None, 24, None) == -1  # not a multiple of 16
    assert L.nkl_stream_copy(None, None, 32, None) == -1  # null pointers
    assert L.nkl_rmsnorm(None, None, None, 4, 4, 4, 4, ctypes.c_float(1e-6), 1, 0, None) == -2  # bf16 -> f32
    assert L.nkl_flash_attn_causal(None, None, None, None, 1, 16, 256, 0, 0, 0, 0, 0, 0, 0, 0,
                                   ctypes.c_float(0.1), 1, None) == -1  # d > 128
    assert b"head dim" in L.nkl_last_error_string()
    assert L.nkl_attention_naive(None, None, None, None, None, 0, 1, 16, 64, 0, 0, 0, 0, 0, 0, 0, 0,
                                 ctypes.c_float(0.1), 1, None) in (-1, -4)
    assert L.nkl_softmax_unfused_workspace_bytes(4, 8) >= 4 * 8 * 4 + 2 * 4 * 4
    assert L.nkl_attention_naive_workspace_bytes(2, 16, 1) >= 2 * 16 * 16 * 6


def test_flash_scratch_sizes():
    """Balanced (split-block) scratch except for the largest shapes, where one
    workgroup per block needs none: 8 x 2048 has 17 units (128 queries x 32
    keys) per CU, 32 x 16384 has 4128 (the sizes assume a 256-CU device, which
    is what the library assumes with no GPU).  One arrival counter per
    64-query block (the smallest block of any kernel), whatever the head dim."""
    from nkilab import _lib

    L = _lib.lib()
    assert L.nkl_flash_attn_causal_workspace_bytes(8, 2048, 128, 1) > 0
    assert L.nkl_flash_attn_causal_counter_bytes(8, 2048, 1) == 8 * 32 * 4
    assert L.nkl_flash_attn_causal_counter_bytes(1, 4096, 1) == 64 * 4
    # more query blocks (256) than CUs, still the balanced schedule: scratch needed
    assert L.nkl_flash_attn_causal_workspace_bytes(16, 2048, 128, 1) > 0
    assert L.nkl_flash_attn_causal_counter_bytes(16, 2048, 1) == 16 * 32 * 4
    assert L.nkl_flash_attn_causal_workspace_bytes(32, 16384, 128, 1) == 0
    assert L.nkl_flash_attn_causal_counter_bytes(32, 16384, 1) == 0
    assert L.nkl_flash_attn_causal_workspace_bytes(8, 2048, 128, 0) == 0  # f32 needs none
    assert L.nkl_flash_attn_causal_workspace_bytes(0, 2048, 128, 1) == 0


def test_pack_gate_up_interleaves_groups_of_32():
    """Rows 64 j .. 64 j + 31 of the packed weight are Wg's rows 32 j .., the
    next 32 are Wu's, as nkl_gemm_swiglu expects."""
    import torch

    from nkilab import ops

    N, K = 96, 5
    wg = torch.arange(N * K, dtype=torch.float32).reshape(N, K)
    wu = -wg - 1
    p = ops.pack_gate_up(wg, wu)
    assert p.shape == (2 * N, K)
    for j in range(N // 32):
        assert torch.equal(p[64 * j:64 * j + 32], wg[32 * j:32 * j + 32])
        assert torch.equal(p[64 * j + 32:64 * j + 64], wu[32 * j:32 * j + 32])
    with pytest.raises(ValueError):
        ops.pack_gate_up(wg[:40], wu[:40])


def test_gemm_swiglu_abi_checks():
    from nkilab import _lib

    L = _lib.lib()
    assert L.nkl_gemm_swiglu(None, None, None, 4, 48, 64, 64, 64, 48, 1, None) == -1  # N % 32
    assert b"multiple of 32" in L.nkl_last_error_string()
    assert L.nkl_gemm_swiglu(None, None, None, 4, 64, 64, 64, 64, 64, 0, None) == -2  # fp32
    assert L.nkl_gemm_swiglu(None, None, None, 0, 64, 64, 64, 64, 64, 1, None) == 0   # empty


def test_noalloc_attention_rejects_shapes_beyond_its_static_scratch():
    """The allocation-free entry holds 1 MiB of arrival counters (one per
    64-query block): a balanced launch over 2^24 + 64 positions needs one more
    and is refused before any device memory is touched."""
    from nkilab import _lib

    L = _lib.lib()
    _lib.flash_configure(kernel="teams", schedule="balanced")
    try:
        S = (1 << 24) + 64
        fake = ctypes.c_void_p(1 << 12)  # never dereferenced: the size check comes first
        rc = L.nkl_flash_attn_causal_noalloc(fake, fake, fake, fake, 1, 1, S, 128, 0, 128, 0, 128, 0, 128, 0, 128,
                                             ctypes.c_float(0.1), 1, None)
        assert rc == -4, L.nkl_last_error_string()
        assert b"static scratch" in L.nkl_last_error_string()
    finally:
        _lib.flash_configure()
    assert L.nkl_flash_attn_causal_noalloc(None, None, None, None, 1, 1, 16, 256, 0, 0, 0, 0, 0, 0, 0, 0,
                                           ctypes.c_float(0.1), 1, None) == -1  # d > 128


def test_rope_and_gqa_abi_checks():
    from nkilab import _lib

    L = _lib.lib()
    assert L.nkl_rope(None, None, 1, 4, 7, 7, 7, 7, 7, 0, ctypes.c_float(1e4), 0, None) == -1  # odd d
    assert b"even" in L.nkl_last_error_string()
    assert L.nkl_rope(None, None, 1, 4, 8, 8, 8, 8, 8, 0, ctypes.c_float(1.0), 0, None) == -1  # base
    assert L.nkl_rope(None, None, 1, 4, 8, 8, 8, 8, 8, 0, ctypes.c_float(1e4), 9, None) == -2  # dtype
    assert L.nkl_rope(None, None, 0, 4, 8, 8, 8, 8, 8, 0, ctypes.c_float(1e4), 0, None) == 0   # empty
    fake = ctypes.c_void_p(1 << 12)  # never dereferenced: the head-count check comes first
    assert L.nkl_flash_attn_causal_gqa(fake, fake, fake, fake, None, 0, None, 0, 4, 3, 16, 64, 0, 64, 0, 64, 0, 64,
                                       0, 64, ctypes.c_float(0.1), 1, None) == -1
    assert b"divide" in L.nkl_last_error_string()
    assert L.nkl_attention_naive_gqa(fake, fake, fake, fake, None, 0, 4, 0, 16, 64, 0, 64, 0, 64, 0, 64, 0, 64,
                                     ctypes.c_float(0.1), 1, None) == -1
    assert b"divide" in L.nkl_last_error_string()
    # row strides above 2^21 elements are refused (32-bit offsets within a block)
    assert L.nkl_flash_attn_causal(fake, fake, fake, fake, 1, 16, 64, 64, (1 << 21) + 8, 64, 64, 64, 64, 64, 64,
                                   ctypes.c_float(0.1), 1, None) == -1
    assert b"row stride" in L.nkl_last_error_string()
    assert L.nkl_flash_attn_causal(fake, fake, fake, fake, 1, 16, 64, (1 << 24) + 8, 64, 64, 64, 64, 64, 64, 64,
                                   ctypes.c_float(0.1), 1, None) == -1
    assert b"head stride" in L.nkl_last_error_string()
    # null q/k/v/o with work to do are refused before any launch
    assert L.nkl_flash_attn_causal(None, None, None, None, 1, 16, 64, 64, 64, 64, 64, 64, 64, 64, 64,
                                   ctypes.c_float(0.1), 1, None) == -1
    assert b"null" in L.nkl_last_error_string()


def test_block_config_options_default_to_the_reference_block():
    from nkilab.model import BlockConfig, DecoderBlock

    cfg = BlockConfig()
    assert cfg.n_kv_heads is None and cfg.rope_base is None and cfg.kv_heads == cfg.n_heads
    assert DecoderBlock(cfg).wqkv.weight.shape == (3 * 256, 256)
    with pytest.raises(ValueError):
        DecoderBlock(BlockConfig(n_kv_heads=3))


def test_psum_block_check():
    from nkilab import _lib

    L = _lib.lib()
    assert L.nkl_check_blocks(4, 2) == 0
    assert L.nkl_check_blocks(3, 3) == -5
    assert b"PSUM" in L.nkl_last_error_string()


def test_choose_blocks_respects_psum_banks():
    from nkilab import ops

    for mt in range(1, 9):
        for nt in range(1, 17):
            bm, bn = ops.choose_blocks(mt, nt)
            assert bm * bn <= 8 and mt % bm == 0 and nt % bn == 0
    assert ops.choose_blocks(4, 4) in {(2, 4), (4, 2)}


def test_choose_blocks_agrees_with_oracle():
    import oracle as O
    from nkilab import ops

    for mt in range(1, 17):
        for nt in range(1, 17):
            assert ops.choose_blocks(mt, nt) == O.choose_blocks(mt, nt)


def test_pad_to():
    from nkilab import ops

    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    p = ops._pad_to(x, 4, 5)
    assert p.shape == (4, 5) and np.array_equal(p[:2, :3], x) and not p[2:].any() and not p[:, 3:].any()
    same = ops._pad_to(x.T, 3, 2)  # right shape: only made contiguous
    assert same.flags.c_contiguous and np.array_equal(same, x.T)


def test_api_surface_matches_reference_names():
    from nkilab import model, ops

    for name in ("matmul", "choose_blocks", "softmax", "rmsnorm", "swiglu", "attention", "ATTENTION_VARIANTS",
                 "_pad_to"):
        assert hasattr(ops, name), name
    assert list(ops.ATTENTION_VARIANTS) == ["naive", "flash", "flash_kv_resident", "flash_balanced",
                                            "flash_pipelined"]
    for name in ("BlockConfig", "RMSNorm", "DecoderBlock", "nki_forward"):
        assert hasattr(model, name), name
    cfg = model.BlockConfig()
    assert (cfg.d_model, cfg.n_heads, cfg.d_ff, cfg.eps, cfg.head_dim) == (256, 4, 1024, 1e-6, 64)


def test_kernels_module_surface():
    """The kernel-level modules the reference's callers import
    (tests/test_matmul.py:10, bench/run_bench.py:34-36): tile constants,
    kernel names, and the blocked matmul's PSUM check raising before any
    launch (tests/test_matmul.py:34-38)."""
    from nkilab.kernels import attention as attn
    from nkilab.kernels import matmul as mm
    from nkilab.kernels import norm, simulate

    assert (mm.TK, mm.TM, mm.TN, attn.T, norm.P) == (128, 128, 512, 128, 128)
    for name in ("matmul_naive", "matmul_blocked"):
        assert callable(getattr(mm, name))
    for name in ("softmax_unfused", "softmax_fused", "rmsnorm_fused", "swiglu_fused"):
        assert callable(getattr(norm, name))
    for name in ("attention_naive", "flash_attention", "flash_attention_kv_resident", "flash_attention_balanced",
                 "flash_attention_pipelined"):
        assert callable(getattr(attn, name))
    lhsT = np.zeros((128, 384), np.float32)
    rhs = np.zeros((128, 1536), np.float32)
    with pytest.raises(Exception, match="PSUM"):
        simulate(mm.matmul_blocked)(lhsT, rhs, BM=3, BN=3)


def test_fp16_dtype_code_and_policy_names():
    import torch

    from nkilab import _lib, model
    from nkilab._tensors import dtype_code

    assert (_lib.F32, _lib.BF16, _lib.F16) == (0, 1, 2)
    assert dtype_code(torch.float16) == 2
    hdr = open(os.path.join(ROOT, "include", "nkilab_hip.h")).read()
    assert "NKL_F16 = 2" in hdr
    assert model._DTYPES["float16"] == torch.float16
    L = _lib.lib()
    # fp16 operands: the naive GEMM variant and the naive attention take them,
    # and here refuse the null pointers instead (no launch)
    assert L.nkl_gemm(None, None, None, None, 4, 4, 4, 4, 4, 4, 0, 0, 1, 0, 0, 0, 0, 2, 2, 1, None) == -1
    assert L.nkl_attention_naive(None, None, None, None, None, 1 << 20, 1, 16, 64, 64, 64, 64, 64, 64, 64, 64, 64,
                                 ctypes.c_float(0.1), 2, None) == -1
    assert L.nkl_flash_attn_causal_workspace_bytes(8, 2048, 128, 2) > 0


def test_host_validation_happens_before_the_gpu():
    from nkilab import ops

    with pytest.raises(AssertionError):
        ops.matmul(np.zeros((2, 3), np.float32), np.zeros((4, 5), np.float32))
    with pytest.raises(KeyError):
        ops.attention(np.zeros((1, 4, 8), np.float32), np.zeros((1, 4, 8), np.float32),
                      np.zeros((1, 4, 8), np.float32), variant="nope")
    with pytest.raises(ValueError):
        ops.matmul(np.zeros((2, 3), np.float32), np.zeros((3, 5), np.float32), variant="nope")


def test_ops_fail_loudly_without_a_gpu():
    import torch

    from nkilab import ops

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="GPU"):
        ops.softmax(np.zeros((2, 3), np.float32))


def test_decoder_block_eager_matches_closed_form():
    """The eager DecoderBlock (the decoder oracle) against an independent float64 restatement."""
    import torch

    from nkilab.model import BlockConfig, DecoderBlock

    torch.manual_seed(1)
    cfg = BlockConfig(d_model=32, n_heads=2, d_ff=48)
    blk = DecoderBlock(cfg).eval()
    x = torch.randn(10, 32)
    with torch.no_grad():
        y = blk(x).double().numpy()
    W = {n: getattr(blk, n).weight.detach().double().numpy() for n in ("wqkv", "wo", "wg", "wu", "wd")}
    g1, g2 = (blk.norm1.weight.detach().double().numpy(), blk.norm2.weight.detach().double().numpy())
    xd = x.double().numpy()

    def rms(t, g):
        return t / np.sqrt((t ** 2).mean(-1, keepdims=True) + cfg.eps) * g

    qkv = rms(xd, g1) @ W["wqkv"].T
    S, d, H, hd = 10, 32, 2, 16
    out = np.zeros((S, d))
    for h in range(H):
        q, k, v = (qkv[:, i * d + h * hd:i * d + (h + 1) * hd] for i in range(3))
        s = q @ k.T / np.sqrt(hd)
        s[np.triu_indices(S, 1)] = -np.inf
        p = np.exp(s - s.max(-1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (p / p.sum(-1, keepdims=True)) @ v
    x1 = xd + out @ W["wo"].T
    hh = rms(x1, g2)
    gate = hh @ W["wg"].T
    ref = x1 + ((gate / (1 + np.exp(-gate))) * (hh @ W["wu"].T)) @ W["wd"].T
    np.testing.assert_allclose(y, ref, atol=1e-5)


def test_ops_reject_mismatched_operands_before_launching():
    """The C ABI takes bare pointers and sizes, so the Python layer checks every
    operand against the others and raises before any launch (CPU tensors: a
    launch would fail differently)."""
    import torch

    from nkilab import ops

    x = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        ops.rmsnorm_into(x, torch.zeros(7), torch.empty(4, 8))      # weight length != D
    with pytest.raises(ValueError):
        ops.rmsnorm_into(x, torch.zeros(8), torch.empty(4, 7))      # y shape != x shape
    with pytest.raises(ValueError):
        ops.softmax_into(x, torch.empty(4, 7))
    with pytest.raises(ValueError):
        ops.swiglu_into(x, torch.zeros(4, 7), torch.empty(4, 8))    # up shape != gate shape
    with pytest.raises(ValueError):
        ops.swiglu_into(x, x, torch.empty(3, 8))                    # y shape != gate shape
    with pytest.raises(TypeError):
        ops.swiglu_into(x, x.bfloat16(), torch.empty(4, 8))
    q = torch.zeros(2, 16, 8)
    with pytest.raises(ValueError):
        ops.attention_into(q, q, q, torch.empty(2, 16, 4))          # o shape != q shape
    with pytest.raises(ValueError):
        ops.attention_into(q, q, q, torch.empty(2, 16, 8, dtype=torch.bfloat16))
    a = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        ops.gemm_into(a, torch.zeros(8, 5), torch.empty(4, 6))      # c columns != b columns
    with pytest.raises(ValueError):
        ops.gemm_into(a, torch.zeros(8, 5), torch.empty(3, 5))      # c rows != a rows
    with pytest.raises(ValueError):
        ops.gemm_into(a, torch.zeros(7, 5), torch.empty(4, 5))      # b rows != a columns
    with pytest.raises(ValueError):
        ops.linear_into(a, torch.zeros(5, 7), torch.empty(4, 5))    # weight [N, K] with K != 8
    with pytest.raises(ValueError):
        ops.linear_into(a, torch.zeros(5, 8), torch.empty(4, 5), residual=torch.zeros(4, 4))


PLAN_SHAPES = [(1, 1, 128), (1, 64, 128), (1, 128, 128), (1, 4096, 128), (8, 2048, 128), (16, 2048, 128),
               (3, 1000, 128), (5, 77, 64), (7, 333, 32), (64, 512, 128), (128, 128, 64), (2, 8192, 128),
               (1, 65, 96), (40, 2049, 128)]


@pytest.mark.parametrize("kernel", [None, "teams", "teams4", "w1", "w1o2", "w64", "w64x4", "fwd", "pp", "ks", "tiny"])
def test_attention_work_split_covers_every_unit_once(kernel):
    """The host restatement of the kernels' own walk (each range from its last
    segment to its first, split blocks merged by their last range, two
    partial-state slots per range): every (query block, key tile) unit once,
    for every kernel, schedule, block size and block start cost the
    configuration accepts, including ragged sizes and more blocks than CUs."""
    from nkilab import _lib

    try:
        for sched in (None, "balanced", "pairs", "block"):
            for qb in (None, 64, 128):
                for cpb in (None, 0, 1, 7, 40):
                    _lib.flash_configure(kernel=kernel, schedule=sched, qb=qb, cpb=cpb)
                    for H, S, d in PLAN_SHAPES:
                        for f16 in (False, True):
                            grid, units, split, parts, polls = _lib.flash_plan_check(H, S, d, f16)
                            assert grid >= 1 and units >= 1 and parts >= 1
                            if sched != "balanced" and sched is not None:
                                assert split == 0
    finally:
        _lib.flash_configure()


def test_attention_work_split_at_the_largest_shapes():
    """Default plans where 64-bit schedule arithmetic takes over (units past
    2^31 / costs past 2^32 at 32 heads x 2^20 positions) and where the
    32-bit instances run (checked against the 64-bit ones on every range)."""
    from nkilab import _lib

    _lib.flash_configure()
    for H, S in ((32, 16384), (1, 1 << 18), (256, 4096)):
        grid, units, split, parts, polls = _lib.flash_plan_check(H, S, 128)
        assert units > 0 and grid >= 1
    with pytest.raises(ValueError):
        _lib.flash_plan_check(1, 128, 128 + 8)
    with pytest.raises(_lib.NklError):
        _lib.call("nkl_flash_attn_plan_check", 1, 128, 128, 0, None)  # fp32


def test_kernel_choice_rules():
    """The automatic kernel and schedule at the boundaries they were measured
    at (a 256-CU device): the one-pass kernel (one workgroup per 128-query
    block, no scratch) up to 224 positions and up to 256 in the 64-query
    regime, unless its workgroups need two rounds where balanced ranges fill
    every CU; 64-query blocks one workgroup each while the heaviest block
    exceeds a balanced range by at most 18 tiles and every block fits one
    round; 128-query
    teams over balanced ranges past one round of 64-query blocks and up to 100
    units per CU; the 64-key ping-pong kernel beyond.  Units are 32-key tiles
    of a query block for the teams kernel and 64-key tiles for the ping-pong
    kernel."""
    from nkilab import _lib

    _lib.flash_configure()
    _lib.flash_configure_polls()
    plan = lambda H, S: _lib.flash_plan_check(H, S, 128)  # noqa: E731
    assert plan(1, 128)[0] == 1 and plan(1, 128)[2:] == (0, 1, -1)
    assert plan(8, 256)[0] == 8 * 2 and plan(8, 256)[4] == -1       # one-pass, 128-query blocks
    assert plan(257, 128)[0] == 257 and plan(257, 128)[4] == -1     # one-pass: ranges would idle CUs
    assert plan(512, 128)[:2] == (256, 512 * 4)                     # two rounds: balanced 128-query
    assert plan(256, 256)[:2] == (256, 256 * 12)                    # 128-query teams, balanced
    assert plan(14, 1024)[0] == 14 * 16 and plan(14, 1024)[4] == -1  # 64-query blocks, one each
    assert plan(10, 1024)[2] > 0                                    # 32 tiles, ranges of 10: balanced
    assert plan(8, 1536)[2] > 0                                     # 48 tiles, ranges of 18: balanced
    assert plan(64, 512)[1] == 64 * 40 and plan(64, 512)[2] > 0     # 512 64-query blocks: 128-query
    assert plan(24, 2048)[1] == 24 * 544                            # 51 units per CU: teams
    assert plan(16, 4096)[1] == 16 * 2112 // 2                      # 132 units per CU: ping-pong


def test_merge_wait_rule():
    """The workgroup merging a split block waits (a bounded 256 polls) while
    blocks have few parts, and not at all when the longest block spans six or
    more ranges; the configured budget overrides both; schedules without split
    blocks report none."""
    from nkilab import _lib

    _lib.flash_configure()
    _lib.flash_configure_polls()
    try:
        assert _lib.flash_plan_check(8, 2048, 128)[3:] == (4, 256)   # 4 parts at most: wait
        assert _lib.flash_plan_check(4, 2048, 128)[4] == 256
        assert _lib.flash_plan_check(1, 4096, 128)[3:] == (7, 0)    # blocks split 7 ways: no wait
        assert _lib.flash_plan_check(1, 2048, 128)[4] == 0
        assert _lib.flash_plan_check(1, 128, 128)[4] == -1          # one workgroup per block
        assert _lib.flash_plan_check(32, 16384, 128)[4] == -1       # pairs
        _lib.flash_configure_polls(4096)
        assert _lib.flash_plan_check(1, 4096, 128)[4] == 4096
    finally:
        _lib.flash_configure_polls()
