"""The decoder block end to end on the HIP kernels (the reference's
tests/test_model.py, plus the 2048-hidden bf16 block)."""
import numpy as np
import pytest
import torch

import oracle as O
from conftest import load_golden, rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S", [128, 300])
@pytest.mark.parametrize("variant", ["naive", "flash_pipelined"])
def test_decoder_block_matches_pytorch(S, variant):
    from nkilab.model import BlockConfig, DecoderBlock, nki_forward

    torch.manual_seed(0)
    block = DecoderBlock(BlockConfig()).eval()
    x = torch.randn(S, block.cfg.d_model)
    with torch.no_grad():
        ref = block(x).numpy()
    out = nki_forward(block, x.numpy(), attention_variant=variant)
    assert isinstance(out, np.ndarray) and out.dtype == np.float32
    np.testing.assert_allclose(out, ref, atol=1e-5)


def test_decoder_matches_golden_vectors():
    from nkilab.model import BlockConfig, DecoderBlock, nki_forward

    gd = load_golden("decoder")
    d, f = gd["wqkv"].shape[1], gd["wg"].shape[0]
    block = DecoderBlock(BlockConfig(d_model=d, n_heads=int(gd["n_heads"]), d_ff=f)).eval()
    with torch.no_grad():
        for n in ("wqkv", "wo", "wg", "wu", "wd", "norm1", "norm2"):
            getattr(block, n).weight.copy_(torch.from_numpy(gd[n]))
    out = nki_forward(block, gd["x"])
    np.testing.assert_allclose(out, gd["y"], atol=1e-5)


def test_weight_cache_follows_parameter_updates():
    from nkilab.model import BlockConfig, DecoderBlock, nki_forward

    torch.manual_seed(3)
    block = DecoderBlock(BlockConfig(d_model=64, n_heads=2, d_ff=128)).eval()
    x = torch.randn(32, 64)
    first = nki_forward(block, x.numpy())
    with torch.no_grad():
        block.wo.weight.mul_(2.0)
        ref = block(x).numpy()
    np.testing.assert_allclose(nki_forward(block, x.numpy()), ref, atol=1e-5)
    assert np.abs(first - ref).max() > 1e-3


def test_decoder_block_2048_hidden_config():
    """batch 1, seq 2048, hidden 2048, 16 heads x 128, FFN 5632, bf16-valued weights
    from N(0, 0.02): max relative error <= 1e-3 against the fp32 PyTorch block on the
    same weights.  The kernels run with fp32 activations (fp32 MFMA GEMMs and fp32
    flash attention): every bf16 rounding point of the activations alone costs about
    1e-3 of this metric (measured by emulating each one on the CPU), so an all-bf16
    activation path cannot meet the bound."""
    from nkilab import workloads
    from nkilab.model import nki_forward

    block, x = workloads.decoder_inputs()
    block = block.cuda()
    xg = x.cuda()
    with torch.no_grad():
        ref = block(xg).cpu().numpy()
    out = nki_forward(block, xg)
    assert out.dtype == torch.float32 and out.is_cuda
    err = rel_err(out.cpu().numpy(), ref)
    assert err <= 1e-3, err


def test_decoder_block_2048_hidden_split_operands():
    """The split-operand configuration (timed beside the fp16 one, which is the
    reported decoder figure): fp32 activations and residual, every projection on
    bf16 MFMA over hi/lo operand pairs against K-stacked bf16 weights, fp32
    attention -- max relative error <= 1e-3 against the fp32 block."""
    from nkilab import workloads
    from nkilab.model import nki_forward

    block, x = workloads.decoder_inputs()
    block = block.cuda()
    xg = x.cuda()
    with torch.no_grad():
        ref = block(xg).cpu().numpy()
    out = nki_forward(block, xg, compute_dtype="split")
    assert out.dtype == torch.float32 and out.is_cuda
    err = rel_err(out.cpu().numpy(), ref)
    assert err <= 1e-3, err


@pytest.mark.parametrize("S", [64, 300])
def test_decoder_split_small_block_matches_pytorch(S):
    """A small block with bf16-valued weights and uniform(0.5, 1.5) norm weights
    under the split policy, against the fp32 eager block; and a block whose
    weights are not bf16 numbers, which takes the fp32 GEMM for them."""
    from nkilab.model import BlockConfig, DecoderBlock, nki_forward

    torch.manual_seed(5)
    block = DecoderBlock(BlockConfig(d_model=128, n_heads=2, d_ff=256)).eval()
    with torch.no_grad():
        for n in ("wqkv", "wo", "wg", "wu", "wd"):
            w = getattr(block, n).weight
            w.copy_(w.bfloat16().float())
    x = torch.randn(S, 128)
    with torch.no_grad():
        ref = block(x).numpy()
    out = nki_forward(block, x.numpy(), compute_dtype="split")
    assert rel_err(out, ref) <= 1e-4
    with torch.no_grad():
        block.wo.weight.add_(1e-4)  # no longer bf16 numbers
        ref2 = block(x).numpy()
    assert rel_err(nki_forward(block, x.numpy(), compute_dtype="split"), ref2) <= 1e-4


def test_split_bf16_pairs(rng):
    """hi is x rounded to bf16 exactly; hi + lo carries x to 2^-16 relative."""
    from nkilab import ops

    x = torch.from_numpy((rng.standard_normal((37, 96)) * 10.0 ** rng.uniform(-3, 3, (37, 96))).astype(np.float32)).cuda()
    y = torch.empty((37, 192), dtype=torch.bfloat16, device="cuda")
    ops.split_bf16_into(x, y)
    hi, lo = y[:, :96].float(), y[:, 96:].float()
    assert torch.equal(hi, x.bfloat16().float())
    assert float(((hi + lo - x).abs() / x.abs().clamp_min(1e-30)).max()) <= 2.0 ** -16


def test_decoder_block_2048_hidden_bf16_activations():
    """The same block with bf16 GEMM / attention operands and an fp32 residual stream.
    Its error against the fp32 block is set by bf16 rounding of the activations (a CPU
    emulation of this exact policy gives 2.6e-3), so the bound here is 5e-3."""
    from nkilab import workloads
    from nkilab.model import nki_forward

    block, x = workloads.decoder_inputs()
    block = block.cuda()
    xg = x.cuda()
    with torch.no_grad():
        ref = block(xg).cpu().numpy()
    out = nki_forward(block, xg, compute_dtype="bfloat16")
    assert out.dtype == torch.float32
    err = rel_err(out.cpu().numpy(), ref)
    assert err <= 5e-3, err


def test_decoder_bf16_matches_oracle_composition():
    """bf16 compute path against the oracle's composition of the same kernels (small block)."""
    from nkilab.model import BlockConfig, DecoderBlock, nki_forward

    torch.manual_seed(4)
    cfg = BlockConfig(d_model=128, n_heads=2, d_ff=256)
    block = DecoderBlock(cfg).eval()
    x = O.bf16_round(torch.randn(96, 128).numpy())
    out = nki_forward(block, torch.from_numpy(x).to(torch.bfloat16)).float().numpy()
    params = {n: getattr(block, n).weight.detach().numpy() for n in ("wqkv", "wo", "wg", "wu", "wd", "norm1", "norm2")}
    ref = O.nki_forward_ref(params, x, cfg.n_heads, cfg.eps, "flash_pipelined", O.BF16)
    assert rel_err(out, ref) < 2e-2


@pytest.mark.parametrize("n_kv_heads,rope_base", [(2, None), (None, 10000.0), (1, 500000.0)])
def test_decoder_gqa_rope_matches_pytorch(n_kv_heads, rope_base):
    """Grouped-query attention and rotary embeddings (not in the reference) end to
    end: fp32 within 1e-3 of the eager block, bf16 within bf16 tolerance."""
    from nkilab.model import BlockConfig, DecoderBlock, nki_forward

    torch.manual_seed(0)
    block = DecoderBlock(BlockConfig(n_kv_heads=n_kv_heads, rope_base=rope_base)).eval()
    x = torch.randn(300, block.cfg.d_model)
    with torch.no_grad():
        ref = block(x).numpy()
    out = nki_forward(block, x.numpy())
    assert np.abs(out - ref).max() <= 1e-3 * np.abs(ref).max()
    outb = nki_forward(block, x.cuda(), compute_dtype="bfloat16").float().cpu().numpy()
    assert rel_err(outb, ref) < 2e-2
