"""nkl_flash_attn_causal_noalloc (causal attention with the library's static
scratch) against nkl_flash_attn_causal_gqa with a caller workspace: two calls
in a row, the second on a smaller input, through the C ABI."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(H, Hkv, S, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(H, S, d, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(Hkv, S, d, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(Hkv, S, d, generator=g).to(torch.bfloat16).cuda()
    return q, k, v


def _strides(q, k, v, o):
    return (q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1), o.stride(0), o.stride(1))


def _with_workspace(q, k, v):
    from nkilab import _lib
    from nkilab.ops import ptr, stream_handle

    L = _lib.lib()
    H, S, d = q.shape
    nbytes = L.nkl_flash_attn_causal_workspace_bytes(H, S, d, _lib.BF16)
    nc = L.nkl_flash_attn_causal_counter_bytes(H, S, _lib.BF16)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    cnt = torch.zeros(max(nc // 4, 1), dtype=torch.int32, device=q.device)
    o = torch.empty_like(q)
    _lib.call("nkl_flash_attn_causal_gqa", ptr(q), ptr(k), ptr(v), ptr(o), ptr(ws), nbytes, ptr(cnt), nc, H,
              k.shape[0], S, d, *_strides(q, k, v, o), 1.0 / math.sqrt(d), _lib.BF16, stream_handle())
    return o, nbytes


def _no_alloc(q, k, v):
    from nkilab import _lib
    from nkilab.ops import ptr, stream_handle

    H, S, d = q.shape
    o = torch.full_like(q, float("nan"))
    _lib.call("nkl_flash_attn_causal_noalloc", ptr(q), ptr(k), ptr(v), ptr(o), H, k.shape[0], S, d,
              *_strides(q, k, v, o), 1.0 / math.sqrt(d), _lib.BF16, stream_handle())
    return o


# (config, shapes of the two calls): the automatic choice at two head widths,
# and the 64-key-tile kernel over balanced ranges.  Every second call is
# smaller than the first and still splits blocks, so it reads scratch the first
# call left behind.
CASES = [
    (None, [(8, 8, 2048, 128), (2, 2, 1024, 128)]),
    (None, [(8, 2, 1024, 64), (4, 1, 1000, 64)]),
    (dict(kernel="fwd", schedule="balanced"), [(8, 8, 2048, 128), (3, 3, 700, 128)]),
]


@pytest.mark.parametrize("cfg,shapes", CASES)
def test_noalloc_matches_workspace_entry(flash_cfg, cfg, shapes):
    if cfg:
        flash_cfg(**cfg)
    for i, (H, Hkv, S, d) in enumerate(shapes):
        print(f"noalloc call {i}: H={H} Hkv={Hkv} S={S} d={d} cfg={cfg}", flush=True)
        q, k, v = _inputs(H, Hkv, S, d, seed=10 + i)
        want, nbytes = _with_workspace(q, k, v)
        got = _no_alloc(q, k, v)
        torch.cuda.synchronize()
        assert nbytes > 0, "shape does not exercise the scratch"
        assert torch.isfinite(got.float()).all()
        # Same kernels and schedule, and split blocks' partial states are
        # folded in a fixed order whichever workgroup merges them: the same bits.
        assert torch.equal(got, want)
