"""The decode attention entry point that allocates nothing (cir_paged_decode_attention_noalloc).

It must give bitwise the output of cir_paged_decode_attention (same kernels, its
split partials in the library's static per-GPU scratch instead of a workspace),
also on a second call with a smaller input that finds the scratch holding the first
call's partials, and reject sizes beyond CIR_ATTENTION_NOALLOC_MAX_BYTES before
launching anything.
"""
import numpy as np
import pytest
import torch

from oracle import paged

pytestmark = pytest.mark.gpu


def to_dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def _case(device, seed, ctx, hq, hkv, d, dtype):
    rng = np.random.default_rng(seed)
    kp, vp, pt, lens = paged.build_pool(rng, ctx, hkv, d, 16, dtype=dtype, extra_slots=2)
    q = rng.standard_normal((len(ctx), hq, d)).astype(dtype)
    return tuple(to_dev(a, device) for a in (q, kp, vp, pt, lens))


# (contexts, hq, hkv, head_dim, dtype): the fp16 MFMA path with 8 and 4 context splits, then the generic path
# (fp32 pools: one partial per 128-token chunk).  Each pair runs large first, then smaller.
CASES = [
    (([3000, 2500], 32, 8, 128, np.float16), ([700], 32, 8, 128, np.float16)),
    (([1500, 40, 1], 4, 2, 64, np.float32), ([200], 4, 2, 64, np.float32)),
    (([2048] * 6, 28, 4, 128, np.float16), ([300, 17, 1], 28, 4, 128, np.float16)),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_attention_matches_workspace_entry_point(device, first, second):
    from cacheir_amd import kernels

    for i, (ctx, hq, hkv, d, dtype) in enumerate((first, second)):
        print(f"noalloc case {i}: ctx={ctx} hq={hq} hkv={hkv} d={d} {np.dtype(dtype).name}", flush=True)
        q, kp, vp, pt, lens = _case(device, 7 + i, ctx, hq, hkv, d, dtype)
        want = kernels.paged_decode_attention(q, kp, vp, pt, lens, check_tables=True)
        out = torch.full_like(q, float("nan"))
        got = kernels.paged_decode_attention_noalloc(q, kp, vp, pt, lens, out=out)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert torch.equal(got, want), f"case {i}: max |d| {(got.float() - want.float()).abs().max().item()}"
        ref = paged.paged_attention(q.cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy(), pt.cpu().numpy(),
                                    lens.cpu().numpy(), hq, hkv)
        tol = 1e-4 if dtype == np.float32 else 2e-3
        np.testing.assert_allclose(got.float().cpu().numpy(), ref, atol=tol, rtol=tol if dtype == np.float32 else 1e-2)


def test_noalloc_attention_rejects_sizes_beyond_its_scratch(device):
    """The generic path at 32k tokens of context for 4 rows of 32 heads needs 17 MB of partials (> 16 MiB): the
    call fails with a clear error before any launch."""
    from cacheir_amd import hip, kernels

    batch, hq, hkv, d, psize, max_pages = 4, 32, 8, 128, 16, 2048
    need = batch * hq * (max_pages * psize // 128) * (d + 2) * 4
    assert need > hip.ATTENTION_NOALLOC_MAX_BYTES
    q = torch.zeros((batch, hq, d), dtype=torch.float32, device=device)
    kp = torch.zeros((2, hkv, psize, d), dtype=torch.float32, device=device)
    pt = torch.zeros((batch, max_pages), dtype=torch.int32, device=device)
    lens = torch.ones(batch, dtype=torch.int32, device=device)
    with pytest.raises(RuntimeError, match="static scratch"):
        kernels.paged_decode_attention_noalloc(q, kp, kp, pt, lens)
    # the library is still usable afterwards
    small = kernels.paged_decode_attention_noalloc(q, kp, kp, pt[:, :4].contiguous(), lens)
    torch.cuda.synchronize()
    assert torch.isfinite(small).all()
