"""Parity of each HIP kernel against the CPU oracle, called through the C ABI.

Tolerances: integer/byte work (dequant, page gathers, argmax) is bit-exact.
fp16 attention and projections are checked with |got - ref| <= 2e-3 + 1e-2*|ref|
(the north-star bound for fp16 vs the fp32 reference); fp32 paths at 1e-4 (the
reference's own GPU parity tolerance, tests/test_runtime.py:62).
"""
import math

import numpy as np
import pytest
import torch

from oracle import ops, paged, quant

pytestmark = pytest.mark.gpu

ATOL16, RTOL16 = 2e-3, 1e-2


def close16(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref) - (ATOL16 + RTOL16 * np.abs(ref))
    assert np.all(err <= 0), f"max violation {err.max():.3e}, max abs err {np.abs(got - ref).max():.3e}"


def to_dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


# ------------------------------------------------------------------ attention --
def test_attention_reference_case_fp32(device):
    """Shape and table of tests/test_advanced_experiments.py:519-557 (fp32, tol 1e-4)."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(0)
    b, hq, hkv, p, d = 2, 4, 2, 2, 8
    q = rng.standard_normal((b, hq, d)).astype(np.float32)
    kp = rng.standard_normal((5, hkv, p, d)).astype(np.float32)
    vp = rng.standard_normal((5, hkv, p, d)).astype(np.float32)
    pt = np.array([[0, 1, 2], [3, 4, 0]], dtype=np.int32)
    lens = np.array([5, 3], dtype=np.int32)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device), check_tables=True)
    ref = paged.brute_force_attention(q, kp, vp, pt, lens, hq, hkv)
    np.testing.assert_allclose(out.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (28, 4), (8, 8), (16, 2)])
def test_attention_fp16_mfma_ragged(device, hq, hkv):
    from cacheir_amd import kernels

    rng = np.random.default_rng(hq * 100 + hkv)
    ctx = [1, 15, 16, 17, 127, 128, 129, 300, 1000]
    kp, vp, pt, lens = paged.build_pool(rng, ctx, hkv, 128, 16, extra_slots=3)
    q = rng.standard_normal((len(ctx), hq, 128)).astype(np.float16)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device), check_tables=True)
    ref = paged.paged_attention(q, kp, vp, pt, lens, hq, hkv)
    close16(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("ctx", [[1500, 40, 1], [1024, 1023], [17000, 900, 3]])
def test_attention_fp32_many_partials(device, ctx):
    """fp32 pools run 128-token chunks, one partial each: 12 and 8 partials take the merge's
    batched loads (the first with a last group of 4), 133 partials its serial form."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(len(ctx) + ctx[0])
    hq, hkv, d = 4, 2, 64
    kp, vp, pt, lens = paged.build_pool(rng, ctx, hkv, d, 16, dtype=np.float32)
    q = rng.standard_normal((len(ctx), hq, d)).astype(np.float32)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device), check_tables=True)
    ref = paged.paged_attention(q, kp, vp, pt, lens, hq, hkv)
    np.testing.assert_allclose(out.cpu().numpy(), ref, atol=1e-4, rtol=1e-4)


def test_attention_empty_sequence_gives_zeros(device):
    from cacheir_amd import kernels

    rng = np.random.default_rng(3)
    kp, vp, pt, lens = paged.build_pool(rng, [20, 5], 2, 128, 16)
    lens = np.array([0, 5], dtype=np.int32)
    q = rng.standard_normal((2, 8, 128)).astype(np.float16)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device)).float().cpu().numpy()
    assert np.all(out[0] == 0)
    close16(out[1], paged.paged_attention(q[1:], kp, vp, pt[1:], lens[1:], 8, 2)[0])


@pytest.mark.parametrize("seed", range(10))
def test_attention_fp16_random_shapes(device, seed):
    """Seeded sweep of the fp16 MFMA decode attention against the oracle: batch 1-48, every GQA ratio 1-8,
    1-8 KV heads, pages of 16 or 32 tokens, contexts 0-1300 with block and page edges (1, 31-33, 255-257)
    mixed in, so split counts, empty rows, partial tiles and the longest-first dispatch all vary."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(1000 + seed)
    batch = int(rng.integers(1, 49))
    g = int(rng.integers(1, 9))
    hkv = int(rng.choice([1, 2, 4, 8]))
    psize = int(rng.choice([16, 32]))
    edges = np.array([0, 1, 31, 32, 33, 255, 256, 257])
    ctx = np.where(rng.random(batch) < 0.3, rng.choice(edges, batch), rng.integers(0, 1301, batch))
    kp, vp, pt, _ = paged.build_pool(rng, np.maximum(ctx, 1), hkv, 128, psize)
    lens = ctx.astype(np.int32)
    q = rng.standard_normal((batch, g * hkv, 128)).astype(np.float16)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device), check_tables=True).float().cpu().numpy()
    live = lens > 0
    assert np.all(out[~live] == 0)
    if live.any():
        close16(out[live], paged.paged_attention(q[live], kp, vp, pt[live], lens[live], g * hkv, hkv))


@pytest.mark.parametrize("hq,hkv", [(32, 8), (28, 4)])
def test_attention_rows_dispatched_longest_first(device, hq, hkv):
    """More (row, KV head) workgroups than CUs: the kernel reorders rows by decreasing context
    (ties by index) before dispatch.  Ties, empty rows and single tokens still land in their own rows."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(hkv)
    batch = 512 // hkv + 8
    ctx = rng.choice([0, 1, 31, 32, 33, 200, 200, 513, 900], batch).astype(np.int64)
    kp, vp, pt, lens = paged.build_pool(rng, np.maximum(ctx, 1), hkv, 128, 16)
    lens = ctx.astype(np.int32)
    assert batch * hkv > 256
    q = rng.standard_normal((batch, hq, 128)).astype(np.float16)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device), check_tables=True).float().cpu().numpy()
    live = lens > 0
    assert np.all(out[~live] == 0)
    ref = paged.paged_attention(q[live], kp, vp, pt[live], lens[live], hq, hkv)
    close16(out[live], ref)


def test_attention_config2_full_size(device):
    """B=64, Hq 32 / Hkv 8, D 128, ctx U[512,4096], P 16, permuted pool."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(0)
    ctx = rng.integers(512, 4097, 64)
    kp, vp, pt, lens = paged.build_pool(rng, ctx, 8, 128, 16)
    q = rng.standard_normal((64, 32, 128)).astype(np.float16)
    out = kernels.paged_decode_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                         to_dev(lens, device), check_tables=True)
    got = out.float().cpu().numpy()
    ref = paged.paged_attention(q, kp, vp, pt, lens, 32, 8)  # every row (a few seconds of NumPy)
    close16(got, ref)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_prefill_attention_causal(device, dtype):
    from cacheir_amd import kernels

    rng = np.random.default_rng(5)
    past, q_len, hq, hkv, d = [3, 40], 6, 8, 2, 128
    total = [p_ + q_len for p_ in past]
    kp, vp, pt, lens = paged.build_pool(rng, total, hkv, d, 16, dtype=dtype)
    q = rng.standard_normal((2 * q_len, hq, d)).astype(dtype)
    out = kernels.paged_prefill_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                          to_dev(lens, device), q_len, check_tables=True).float().cpu().numpy()
    for b in range(2):
        kh = paged.gather_sequence(kp, pt[b], total[b]).astype(np.float32)[None]
        vh = paged.gather_sequence(vp, pt[b], total[b]).astype(np.float32)[None]
        qh = q[b * q_len:(b + 1) * q_len].astype(np.float32)[None]
        ref = ops.attention(qh, kh, vh, hq, hkv, d, causal=True).reshape(q_len, hq, d)
        if dtype == np.float32:
            np.testing.assert_allclose(out[b * q_len:(b + 1) * q_len], ref, atol=1e-4, rtol=1e-4)
        else:
            close16(out[b * q_len:(b + 1) * q_len], ref)


@pytest.mark.parametrize("seed", range(8))
def test_prefill_attention_fp16_random_shapes(device, seed):
    """Seeded sweep of the fp16 prefill kernel (128-vector query tiles over each sequence's blocks, causal mask)
    against the oracle: batch 1-4, GQA ratio 1-8, 1-8 KV heads, pages of 16 or 32, 1-700 new tokens after 0-900
    tokens of earlier context, so tiles end mid-token, sequences have different lengths and blocks end mid-page."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(4000 + seed)
    batch = int(rng.integers(1, 5))
    g = int(rng.integers(1, 9))
    hkv = int(rng.choice([1, 2, 4, 8]))
    psize = int(rng.choice([16, 32]))
    q_len = int(rng.choice([2, 7, 33, 129, int(rng.integers(1, 701))]))
    past = rng.integers(0, 901, batch)
    total = past + q_len
    kp, vp, pt, lens = paged.build_pool(rng, total, hkv, 128, psize)
    hq = g * hkv
    q = rng.standard_normal((batch * q_len, hq, 128)).astype(np.float16)
    out = kernels.paged_prefill_attention(to_dev(q, device), to_dev(kp, device), to_dev(vp, device), to_dev(pt, device),
                                          to_dev(lens, device), q_len, check_tables=True).float().cpu().numpy()
    for b in range(batch):
        kh = paged.gather_sequence(kp, pt[b], int(total[b])).astype(np.float32)[None]
        vh = paged.gather_sequence(vp, pt[b], int(total[b])).astype(np.float32)[None]
        qh = q[b * q_len:(b + 1) * q_len].astype(np.float32)[None]
        ref = ops.attention(qh, kh, vh, hq, hkv, 128, causal=True).reshape(q_len, hq, 128)
        close16(out[b * q_len:(b + 1) * q_len], ref)


@pytest.mark.parametrize("q_len,batch", [(600, 14), (590, 14), (512, 16), (600, 10)])
def test_prefill_attention_paired_tiles(device, q_len, batch):
    """A prefill grid of at least two workgroups per CU runs tile pairs (tiles - 1 - x, then x) in one workgroup:
    an even and an odd tile count (600 / 590 tokens x 8 query heads over 1 KV head: 38 / 37 tiles of 128 query
    vectors, the odd one with a middle tile run once; 266 paired workgroups, 2 K/V blocks per LDS buffer), and 16
    sequences of 32 tiles (256 paired workgroups, at most one per CU: 4 blocks per buffer), after 0-300 tokens of
    context.  The batch agrees with the oracle, and bit for bit with each sequence launched alone (unpaired, one
    workgroup per CU at most: 4 blocks per buffer).  10 sequences of 38 tiles (380 workgroups) run unpaired with
    2 blocks per buffer, against the same checks."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(q_len)
    hkv, g = 1, 8
    hq = g * hkv
    tiles = -(-q_len * g // 128)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    one_tile = tiles * hkv * batch
    paired = one_tile >= 2 * cus
    assert paired == (batch != 10)
    workgroups = (tiles + 1) // 2 * hkv * batch if paired else one_tile
    assert (workgroups <= cus) == (q_len == 512)  # 4 K/V blocks per LDS buffer
    past = rng.integers(0, 301, batch)
    total = past + q_len
    kp, vp, pt, lens = paged.build_pool(rng, total, hkv, 128, 16)
    q = rng.standard_normal((batch * q_len, hq, 128)).astype(np.float16)
    kpd, vpd, ptd = to_dev(kp, device), to_dev(vp, device), to_dev(pt, device)
    out = kernels.paged_prefill_attention(to_dev(q, device), kpd, vpd, ptd, to_dev(lens, device), q_len,
                                          check_tables=True)
    for b in range(batch):
        alone = kernels.paged_prefill_attention(to_dev(q[b * q_len:(b + 1) * q_len], device), kpd, vpd,
                                                ptd[b:b + 1].contiguous(), to_dev(lens[b:b + 1], device), q_len,
                                                check_tables=True)
        assert torch.equal(alone, out[b * q_len:(b + 1) * q_len]), f"sequence {b}"
    out = out.float().cpu().numpy()
    for b in range(batch):
        kh = paged.gather_sequence(kp, pt[b], int(total[b])).astype(np.float32)[None]
        vh = paged.gather_sequence(vp, pt[b], int(total[b])).astype(np.float32)[None]
        qh = q[b * q_len:(b + 1) * q_len].astype(np.float32)[None]
        ref = ops.attention(qh, kh, vh, hq, hkv, 128, causal=True).reshape(q_len, hq, 128)
        close16(out[b * q_len:(b + 1) * q_len], ref)


# -------------------------------------------------------------- block weights --
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_dequant_bit_exact(device, fmt):
    from cacheir_amd import kernels

    rng = np.random.default_rng(11)
    n, k = 37, 384
    if fmt == "q4_0":
        blocks, _, _ = quant.random_q4_0(rng, n, k)
        ref = quant.decode_q4_0(blocks, k)
    else:
        blocks, _, _ = quant.random_q8_0(rng, n, k)
        ref = quant.decode_q8_0(blocks, k)
    code = kernels.FMT_NAMES[fmt]
    dblocks = to_dev(blocks.reshape(-1), device)
    got = kernels.dequant_blocks(dblocks, code, n, k).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    w = kernels.QWeight.from_blocks(dblocks, code, n, k)
    got_t = kernels.dequant_tiled(w).cpu().numpy()
    assert np.array_equal(got_t.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m,n,k,splits", [(1, 64, 128, 1), (5, 100, 256, 2), (16, 48, 512, 4), (32, 80, 384, 3),
                                          (33, 16, 128, 1), (70, 40, 256, 1), (64, 48, 256, 2), (128, 100, 512, 4),
                                          (100, 200, 1280, 5), (200, 24, 384, 3), (64, 4608, 512, 1),
                                          (128, 4610, 896, 7), (150, 4608, 384, 3)])
def test_qgemm_small(device, fmt, m, n, k, splits):
    from cacheir_amd import kernels

    rng = np.random.default_rng(m * 1000 + n + k)
    if fmt == "q4_0":
        blocks, _, _ = quant.random_q4_0(rng, n, k)
        wf = quant.decode_q4_0(blocks, k)
    else:
        blocks, _, _ = quant.random_q8_0(rng, n, k)
        wf = quant.decode_q8_0(blocks, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), kernels.FMT_NAMES[fmt], n, k)
    part = kernels.qgemm_partial(to_dev(x, device), w, splits=splits)
    got = part.sum(0).cpu().numpy()
    ref = ops.matmul(x.astype(np.float32), wf)
    close16(got, ref)
    # products and block scales are exact in fp32: only summation order differs from an fp64 product
    wop = wf.astype(np.float64)
    ref64 = x.astype(np.float64) @ wop.T
    bound = 1e-5 * (np.abs(x.astype(np.float64)) @ np.abs(wop).T) + 1e-6
    assert np.all(np.abs(got - ref64) <= bound)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("n,k", [(14336, 4096), (4096, 14336)])
@pytest.mark.parametrize("m", [1, 8, 32])
def test_qgemm_config3_shapes(device, fmt, n, k, m):
    """Llama-3-8B gate/up/down shapes, nibbles U[0,15], d=|N(0,0.01)|, x fp16 N(0,1)."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(7)
    if fmt == "q4_0":
        blocks, _, _ = quant.random_q4_0(rng, n, k)
        wf = quant.decode_q4_0(blocks, k)
    else:
        blocks, _, _ = quant.random_q8_0(rng, n, k)
        wf = quant.decode_q8_0(blocks, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), kernels.FMT_NAMES[fmt], n, k)
    part = kernels.qgemm_partial(to_dev(x, device), w)
    got = part.sum(0).cpu().numpy()
    close16(got, ops.matmul(x.astype(np.float32), wf))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_qgemv_every_small_batch(device, fmt):
    """Batches of 1..8 rows (the GEMV kernel, whose scaled accumulator registers depend on the row count): every
    row count, a ragged n, k-splits 1, 2 and 5 of 10 quads (ring tails of every length), and one split too long
    for the GEMV's activation stage (m * quads > 128, served by the MFMA GEMM). Each split's partials are checked,
    not only their sum, against the exact-product bound of fp64 and the fp16 bound of the oracle."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(4242)
    n, k = 200, 1280
    enc, dec = (quant.random_q4_0, quant.decode_q4_0) if fmt == "q4_0" else (quant.random_q8_0, quant.decode_q8_0)
    blocks = enc(rng, n, k)[0]
    wf = dec(blocks, k).astype(np.float64)
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), kernels.FMT_NAMES[fmt], n, k)
    for m in range(1, 9):
        x = rng.standard_normal((m, k)).astype(np.float16)
        xd = to_dev(x, device)
        for splits in (1, 2, 5):
            part = kernels.qgemm_partial(xd, w, splits=splits).double().cpu().numpy()
            kq = k // 128 // splits
            for s in range(splits):
                xs = x[:, s * kq * 128:(s + 1) * kq * 128].astype(np.float64)
                ws_ = wf[:, s * kq * 128:(s + 1) * kq * 128]
                bound = 1e-5 * (np.abs(xs) @ np.abs(ws_).T) + 1e-6
                assert np.all(np.abs(part[s] - xs @ ws_.T) <= bound), (m, splits, s)
            close16(part.sum(0), ops.matmul(x.astype(np.float32), wf.astype(np.float32)))
    x = rng.standard_normal((8, 4096)).astype(np.float16)
    blocks = enc(rng, 48, 4096)[0]
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), kernels.FMT_NAMES[fmt], 48, 4096)
    got = kernels.qgemm_partial(to_dev(x, device), w, splits=1)[0].cpu().numpy()
    close16(got, ops.matmul(x.astype(np.float32), dec(blocks, 4096)))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m,n,k,splits", [(128, 100, 8192, 10), (40, 64, 8448, 7), (128, 3584, 18944, 9),
                                          (70, 200, 8320, 4)])
def test_qgemm_large_m_ragged_splits(device, fmt, m, n, k, splits):
    """The large-m kernel's k-splits need not divide k/128: split s covers quads s * ceil(kq / S) onward and the
    last one fewer (down to one quad).  Each split's partials against the exact-product bound of fp64 over that
    range, and their sum against the oracle."""
    from cacheir_amd import hip, kernels

    code = kernels.FMT_NAMES[fmt]
    assert kernels.gemm_plan(hip.GEMM_PARTIALS, code, m, n, k, splits).startswith("qgemm_xl_kernel")
    rng = np.random.default_rng(m + n + k + splits)
    enc, dec = (quant.random_q4_0, quant.decode_q4_0) if fmt == "q4_0" else (quant.random_q8_0, quant.decode_q8_0)
    blocks = enc(rng, n, k)[0]
    wf = dec(blocks, k).astype(np.float64)
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), code, n, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    part = kernels.qgemm_partial(to_dev(x, device), w, splits=splits).double().cpu().numpy()
    kq = k // 128
    per = -(-kq // splits)
    for s in range(splits):
        lo, hi = 128 * s * per, 128 * min(kq, (s + 1) * per)
        assert hi > lo
        xs, ws_ = x[:, lo:hi].astype(np.float64), wf[:, lo:hi]
        bound = 1e-5 * (np.abs(xs) @ np.abs(ws_).T) + 1e-6
        assert np.all(np.abs(part[s] - xs @ ws_.T) <= bound), s
    close16(part.sum(0), ops.matmul(x.astype(np.float32), wf.astype(np.float32)))


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_qgemm_large_m_multi_round_matches_one_round(device, fmt):
    """Launches of more workgroups than CUs (1100 rows: 36 column groups x 9 row blocks = 324 workgroups) take the
    large-m kernel's plain-FMA scaling form; 512-row slices of the same inputs at one split (144 workgroups, one
    round: the default form, for Q8_0 partials the interleave-hinted one) must give the same bits, for the partials
    and for the fused SwiGLU.  At 4 splits both launches are multi-round: the slices check the row blocks (the last
    one partly filled).  The partials' sum also within the fp16 bound of the oracle."""
    from cacheir_amd import hip, kernels

    rng = np.random.default_rng(1100 if fmt == "q4_0" else 1101)
    enc, dec = (quant.random_q4_0, quant.decode_q4_0) if fmt == "q4_0" else (quant.random_q8_0, quant.decode_q8_0)
    code = kernels.FMT_NAMES[fmt]
    m, n, k = 1100, 4608, 1024
    assert kernels.gemm_plan(hip.GEMM_PARTIALS, code, m, n, k, 1).startswith("qgemm_xl_kernel")
    blocks = enc(rng, n, k)[0]
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), code, n, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    xd = to_dev(x, device)
    for splits in (1, 4):
        got = kernels.qgemm_partial(xd, w, splits=splits)
        for a in (0, 300, m - 512):
            ref = kernels.qgemm_partial(xd[a:a + 512].contiguous(), w, splits=splits)
            assert torch.equal(got[:, a:a + 512], ref), (splits, a)
    close16(got.sum(0).cpu().numpy(), ops.matmul(x.astype(np.float32), dec(blocks, k).astype(np.float32)))
    inter = n // 2
    g_dev, u_dev = to_dev(enc(rng, inter, k)[0], device), to_dev(enc(rng, inter, k)[0], device)
    w_il = kernels.QWeight.from_blocks(kernels.interleave_gate_up(g_dev, u_dev, inter).reshape(-1), code, n, k)
    act = kernels.qgemm_swiglu(xd, w_il, torch.float16)
    for a in (0, m - 512):
        assert torch.equal(act[a:a + 512], kernels.qgemm_swiglu(xd[a:a + 512].contiguous(), w_il, torch.float16)), a


@pytest.mark.parametrize("seed", range(12))
def test_qgemm_planner_random_shapes(device, seed):
    """Seeded random shapes through the planner's own choices (``choose_splits``, then whichever kernel
    ``gemm_plan`` names: GEMV, the m <= 32 kernel with one or two row tiles, the large-m kernel at 64 or 128 rows
    with splits that need not divide k/128): m in 1..200, ragged n up to ~5100, k up to 64 quads, both block
    formats. The
    partials' sum against the exact-product bound of fp64 and the fp16 bound of the oracle; the fused SwiGLU
    (interleaved gate/up tiles) and the fused greedy head against the same products."""
    from cacheir_amd import hip, kernels

    rng = np.random.default_rng(900 + seed)
    fmt = ("q4_0", "q8_0")[seed % 2]
    code = kernels.FMT_NAMES[fmt]
    enc, dec = (quant.random_q4_0, quant.decode_q4_0) if fmt == "q4_0" else (quant.random_q8_0, quant.decode_q8_0)
    m = int(rng.choice([1, 2, 5, 8, 9, 16, 17, 31, 32, 33, 48, 64, 65, 100, 128, 129, 200]))
    n = int(rng.integers(1, 321)) * 16 + int(rng.integers(0, 16))
    k = 128 * int(rng.integers(1, 65))
    inter = 16 * max(1, n // 32)
    splits = kernels.choose_splits(m, n, k)
    plan = kernels.gemm_plan(hip.GEMM_PARTIALS, code, m, n, k, splits)
    plans = (plan, kernels.gemm_plan(hip.GEMM_SWIGLU, code, m, 2 * inter, k, 1),
             kernels.gemm_plan(hip.GEMM_ARGMAX, code, m, n, k, 1))
    print(f"seed {seed}: {fmt} m={m} n={n} k={k} splits={splits} -> {' | '.join(plans)}", flush=True)
    assert "invalid" not in plans
    blocks = enc(rng, n, k)[0]
    wf = dec(blocks, k).astype(np.float64)
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), code, n, k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    xd = to_dev(x, device)
    x64 = x.astype(np.float64)
    got = kernels.qgemm_partial(xd, w, splits=splits).double().sum(0).cpu().numpy()
    ref64 = x64 @ wf.T
    assert np.all(np.abs(got - ref64) <= 1e-5 * (np.abs(x64) @ np.abs(wf).T) + 1e-6)
    close16(got, ops.matmul(x.astype(np.float32), wf.astype(np.float32)))

    # SwiGLU over interleaved gate/up tiles (inter columns each, a multiple of 16)
    g_blocks, u_blocks = enc(rng, inter, k)[0], enc(rng, inter, k)[0]
    g_dev, u_dev = to_dev(g_blocks, device), to_dev(u_blocks, device)
    w_il = kernels.QWeight.from_blocks(kernels.interleave_gate_up(g_dev, u_dev, inter).reshape(-1), code, 2 * inter, k)
    act = kernels.qgemm_swiglu(xd, w_il, torch.float32).double().cpu().numpy()
    gw, uw = dec(g_blocks, k).astype(np.float64), dec(u_blocks, k).astype(np.float64)
    g, u = x64 @ gw.T, x64 @ uw.T
    sig = 1.0 / (1.0 + np.exp(-g))
    want = g * sig * u
    # g and u carry the exact-product bound of their fp32 sums; |d silu/dg| <= 1.1 carries it through
    bg = 1e-5 * (np.abs(x64) @ np.abs(gw).T) + 1e-6
    bu = 1e-5 * (np.abs(x64) @ np.abs(uw).T) + 1e-6
    bound = 1.1 * bg * np.abs(u) + np.abs(g * sig) * bu + 1e-5 * np.abs(want) + 1e-6
    assert np.all(np.abs(act - want) <= bound), np.abs(act - want).max()

    # fused greedy head: the chosen column's product is the row maximum up to fp32 summation (ties resolve to
    # the smallest column, so only rows whose top two products are apart are compared by id)
    ids = torch.empty(m, dtype=torch.int64, device=device)
    kernels.qgemm_argmax(xd, w, out=ids, workspace=kernels.qgemm_argmax_workspace(m, n, device))
    ids = ids.cpu().numpy()
    top2 = np.sort(ref64, axis=1)[:, -2:]
    slack = 1e-5 * (np.abs(x64) @ np.abs(wf).T).max(axis=1) + 1e-6
    assert np.all(ref64[np.arange(m), ids] >= top2[:, 1] - 2 * slack)
    clear = (top2[:, 1] - top2[:, 0]) > 2 * slack
    assert np.array_equal(ids[clear], ref64.argmax(axis=1)[clear])


@pytest.mark.parametrize("seed", range(8))
def test_qgemm_planner_random_shapes_row_formats(device, seed):
    """The same seeded sweep over the reference's per-row asymmetric int4/int8 packing (quantization.py; codes
    times activations on MFMA, scale and zero point applied after the k loop): partials through the planner's
    k-split and the fused greedy head, against fp64 on the dequantized weights within the fp16 bound."""
    from cacheir_amd import hip, kernels

    rng = np.random.default_rng(1900 + seed)
    bits = (4, 8)[seed % 2]
    code = hip.CIR_I4_ROW if bits == 4 else hip.CIR_I8_ROW
    m = int(rng.choice([1, 3, 8, 9, 16, 17, 32, 33, 64, 100, 128, 129, 200]))
    n = int(rng.integers(1, 321)) * 16 + int(rng.integers(0, 16))
    k = 128 * int(rng.integers(1, 65))
    splits = kernels.choose_splits(m, n, k)
    plans = (kernels.gemm_plan(hip.GEMM_PARTIALS, code, m, n, k, splits), kernels.gemm_plan(hip.GEMM_ARGMAX, code, m, n, k, 1))
    print(f"seed {seed}: int{bits} rows m={m} n={n} k={k} splits={splits} -> {' | '.join(plans)}", flush=True)
    assert "invalid" not in plans
    pk = quant.asymmetric_pack(rng.standard_normal((n, k)).astype(np.float32) * 0.05, bits)
    w = kernels.QWeight.from_rows(to_dev(pk["packed_values"], device), to_dev(pk["scales"], device),
                                  to_dev(pk["zero_points"], device), bits, n, k)
    wd = quant.asymmetric_dequant(pk).astype(np.float64)
    x = rng.standard_normal((m, k)).astype(np.float16)
    xd = to_dev(x, device)
    ref64 = x.astype(np.float64) @ wd.T
    got = kernels.qgemm_partial(xd, w, splits=splits).double().sum(0).cpu().numpy()
    close16(got, ref64)
    ids = torch.empty(m, dtype=torch.int64, device=device)
    kernels.qgemm_argmax(xd, w, out=ids, workspace=kernels.qgemm_argmax_workspace(m, n, device))
    ids = ids.cpu().numpy()
    top2 = np.sort(ref64, axis=1)[:, -2:]
    slack = ATOL16 + RTOL16 * np.abs(top2[:, 1])
    assert np.all(ref64[np.arange(m), ids] >= top2[:, 1] - 2 * slack)
    clear = (top2[:, 1] - top2[:, 0]) > 2 * slack
    assert np.array_equal(ids[clear], ref64.argmax(axis=1)[clear])


def test_gemm_f32(device):
    from cacheir_amd import kernels

    rng = np.random.default_rng(1)
    x = rng.standard_normal((16, 688)).astype(np.float32)
    w = rng.standard_normal((256, 688)).astype(np.float32)
    for splits in (1, 3):
        part = kernels.gemm_f32_partial(to_dev(x, device), to_dev(w, device), splits=splits)
        np.testing.assert_allclose(part.sum(0).cpu().numpy(), ops.matmul(x, w), rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ epilogues --
def test_epilogue_store_residual_and_swiglu(device):
    from cacheir_amd import kernels

    rng = np.random.default_rng(2)
    part = rng.standard_normal((3, 4, 64)).astype(np.float32)
    resid = rng.standard_normal((4, 64)).astype(np.float32)
    out = kernels.epilogue_store(to_dev(part, device), torch.float32, residual=to_dev(resid, device))
    np.testing.assert_allclose(out.cpu().numpy(), resid + part.sum(0), rtol=1e-6, atol=1e-6)
    sw = kernels.epilogue_swiglu(to_dev(part, device), torch.float32).cpu().numpy()
    tot = part.sum(0)
    np.testing.assert_allclose(sw, ops.silu_mul(tot[:, :32], tot[:, 32:]), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kvdt", [torch.float32, torch.float16])
def test_epilogue_qkv_rope_append(device, kvdt):
    from cacheir_amd import kernels

    rng = np.random.default_rng(4)
    batch, q_len, hq, hkv, d, psize = 2, 3, 4, 2, 64, 16
    n = (hq + 2 * hkv) * d
    part = rng.standard_normal((2, batch * q_len, n)).astype(np.float32)
    positions = np.array([0, 37], dtype=np.int32)
    pt = np.array([[5, 1, 0, 0], [2, 3, 4, 6]], dtype=np.int32)
    theta = 10000.0
    inv_freq = (1.0 / (theta ** (np.arange(0, d // 2, dtype=np.float32) * 2.0 / d))).astype(np.float32)
    kp = torch.zeros((8, hkv, psize, d), dtype=kvdt, device=device)
    vp = torch.zeros_like(kp)
    q_out = torch.empty((batch * q_len, hq * d), dtype=torch.float32, device=device)
    kernels.epilogue_qkv_rope_append(to_dev(part, device), to_dev(inv_freq, device), to_dev(positions, device),
                                     to_dev(pt, device), q_out, kp, vp, batch=batch, q_len=q_len, num_heads=hq,
                                     num_kv_heads=hkv, head_dim=d)
    tot = part.sum(0)
    kpn, vpn = kp.float().cpu().numpy(), vp.float().cpu().numpy()
    for b in range(batch):
        rows = tot[b * q_len:(b + 1) * q_len][None]
        q_ref = ops.rope_one(rows[..., :hq * d], d, theta, int(positions[b]))[0]
        k_ref = ops.rope_one(rows[..., hq * d:(hq + hkv) * d], d, theta, int(positions[b]))[0]
        v_ref = rows[0, :, (hq + hkv) * d:]
        np.testing.assert_allclose(q_out.cpu().numpy()[b * q_len:(b + 1) * q_len], q_ref, rtol=2e-5, atol=2e-5)
        for s in range(q_len):
            pos = int(positions[b]) + s
            slot, off = pt[b, pos // psize], pos % psize
            tol = 1e-3 if kvdt == torch.float16 else 2e-5
            np.testing.assert_allclose(kpn[slot, :, off].reshape(-1), k_ref[s], rtol=tol, atol=tol)
            np.testing.assert_allclose(vpn[slot, :, off].reshape(-1), v_ref[s], rtol=tol, atol=tol)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,hq,hkv,splits", [(32, 32, 8, 3), (2, 32, 8, 1), (5, 28, 4, 2), (3, 8, 8, 1),
                                                 (96, 28, 4, 2), (4, 32, 8, 12)])
def test_fused_qkv_decode_attention_matches_epilogue_then_attention(device, batch, hq, hkv, splits):
    """cir_paged_decode_attention_qkv == cir_epilogue_qkv_rope_append + cir_paged_decode_attention, bitwise:
    attention output and the pool contents (the appended k/v), incl. small batches that split the context,
    (96 rows x 4 KV heads: more workgroups than CUs) rows dispatched longest first, and 12 QKV splits (more than
    the kernel loads ahead of the first K/V block: the rest are loaded when summed)."""
    rng = np.random.default_rng(batch * 100 + hq)
    _fused_equals_two_kernels(device, rng, rng.integers(1, 700, batch), hq, hkv, splits, psize=16)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(8))
def test_fused_qkv_decode_attention_random_shapes(device, seed):
    """The same bitwise check over a seeded sweep: batch 1-40, GQA 1-8, 1-8 KV heads, 1-10 QKV splits, pages of
    16 or 32 tokens, contexts 1-600 with the new token on block and page edges (first token of a sequence, last of
    a tile or block, first of the next) so that it lands in every wavefront position, past-the-end tiles included."""
    rng = np.random.default_rng(2000 + seed)
    batch = int(rng.integers(1, 41))
    g, hkv = int(rng.integers(1, 9)), int(rng.choice([1, 2, 4, 8]))
    edges = np.array([1, 2, 16, 17, 31, 32, 33, 64, 65, 256, 257])
    lens = np.where(rng.random(batch) < 0.4, rng.choice(edges, batch), rng.integers(1, 601, batch))
    _fused_equals_two_kernels(device, rng, lens, g * hkv, hkv, int(rng.integers(1, 11)),
                              psize=int(rng.choice([16, 32])))


def _fused_equals_two_kernels(device, rng, lens, hq, hkv, splits, psize):
    from cacheir_amd import kernels

    d = 128
    batch = len(lens)
    lens = np.asarray(lens).astype(np.int32)                        # after the append
    positions = (lens - 1).astype(np.int32)
    pages = [-(-int(n) // psize) for n in lens]
    max_pages = max(pages) + 1
    slots = sum(pages) + 3
    perm = rng.permutation(slots).astype(np.int32)
    pt = np.zeros((batch, max_pages), np.int32)
    o = 0
    for b, n in enumerate(pages):
        pt[b, :n] = perm[o:o + n]
        o += n
    n_cols = (hq + 2 * hkv) * d
    part = rng.standard_normal((splits, batch, n_cols)).astype(np.float32)
    inv = (1.0 / (500000.0 ** (np.arange(0, d // 2, dtype=np.float32) * 2.0 / d))).astype(np.float32)
    kp0 = torch.randn((slots, hkv, psize, d), device=device).half()
    vp0 = torch.randn((slots, hkv, psize, d), device=device).half()
    P, I, POS, PT, L = (to_dev(a, device) for a in (part, inv, positions, pt, lens))

    kp1, vp1 = kp0.clone(), vp0.clone()
    q = torch.empty((batch, hq * d), dtype=torch.float16, device=device)
    kernels.epilogue_qkv_rope_append(P, I, POS, PT, q, kp1, vp1, batch=batch, q_len=1, num_heads=hq,
                                     num_kv_heads=hkv, head_dim=d)
    ref = kernels.paged_decode_attention(q.view(batch, hq, d), kp1, vp1, PT, L)

    kp2, vp2 = kp0.clone(), vp0.clone()
    got = kernels.paged_decode_attention_qkv(P, I, POS, kp2, vp2, PT, L, num_heads=hq, check_tables=True)
    torch.cuda.synchronize()
    assert torch.equal(kp2, kp1) and torch.equal(vp2, vp1), "appended K/V differ"
    assert torch.equal(got, ref), f"max |d| {(got.float() - ref.float()).abs().max().item()}"


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("lens,hq,hkv,want_s", [
    ([2048], 32, 8, 8), ([2048, 1700, 2048, 1300], 32, 8, 8), ([1500, 900, 1200, 1400, 1500, 1100, 800, 1000], 32, 8, 4),
    ([900, 600], 28, 4, 4), ([300], 32, 8, 2), ([1100], 32, 8, 5), ([1300, 20, 1], 32, 8, 6)])
def test_o_projection_from_attention_parts(device, fmt, lens, hq, hkv, want_s):
    """cir_paged_decode_attention_qkv_parts + cir_qgemm_attn (the O projection merging the attention's split
    partials while it stages its input), against
    * the oracle: RoPE(sum of the QKV partials) -> paged attention over the pool -> matmul with the decoded W_o,
      within the fp16 bound;
    * the merged path (cir_paged_decode_attention_qkv, then cir_qgemm on its fp16 output) bitwise, with the appended
      K/V bitwise too.
    Lengths are fixed so the split counts S = 2, 4, 5, 6 and 8 all run (S = 5 leaves 3 of the 8 partial slots
    masked)."""
    from cacheir_amd import kernels

    batch = len(lens)
    rng = np.random.default_rng(sum(lens) + hq + (fmt == "q8_0"))
    d, psize, theta = 128, 16, 500000.0
    lens = np.asarray(lens, np.int32)
    positions = (lens - 1).astype(np.int32)
    pages = [-(-int(n) // psize) for n in lens]
    max_pages = max(pages)
    slots = sum(pages) + 2
    perm = rng.permutation(slots).astype(np.int32)
    pt = np.zeros((batch, max_pages), np.int32)
    o = 0
    for b, n in enumerate(pages):
        pt[b, :n] = perm[o:o + n]
        o += n
    part = rng.standard_normal((2, batch, (hq + 2 * hkv) * d)).astype(np.float32)
    inv = (1.0 / (theta ** (np.arange(0, d // 2, dtype=np.float32) * 2.0 / d))).astype(np.float32)
    kp0 = torch.randn((slots, hkv, psize, d), device=device).half()
    vp0 = torch.randn((slots, hkv, psize, d), device=device).half()
    P, I, POS, PT, L = (to_dev(a, device) for a in (part, inv, positions, pt, lens))
    S = kernels.paged_decode_splits(batch, hq, hkv, d, psize, max_pages, torch.float16)
    assert S == want_s
    n = 4096
    enc = quant.random_q4_0 if fmt == "q4_0" else quant.random_q8_0
    blocks = enc(rng, n, hq * d)[0]
    w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), kernels.FMT_NAMES[fmt], n, hq * d)
    splits = kernels.choose_splits(batch, n, hq * d)

    kp1, vp1 = kp0.clone(), vp0.clone()
    attn = kernels.paged_decode_attention_qkv(P, I, POS, kp1, vp1, PT, L, num_heads=hq)
    ref = kernels.qgemm_partial(attn.view(batch, hq * d), w, splits=splits)

    kp2, vp2 = kp0.clone(), vp0.clone()
    ws = kernels.attention_workspace(batch, hq, d, max_pages * psize, device)
    got_s = kernels.paged_decode_attention_qkv_parts(P, I, POS, kp2, vp2, PT, L, num_heads=hq, workspace=ws)
    got = kernels.qgemm_attn(ws, got_s, hq, w, batch, splits=splits)
    torch.cuda.synchronize()
    assert got_s == S
    assert torch.equal(kp2, kp1) and torch.equal(vp2, vp1), "appended K/V differ"
    assert torch.equal(got, ref), f"max |d| {(got - ref).abs().max().item()}"

    # oracle: q = RoPE(sum of the q partials) at each row's position, attention over the pool as the call left it
    # (the appended K/V are checked against the oracle's RoPE in test_epilogue_qkv_rope_append): the attention the
    # O projection merged (bitwise the merged path's fp16 output, above) within the fp16 bound; then the
    # projection of that fp16 input with the decoded W_o within the bound (with Q8_0's |w| ~ 0.7, the fp16
    # rounding of the attention output alone moves outputs near zero past 2e-3, so W_o is applied to the
    # backend's own fp16 input, as the GEMM tests do)
    qsum = part.sum(axis=0)[:, : hq * d]
    q = np.concatenate([ops.rope_one(qsum[b][None, None], d, theta, int(positions[b])) for b in range(batch)])
    att = paged.paged_attention(q.reshape(batch, hq, d), kp2.float().cpu().numpy(), vp2.float().cpu().numpy(), pt,
                                lens, hq, hkv)
    close16(attn.float().cpu().numpy(), att)
    dec = quant.decode_q4_0(blocks, hq * d) if fmt == "q4_0" else quant.decode_q8_0(blocks, hq * d)
    close16(got.sum(dim=0).cpu().numpy(), ops.matmul(attn.float().cpu().numpy().reshape(batch, hq * d), dec))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m,k", [(1, 512), (8, 512), (32, 512), (48, 512), (100, 640), (128, 640), (200, 640),
                                 (1, 4096), (3, 4096), (8, 4096), (16, 4096), (32, 4096)])
def test_qgemm_swiglu_matches_gemm_then_epilogue(device, fmt, m, k):
    """cir_qgemm_swiglu over interleaved gate/up tiles == cir_qgemm (splits 1) + cir_epilogue_swiglu, bitwise,
    and within the fp16 bound of the fp64 oracle. At m <= 8 the reference side runs the GEMV (k = 4096 stages
    all of an 8-row activation in 64 KiB of LDS): with 32 quads or more the fused kernel sums two k-groups (even
    and odd quads) and then adds them, the GEMV sums the quads in order, so there the outputs agree to one fp16
    ulp (the fp32 sums differ in rounding only); with fewer quads, bit for bit.  m = 48, 100 and 128 run the
    balanced large-m SwiGLU (64- and 128-row blocks, a partly filled one at 100) against the large-m kernel's
    partials, m = 200 the large-m SwiGLU in 128-row blocks."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(11 + m + k)
    inter = 160 if m <= 32 else 2304  # m > 32: wide enough (n 4608) for the large-m kernel
    enc = quant.random_q4_0 if fmt == "q4_0" else quant.random_q8_0
    dec = quant.decode_q4_0 if fmt == "q4_0" else quant.decode_q8_0
    code = kernels.FMT_NAMES[fmt]
    gate, up = enc(rng, inter, k)[0], enc(rng, inter, k)[0]
    x = rng.standard_normal((m, k)).astype(np.float16)
    xd = to_dev(x, device)
    g_dev, u_dev = to_dev(gate, device), to_dev(up, device)
    w_cat = kernels.QWeight.from_blocks(torch.cat([g_dev.reshape(-1), u_dev.reshape(-1)]), code, 2 * inter, k)
    part = kernels.qgemm_partial(xd, w_cat, splits=1)
    ref = kernels.epilogue_swiglu(part, torch.float16)
    w_il = kernels.QWeight.from_blocks(kernels.interleave_gate_up(g_dev, u_dev, inter).reshape(-1), code, 2 * inter, k)
    got = kernels.qgemm_swiglu(xd, w_il, torch.float16)
    torch.cuda.synchronize()
    if m <= 8 and k // 128 >= 32:
        d = (got.float() - ref.float()).abs()
        assert torch.all(d <= ref.float().abs() * 2.0 ** -10 + 2.0 ** -24), d.max().item()
    else:
        assert torch.equal(got, ref)
    xf = x.astype(np.float64)
    g64, u64 = xf @ dec(gate, k).astype(np.float64).T, xf @ dec(up, k).astype(np.float64).T
    want = g64 / (1.0 + np.exp(-g64)) * u64
    err = np.abs(got.double().cpu().numpy() - want) - (2e-3 + 1e-2 * np.abs(want))
    assert np.all(err <= 0), err.max()


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
@pytest.mark.parametrize("m,inter", [(40, 17600), (128, 17600), (100, 5008), (128, 2304), (130, 17600)])
def test_qgemm_swiglu_large_m_column_runs(device, fmt, m, inter):
    """The fused SwiGLU at m > 32 over intermediate sizes that give each workgroup 4-5 gate/up pairs (17600: 1100
    pairs over 256 workgroups), 1-2 pairs (5008) and one (2304), with 64- and 128-row blocks and a second, partly
    filled row block at m = 130: bitwise equal to the partials of cir_qgemm (splits 1) + cir_epilogue_swiglu, and
    within the fp16 bound of the fp64 oracle on a sample of columns."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(m + inter)
    k = 512
    enc = quant.random_q4_0 if fmt == "q4_0" else quant.random_q8_0
    dec = quant.decode_q4_0 if fmt == "q4_0" else quant.decode_q8_0
    code = kernels.FMT_NAMES[fmt]
    gate, up = enc(rng, inter, k)[0], enc(rng, inter, k)[0]
    x = rng.standard_normal((m, k)).astype(np.float16)
    xd = to_dev(x, device)
    g_dev, u_dev = to_dev(gate, device), to_dev(up, device)
    w_cat = kernels.QWeight.from_blocks(torch.cat([g_dev.reshape(-1), u_dev.reshape(-1)]), code, 2 * inter, k)
    ref = kernels.epilogue_swiglu(kernels.qgemm_partial(xd, w_cat, splits=1), torch.float16)
    w_il = kernels.QWeight.from_blocks(kernels.interleave_gate_up(g_dev, u_dev, inter).reshape(-1), code, 2 * inter, k)
    got = kernels.qgemm_swiglu(xd, w_il, torch.float16)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    cols = np.unique(np.concatenate([np.arange(0, inter, 97), np.arange(inter - 40, inter)]))
    xf = x.astype(np.float64)
    g64 = xf @ dec(gate[cols], k).astype(np.float64).T
    u64 = xf @ dec(up[cols], k).astype(np.float64).T
    want = g64 / (1.0 + np.exp(-g64)) * u64
    err = np.abs(got.double().cpu().numpy()[:, cols] - want) - (2e-3 + 1e-2 * np.abs(want))
    assert np.all(err <= 0), err.max()


@pytest.mark.gpu
@pytest.mark.parametrize("proj,n,k", [("qkv", 4608, 3584), ("down", 3584, 18944), ("gate_up", 18944, 3584)])
def test_config5_projections_full_size(device, proj, n, k):
    """BASELINE config 5's Q8_0 projections at batch 128, full Qwen2-7B shapes: QKV (the large-m kernel), down
    (the large-m kernel over 9 k-splits of 17 quads, the last 12) and gate|up with the fused SwiGLU, against the
    dequantized oracle.  Scales are |N(0, 5e-4)| so that int8 codes give weights of config 3's size (RMS ~0.03);
    with config 3's 0.01, |g| and |u| reach ~150 and fp32 accumulation alone moves silu(g) * u by ~2e-3."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(13)
    m = 128
    code = kernels.FMT_NAMES["q8_0"]
    x = rng.standard_normal((m, k)).astype(np.float16)
    xd = to_dev(x, device)
    xf = x.astype(np.float32)
    if proj != "gate_up":
        blocks = quant.random_q8_0(rng, n, k, scale_sigma=5e-4)[0]
        w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), code, n, k)
        got = kernels.qgemm_partial(xd, w).sum(0).cpu().numpy()
        close16(got, ops.matmul(xf, quant.decode_q8_0(blocks, k)))
        return
    gate, up = quant.random_q8_0(rng, n, k, scale_sigma=5e-4)[0], quant.random_q8_0(rng, n, k, scale_sigma=5e-4)[0]
    w_il = kernels.QWeight.from_blocks(kernels.interleave_gate_up(to_dev(gate, device), to_dev(up, device), n)
                                       .reshape(-1), code, 2 * n, k)
    got = kernels.qgemm_swiglu(xd, w_il, torch.float16).float().cpu().numpy()
    x64 = x.astype(np.float64)
    g = ops.matmul(x64, quant.decode_q8_0(gate, k).astype(np.float64))
    u = ops.matmul(x64, quant.decode_q8_0(up, k).astype(np.float64))
    close16(got, g / (1.0 + np.exp(-g)) * u)


def _shared_prefix_case(device, rng, batch, prefix_pages, suffix_lo, suffix_hi, hkv=4, d=128, psize=16):
    """BASELINE config 5 layout: every sequence's first ``prefix_pages`` pages are the same slots; suffix pages
    are distinct and permuted.  Returns pools (torch fp16), page table, lengths and the slot count."""
    suffix = rng.integers(suffix_lo, suffix_hi + 1, batch)
    lens = prefix_pages * psize + suffix
    spages = -(-suffix // psize)
    slots = prefix_pages + int(spages.sum())
    perm = rng.permutation(slots).astype(np.int32)
    shared = perm[:prefix_pages]
    max_pages = prefix_pages + int(spages.max())
    pt = np.zeros((batch, max_pages), np.int32)
    o = prefix_pages
    for b in range(batch):
        pt[b, :prefix_pages] = shared
        pt[b, prefix_pages:prefix_pages + spages[b]] = perm[o:o + spages[b]]
        o += spages[b]
    kp = torch.randn((slots, hkv, psize, d), device=device).half()
    vp = torch.randn((slots, hkv, psize, d), device=device).half()
    return kp, vp, pt, lens.astype(np.int32), slots


@pytest.mark.gpu
def test_config5_shared_prefix_attention_matches_oracle(device):
    """Qwen2-7B heads (28 query / 4 KV, GQA 7), batch 128, all sequences share a 64-page (1024-token) prefix
    held once in the pool; suffixes 64..1024 tokens here so the oracle finishes quickly."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(5)
    kp, vp, pt, lens, _ = _shared_prefix_case(device, rng, 128, 64, 64, 1024)
    q = rng.standard_normal((128, 28, 128)).astype(np.float16)
    got = kernels.paged_decode_attention(to_dev(q, device), kp, vp, to_dev(pt, device), to_dev(lens, device),
                                         check_tables=True).float().cpu().numpy()
    ref = paged.paged_attention(q, kp.cpu().numpy(), vp.cpu().numpy(), pt, lens, 28, 4)
    err = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert np.all(err <= 0), err.max()


@pytest.mark.gpu
def test_config5_full_size_aliasing_is_transparent(device):
    """Full config-5 attention shape (batch 128, 1024-token shared prefix, suffixes 64..7168): reading the prefix
    through aliased page-table entries gives bitwise the result of private copies of the prefix pages, and the
    shortest/longest rows match the oracle."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(7)
    kp, vp, pt, lens, slots = _shared_prefix_case(device, rng, 128, 64, 64, 7168)
    q = to_dev(rng.standard_normal((128, 28, 128)).astype(np.float16), device)
    got = kernels.paged_decode_attention(q, kp, vp, to_dev(pt, device), to_dev(lens, device), check_tables=True)
    # de-alias: every row gets its own copy of the 64 prefix pages
    shared = pt[0, :64].copy()
    pt2 = pt.copy()
    extra = slots + np.arange(128 * 64, dtype=np.int32).reshape(128, 64)
    pt2[:, :64] = extra
    idx = torch.from_numpy(np.tile(shared, 128).astype(np.int64)).to(device)
    kp2 = torch.cat([kp, kp.index_select(0, idx)])
    vp2 = torch.cat([vp, vp.index_select(0, idx)])
    got2 = kernels.paged_decode_attention(q, kp2, vp2, to_dev(pt2, device), to_dev(lens, device), check_tables=True)
    torch.cuda.synchronize()
    assert torch.equal(got, got2)
    qn = q.cpu().numpy()
    for b in (int(np.argmin(lens)), int(np.argmax(lens))):
        n_pages = -(-int(lens[b]) // 16)
        sl = torch.from_numpy(pt[b, :n_pages].astype(np.int64)).to(device)
        kb, vb = kp.index_select(0, sl).cpu().numpy(), vp.index_select(0, sl).cpu().numpy()
        ref = paged.paged_attention(qn[b:b + 1], kb, vb, np.arange(n_pages, dtype=np.int32)[None], lens[b:b + 1], 28, 4)
        err = np.abs(got[b:b + 1].float().cpu().numpy() - ref) - (2e-3 + 1e-2 * np.abs(ref))
        assert np.all(err <= 0), (b, err.max())


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_row_packed_dequant_bit_exact_and_gemm(device, bits):
    """The reference's per-row asymmetric int4/int8 packing through cir_qweight_repack_rows: dequant equals
    quantization.py's (q - zp) * scale bit for bit; the GEMM is within the fp16 bound of fp64 on those weights."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(bits)
    n, k = 200, 384  # n not a multiple of 16
    w = rng.standard_normal((n, k)).astype(np.float32) * 0.05
    w[0] = np.abs(w[0]) + 0.01
    pk = quant.asymmetric_pack(w, bits)
    qw = kernels.QWeight.from_rows(to_dev(pk["packed_values"], device), to_dev(pk["scales"], device),
                                   to_dev(pk["zero_points"], device), bits, n, k)
    deq = quant.asymmetric_dequant(pk)
    got = kernels.dequant_tiled(qw).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), deq.astype(np.float32).view(np.uint32))
    for m in (1, 8, 32, 64, 128):
        x = rng.standard_normal((m, k)).astype(np.float16)
        for splits in (1, 3):
            y = kernels.qgemm_partial(to_dev(x, device), qw, splits=splits).sum(0).double().cpu().numpy()
            ref = x.astype(np.float64) @ deq.astype(np.float64).T
            err = np.abs(y - ref) - (2e-3 + 1e-2 * np.abs(ref))
            assert np.all(err <= 0), (m, splits, err.max())
    # n 4608 at m 128: the large-m kernel (row scales after the k loop, activation sums by MFMA)
    n2, k2 = 4608, 256
    w2 = rng.standard_normal((n2, k2)).astype(np.float32) * 0.05
    pk2 = quant.asymmetric_pack(w2, bits)
    qw2 = kernels.QWeight.from_rows(to_dev(pk2["packed_values"], device), to_dev(pk2["scales"], device),
                                    to_dev(pk2["zero_points"], device), bits, n2, k2)
    x2 = rng.standard_normal((128, k2)).astype(np.float16)
    y2 = kernels.qgemm_partial(to_dev(x2, device), qw2).sum(0).double().cpu().numpy()
    ref2 = x2.astype(np.float64) @ quant.asymmetric_dequant(pk2).astype(np.float64).T
    assert np.all(np.abs(y2 - ref2) - (2e-3 + 1e-2 * np.abs(ref2)) <= 0)


@pytest.mark.parametrize("splits", [1, 3, 8, 9, 16])
@pytest.mark.parametrize("n", [256, 3584, 4096, 5120])
def test_residual_rmsnorm_epilogue(device, splits, n):
    """cir_epilogue_residual_rmsnorm: h = residual + the split partials summed in split order (fp32, bit for bit
    against the same order in numpy), xn = RMSNorm(h) * w against the oracle, fp32 and fp16 outputs.  Covers 1-16
    splits (the 16-split variant serves the 9 of the large-m down projection) and rows past 4096 (a second column
    group per thread)."""
    from cacheir_amd import kernels

    rng = np.random.default_rng(splits * 10000 + n)
    m = 5
    part = rng.standard_normal((splits, m, n)).astype(np.float32)
    resid = rng.standard_normal((m, n)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float16)
    p = part[0].copy()
    for s_ in range(1, splits):
        p = p + part[s_]
    h_want = resid + p
    for odt in (torch.float32, torch.float16):
        h = torch.empty((m, n), device=device, dtype=torch.float32)
        xn = torch.empty((m, n), device=device, dtype=odt)
        kernels.epilogue_residual_rmsnorm(to_dev(part, device), to_dev(resid, device), to_dev(w, device), 1e-5, h, xn)
        assert np.array_equal(h.cpu().numpy().view(np.uint32), h_want.view(np.uint32))
        want = ops.rms_norm(h_want, w.astype(np.float32), 1e-5)
        if odt == torch.float32:
            np.testing.assert_allclose(xn.cpu().numpy(), want, rtol=1e-5, atol=1e-5)
        else:
            close16(xn.float().cpu().numpy(), want)


def test_row_kernels(device):
    from cacheir_amd import kernels

    rng = np.random.default_rng(8)
    # reference fixed-input RMSNorm case (tests/test_advanced_experiments.py:443-447)
    x = (np.arange(24, dtype=np.float32).reshape(3, 8) / 10.0).astype(np.float32)
    y = kernels.rmsnorm(to_dev(x, device), to_dev(np.ones(8, np.float32), device), 1e-6, torch.float32).cpu().numpy()
    np.testing.assert_allclose(y, x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6), rtol=1e-5, atol=1e-6)
    xx = rng.standard_normal((5, 4096)).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float16)
    y16 = kernels.rmsnorm(to_dev(xx, device), to_dev(w, device), 1e-5, torch.float16).float().cpu().numpy()
    close16(y16, ops.rms_norm(xx, w.astype(np.float32), 1e-5))
    table = rng.standard_normal((50, 16)).astype(np.float16)
    ids = np.array([3, 0, 49, 7], dtype=np.int64)
    emb = kernels.embedding(to_dev(ids, device), to_dev(table, device), torch.float32).cpu().numpy()
    assert np.array_equal(emb, table[ids].astype(np.float32))
    # 4-value accesses (hidden % 4 == 0, rows past one unrolled pass) and the one-value path (hidden 4099), every
    # table/output dtype pair, bit for bit
    for hidden in (4096, 5120, 4099):
        tab = rng.standard_normal((64, hidden)).astype(np.float32)
        ids = rng.integers(0, 64, 9).astype(np.int64)
        for tdt in (torch.float16, torch.float32):
            t = to_dev(tab, device).to(tdt)
            ref = t.cpu()[torch.from_numpy(ids)]
            for odt in (torch.float16, torch.float32):
                got = kernels.embedding(to_dev(ids, device), t, odt).cpu()
                assert torch.equal(got, ref.to(odt)), (hidden, tdt, odt)
    logits = rng.standard_normal((3, 1000)).astype(np.float32)
    logits[1, 10] = logits[1, 20] = 50.0  # tie -> first index
    got = kernels.argmax(to_dev(logits, device)).cpu().numpy()
    assert np.array_equal(got, ops.greedy(logits, 1000))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["q4_0", "q8_0", "i4_row", "i8_row"])
@pytest.mark.parametrize("m,k", [(1, 256), (5, 256), (8, 256), (16, 256), (17, 256), (32, 256), (2, 4096), (8, 4096),
                                 (40, 256), (130, 384)])
def test_qgemm_argmax_matches_gemm_then_argmax(device, fmt, m, k):
    """cir_qgemm_argmax (LM head + greedy argmax, no logits stored) == the oracle's greedy pick over the logits
    of cir_qgemm (splits 1): bitwise the same ids, with a planted tie between a near and a far column (first
    index wins), a row of NaN logits (numpy picks the first NaN, index 0) and a ragged vocabulary. Block formats
    at m <= 8 run the GEMV's argmax epilogue, m <= 32 the small GEMM's, and m > 32 over 37 column groups the
    large-m GEMM's (64- and 128-row blocks, a ragged last block at m = 130)."""
    from cacheir_amd import hip, kernels

    rng = np.random.default_rng(17 * m + len(fmt) + k)
    n = 1000 if m <= 32 else 4610  # not a multiple of the 32- or 64-column wavefront groups
    if fmt in ("q4_0", "q8_0"):
        enc = quant.random_q4_0 if fmt == "q4_0" else quant.random_q8_0
        blocks = enc(rng, n, k)[0].reshape(n, -1)
        # rows 3 and n-2: identical and dominant for positive x
        bb = 18 if fmt == "q4_0" else 34
        dom = np.zeros((k // 32, bb), np.uint8)
        dom[:, :2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
        dom[:, 2:] = 0xFF if fmt == "q4_0" else 0x7F
        blocks[3] = blocks[n - 2] = dom.reshape(-1)
        w = kernels.QWeight.from_blocks(to_dev(blocks.reshape(-1), device), kernels.FMT_NAMES[fmt], n, k)
    else:
        bits = 4 if fmt == "i4_row" else 8
        wf = rng.standard_normal((n, k)).astype(np.float32) * 0.05
        wf[3] = wf[n - 2] = np.linspace(0.4, 0.6, k, dtype=np.float32)
        pk = quant.asymmetric_pack(wf, bits)
        w = kernels.QWeight.from_rows(to_dev(pk["packed_values"], device), to_dev(pk["scales"], device),
                                      to_dev(pk["zero_points"], device), bits, n, k)
    if m > 32:
        assert kernels.gemm_plan(hip.GEMM_ARGMAX, w.fmt, m, n, k).startswith("qgemm_xl_kernel")
    x = np.abs(rng.standard_normal((m, k))).astype(np.float16)
    if m > 2:
        x[1] = rng.standard_normal(k).astype(np.float16)  # a row with an ordinary (random) winner
    if m > 4:
        x[4, 7] = np.float16(np.nan)  # every logit of row 4 is NaN
    xd = to_dev(x, device)
    logits = kernels.qgemm_partial(xd, w, splits=1)[0]
    want = ops.greedy(logits.cpu().numpy(), n)
    got = kernels.qgemm_argmax(xd, w).cpu().numpy()
    assert np.array_equal(got, want), (got, want)
    assert got[0] == 3  # tie between columns 3 and n-2 goes to the first
    if m > 4:
        assert got[4] == 0
    # the fused kernel's ids also equal cir_argmax over the same logits
    assert np.array_equal(kernels.argmax(logits).cpu().numpy(), want)


def test_stream_read_calibration_runs(device):
    """cir_stream_read (the bench's read ceiling) reads a buffer in both layouts and leaves its output alone."""
    from cacheir_amd import kernels

    buf = torch.arange(1 << 20, dtype=torch.int32, device=device)
    out = torch.zeros(1, dtype=torch.int32, device=device)
    for layout in (0, 1):
        for wgs, threads in ((224, 256), (1024, 512), (7, 64)):
            kernels.stream_read(buf, wgs, threads, layout, out)
            kernels.stream_read(buf, wgs, threads, layout, out, side=buf[: 1 << 16], side_ratio=3)
    torch.cuda.synchronize()
    assert int(out.item()) == 0
    with pytest.raises(Exception):
        kernels.stream_read(buf, 0, 256, 0, out)
    with pytest.raises(Exception):  # the side buffer must hold a power of two of 16-byte chunks
        kernels.stream_read(buf, 224, 256, 0, out, side=buf[:1000], side_ratio=2)
