"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Each oracle function is checked against something other than its own formula:
the reference's golden vectors and fixed-input tests, the reference's compiled
C++ kernels (oracle/_ref, when built), brute force, or identities the
mathematics fixes.
"""
import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import ops, paged, quant

GOLDEN = Path(__file__).with_name("golden")
REF_LIB = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libcacheir_ref.so"


# ----------------------------------------------------------- GGUF blocks ------
def test_gguf_kat_vectors():
    kat = json.loads((GOLDEN / "gguf_kat.json").read_text())
    q8 = np.frombuffer(bytes.fromhex(kat["q8_0"]["block_hex"]), dtype=np.uint8)
    q4 = np.frombuffer(bytes.fromhex(kat["q4_0"]["block_hex"]), dtype=np.uint8)
    exp8 = np.array(kat["q8_0"]["expected"], dtype=np.float32)
    exp4 = np.array(kat["q4_0"]["expected"], dtype=np.float32)
    assert np.array_equal(quant.decode_q8_0(q8[None], 32)[0], exp8)
    assert np.array_equal(quant.decode_q8_0_loop(q8.tobytes(), 32), exp8)
    assert np.array_equal(quant.decode_q4_0(q4[None], 32)[0], exp4)
    assert np.array_equal(quant.decode_q4_0_loop(q4.tobytes(), 32), exp4)


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_block_decode_vectorised_matches_loop_and_closed_form(fmt):
    rng = np.random.default_rng(0)
    n, k = 7, 96
    if fmt == "q4_0":
        blocks, nib, d = quant.random_q4_0(rng, n, k)
        vec = quant.decode_q4_0(blocks, k)
        loop = quant.decode_q4_0_loop(blocks.tobytes(), n * k).reshape(n, k)
        closed = (nib.astype(np.float64) - 8.0) * np.repeat(d.astype(np.float64), 32, axis=1)
    else:
        blocks, q, d = quant.random_q8_0(rng, n, k)
        vec = quant.decode_q8_0(blocks, k)
        loop = quant.decode_q8_0_loop(blocks.tobytes(), n * k).reshape(n, k)
        closed = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32, axis=1)
    assert np.array_equal(vec, loop)
    # products are exact in fp32 (<= 15 / 19 significant bits), so the fp64 closed form agrees bit for bit
    assert np.array_equal(vec.astype(np.float64), closed)


def test_q4_0_nibble_placement_roundtrip():
    """Element j sits in the low nibble of byte j, element j+16 in its high nibble (gguf.py:258-261,305-308)."""
    nib = np.tile(np.arange(32, dtype=np.uint8) % 16, (2, 1))
    nib[1] = np.arange(31, -1, -1) % 16
    d = np.ones((2, 1), dtype=np.float16)
    blocks = quant.encode_q4_0(nib, d)
    assert blocks[0, 2] == (0 | (0 << 4))  # element 0 low, element 16 (=0) high
    assert blocks[0, 3] == (1 | (1 << 4))
    dec = quant.decode_q4_0(blocks, 32)
    assert np.array_equal(dec + 8, nib.astype(np.float32))


def test_asymmetric_pack_reference_case():
    """tests/test_project_surfaces.py:73-82 shapes and int8 round trip."""
    w = np.linspace(-1.5, 2.0, num=30, dtype=np.float32).reshape(3, 10)
    q4 = quant.asymmetric_pack(w, 4)
    q8 = quant.asymmetric_pack(w, 8)
    assert q4["packed_values"].shape == (3, 5)
    assert q8["packed_values"].shape == w.shape
    assert q4["zero_points"].shape == (3,)
    np.testing.assert_allclose(quant.asymmetric_dequant(q8), w, rtol=0.02, atol=0.02)
    # int4 error is bounded by half a quantisation step per row
    step = q4["scales"][:, None]
    assert np.all(np.abs(quant.asymmetric_dequant(q4) - w) <= 0.5 * step + 1e-6)


# ----------------------------------------------------------- CPU ops ----------
def test_rms_norm_and_matmul_reference_fixed_inputs():
    """tests/test_advanced_experiments.py:440-452 inputs and closed forms."""
    x = (np.arange(24, dtype=np.float32).reshape(1, 3, 8) / 10.0).astype(np.float32)
    y = ops.rms_norm(x, np.ones(8, np.float32), 1e-6)
    np.testing.assert_allclose(y, x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6), rtol=1e-5, atol=1e-6)
    w = (np.arange(32, dtype=np.float32).reshape(4, 8) / 100.0).astype(np.float32)
    z = ops.matmul(x, w)
    brute = np.array([[[sum(float(x[0, s, i]) * float(w[o, i]) for i in range(8)) for o in range(4)] for s in range(3)]])
    np.testing.assert_allclose(z, brute, rtol=1e-5, atol=1e-6)


def test_silu_mul_reference_inputs():
    """tests/test_runtime.py:34-41 inputs; compared with float64 logistic form."""
    gate = np.linspace(-3.0, 3.0, num=24, dtype=np.float32).reshape(2, 3, 4)
    up = np.linspace(0.5, 2.0, num=24, dtype=np.float32).reshape(2, 3, 4)
    g = gate.astype(np.float64)
    np.testing.assert_allclose(ops.silu_mul(gate, up), g * (1 / (1 + np.exp(-g))) * up, rtol=1e-6, atol=1e-6)


@pytest.mark.skipif(not REF_LIB.exists(), reason="oracle/_ref not built (reference sources absent)")
def test_oracle_matches_reference_cpp_kernels():
    lib = ctypes.CDLL(str(REF_LIB))
    fp = ctypes.POINTER(ctypes.c_float)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 64)).astype(np.float32)
    w = rng.standard_normal(64).astype(np.float32)
    out = np.empty_like(x)
    assert lib.cir_ref_rms_norm(x.ctypes.data_as(fp), w.ctypes.data_as(fp), out.ctypes.data_as(fp),
                                ctypes.c_size_t(2), ctypes.c_size_t(3), ctypes.c_size_t(64), ctypes.c_float(1e-5)) == 0
    np.testing.assert_allclose(ops.rms_norm(x, w, 1e-5), out, rtol=2e-6, atol=2e-6)
    g = rng.standard_normal(100).astype(np.float32)
    u = rng.standard_normal(100).astype(np.float32)
    o2 = np.empty_like(g)
    assert lib.cir_ref_silu_mul(g.ctypes.data_as(fp), u.ctypes.data_as(fp), o2.ctypes.data_as(fp), ctypes.c_size_t(100)) == 0
    np.testing.assert_allclose(ops.silu_mul(g, u), o2, rtol=1e-6, atol=1e-6)
    wm = rng.standard_normal((48, 64)).astype(np.float32)
    o3 = np.empty((2, 3, 48), dtype=np.float32)
    assert lib.cir_ref_matmul_out_in(x.ctypes.data_as(fp), wm.ctypes.data_as(fp), o3.ctypes.data_as(fp),
                                     ctypes.c_size_t(2), ctypes.c_size_t(3), ctypes.c_size_t(64), ctypes.c_size_t(48)) == 0
    np.testing.assert_allclose(ops.matmul(x, wm), o3, rtol=1e-4, atol=1e-4)


def test_rope_properties():
    """Interleaved RoPE is pinned by identities, not by re-typing cpu.py:324-340."""
    rng = np.random.default_rng(2)
    d, theta = 16, 10000.0
    x = rng.standard_normal((1, 1, 2 * d)).astype(np.float32)
    # position 0 is the identity
    np.testing.assert_array_equal(ops.rope_one(x, d, theta, 0), x)
    # pair (x[2i], x[2i+1]) is a complex number rotated by pos * theta^(-2i/d)
    pos = 37
    got = ops.rope_one(x, d, theta, pos).reshape(2, d // 2, 2)
    z = x.reshape(2, d // 2, 2).astype(np.float64)
    zc = z[..., 0] + 1j * z[..., 1]
    freq = theta ** (-2.0 * np.arange(d // 2) / d)
    expect = zc * np.exp(1j * pos * freq)
    np.testing.assert_allclose(got[..., 0], expect.real, rtol=2e-4, atol=2e-4)
    np.testing.assert_allclose(got[..., 1], expect.imag, rtol=2e-4, atol=2e-4)
    # norms preserved per pair; rotations compose (a then b == a+b)
    np.testing.assert_allclose(np.abs(got[..., 0] + 1j * got[..., 1]), np.abs(zc), rtol=1e-5)
    a = ops.rope_one(ops.rope_one(x, d, theta, 5), d, theta, 7)
    np.testing.assert_allclose(a, ops.rope_one(x, d, theta, 12), rtol=1e-5, atol=1e-5)
    # a rotate-half convention would mix x[i] with x[i + d/2]; interleaved leaves other pairs alone
    e = np.zeros((1, 1, d), dtype=np.float32)
    e[0, 0, 2] = 1.0
    r = ops.rope_one(e, d, theta, 3)[0, 0]
    assert np.count_nonzero(r) == 2 and r[2] != 0 and r[3] != 0


# ----------------------------------------------------------- paged KV ---------
def test_extend_pages_reference_case():
    """kv_cache.py:110-122 / tests/test_advanced_experiments.py:170-176: 3 tokens, P=2."""
    pages: list[dict] = []
    nxt = paged.extend_pages(pages, 0, 3, 2, 0)
    assert nxt == 2 and [(p["start"], p["length"]) for p in pages] == [(0, 2), (2, 1)]
    nxt = paged.extend_pages(pages, 3, 1, 2, nxt)  # fills the partial page, no new id
    assert nxt == 2 and pages[-1]["length"] == 2
    nxt = paged.extend_pages(pages, 4, 1, 2, nxt)
    assert nxt == 3 and pages[-1]["start"] == 4


def test_paged_gather_equals_contiguous_and_permutation_invariance():
    rng = np.random.default_rng(3)
    ctx = [5, 33, 16]
    kp, vp, pt, lens = paged.build_pool(rng, ctx, 2, 8, 4, dtype=np.float32)
    contiguous = [paged.gather_sequence(kp, pt[b], ctx[b]) for b in range(3)]
    for b in range(3):
        for t in range(ctx[b]):
            assert np.array_equal(contiguous[b][t], kp[pt[b, t // 4], :, t % 4])
    q = rng.standard_normal((3, 4, 8)).astype(np.float32)
    out = paged.paged_attention(q, kp, vp, pt, lens, 4, 2)
    # relabel slots: same outputs
    perm = rng.permutation(kp.shape[0])
    inv = np.argsort(perm)
    out2 = paged.paged_attention(q, kp[perm], vp[perm], inv[pt].astype(np.int32), lens, 4, 2)
    np.testing.assert_allclose(out, out2, rtol=1e-6, atol=1e-6)


def test_paged_attention_matches_brute_force_and_limits():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((2, 4, 8)).astype(np.float32)
    kp = rng.standard_normal((5, 2, 2, 8)).astype(np.float32)
    vp = rng.standard_normal((5, 2, 2, 8)).astype(np.float32)
    pt = np.array([[0, 1, 2], [3, 4, 0]], dtype=np.int32)
    lens = np.array([5, 3], dtype=np.int32)
    np.testing.assert_allclose(paged.paged_attention(q, kp, vp, pt, lens, 4, 2),
                               paged.brute_force_attention(q, kp, vp, pt, lens, 4, 2), rtol=1e-5, atol=1e-5)
    # one visible token -> that token's V exactly; identical keys -> mean of V
    one = paged.paged_attention(q, kp, vp, pt, np.array([1, 1], np.int32), 4, 2)
    assert np.allclose(one[0, 0], vp[0, 0, 0]) and np.allclose(one[1, 3], vp[3, 1, 0])
    kz = np.zeros_like(kp)
    mean = paged.paged_attention(q, kz, vp, pt, lens, 4, 2)
    np.testing.assert_allclose(mean[0, 0], np.mean([vp[pt[0, t // 2], 0, t % 2] for t in range(5)], axis=0), rtol=1e-5)


def test_softmax_attention_causal_mask():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((1, 3, 2, 4)).astype(np.float32)
    k = rng.standard_normal((1, 3, 1, 4)).astype(np.float32)
    v = rng.standard_normal((1, 3, 1, 4)).astype(np.float32)
    out = ops.attention(q, k, v, 2, 1, 4, causal=True).reshape(3, 2, 4)
    # first query sees only the first key
    np.testing.assert_allclose(out[0, 0], v[0, 0, 0], rtol=1e-6)
    np.testing.assert_allclose(out[0, 1], v[0, 0, 0], rtol=1e-6)
