"""The C/OpenMP restatement timed as bench.py's CPU baseline computes what the NumPy oracle computes.

Both builds (AVX2 + F16C and AVX-512) are checked when the host can run them: the Q4_0 GEMM (with and without the
residual accumulate) against the oracle's exact dequant followed by a float64 matmul, and the paged attention over
fp16 pages against ``oracle.paged.paged_attention``, at shapes the oracle finishes in milliseconds.
"""
import ctypes

import numpy as np
import pytest

from oracle import cbase, paged
from oracle import quant as oq


def _libs():
    libs = [cbase.LIB_AVX2]
    if cbase._V4_FLAGS <= cbase.cpu_flags():
        libs.append(cbase.LIB_AVX512)
    return libs


@pytest.mark.parametrize("path", _libs(), ids=lambda p: p.name)
def test_c_baseline_matches_the_numpy_oracle(path, monkeypatch):
    if not path.exists():
        pytest.skip("C oracle not built (make -C oracle cpu)")
    monkeypatch.setattr(cbase, "_lib", None)
    monkeypatch.setattr(cbase, "library_path", lambda: path)
    rng = np.random.default_rng(3)
    m, k, n = 5, 256, 48
    blocks = oq.random_q4_0(rng, n, k)[0]
    x = rng.standard_normal((m, k)).astype(np.float32)
    ref = x.astype(np.float64) @ oq.decode_q4_0(blocks, k).astype(np.float64).T
    y = cbase.q4_0_gemm(x, blocks, n)
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)
    base = rng.standard_normal((m, n)).astype(np.float32)
    y2 = cbase.q4_0_gemm(x, blocks, n, out=base.copy(), accumulate=True)
    np.testing.assert_allclose(y2, base + ref, rtol=1e-5, atol=1e-5)

    kp, vp, pt, lens = paged.build_pool(rng, [1, 37, 300], 2, 128, 16)
    q = rng.standard_normal((3, 8, 128)).astype(np.float32)
    got = cbase.paged_attention(q, kp, vp, pt, lens, 8, 2)
    np.testing.assert_allclose(got, paged.paged_attention(q, kp, vp, pt, lens, 8, 2), rtol=1e-5, atol=1e-5)
    assert isinstance(cbase.load(), ctypes.CDLL)


def test_host_info_names_the_build():
    info = cbase.host_info()
    assert info["os_cpu_count"] >= 1 and info["isa"].startswith(("avx512", "avx2"))
