"""ctypes bridge to the C/OpenMP oracle (``oracle/c/oracle_cpu.c``) and the timed
CPU baseline of one decode step -- TEST INFRASTRUCTURE ONLY.

``time_decode_step`` runs one Llama decoder layer for the whole batch (RMSNorm,
Q4_0 Q|K|V GEMM, RoPE, KV append, paged attention over fp16 pages, O GEMM +
residual, RMSNorm, gate|up GEMM, SiLU-mul, down GEMM + residual) plus the final
norm, lm_head GEMM and argmax, on random inputs of the workload's shapes, and scales
the layer time by the layer count: cpu_step = layers * t_layer + t_head.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_AVX2 = HERE / "_lib" / "liboracle_cpu.so"
LIB_AVX512 = HERE / "_lib" / "liboracle_cpu_avx512.so"
_V4_FLAGS = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}  # what -march=x86-64-v4 assumes


def cpu_flags() -> set[str]:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("flags"):
                return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def library_path() -> Path:
    """The AVX-512 build when the host has every x86-64-v4 feature, else the AVX2 build."""
    return LIB_AVX512 if _V4_FLAGS <= cpu_flags() else LIB_AVX2


def host_info() -> dict:
    """Facts about the host the CPU baseline ran on: logical CPUs, the lscpu model name, the ISA build used."""
    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().lower().startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            for line in Path("/proc/cpuinfo").read_text().splitlines():
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "isa": _isa_name(_chosen or library_path())}


def _isa_name(path: Path) -> str:
    return "avx512 (x86-64-v4)" if path == LIB_AVX512 else "avx2+f16c (x86-64-v3)"


_chosen: Path | None = None  # the build time_decode_step picked on this host


def choose_fastest_build(m: int, n: int, k: int, log=print) -> dict:
    """Time one Q4_0 GEMM of [m, k] x [n, k] (best of 2) with each build this host can run and keep the faster
    for the rest of the process; returns {isa: seconds}."""
    global _lib, _chosen
    builds = [LIB_AVX2] + ([LIB_AVX512] if _V4_FLAGS <= cpu_flags() and LIB_AVX512.exists() else [])
    rng = np.random.default_rng(0)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = _rand_q4(rng, n, k)
    times = {}
    for path in builds:
        _lib, _chosen = None, path
        y = np.empty((m, n), np.float32)
        q4_0_gemm(x, w, n, out=y)  # warm-up
        best = min(_timed_once(lambda: q4_0_gemm(x, w, n, out=y)) for _ in range(2))
        times[_isa_name(path)] = best
    fastest = min(builds, key=lambda p: times[_isa_name(p)])
    _lib, _chosen = None, fastest
    log("cpu: build choice " + ", ".join(f"{k} {v * 1e3:.1f} ms" for k, v in times.items()) + f" -> {_isa_name(fastest)}")
    return times


def _timed_once(fn) -> float:
    t0 = time.perf_counter()
    fn()
    return time.perf_counter() - t0

_f = ctypes.POINTER(ctypes.c_float)
_u8 = ctypes.POINTER(ctypes.c_uint8)
_u16 = ctypes.POINTER(ctypes.c_uint16)
_i32 = ctypes.POINTER(ctypes.c_int)
_i64 = ctypes.POINTER(ctypes.c_int64)
_lib = None


def load():
    global _lib
    if _lib is None:
        path = _chosen or library_path()
        if not path.exists():
            subprocess.run(["make", "-s", "-C", str(HERE), "cpu"], check=True)
        lib = ctypes.CDLL(str(path))
        lib.orc_rmsnorm.argtypes = [_f, _f, _f, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        lib.orc_q4_0_gemm.argtypes = [_f, ctypes.c_int, ctypes.c_int, _u8, ctypes.c_int, _f, ctypes.c_int]
        lib.orc_rope.argtypes = [_f, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32, _f]
        lib.orc_kv_append.argtypes = [_f, _f, _u16, _u16, _i32, ctypes.c_int, _i32, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int]
        lib.orc_paged_attention.argtypes = [_f, _u16, _u16, _i32, ctypes.c_int, _i32, _f, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f, ctypes.c_int]
        lib.orc_silu_mul.argtypes = [_f, _f, ctypes.c_int, ctypes.c_int]
        lib.orc_argmax.argtypes = [_f, ctypes.c_int, ctypes.c_int, _i64]
        lib.orc_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def P(a, t):
    return a.ctypes.data_as(t)


def q4_0_gemm(x: np.ndarray, blocks: np.ndarray, n: int, out: np.ndarray | None = None, accumulate=False):
    lib = load()
    m, k = x.shape
    y = np.zeros((m, n), np.float32) if out is None else out
    lib.orc_q4_0_gemm(P(x, _f), m, k, P(blocks, _u8), n, P(y, _f), int(accumulate))
    return y


def paged_attention(q, kp, vp, pt, lens, num_heads, num_kv_heads):
    lib = load()
    b, hq, d = q.shape
    p = kp.shape[2]
    out = np.zeros_like(q, dtype=np.float32)
    max_ctx = int(pt.shape[1] * p)
    scratch = np.zeros((lib.orc_threads(), max_ctx), np.float32)
    lib.orc_paged_attention(P(np.ascontiguousarray(q, np.float32), _f), P(kp.view(np.uint16), _u16),
                            P(vp.view(np.uint16), _u16), P(np.ascontiguousarray(pt, np.int32), _i32), pt.shape[1],
                            P(np.ascontiguousarray(lens, np.int32), _i32), P(out, _f), b, hq, num_kv_heads, d, p,
                            float(1.0 / np.sqrt(d)), P(scratch, _f), max_ctx)
    return out


def _rand_q4(rng, n, k):
    nb = k // 32
    raw = rng.integers(0, 256, size=(n, nb, 18), dtype=np.uint8)
    d = np.abs(rng.normal(0, 0.01, size=(n, nb))).astype(np.float16).view(np.uint8).reshape(n, nb, 2)
    raw[:, :, :2] = d
    return raw.reshape(n, -1)


def time_decode_step(*, batch, ctx, hidden, ffn, heads, kv_heads, vocab, layers, budget_s=12.0, log=print) -> dict:
    build_times = choose_fastest_build(batch, 2 * ffn, hidden, log=log)
    lib = load()
    rng = np.random.default_rng(0)
    D, Pg = hidden // heads, 16
    kvd = kv_heads * D
    qkv = _rand_q4(rng, hidden + 2 * kvd, hidden)
    wo = _rand_q4(rng, hidden, hidden)
    gu = _rand_q4(rng, 2 * ffn, hidden)
    wd = _rand_q4(rng, hidden, ffn)
    head = _rand_q4(rng, vocab, hidden)
    norm = np.ones(hidden, np.float32)
    pages = -(-ctx // Pg)
    pt = np.arange(batch * pages, dtype=np.int32).reshape(batch, pages)
    kp = rng.standard_normal((batch * pages, kv_heads, Pg, D)).astype(np.float16)
    vp = rng.standard_normal((batch * pages, kv_heads, Pg, D)).astype(np.float16)
    x = rng.standard_normal((batch, hidden)).astype(np.float32)
    pos = np.full(batch, ctx - 1, np.int32)
    lens = pos + 1
    inv = (1.0 / (500000.0 ** (np.arange(0, D // 2, dtype=np.float32) * 2.0 / D))).astype(np.float32)
    h = np.empty_like(x)
    y_qkv = np.empty((batch, hidden + 2 * kvd), np.float32)
    attn = np.empty((batch, hidden), np.float32)
    y_gu = np.empty((batch, 2 * ffn), np.float32)
    act = np.empty((batch, ffn), np.float32)
    logits = np.empty((batch, vocab), np.float32)
    ids = np.empty(batch, np.int64)
    threads = lib.orc_threads()
    scratch = np.zeros((threads, pages * Pg), np.float32)

    def layer():
        lib.orc_rmsnorm(P(x, _f), P(norm, _f), P(h, _f), batch, hidden, 1e-5)
        lib.orc_q4_0_gemm(P(h, _f), batch, hidden, P(qkv, _u8), hidden + 2 * kvd, P(y_qkv, _f), 0)
        q = np.ascontiguousarray(y_qkv[:, :hidden])
        k = np.ascontiguousarray(y_qkv[:, hidden:hidden + kvd])
        v = np.ascontiguousarray(y_qkv[:, hidden + kvd:])
        lib.orc_rope(P(q, _f), batch, heads, D, P(pos, _i32), P(inv, _f))
        lib.orc_rope(P(k, _f), batch, kv_heads, D, P(pos, _i32), P(inv, _f))
        lib.orc_kv_append(P(k, _f), P(v, _f), P(kp.view(np.uint16), _u16), P(vp.view(np.uint16), _u16), P(pt, _i32),
                          pages, P(pos, _i32), batch, kv_heads, D, Pg)
        lib.orc_paged_attention(P(q, _f), P(kp.view(np.uint16), _u16), P(vp.view(np.uint16), _u16), P(pt, _i32),
                                pages, P(lens, _i32), P(attn, _f), batch, heads, kv_heads, D, Pg,
                                float(1.0 / np.sqrt(D)), P(scratch, _f), pages * Pg)
        lib.orc_q4_0_gemm(P(attn, _f), batch, hidden, P(wo, _u8), hidden, P(x, _f), 1)
        lib.orc_rmsnorm(P(x, _f), P(norm, _f), P(h, _f), batch, hidden, 1e-5)
        lib.orc_q4_0_gemm(P(h, _f), batch, hidden, P(gu, _u8), 2 * ffn, P(y_gu, _f), 0)
        lib.orc_silu_mul(P(y_gu, _f), P(act, _f), batch, ffn)
        lib.orc_q4_0_gemm(P(act, _f), batch, ffn, P(wd, _u8), hidden, P(x, _f), 1)

    def final():
        lib.orc_rmsnorm(P(x, _f), P(norm, _f), P(h, _f), batch, hidden, 1e-5)
        lib.orc_q4_0_gemm(P(h, _f), batch, hidden, P(head, _u8), vocab, P(logits, _f), 0)
        lib.orc_argmax(P(logits, _f), batch, vocab, P(ids, _i64))

    def timed(fn, budget):
        fn()  # warm-up
        t0, n = time.perf_counter(), 0
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget or n >= 20:
                return el / n, n

    t_layer, n_layer = timed(layer, budget_s * 0.7)
    t_head, n_head = timed(final, budget_s * 0.3)
    step = layers * t_layer + t_head
    log(f"cpu: layer {t_layer * 1e3:.1f} ms x{n_layer}, head {t_head * 1e3:.1f} ms x{n_head}, "
        f"step {step * 1e3:.1f} ms on {threads} threads")
    info = host_info()
    info["gate_up_gemm_ms_by_build"] = {k: round(v * 1e3, 2) for k, v in build_times.items()}
    return {"value": round(batch / step, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"one full decoder layer for all {batch} sequences ({n_layer} timed runs) + final norm/lm_head/"
                      f"argmax ({n_head} runs) at the bench shapes, step = {layers} x layer + head",
            "ms_per_step": round(step * 1e3, 2), **info,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "openmp_threads_used": threads,
            "blas_threads": "none (no BLAS: the C kernels are the whole computation)"}
