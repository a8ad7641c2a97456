"""Decode-step benchmark for the MI355X backend (BASELINE.json metric).

Workload (one GPU): Llama-3-8B-shaped decoder -- 32 layers, hidden
4096, 32 query / 8 KV heads (head_dim 128), SwiGLU ffn 14336, vocab 128256, every
linear weight (QKV, O, gate, up, down, lm_head) Q4_0 blocks, norms and embeddings
fp16, random-init weights generated on the device.  Batch 32, every sequence at 2048
tokens of context (2047 cached + the new one), page size 16, greedy sampling.  The KV
pages hold synthetic N(0,1) fp16 values (no prompt is prefilled; the measured step
is a real decode step over that paged context).

A "step" = one HIP-graph replay of the whole decode graph: token embedding, 32 x
(RMSNorm + QKV GEMM + RoPE/KV-append, paged attention, O GEMM + residual, RMSNorm +
gate|up GEMM + SwiGLU, down GEMM + residual), final norm, the lm_head GEMM fused with the
greedy argmax (the logits are not stored), and the copy of the ids into the next step's
input.  Before timing, one step through the unfused path (logits stored, then argmax)
checks that both pick the same ids.  Positions are held at 2047, so
every step re-appends at the same slot and attends over exactly 2048 tokens.

Printed: one JSON line with value = decode tokens/s (32 tokens per step), the
paged-attention roofline (algorithmic bytes / live HIP-event time of the attention
kernel, launches captured in a HIP graph so no host gap is timed, rotated over the 32
layers' KV so the 256 MB MALL cannot hold it), the same kernel at BASELINE configs 2 and 5
(ragged contexts over randomly permuted pages; config 5 with a shared 1024-token prefix, its
bytes counted once), the same for the largest projection (the
fused gate|up Q4_0 GEMM + SwiGLU at m = batch, rotated
over the 32 layers' weights), the same for the dequant GEMV at m = 1, 8 and 32 (BASELINE
config 3's 14336 -> 4096 and 4096 -> 14336 projections, rotated over the layers' down and gate weights; m = 32
takes the MFMA GEMM), the batched GEMM
on MFMA (BASELINE config 5's Q8_0 gate|up + SwiGLU at batch 128: TFLOP/s against the dense fp16
MFMA peak), the same decode
step at batch 1 (decode_batch1: the projections and greedy head then run the GEMV), BASELINE config 5's
full decode step (decode_config5: Qwen2-7B shape, Q8_0, batch 128 over a shared 1024-token prefix and ragged
suffixes, against its HBM floor of unique bytes), and a CPU
baseline (the C/OpenMP oracle restatement timed on this
host over one layer and the lm_head, scaled to a full step).

roofline.traffic is the HBM bytes per attention launch measured by rocprofv3
FETCH_SIZE / WRITE_SIZE runs of this script, each scaled by the factor the same
counter shows for a copy of known size (--copy-calibration adds that copy); the
figures are read from the committed summary in profiles/ (null if it is absent).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, MI355X
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "attn_f16_d128_decode_b32_ctx2048_traffic.txt")


def measured_traffic(path: str) -> dict | None:
    """HBM bytes per attention launch from the committed counter summary: lines
    ``key: value`` with fetch_kib, write_kib (per dispatch) and fetch_scale, write_scale."""
    try:
        kv = {}
        with open(path) as f:
            for line in f:
                if ":" in line and not line.lstrip().startswith("#"):
                    k, v = line.split(":", 1)
                    kv[k.strip()] = v.strip()
        fetch = float(kv["fetch_kib"]) * float(kv["fetch_scale"]) * 1024
        write = float(kv["write_kib"]) * float(kv["write_scale"]) * 1024
        return {"bytes": round(fetch + write), "fetch": round(fetch), "write": round(write),
                "source": os.path.relpath(path, os.path.dirname(os.path.abspath(__file__)))}
    except (OSError, KeyError, ValueError):
        return None


COUNTERS_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                             "qgemm_counters_config5_gateup_m128_config4_m32.txt")


def measured_counters(path: str, prefix: str) -> dict | None:
    """The ``<prefix>_*`` figures (MFMA busy, VALU busy, L1 pending, ...) of one kernel from the committed rocprofv3
    counter summary; null when the file is absent."""
    try:
        out = {}
        with open(path) as f:
            for line in f:
                if ":" in line and not line.lstrip().startswith("#"):
                    k, v = (x.strip() for x in line.split(":", 1))
                    if k.startswith(prefix + "_"):
                        out[k[len(prefix) + 1:]] = float(v)
        if not out:
            return None
        out["source"] = os.path.relpath(path, os.path.dirname(os.path.abspath(__file__)))
        return out
    except (OSError, ValueError):
        return None


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--attn-iters", type=int, default=64)
    ap.add_argument("--gemm-iters", type=int, default=64)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first copy 256 MiB four times (the known-size kernel for FETCH_SIZE/WRITE_SIZE scaling)")
    ap.add_argument("--only", choices=["gemm", "config5"], default=None,
                    help="run only the projection rooflines (gemm) or only BASELINE config 5's decode step "
                         "(config5), for rocprofv3 runs of those kernels, and print their JSON; not a bench line")
    return ap.parse_args()


def llama3_8b(layers: int):
    from cacheir_amd.artifact import ModelConfig

    return ModelConfig(architecture="Llama3-8B-shape", hidden_size=4096, intermediate_size=14336, num_layers=layers,
                       num_attention_heads=32, num_key_value_heads=8, vocab_size=128256,
                       max_position_embeddings=8192, rope_theta=500000.0, rms_norm_eps=1e-5, dtype="float16")


def qwen2_7b(layers: int):
    from cacheir_amd.artifact import ModelConfig

    return ModelConfig(architecture="Qwen2-7B-shape", hidden_size=3584, intermediate_size=18944, num_layers=layers,
                       num_attention_heads=28, num_key_value_heads=4, vocab_size=152064,
                       max_position_embeddings=32768, rope_theta=1000000.0, rms_norm_eps=1e-6, dtype="float16")


def graph_us_per_launch(launch, iters: int, replays: int = 3, warm_replays: int = 2) -> float:
    """GPU time per launch of ``launch(i)``: ``iters`` launches captured in one HIP graph, replayed ``warm_replays``
    times untimed (the first replays after a pause run ~2-4% slow while the clocks come up), then ``replays`` times
    between HIP events on the launch stream (no host launch gaps inside the timed region)."""
    import torch

    for i in range(4):
        launch(i)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch(0)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(iters):
            launch(i)
    for _ in range(warm_replays):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / (iters * replays)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_greedy_steps(plan, steps: int, warmup: int) -> float:
    """ms per greedy decode step of `plan`: the step (and the copy of its ids into the next step's input) captured
    in one HIP graph, `warmup` untimed replays, then `steps` replays between two events."""
    import torch

    def body():
        plan.launch_greedy()
        plan.ids.copy_(plan.next_ids)

    # capture (warm-up on a side stream first, as torch requires)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        body()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_runtime_steps(base, sessions, ids: list[int], steps: int, warmup: int) -> dict:
    """Wall time per step of the runtime API with its host work: ``decode_greedy`` (inputs staged and copied,
    the step's graph replayed, the ids copied back: a scheduler's greedy loop) and ``run_decode_batch`` followed by
    a synchronize (logits left on the device).  Each step is rolled back one token afterwards, so every step decodes
    at the same position over the same pages, as the graph-step timing does."""
    import torch

    def rollback():
        for s in sessions:
            s.kv_cache.tokens -= 1

    out = {}
    for name, fn in (("decode_greedy_ms", lambda: base.decode_greedy(sessions, ids)),
                     ("run_decode_batch_ms", lambda: (base.run_decode_batch(sessions, ids), torch.cuda.synchronize()))):
        for _ in range(max(2, warmup)):  # the first call captures the step's graph
            fn()
            rollback()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
            rollback()
        out[name] = round((time.perf_counter() - t0) * 1000.0 / steps, 4)
    return out


def ragged_attention_case(config: int, dev, iters: int) -> dict:
    """Paged decode attention at BASELINE config 2 (batch 64, Llama-3-8B heads, contexts
    U[512, 4096], pages permuted at random over the pool) or config 5 (batch 128, Qwen2-7B
    heads, one 1024-token prefix in 64 pages shared by every page table, suffixes U[64, 7168]
    in pages of their own, permuted).  Context lengths and page tables are numpy draws with
    seed 0; q and the K/V pools are N(0,1) fp16 drawn on the device.  Two copies of the pools
    alternate so the 256 MB MALL holds neither.  Returns bytes and live time per launch."""
    import torch

    from cacheir_amd import kernels

    rng = np.random.default_rng(0)
    P, D = 16, 128
    if config == 2:
        B, H, Hkv = 64, 32, 8
        ctx = rng.integers(512, 4097, B)
        npg = -(-ctx // P)
        slots = int(npg.sum())
        perm = rng.permutation(slots)
        max_pages = 4096 // P
        pt = np.zeros((B, max_pages), np.int32)
        off = 0
        for b in range(B):
            pt[b, : npg[b]] = perm[off: off + npg[b]]
            off += npg[b]
        unique_tokens = int(ctx.sum())
    else:
        B, H, Hkv, prefix = 128, 28, 4, 1024
        suffix = rng.integers(64, 7169, B)
        ctx = prefix + suffix
        npg = -(-suffix // P)
        slots = prefix // P + int(npg.sum())
        perm = prefix // P + rng.permutation(slots - prefix // P)
        max_pages = (prefix + 7168) // P
        pt = np.zeros((B, max_pages), np.int32)
        off = 0
        for b in range(B):
            pt[b, : prefix // P] = np.arange(prefix // P)
            pt[b, prefix // P: prefix // P + npg[b]] = perm[off: off + npg[b]]
            off += npg[b]
        unique_tokens = prefix + int(suffix.sum())
    g = torch.Generator(device=dev)
    g.manual_seed(config)
    pools = [(torch.randn((slots, Hkv, P, D), device=dev, generator=g).half(),
              torch.randn((slots, Hkv, P, D), device=dev, generator=g).half()) for _ in range(2)]
    q = torch.randn((B, H, D), device=dev, generator=g).half()
    out = torch.empty_like(q)
    table = torch.from_numpy(pt).to(dev)
    lens = torch.from_numpy(ctx.astype(np.int32)).to(dev)
    ws = kernels.attention_workspace(B, H, D, max_pages * P, dev)
    us = graph_us_per_launch(lambda it: kernels.paged_decode_attention(
        q, pools[it % 2][0], pools[it % 2][1], table, lens, out=out, workspace=ws), iters)
    per_token = 2 * Hkv * D * 2  # K + V, fp16
    side = 2 * B * H * D * 2 + 4 * int(npg.sum()) + 4 * B  # q, out, page-table entries, lengths
    unique = per_token * unique_tokens + side
    logical = per_token * int(ctx.sum()) + side
    res = {"config": config, "batch": B, "heads": [H, Hkv], "context_sum": int(ctx.sum()),
           "context_max": int(ctx.max()), "us_per_launch": round(us, 3), "bytes_per_launch": unique,
           "achieved": round(unique / (us * 1e-6) / 1e9, 1),
           "frac": round(unique / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    if config == 5:
        res["logical_bytes_per_launch"] = logical
        res["logical_gbs"] = round(logical / (us * 1e-6) / 1e9, 1)
    del pools
    torch.cuda.empty_cache()
    return res


def read_ceiling_mixed(dev, nbytes: int, side_bytes: int, side_ratio: int, iters: int = 24) -> dict:
    """The same best-shape read of ``nbytes`` with ``side_ratio`` reads of an L2-resident ``side_bytes`` buffer per 8
    chunks streamed (all issued before any is consumed): the loads of the m = 32 gate|up GEMM, whose 224
    workgroups each re-read the 256 KB of activations beside their share of the weights (side_ratio 7: 0.875 bytes
    of activations per weight byte)."""
    import torch
    from cacheir_amd import kernels

    out = torch.zeros(1, dtype=torch.int32, device=dev)
    nbytes = nbytes // 16 * 16
    copies = max(4, -(-1_500_000_000 // nbytes))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(c + 1) for c in range(copies)]
    side = torch.ones(side_bytes, dtype=torch.uint8, device=dev)
    best = None
    for layout in (0, 1):
        for wgs in (224, 256, 512):
            for threads in (256, 512):
                us = graph_us_per_launch(lambda i: kernels.stream_read(bufs[i % copies], wgs, threads, layout, out,
                                                                       side=side, side_ratio=side_ratio), iters)
                if best is None or us < best[0]:
                    best = (us, layout, wgs, threads)
    us, layout, wgs, threads = best
    side_total = nbytes * side_ratio // 8
    res = {"bytes": nbytes, "side_bytes_read": side_total, "us": round(us, 3),
           "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
           "shape": f"{'grid-stride' if layout == 0 else 'chunked'} {wgs} x {threads}"}
    log(f"read ceiling with L2 re-reads: {nbytes / 1e6:.1f} MB + {side_total / 1e6:.1f} MB from a "
        f"{side_bytes // 1024} KB buffer in {us:.2f} us = {res['gbs']:.0f} GB/s of the stream ({res['shape']})")
    del bufs
    torch.cuda.empty_cache()
    return res


def read_ceiling(dev, sizes: dict[str, int], iters: int = 24) -> dict:
    """Best rate of a plain read of each byte count (``cir_stream_read``): grid-stride and chunked layouts over
    224-2048 workgroups of 256 or 512 threads, each launch reading a different buffer of a set larger than the
    256 MB MALL.  The hot kernels' rates are read against these as well as against the 8 TB/s peak."""
    import torch
    from cacheir_amd import kernels

    out = torch.zeros(1, dtype=torch.int32, device=dev)
    res = {}
    for name, nbytes in sizes.items():
        nbytes = nbytes // 16 * 16
        copies = max(4, -(-1_500_000_000 // nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(c + 1) for c in range(copies)]
        best = None
        for layout in (0, 1):
            for wgs in (224, 256, 512, 1024, 2048):
                for threads in (256, 512):
                    us = graph_us_per_launch(
                        lambda i: kernels.stream_read(bufs[i % copies], wgs, threads, layout, out), iters)
                    if best is None or us < best[0]:
                        best = (us, layout, wgs, threads)
        us, layout, wgs, threads = best
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"bytes": nbytes, "us": round(us, 3), "gbs": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
                     "shape": f"{'grid-stride' if layout == 0 else 'chunked'} {wgs} x {threads}"}
        log(f"read ceiling {name}: {nbytes / 1e6:.1f} MB in {us:.2f} us = {gbs:.0f} GB/s "
            f"({gbs / HBM_PEAK_GBS:.1%} of peak; {res[name]['shape']})")
        del bufs
        torch.cuda.empty_cache()
    return res


def prefill_case(base, cfg, tokens: int, dev) -> dict:
    """Prefill measured (the step before decode): one prompt of ``tokens`` ids through ``HipRuntime.run`` on the
    base session (causal paged attention writing the pool, projections on the large-m MFMA GEMM, logits for every
    position), best of 3 timed runs after a warm-up, host launches included.  FLOPs: 2 per weight per token for the
    linear layers and the lm_head, plus q.k and p.v over the causal context."""
    import torch

    ids = np.random.default_rng(3).integers(0, cfg.vocab_size, size=(1, tokens))
    out = base.run(ids, mode="prefill")
    torch.cuda.synchronize()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        out = base.run(ids, mode="prefill")
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    if not bool(torch.isfinite(out).all()):
        raise RuntimeError("prefill: non-finite logits")
    del out
    ms = min(times) * 1e3
    h, f, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    per_layer = h * (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * d + cfg.num_attention_heads * d * h \
        + 3 * h * f
    params = cfg.num_layers * per_layer + cfg.vocab_size * h
    attn = cfg.num_layers * 4 * cfg.num_attention_heads * d * tokens * (tokens + 1) // 2
    tflops = (2 * tokens * params + attn) / (ms * 1e-3) / 1e12
    torch.cuda.empty_cache()
    return {"tokens": tokens, "batch": 1, "ms": round(ms, 3), "tokens_per_s": round(tokens / ms * 1e3, 1),
            "tflops": round(tflops, 1), "frac_mfma": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "note": "HipRuntime.run(mode='prefill') wall time, host launches included; logits for every position"}


def config5_step_case(dev, steps: int, warmup: int) -> dict:
    """BASELINE config 5's full decode step: the Qwen2-7B shape (28 layers, Q8_0, random-init: int8 uniform,
    d = |N(0, 3e-4)|, so weights have std ~0.02), batch 128; one 1024-token prefix in 64 pages that every page
    table shares (forks aliasing the base session's pages, no copies), suffixes U[64, 7168] (numpy seed 0, the
    draw of the config-5 attention case) in pages of each session's own lane; N(0, 1) fp16 K/V.  The greedy step
    (fused LM head + argmax) captured in a HIP graph, as for config 4.  The HBM floor counts every weight once and
    the K/V of the prefix once per layer (the unique bytes)."""
    import torch

    from cacheir_amd.compiler import compile_config
    from cacheir_amd.runtime import HipRuntime
    from cacheir_amd.weights import GGML_Q8_0, SyntheticQuant

    B, prefix, P = 128, 1024, 16
    cfg = qwen2_7b(28)
    sfx = np.random.default_rng(0).integers(64, 7169, B)
    t0 = time.time()
    art = compile_config(cfg, quant="q8_0", modes=("decode",))
    pages = prefix // P + int((-(-sfx // P)).sum()) + 33 * 8
    base = HipRuntime(art, source=SyntheticQuant(GGML_Q8_0, dev, seed=0, scale_sigma=3e-4), kv_capacity_pages=pages)
    base.kv_cache.ensure_capacity(prefix)
    base.kv_cache.tokens = prefix
    sessions = []
    for n in sfx:
        s = base.fork()
        s.kv_cache.alias_prefix(base.kv_cache.slots, prefix)
        s.kv_cache.ensure_capacity(prefix + int(n))
        s.kv_cache.tokens = prefix + int(n) - 1
        sessions.append(s)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    for layer in range(cfg.num_layers):
        base.kv_allocator.k[layer].normal_(generator=g)
        base.kv_allocator.v[layer].normal_(generator=g)
    max_pages = base._bucket(max(len(s.kv_cache.slots) for s in sessions))
    plan = base.plan("decode", B, 1, max_pages)
    rows = np.zeros((B, max_pages), np.int32)
    for b, s in enumerate(sessions):
        rows[b, : len(s.kv_cache.slots)] = s.kv_cache.slots
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, size=(B, 1))
    plan.set_inputs(ids, rows, np.array([s.kv_cache.tokens for s in sessions], np.int32))
    plan.launch_with_argmax()
    torch.cuda.synchronize()
    assert torch.isfinite(plan.logits).all().item(), "config 5: non-finite logits"
    want = plan.next_ids.clone()
    plan.next_ids.zero_()
    plan.launch_greedy()
    torch.cuda.synchronize()
    assert torch.equal(plan.next_ids, want), "config 5: fused greedy head disagrees with argmax(logits)"
    log(f"config 5 model ready in {time.time() - t0:.1f}s; weights {base.weights.nbytes() / 1e9:.3f} GB")
    ms = time_greedy_steps(plan, steps, warmup)
    embed = base.weights.dense("tok_embeddings", torch.float16)
    weight_bytes = base.weights.nbytes() - embed.numel() * embed.element_size() + B * cfg.hidden_size * 2
    per_token = cfg.num_layers * 2 * cfg.num_key_value_heads * cfg.head_dim * 2  # K + V over all layers
    unique = per_token * (prefix + int(sfx.sum()))
    logical = per_token * int((prefix + sfx).sum())
    floor_ms = (weight_bytes + unique) / HBM_PEAK_GBS / 1e6
    res = {"workload": "BASELINE config 5: Qwen2-7B-shape Q8_0 full decode step, shared 1024-token prefix",
           "batch": B, "layers": cfg.num_layers, "context_sum": int((prefix + sfx).sum()),
           "context_max": int((prefix + sfx).max()), "ms_per_step": round(ms, 4),
           "tokens_per_s": round(B * 1000.0 / ms, 2), "weight_bytes": weight_bytes, "kv_unique_bytes": unique,
           "kv_logical_bytes": logical, "hbm_floor_ms": round(floor_ms, 4), "frac_of_floor": round(floor_ms / ms, 4),
           "gemm_plans": base.cache_stats()["gemm_plans"]}
    del plan, sessions, base, embed
    torch.cuda.empty_cache()
    return res


def gemm_rooflines(base, cfg, B, dev, args) -> dict:
    """The projection rooflines: the fused gate|up GEMM + SwiGLU at m = batch, BASELINE config 3 (m = 1, 8, 32)
    and the batched GEMM of config 5 (Q8_0 gate|up at m = 128), each timed live as HIP-graph replays."""
    import torch

    from cacheir_amd import kernels

    # ---- the same for the fused gate|up GEMM + SwiGLU (m = batch), rotated over the layers' weights ----
    gu = [base.weights.swiglu_weight(f"layer{i}_gate_w", f"layer{i}_up_w") for i in range(cfg.num_layers)]
    xg = torch.randn((B, cfg.hidden_size), device=dev, dtype=torch.float16)
    g_out = torch.empty((B, gu[0].n // 2), device=dev, dtype=torch.float16)
    gemm_us = graph_us_per_launch(lambda it: kernels.qgemm_swiglu(xg, gu[it % len(gu)], out=g_out), args.gemm_iters)
    gemm_bytes = gu[0].nbytes + 2 * B * gu[0].k + 2 * B * (gu[0].n // 2)
    gemm_gbs = gemm_bytes / (gemm_us * 1e-6) / 1e9
    log(f"gate|up GEMM + SwiGLU {gemm_us:.2f} us/launch (m={B}), {gemm_gbs:.0f} GB/s")

    # ---- the Q4_0 projections 14336 -> 4096 (the layers' down weights) and 4096 -> 14336 (16
    # layers' gate weights, tiled on their own) at m = 1 and 8 (the dequant GEMV) and m = 32 (the MFMA GEMM) ----
    dn = [base.weights.matmul_weight((f"layer{i}_down_w",)) for i in range(cfg.num_layers)]
    gt = [base.weights.matmul_weight((f"layer{i}_gate_w",)) for i in range(min(16, cfg.num_layers))]
    gemv = []
    for shape, ws_ in (("down", dn), ("gate", gt)):
        n3, k3 = ws_[0].n, ws_[0].k
        for m in (1, 8, 32):
            xv = torch.randn((m, k3), device=dev, dtype=torch.float16)
            sp = kernels.choose_splits(m, n3, k3)
            pv = torch.empty((sp, m, n3), device=dev)
            us = graph_us_per_launch(lambda it: kernels.qgemm_partial(xv, ws_[it % len(ws_)], splits=sp, out=pv),
                                     args.gemm_iters)
            by = ws_[0].nbytes + 2 * m * k3 + 4 * m * n3  # weights, x, y once
            gbs = by / (us * 1e-6) / 1e9
            row = {"shape": shape, "m": m, "n": n3, "k": k3, "splits": sp,
                   "kernel": "qgemv_kernel" if m <= 8 else "qgemm_xs_kernel (MFMA)", "us_per_launch": round(us, 3),
                   "bytes_per_launch": by, "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
            if m > 8:
                row["tflops"] = round(2.0 * m * n3 * k3 / (us * 1e-6) / 1e12, 1)
            gemv.append(row)
            log(f"{row['kernel']} m={m} {n3}x{k3} {us:.2f} us/launch, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of peak)")
    del gt

    # ---- the batched GEMM on MFMA: BASELINE config 5's gate|up (Qwen2-7B, Q8_0) + SwiGLU at batch 128 ----
    n5, k5, m5 = 2 * 18944, 3584, 128

    def random_q8_0(seed: int):
        g5 = torch.Generator(device=dev)
        g5.manual_seed(seed)
        nb = n5 * (k5 // 32)
        blocks = torch.randint(0, 256, (nb, 34), dtype=torch.uint8, device=dev, generator=g5)
        d = (torch.rand(nb, device=dev, generator=g5) * 0.02 + 0.001).half()
        blocks[:, :2] = d.view(torch.uint8).view(nb, 2)
        return kernels.QWeight.from_blocks(blocks.reshape(-1), kernels.FMT_NAMES["q8_0"], n5, k5)

    w5 = [random_q8_0(100 + i) for i in range(4)]  # 4 x 144 MB: rotated past the 256 MB MALL
    x5 = torch.randn((m5, k5), device=dev, dtype=torch.float16)
    o5 = torch.empty((m5, n5 // 2), device=dev, dtype=torch.float16)
    from cacheir_amd import hip

    plan5 = kernels.gemm_plan(hip.GEMM_SWIGLU, kernels.FMT_NAMES["q8_0"], m5, n5, k5)
    us5 = graph_us_per_launch(lambda it: kernels.qgemm_swiglu(x5, w5[it % len(w5)], out=o5), args.gemm_iters)
    flop5 = 2.0 * m5 * n5 * k5
    bytes5 = w5[0].nbytes + 2 * m5 * k5 + 2 * m5 * (n5 // 2)
    tflops5 = flop5 / (us5 * 1e-6) / 1e12
    gbs5 = bytes5 / (us5 * 1e-6) / 1e9
    log(f"batched GEMM (config 5 gate|up Q8_0, m={m5}) {us5:.2f} us/launch, {gbs5:.0f} GB/s "
        f"({gbs5 / HBM_PEAK_GBS:.1%} of HBM peak; {flop5 / bytes5:.0f} flop/B), {tflops5:.0f} TFLOP/s "
        f"({tflops5 / MFMA_F16_PEAK_TFLOPS:.1%} of fp16 MFMA)")
    del w5
    return {"us": gemm_us, "bytes": gemm_bytes, "gbs": gemm_gbs, "gemv": gemv, "us5": us5, "tflops5": tflops5,
            "gbs5": gbs5, "plan5": plan5, "flop5": flop5, "bytes5": bytes5}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              flush=True)
        return 2
    import torch

    from cacheir_amd.compiler import compile_config
    from cacheir_amd.runtime import HipRuntime
    from cacheir_amd.weights import GGML_Q4_0, SyntheticQuant

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"calibration: copied {src.numel() * 4} bytes x4")
        del src, dst
    if args.only == "config5":
        print(json.dumps({"only": "config5", **config5_step_case(dev, args.steps, args.warmup)}), flush=True)
        return 0
    cfg = llama3_8b(args.layers)
    B, ctx, P = args.batch, args.ctx, 16
    art = compile_config(cfg, quant="q4_0", modes=("prefill", "decode"))
    pages_per_seq = -(-ctx // P)
    t0 = time.time()
    # one lane of pages_per_seq slots for each session (the base runtime's own included), so no lane runs dry
    base = HipRuntime(art, source=SyntheticQuant(GGML_Q4_0, dev, seed=0),
                      kv_capacity_pages=(B + 1) * pages_per_seq)
    sessions = [base.fork() for _ in range(B)]
    for s in sessions:
        s.kv_cache.ensure_capacity(ctx)
        s.kv_cache.tokens = ctx - 1
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    for layer in range(cfg.num_layers):  # synthetic context: N(0,1) fp16 K/V in every page
        base.kv_allocator.k[layer].normal_(generator=g)
        base.kv_allocator.v[layer].normal_(generator=g)
    max_pages = base._bucket(pages_per_seq)
    plan = base.plan("decode", B, 1, max_pages)
    rows = np.zeros((B, max_pages), np.int32)
    for b, s in enumerate(sessions):
        rows[b, : len(s.kv_cache.slots)] = s.kv_cache.slots
    ids = np.random.default_rng(0).integers(0, cfg.vocab_size, size=(B, 1))
    plan.set_inputs(ids, rows, np.full(B, ctx - 1, np.int32))
    torch.cuda.synchronize()
    log(f"model ready in {time.time() - t0:.1f}s; weights {base.weights.nbytes() / 1e9:.3f} GB, "
        f"KV pool {base.kv_allocator.stats()['persistent_pools'][0]['bytes'] / 1e9:.3f} GB")

    if args.only == "gemm":
        gemm = gemm_rooflines(base, cfg, B, dev, args)
        print(json.dumps({"only": "gemm", **gemm}), flush=True)
        return 0

    # the timed step is the greedy one (LM head fused with the argmax); check once that it picks the ids the
    # logits path picks, and that the logits are finite
    plan.launch_with_argmax()
    torch.cuda.synchronize()
    assert torch.isfinite(plan.logits).all().item(), "non-finite logits"
    want = plan.next_ids.clone()
    plan.next_ids.zero_()
    plan.launch_greedy()
    torch.cuda.synchronize()
    assert torch.equal(plan.next_ids, want), "fused greedy head disagrees with argmax(logits)"

    # Bytes a step must move: every linear weight and norm once, the embedding rows of
    # the batch only (the table itself is never streamed), and every layer's K/V.  Taken
    # before the roofline loops below tile extra weight copies into the same store.
    embed = base.weights.dense("tok_embeddings", torch.float16)
    weight_bytes = base.weights.nbytes() - embed.numel() * embed.element_size() + B * cfg.hidden_size * 2

    ms_step = time_greedy_steps(plan, args.steps, args.warmup)
    toks = B * 1000.0 / ms_step
    assert bool(((plan.next_ids >= 0) & (plan.next_ids < cfg.vocab_size)).all().item()), "ids out of range"
    log(f"step {ms_step:.3f} ms -> {toks:.1f} tok/s")

    # ---- live roofline of the paged-attention kernel (HIP events on the launch stream) ----
    from cacheir_amd import kernels

    H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    q = torch.randn((B, H, D), device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    ws = kernels.attention_workspace(B, H, D, max_pages * P, dev)
    def attn(it):
        kp, vp = base.kv_allocator.layer_pools(it % cfg.num_layers)
        kernels.paged_decode_attention(q, kp, vp, plan.page_table, plan.seq_lens, out=out, workspace=ws)

    attn_us = graph_us_per_launch(attn, args.attn_iters)
    kv_bytes = 2 * Hkv * D * 2 * B * ctx  # K + V fp16 over every visible token
    qo_bytes = 2 * B * H * D * 2
    table_bytes = 4 * B * pages_per_seq + 4 * B
    attn_bytes = kv_bytes + qo_bytes + table_bytes
    achieved = attn_bytes / (attn_us * 1e-6) / 1e9
    log(f"attention {attn_us:.2f} us/launch, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of peak)")

    gemm = gemm_rooflines(base, cfg, B, dev, args)
    gemm_us, gemm_bytes, gemm_gbs = gemm['us'], gemm['bytes'], gemm['gbs']
    gemv, us5, tflops5, gbs5 = gemm['gemv'], gemm['us5'], gemm['tflops5'], gemm['gbs5']
    flop5, bytes5 = gemm['flop5'], gemm['bytes5']

    # ---- the attention kernel at BASELINE configs 2 and 5 (ragged contexts, permuted / shared pages) ----
    ragged = []
    for c in (2, 5):
        r = ragged_attention_case(c, dev, max(8, args.attn_iters // 4))
        ragged.append(r)
        extra = f", logical {r['logical_gbs']:.0f} GB/s" if "logical_gbs" in r else ""
        log(f"attention config {c} (batch {r['batch']}, context sum {r['context_sum']}) {r['us_per_launch']:.2f} "
            f"us/launch, {r['achieved']:.0f} GB/s unique ({r['frac']:.1%} of peak){extra}")

    # ---- the same decode step at batch 1 (sequence 0's context): QKV, O, down and the greedy head run the GEMV ----
    plan1 = base.plan("decode", 1, 1, max_pages)
    plan1.set_inputs(ids[:1], rows[:1], np.full(1, ctx - 1, np.int32))
    plan1.launch_with_argmax()  # the same checks as the batch-B plan: finite logits, fused head == argmax
    torch.cuda.synchronize()
    assert torch.isfinite(plan1.logits).all().item(), "non-finite logits at batch 1"
    want1 = plan1.next_ids.clone()
    plan1.next_ids.zero_()
    plan1.launch_greedy()
    torch.cuda.synchronize()
    assert torch.equal(plan1.next_ids, want1), "fused greedy head disagrees with argmax(logits) at batch 1"
    ms_b1 = time_greedy_steps(plan1, args.steps, args.warmup)
    kv_b1 = 2 * Hkv * D * 2 * ctx * cfg.num_layers
    log(f"batch-1 step {ms_b1:.3f} ms -> {1000.0 / ms_b1:.1f} tok/s")

    # ---- the runtime API a scheduler calls, host work included (graph replay per step) ----
    host_steps = {}
    for name, sess, graph_ms in (("batch32", sessions, ms_step), ("batch1", sessions[:1], ms_b1)):
        r = time_runtime_steps(base, sess, ids[: len(sess), 0].tolist(), args.steps, args.warmup)
        r["graph_step_ms"] = round(graph_ms, 4)
        r["decode_greedy_overhead"] = round(r["decode_greedy_ms"] / graph_ms - 1.0, 4)
        host_steps[name] = r
        log(f"runtime API {name}: decode_greedy {r['decode_greedy_ms']:.3f} ms, run_decode_batch "
            f"{r['run_decode_batch_ms']:.3f} ms (graph step {graph_ms:.3f} ms)")
    prefill = prefill_case(base, cfg, ctx, dev)
    log(f"prefill {prefill['tokens']} tokens {prefill['ms']:.2f} ms -> {prefill['tokens_per_s']:.0f} tok/s, "
        f"{prefill['tflops']:.0f} TFLOP/s ({prefill['frac_mfma']:.1%} of fp16 MFMA)")
    gemm_plans = base.cache_stats()["gemm_plans"]
    c5 = config5_step_case(dev, args.steps, args.warmup)
    log(f"config 5 step {c5['ms_per_step']:.3f} ms -> {c5['tokens_per_s']:.1f} tok/s "
        f"({c5['frac_of_floor']:.1%} of its {c5['hbm_floor_ms']:.2f} ms HBM floor)")

    traffic = measured_traffic(TRAFFIC_FILE)
    ceiling = read_ceiling(dev, {"attention": attn_bytes, "gate_up": gemm_bytes,
                                 "config3": gemv[0]["bytes_per_launch"] if gemv else 33075200})
    # the activations the gate|up GEMM re-reads: B rows x hidden fp16 = 256 KB at batch 32
    ceiling["gate_up_with_activations"] = read_ceiling_mixed(dev, gemm_bytes, B * cfg.hidden_size * 2, 7)
    for row in gemv:  # config-3 projections against the read of their own size (33.0-35.1 MB, one ceiling)
        row["frac_of_read_ceiling"] = round(row["achieved"] / ceiling["config3"]["gbs"], 4)

    # ---- CPU baseline: C/OpenMP restatement, one layer + lm_head, scaled to the step ----
    cpu = None
    if not args.no_cpu:
        from oracle import cbase

        cpu = cbase.time_decode_step(batch=B, ctx=ctx, hidden=4096, ffn=14336, heads=H, kv_heads=Hkv, vocab=128256,
                                     layers=cfg.num_layers, budget_s=12.0, log=log)

    line = {
        "metric": "decode tokens/s, batch 32, Llama-3-8B-shape Q4_0; paged-attn HBM GB/s",
        "value": round(toks, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 activations/KV, Q4_0 weights (int4 x fp16 MFMA, fp32 accumulate)",
        "data": "synthetic: random-init Q4_0 weights, N(0,1) fp16 KV context",
        "config": {"workload": "BASELINE config 4: Llama-3-8B-shape Q4_0 full decode step", "batch": B,
                   "context": ctx, "layers": cfg.num_layers, "page_size": P, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "paged decode attention (attn_f16_d128<4>)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_detail": traffic,
                     "bytes_per_launch": attn_bytes, "us_per_launch": round(attn_us, 3),
                     "frac_of_read_ceiling": round(achieved / ceiling["attention"]["gbs"], 4)},
        "read_ceiling": {"note": "best plain read of each byte count on this GPU (cir_stream_read, buffers rotated "
                                 "past the MALL): what a kernel moving those bytes could reach at most",
                         **ceiling},
        "roofline_attention_ragged": {"bound": "hbm", "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                      "note": "BASELINE configs 2 and 5; achieved on unique K/V bytes (config 5's "
                                              "shared prefix counted once), logical bytes beside it",
                                      "cases": ragged},
        "roofline_gemm": {"bound": "hbm", "kernel": f"Q4_0 gate|up GEMM + SwiGLU m={B} (qgemm_xs_kernel, EPI=1)",
                          "achieved": round(gemm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gemm_gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": gemm_bytes,
                          "us_per_launch": round(gemm_us, 3),
                          "frac_of_read_ceiling": round(gemm_gbs / ceiling["gate_up"]["gbs"], 4),
                          "frac_of_read_ceiling_with_activations":
                              round(gemm_gbs / ceiling["gate_up_with_activations"]["gbs"], 4),
                          "counters": measured_counters(COUNTERS_FILE, "xs_swiglu")},
        "roofline_gemv": {"bound": "hbm", "kernel": "Q4_0 projections, BASELINE config 3 (n x k, y = x W^T): dequant "
                                                    "GEMV at m <= 8, MFMA GEMM at m = 32",
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "shapes": gemv},
        # 2 * 128 FLOP per Q8_0 weight of 34/32 B: ~232 flop/B of weights + activations, left of the ~312 flop/B
        # ridge, so HBM bounds it; the MFMA figures ride along (utilisation is the secondary counter)
        "roofline_batched_gemm": {"bound": "hbm",
                                  "kernel": f"Q8_0 gate|up GEMM + SwiGLU m=128 ({gemm['plan5']}), "
                                            "BASELINE config 5 shape (n 37888, k 3584)",
                                  "achieved": round(gbs5, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                  "frac": round(gbs5 / HBM_PEAK_GBS, 4), "us_per_launch": round(us5, 3),
                                  "arithmetic_intensity": round(flop5 / bytes5, 1),
                                  "mfma_tflops": round(tflops5, 1), "mfma_peak": MFMA_F16_PEAK_TFLOPS,
                                  "mfma_frac": round(tflops5 / MFMA_F16_PEAK_TFLOPS, 4),
                                  "counters": measured_counters(COUNTERS_FILE, "xw")},
        "step_bytes": {"weights": weight_bytes, "kv": kv_bytes * cfg.num_layers,
                       "hbm_floor_ms": round((weight_bytes + kv_bytes * cfg.num_layers) / HBM_PEAK_GBS / 1e6, 4)},
        "decode_batch1": {"ms_per_step": round(ms_b1, 4), "tokens_per_s": round(1000.0 / ms_b1, 2),
                          "hbm_floor_ms": round((weight_bytes + kv_b1) / HBM_PEAK_GBS / 1e6, 4),
                          "note": "same model and context, one sequence; projections on the dequant GEMV"},
        "prefill": prefill,
        "decode_config5": c5,
        "runtime_api_steps": {"note": "wall ms per step through HipRuntime.decode_greedy / run_decode_batch (+ "
                                      "synchronize), host work included, graph replay per step",
                              **host_steps},
        "gemm_plans": gemm_plans,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
