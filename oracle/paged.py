"""Paged KV cache math and paged decode attention (test infrastructure only).

* ``extend_pages`` restates ``cacheir/runtime/kv_cache.py:110-122`` (a new page
  starts whenever the cursor is page-aligned; otherwise the last page grows).
* The pool layout is the reference's persistent pool
  ``[slots, kv_heads, page_size, head_dim]`` (``cacheir/runtime/cuda.py:266-290``);
  token ``t`` of sequence ``b`` lives at
  ``pool[page_table[b, t // P], kvh, t % P, :]`` (``triton_kernels.py:201-209``).
* ``brute_force_attention`` is the loop of
  ``tests/test_advanced_experiments.py:541-557`` (gather per position, softmax of
  ``q.k / sqrt(D)``, weighted V sum), computed in float64.
* ``paged_attention`` gathers to contiguous ``[T, Hkv, D]`` per sequence and calls
  ``oracle.ops.attention`` (``cpu.py:342-371``), in float32.

Pinning: gather == contiguous cache bit-for-bit; the vectorised form agrees with
the float64 brute force; a single-position context returns V exactly; uniform
scores return the mean of V; permuting page slots leaves the output unchanged.
"""
from __future__ import annotations

import numpy as np

from oracle import ops


def extend_pages(pages: list[dict], start: int, length: int, page_size: int, next_page_id: int) -> int:
    """``kv_cache.py:110-122``.  Mutates ``pages`` (dicts with page_id/start/length); returns the next id."""
    remaining = length
    cursor = start
    while remaining > 0:
        page_offset = cursor % page_size
        take = min(remaining, page_size - page_offset)
        if page_offset == 0:
            pages.append({"page_id": next_page_id, "start": cursor, "length": take})
            next_page_id += 1
        else:
            pages[-1]["length"] += take
        cursor += take
        remaining -= take
    return next_page_id


def gather_sequence(pool: np.ndarray, page_row: np.ndarray, seq_len: int) -> np.ndarray:
    """Contiguous ``[T, Hkv, D]`` view of one sequence's tokens from ``pool [S, Hkv, P, D]``."""
    page_size = pool.shape[2]
    t = np.arange(seq_len)
    slots = page_row[t // page_size]
    return pool[slots, :, t % page_size, :]


def build_pool(rng: np.random.Generator, ctx_lens, kv_heads: int, head_dim: int, page_size: int,
               dtype=np.float16, permute: bool = True, extra_slots: int = 0):
    """BASELINE config-2 style inputs: pool slots = sum(ceil(ctx/P)) (+extra); page tables
    are a random permutation of the slots dealt to sequences in order.

    Returns ``(k_pool, v_pool, page_table[B, max_pages] int32, seq_lens int32)``; unused
    page-table entries are 0 (as the reference pads, ``cuda.py:1231-1234``).
    """
    ctx_lens = np.asarray(ctx_lens, dtype=np.int64)
    pages_per = (ctx_lens + page_size - 1) // page_size
    total = int(pages_per.sum()) + extra_slots
    order = rng.permutation(total) if permute else np.arange(total)
    max_pages = max(1, int(pages_per.max()) if len(pages_per) else 1)
    page_table = np.zeros((len(ctx_lens), max_pages), dtype=np.int32)
    cursor = 0
    for b, n in enumerate(pages_per):
        page_table[b, :n] = order[cursor : cursor + n]
        cursor += n
    k_pool = rng.standard_normal((total, kv_heads, page_size, head_dim)).astype(dtype)
    v_pool = rng.standard_normal((total, kv_heads, page_size, head_dim)).astype(dtype)
    return k_pool, v_pool, page_table, ctx_lens.astype(np.int32)


def paged_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, page_table: np.ndarray,
                    seq_lens: np.ndarray, num_heads: int, num_kv_heads: int) -> np.ndarray:
    """Decode attention for ``q [B, Hq, D]`` over each sequence's paged context, float32 math.

    Sequences with ``seq_len == 0`` produce zeros (the HIP kernel's documented
    behaviour for an empty context; the reference never issues one).
    """
    batch, _, head_dim = q.shape
    out = np.zeros((batch, num_heads, head_dim), dtype=np.float32)
    for b in range(batch):
        n = int(seq_lens[b])
        if n == 0:
            continue
        kh = gather_sequence(k_pool, page_table[b], n).astype(np.float32)[None]
        vh = gather_sequence(v_pool, page_table[b], n).astype(np.float32)[None]
        qh = q[b].astype(np.float32)[None, None]
        out[b] = ops.attention(qh, kh, vh, num_heads, num_kv_heads, head_dim, causal=False).reshape(num_heads, head_dim)
    return out


def brute_force_attention(q, k_pool, v_pool, page_table, seq_lens, num_heads, num_kv_heads) -> np.ndarray:
    """``tests/test_advanced_experiments.py:541-557`` loop, in float64."""
    batch, _, head_dim = q.shape
    page_size = k_pool.shape[2]
    repeat = num_heads // num_kv_heads
    out = np.zeros((batch, num_heads, head_dim), dtype=np.float64)
    for b in range(batch):
        seq = int(seq_lens[b])
        for h in range(num_heads):
            if seq == 0:
                continue
            kv_head = h // repeat
            ks, vs = [], []
            for pos in range(seq):
                page = int(page_table[b, pos // page_size])
                slot = pos % page_size
                ks.append(k_pool[page, kv_head, slot].astype(np.float64))
                vs.append(v_pool[page, kv_head, slot].astype(np.float64))
            k_ref = np.stack(ks)
            v_ref = np.stack(vs)
            scores = (q[b, h].astype(np.float64)[None, :] * k_ref).sum(axis=-1) / (head_dim ** 0.5)
            scores = scores - scores.max()
            p = np.exp(scores)
            p /= p.sum()
            out[b, h] = (p[:, None] * v_ref).sum(axis=0)
    return out
