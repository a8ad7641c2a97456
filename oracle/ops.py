"""NumPy restatement of CacheIR's CPU op semantics (test infrastructure only).

Each function follows the reference NumPy branch cited in its docstring
(``cacheir/runtime/cpu.py``), in float32 like the reference.

Pinning:
* ``rms_norm`` / ``matmul`` -- reference fixed-input tests
  ``tests/test_advanced_experiments.py:440-452`` (reproduced in tests/test_oracle.py)
  and the reference C++ kernels built into ``oracle/_ref`` when available.
* ``silu_mul`` -- ``tests/test_runtime.py:34-41`` inputs; reference C++ ``silu_mul``.
* ``rope_one`` -- no reference test pins it.  Pinned by properties the mathematics
  fixes: position 0 is the identity, each pair's norm is preserved, rotating by
  ``a`` then ``b`` equals rotating by ``a+b`` (checked through complex
  multiplication), and pair ``i`` turns at ``theta**(-2i/D)`` per position
  (checked against ``numpy`` complex exponentials).  A rotate-half layout or a
  wrong frequency exponent fails these.
* ``attention`` -- brute-force loop of ``tests/test_advanced_experiments.py:541-557``
  (``brute_force_attention`` in ``oracle/paged.py``) and softmax invariants.
"""
from __future__ import annotations

import numpy as np


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """``cpu.py:284-289`` NumPy branch: ``(x * 1/sqrt(mean(x^2)+eps)) * w``."""
    scale = 1.0 / np.sqrt(np.mean(np.square(x), axis=-1, keepdims=True) + eps)
    return (x * scale) * weight


def matmul(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """``cpu.py:291-304``: ``einsum('...i,oi->...o')`` with weight stored ``[out, in]``."""
    return np.einsum("...i,oi->...o", x, weight, optimize=True)


def silu(x: np.ndarray) -> np.ndarray:
    """``cpu.py:258-260``."""
    return x / (1.0 + np.exp(-x))


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``cpu.py:266-272`` NumPy branch: ``(g / (1 + e^-g)) * u``."""
    return (gate / (1.0 + np.exp(-gate))) * up


def rope_one(x: np.ndarray, head_dim: int, theta: float, offset: int) -> np.ndarray:
    """``cpu.py:324-340``: interleaved (GPT-J) RoPE on ``[B, S, H*D]``.

    Pair ``i`` is ``(x[2i], x[2i+1])``; ``freq_i = 1/theta**(2i/D)`` in float32;
    positions are ``offset + s``.
    """
    batch, seq, flat = x.shape
    heads = flat // head_dim
    view = x.reshape(batch, seq, heads, head_dim)
    half = head_dim // 2
    freq = 1.0 / (theta ** (np.arange(0, half, dtype=np.float32) * 2.0 / head_dim))
    pos = (np.arange(seq, dtype=np.float32) + float(offset))[:, None]
    angles = pos * freq[None, :]
    cos = np.cos(angles)[None, :, None, :]
    sin = np.sin(angles)[None, :, None, :]
    even = view[..., 0::2]
    odd = view[..., 1::2]
    rotated = np.empty_like(view)
    rotated[..., 0::2] = even * cos - odd * sin
    rotated[..., 1::2] = even * sin + odd * cos
    return rotated.reshape(batch, seq, flat)


def rope_offsets(x: np.ndarray, head_dim: int, theta: float, offsets: list[int]) -> np.ndarray:
    """Per-row offsets, as ``cuda.py:1084-1102`` uses for batched decode.

    Row ``b`` is rotated exactly as ``rope_one(x[b:b+1], ..., offsets[b])``.
    """
    return np.concatenate(
        [rope_one(x[b : b + 1], head_dim, theta, int(offsets[b])) for b in range(x.shape[0])], axis=0
    )


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """``cpu.py:373-377``."""
    shifted = x - np.max(x, axis=axis, keepdims=True)
    exp = np.exp(shifted)
    return exp / np.sum(exp, axis=axis, keepdims=True)


def attention(
    qh: np.ndarray, kh: np.ndarray, vh: np.ndarray, heads: int, kv_heads: int, head_dim: int, causal: bool
) -> np.ndarray:
    """``cpu.py:342-371`` after the cache append.

    ``qh`` is ``[B, Sq, Hq, D]``; ``kh``/``vh`` are the whole cache ``[B, T, Hkv, D]``.
    GQA by ``np.repeat`` along heads (``kvh = h // (Hq/Hkv)``), scores divided by
    ``sqrt(D)``, prefill masks ``key > past + q`` with -1e30.  Returns ``[B, Sq, Hq*D]``.
    """
    batch, q_len = qh.shape[:2]
    repeat = heads // kv_heads
    if repeat > 1:
        kh = np.repeat(kh, repeat, axis=2)
        vh = np.repeat(vh, repeat, axis=2)
    scores = np.einsum("bqhd,bkhd->bhqk", qh, kh, optimize=True) / float(np.sqrt(float(head_dim)))
    if causal:
        k_len = kh.shape[1]
        past = max(0, k_len - q_len)
        qpos = past + np.arange(q_len, dtype=np.int64)[:, None]
        kpos = np.arange(k_len, dtype=np.int64)[None, :]
        scores = np.where((kpos > qpos)[None, None, :, :], -1.0e30, scores)
    probs = softmax(scores, axis=-1)
    ctx = np.einsum("bhqk,bkhd->bqhd", probs, vh, optimize=True)
    return ctx.reshape(batch, q_len, heads * head_dim)


def greedy(logits_last: np.ndarray, vocab: int) -> np.ndarray:
    """``cpu.py:181-182`` / ``scheduler.py:535-543``: first-index argmax modulo vocab."""
    return np.argmax(logits_last, axis=-1) % vocab
