"""Q4_0 / Q8_0 block formats and the reference per-row int4/int8 packing (test infrastructure only).

Block layouts follow ``cacheir/importers/gguf.py:36,40`` (32 values per block;
Q4_0 = 18 bytes: fp16 ``d`` then 16 bytes ``qs``; Q8_0 = 34 bytes: fp16 ``d`` then
32 int8) and the decoders ``gguf.py:273-282`` (Q8_0) and ``gguf.py:297-310`` (Q4_0):

* Q4_0: ``w[j] = ((qs[j] & 15) - 8) * d`` and ``w[j+16] = ((qs[j] >> 4) - 8) * d``, j < 16.
* Q8_0: ``w[j] = int8(q[j]) * d``.

``d`` is widened fp16 -> fp32 (``gguf.py:249-250``) and the product is taken in
fp32; both products are exact in fp32 (at most 11+4 resp. 11+8 significant bits).

Pinning: the reference known-answer vectors of
``tests/test_advanced_experiments.py:85-92,116-121`` (reproduced as fixtures in
``tests/golden/gguf_kat.json``), the per-block loop ``decode_*_loop`` (a literal
block-at-a-time walk, compared with the vectorised form on random data), exact
integer re-encoding (decode -> nibble recovery -> encode round trip), and the
closed form ``(n - 8) * d`` evaluated in float64.

Per-row asymmetric packing follows ``cacheir/quantization.py:96-139`` (used by the
reference runtime when ``--quant int4/int8`` is set).
"""
from __future__ import annotations

import struct

import numpy as np

QK = 32
Q4_0_BLOCK_BYTES = 18
Q8_0_BLOCK_BYTES = 34
GGML_TYPE_F32 = 0
GGML_TYPE_F16 = 1
GGML_TYPE_Q4_0 = 2
GGML_TYPE_Q8_0 = 8


# ---------------------------------------------------------------- Q4_0 ----------
def encode_q4_0(nibbles: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Pack ``nibbles [N, K]`` (0..15) and fp16 ``scales [N, K/32]`` into GGUF Q4_0 bytes ``[N, K/32*18]``.

    Element ``j`` of a block goes to the low nibble of byte ``j`` and element ``j+16``
    to the high nibble (the inverse of ``gguf.py:297-310``).
    """
    n, k = nibbles.shape
    assert k % QK == 0
    nb = k // QK
    nib = nibbles.astype(np.uint8).reshape(n, nb, QK)
    qs = (nib[:, :, :16] & 0x0F) | ((nib[:, :, 16:] & 0x0F) << 4)
    d = np.ascontiguousarray(scales.astype(np.float16).reshape(n, nb)).view(np.uint8).reshape(n, nb, 2)
    return np.ascontiguousarray(np.concatenate([d, qs], axis=2).reshape(n, nb * Q4_0_BLOCK_BYTES))


def decode_q4_0(blocks: np.ndarray, k: int) -> np.ndarray:
    """Vectorised ``gguf.py:297-310``: GGUF Q4_0 bytes ``[N, K/32*18]`` -> fp32 ``[N, K]``."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.shape[0]
    nb = k // QK
    raw = blocks.reshape(n, nb, Q4_0_BLOCK_BYTES)
    d = np.ascontiguousarray(raw[:, :, :2]).view(np.float16).reshape(n, nb).astype(np.float32)
    qs = raw[:, :, 2:]
    low = (qs & 0x0F).astype(np.int16)
    high = (qs >> 4).astype(np.int16)
    vals = np.concatenate([low - 8, high - 8], axis=2).astype(np.float32)
    return (vals * d[:, :, None]).reshape(n, k)


def decode_q4_0_loop(data: bytes, count: int) -> np.ndarray:
    """Block-at-a-time walk over the byte stream, as ``gguf.py:297-310`` does."""
    out = np.empty(count, dtype=np.float32)
    cursor = 0
    for block in range(count // QK):
        scale = float(np.frombuffer(data[cursor : cursor + 2], dtype=np.float16, count=1).astype(np.float32)[0])
        cursor += 2
        packed = np.frombuffer(data[cursor : cursor + 16], dtype=np.uint8, count=16)
        cursor += 16
        vals = np.empty(QK, dtype=np.float32)
        vals[:16] = ((packed & 0x0F).astype(np.int16) - 8).astype(np.float32)
        vals[16:] = ((packed >> 4).astype(np.int16) - 8).astype(np.float32)
        out[block * QK : (block + 1) * QK] = vals * np.float32(scale)
    return out


# ---------------------------------------------------------------- Q8_0 ----------
def encode_q8_0(values: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Pack int8 ``values [N, K]`` and fp16 ``scales [N, K/32]`` into GGUF Q8_0 bytes ``[N, K/32*34]``."""
    n, k = values.shape
    nb = k // QK
    q = values.astype(np.int8).reshape(n, nb, QK).view(np.uint8)
    d = np.ascontiguousarray(scales.astype(np.float16).reshape(n, nb)).view(np.uint8).reshape(n, nb, 2)
    return np.ascontiguousarray(np.concatenate([d, q], axis=2).reshape(n, nb * Q8_0_BLOCK_BYTES))


def decode_q8_0(blocks: np.ndarray, k: int) -> np.ndarray:
    """Vectorised ``gguf.py:273-282``: GGUF Q8_0 bytes -> fp32 ``[N, K]``."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.shape[0]
    nb = k // QK
    raw = blocks.reshape(n, nb, Q8_0_BLOCK_BYTES)
    d = np.ascontiguousarray(raw[:, :, :2]).view(np.float16).reshape(n, nb).astype(np.float32)
    q = np.ascontiguousarray(raw[:, :, 2:]).view(np.int8).astype(np.float32)
    return (q * d[:, :, None]).reshape(n, k)


def decode_q8_0_loop(data: bytes, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    cursor = 0
    for block in range(count // QK):
        scale = float(np.frombuffer(data[cursor : cursor + 2], dtype=np.float16, count=1).astype(np.float32)[0])
        cursor += 2
        vals = np.frombuffer(data[cursor : cursor + 32], dtype=np.int8, count=32).astype(np.float32)
        cursor += 32
        out[block * QK : (block + 1) * QK] = vals * np.float32(scale)
    return out


def random_q4_0(rng: np.random.Generator, n: int, k: int, scale_sigma: float = 0.01) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """BASELINE config 3 draw: nibbles uniform in [0,15], ``d = |N(0, sigma)|`` as fp16.

    Returns ``(blocks, nibbles, scales)``.
    """
    nib = rng.integers(0, 16, size=(n, k), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, scale_sigma, size=(n, k // QK))).astype(np.float16)
    return encode_q4_0(nib, d), nib, d


def random_q8_0(rng: np.random.Generator, n: int, k: int, scale_sigma: float = 0.01) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    q = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
    d = np.abs(rng.normal(0.0, scale_sigma, size=(n, k // QK))).astype(np.float16)
    return encode_q8_0(q, d), q, d


# ------------------------------------------------------ minimal GGUF writer ----------
def _gguf_string(value: str) -> bytes:
    data = value.encode("utf-8")
    return struct.pack("<Q", len(data)) + data


def write_gguf(path, tensors: list[tuple[str, int, tuple[int, ...], bytes]], metadata: dict | None = None, alignment: int = 32) -> None:
    """Write a GGUF v3 file with the header layout the reference parser reads
    (``gguf.py:128-167``; built the same way as ``tests/test_advanced_experiments.py:69-84``).

    ``tensors``: ``(name, ggml_type, gguf_dims, raw_bytes)`` with ``gguf_dims`` in GGUF
    order (fastest dimension first).  Metadata values may be int (uint32), float
    (float32) or str.
    """
    metadata = metadata or {}
    header = bytearray()
    header += b"GGUF"
    header += struct.pack("<I", 3)
    header += struct.pack("<Q", len(tensors))
    header += struct.pack("<Q", len(metadata))
    for key, value in metadata.items():
        header += _gguf_string(key)
        if isinstance(value, bool):
            header += struct.pack("<I", 7) + struct.pack("<?", value)
        elif isinstance(value, int):
            header += struct.pack("<I", 4) + struct.pack("<I", value)
        elif isinstance(value, float):
            header += struct.pack("<I", 6) + struct.pack("<f", value)
        else:
            header += struct.pack("<I", 8) + _gguf_string(str(value))
    cursor = 0
    offsets = []
    for _name, _t, _dims, raw in tensors:
        offsets.append(cursor)
        cursor += len(raw)
        cursor = (cursor + alignment - 1) // alignment * alignment
    for (name, ggml_type, dims, _raw), off in zip(tensors, offsets):
        header += _gguf_string(name)
        header += struct.pack("<I", len(dims))
        for dim in dims:
            header += struct.pack("<Q", int(dim))
        header += struct.pack("<I", int(ggml_type))
        header += struct.pack("<Q", off)
    while len(header) % alignment:
        header += b"\x00"
    body = bytearray()
    for (_name, _t, _dims, raw), off in zip(tensors, offsets):
        while len(body) < off:
            body += b"\x00"
        body += raw
    with open(path, "wb") as handle:
        handle.write(bytes(header) + bytes(body))


# ------------------------------------------- reference per-row asymmetric pack ----------
def asymmetric_pack(weight: np.ndarray, bits: int) -> dict:
    """``quantization.py:96-120``: per-row ``scale = max((max-min)/qmax, 1e-8)``,
    ``zp = round(-min/scale)``, ``q = clip(round(w/scale + zp), 0, qmax)``; int4 packs
    even columns in the low nibble (``quantization.py:123-130``)."""
    array = np.asarray(weight, dtype=np.float32)
    qmax = (1 << bits) - 1
    mins = np.min(array, axis=1)
    maxs = np.max(array, axis=1)
    scales = np.maximum((maxs - mins) / float(qmax), 1.0e-8).astype(np.float32)
    zero_points = np.round(0 - mins / scales).astype(np.int32)
    qvalues = np.round(array / scales[:, None] + zero_points[:, None]).clip(0, qmax).astype(np.uint8)
    if bits == 4:
        rows, cols = qvalues.shape
        padded = np.zeros((rows, cols + (cols % 2)), dtype=np.uint8)
        padded[:, :cols] = qvalues & 0x0F
        packed = (padded[:, 0::2] | (padded[:, 1::2] << 4)).astype(np.uint8)
    else:
        packed = qvalues
    return {"packed_values": packed, "scales": scales, "zero_points": zero_points, "bits": bits, "shape": array.shape}


def asymmetric_dequant(packed: dict) -> np.ndarray:
    """``quantization.py:74-84`` with ``_unpack_int4`` (``quantization.py:133-139``)."""
    rows, cols = packed["shape"]
    pv = packed["packed_values"]
    if packed["bits"] == 4:
        q = np.empty((rows, pv.shape[1] * 2), dtype=np.float32)
        q[:, 0::2] = (pv & 0x0F).astype(np.float32)
        q[:, 1::2] = ((pv >> 4) & 0x0F).astype(np.float32)
        q = q[:, :cols]
    else:
        q = pv.astype(np.float32)
    scale = packed["scales"].astype(np.float32)[:, None]
    zero = packed["zero_points"].astype(np.float32)[:, None]
    return (q[:rows, :cols] - zero) * scale
