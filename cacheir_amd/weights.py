"""Weight loading for the ROCm backend: GGUF blocks kept packed, dense tensors, synthetic models.

Sources:
* ``GGUFFile`` -- header / metadata / tensor directory reader restating the
  layout parsed by ``cacheir/importers/gguf.py:71-211`` (little-endian, v2/v3,
  ``general.alignment`` default 32, logical shape = reversed GGUF dims).  Q4_0 and
  Q8_0 tensors are returned as raw blocks (no host dequant, unlike
  ``gguf.py:273-310`` which decodes to fp32 at load); F32/F16 as arrays.
* ``NpzDir`` -- ``weights.npz`` next to ``config.json`` (``cacheir/runtime/cpu.py:69-75``).
* ``SyntheticQuant`` -- random-init block weights generated on the device (bench).

``HipWeightStore`` turns a graph's WeightSpecs into device tensors: 2-D matmul
weights become ``kernels.QWeight`` (tiled Q4_0/Q8_0) when the source holds blocks or
when the artifact's quant is ``q4_0``/``q8_0``; otherwise dense tensors.  Fused
projections (Q|K|V, gate|up) are concatenated as GGUF blocks before the repack so
one GEMM launch covers them (the reference packs dense weights the same way,
``cacheir/runtime/cuda.py:1017-1023``).
"""
from __future__ import annotations

import struct
from pathlib import Path
from typing import Any

import numpy as np
import torch

from cacheir_amd import kernels
from cacheir_amd.hip import CIR_Q4_0, CIR_Q8_0

QK = 32
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8
_BLOCK = {GGML_Q4_0: 18, GGML_Q8_0: 34}
_SCALAR_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


# ------------------------------------------------------------------- GGUF -----
class GGUFFile:
    """Minimal GGUF reader (header, metadata, tensor directory, raw tensor bytes)."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        with self.path.open("rb") as f:
            if f.read(4) != b"GGUF":
                raise ValueError(f"{self.path} is not a GGUF file")
            self.version = struct.unpack("<I", f.read(4))[0]
            n_tensors, n_kv = struct.unpack("<QQ", f.read(16))
            self.metadata: dict[str, Any] = {}
            for _ in range(n_kv):
                key = self._str(f)
                self.metadata[key] = self._value(f)
            self.tensors: dict[str, dict[str, Any]] = {}
            for _ in range(n_tensors):
                name = self._str(f)
                ndim = struct.unpack("<I", f.read(4))[0]
                dims = struct.unpack(f"<{ndim}Q", f.read(8 * ndim))
                ggml_type, offset = struct.unpack("<IQ", f.read(12))
                self.tensors[name] = {"dims": tuple(int(d) for d in dims), "type": int(ggml_type), "offset": int(offset)}
            align = int(self.metadata.get("general.alignment", 32))
            pos = f.tell()
            self.data_offset = (pos + align - 1) // align * align

    @staticmethod
    def _str(f) -> str:
        n = struct.unpack("<Q", f.read(8))[0]
        return f.read(n).decode("utf-8", errors="replace")

    def _scalar(self, f, t: int):
        if t == 8:
            return self._str(f)
        fmt = _SCALAR_FMT.get(t)
        if fmt is None:
            raise ValueError(f"unsupported GGUF metadata type {t}")
        return struct.unpack(fmt, f.read(struct.calcsize(fmt)))[0]

    def _value(self, f):
        t = struct.unpack("<I", f.read(4))[0]
        if t == 9:
            et = struct.unpack("<I", f.read(4))[0]
            n = struct.unpack("<Q", f.read(8))[0]
            return [self._scalar(f, et) for _ in range(n)]
        return self._scalar(f, t)

    def shape(self, name: str) -> tuple[int, ...]:
        dims = self.tensors[name]["dims"]
        return tuple(reversed(dims)) if len(dims) > 1 else dims

    def ggml_type(self, name: str) -> int:
        return self.tensors[name]["type"]

    def raw(self, name: str) -> np.ndarray:
        info = self.tensors[name]
        count = int(np.prod(info["dims"], dtype=np.int64))
        t = info["type"]
        if t in _BLOCK:
            nbytes = count // QK * _BLOCK[t]
        elif t == GGML_F32:
            nbytes = count * 4
        elif t == GGML_F16:
            nbytes = count * 2
        else:
            raise NotImplementedError(f"GGUF tensor {name!r} has type {t}; the ROCm backend reads F32, F16, Q4_0, Q8_0")
        # read into a writable array of our own (torch.from_numpy warns on read-only buffers)
        data = np.empty(nbytes, dtype=np.uint8)
        with self.path.open("rb") as f:
            f.seek(self.data_offset + info["offset"])
            got = f.readinto(memoryview(data))
        if got != nbytes:
            raise ValueError(f"GGUF tensor {name!r} ended early")
        return data

    def dense(self, name: str) -> np.ndarray:
        t = self.ggml_type(name)
        raw = self.raw(name)
        if t == GGML_F32:
            return raw.view(np.float32).reshape(self.shape(name))
        if t == GGML_F16:
            return raw.view(np.float16).reshape(self.shape(name))
        raise TypeError(f"{name!r} is block-quantized; use blocks()")


# ---------------------------------------------------------- host quantizers ----
def row_bits(quant: str | None) -> int | None:
    """Bit width of the reference's per-row asymmetric packing for a ``--quant`` name
    (``quantization.py:63-71``: int4 / awq / gptq -> 4, int8 / 8bit -> 8), else None."""
    name = (quant or "").lower()
    if not name or name in ("q4_0", "q8_0"):
        return None
    if "int4" in name or "awq" in name or "gptq" in name:
        return 4
    if "int8" in name or "8bit" in name:
        return 8
    return None


def pack_rows(w: np.ndarray, bits: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The reference's per-row asymmetric packing of ``W[out, in]`` (``quantization.py:96-139``):
    scale = max((max - min) / qmax, 1e-8), zero_point = round(-min / scale), q = clip(round(w / scale + zp),
    0, qmax); 4-bit codes two per byte (even column low nibble).  Returns (packed uint8, scales fp32,
    zero_points int32), the ``PackedQuantizedTensor`` fields."""
    a = np.asarray(w, dtype=np.float32)
    qmax = (1 << bits) - 1
    mins, maxs = a.min(axis=1), a.max(axis=1)
    scales = np.maximum((maxs - mins) / np.float32(qmax), np.float32(1.0e-8)).astype(np.float32)
    zps = np.round(np.float32(0) - mins / scales).astype(np.int32)
    q = np.round(a / scales[:, None] + zps[:, None]).clip(0, qmax).astype(np.uint8)
    if bits == 4:
        rows, cols = q.shape
        padded = np.zeros((rows, cols + (cols % 2)), dtype=np.uint8)
        padded[:, :cols] = q & 0x0F
        q = (padded[:, 0::2] | (padded[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(q), np.ascontiguousarray(scales), np.ascontiguousarray(zps)


def unpack_rows(packed: np.ndarray, scales: np.ndarray, zero_points: np.ndarray, bits: int, k: int) -> np.ndarray:
    """``(q - zero_point) * scale`` in fp32 for ``pack_rows`` output: the reference's
    ``dequantize_packed_weight`` (``quantization.py:74-84``, int4 unpack ``quantization.py:133-139``)."""
    packed = np.asarray(packed, dtype=np.uint8)
    if bits == 4:
        q = np.empty((packed.shape[0], packed.shape[1] * 2), dtype=np.float32)
        q[:, 0::2] = packed & 0x0F
        q[:, 1::2] = packed >> 4
        q = q[:, :k]
    else:
        q = packed.astype(np.float32)
    return (q - zero_points.astype(np.float32)[:, None]) * scales.astype(np.float32)[:, None]


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """Dense ``[n, k]`` -> GGUF Q4_0 bytes: per block d = m / -8 where m is the value of
    largest magnitude, q = min(15, floor(x/d + 8.5)) (the ggml reference quantizer)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blk = w.reshape(n, k // QK, QK)
    idx = np.argmax(np.abs(blk), axis=2)
    m = np.take_along_axis(blk, idx[..., None], axis=2)[..., 0]
    d = (m / -8.0).astype(np.float32)
    inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1.0), 0.0).astype(np.float32)
    q = np.minimum(15, np.floor(blk * inv[..., None] + 8.5)).clip(0, 15).astype(np.uint8)
    qs = (q[:, :, :16] | (q[:, :, 16:] << 4)).astype(np.uint8)
    dh = d.astype(np.float16).view(np.uint8).reshape(n, k // QK, 2)
    return np.concatenate([dh, qs], axis=2).reshape(n, -1)


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """Dense ``[n, k]`` -> GGUF Q8_0 bytes: d = amax/127, q = round(x/d)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blk = w.reshape(n, k // QK, QK)
    d = (np.max(np.abs(blk), axis=2) / 127.0).astype(np.float32)
    inv = np.where(d != 0, 1.0 / np.where(d != 0, d, 1.0), 0.0).astype(np.float32)
    q = np.round(blk * inv[..., None]).clip(-127, 127).astype(np.int8).view(np.uint8)
    dh = d.astype(np.float16).view(np.uint8).reshape(n, k // QK, 2)
    return np.concatenate([dh, q], axis=2).reshape(n, -1)


# --------------------------------------------------------------- sources ------
class NpzDir:
    """``weights.npz`` + ``config.json`` model directory (the tiny-model format)."""

    def __init__(self, path: str | Path):
        p = Path(path)
        self.npz = p if p.suffix == ".npz" else p / "weights.npz"
        with np.load(self.npz) as data:
            self._arrays = {k: data[k] for k in data.files}

    def has_blocks(self, key: str) -> bool:
        return False

    def dense(self, key: str) -> np.ndarray:
        return self._arrays[key]


class GGUFSource:
    def __init__(self, path: str | Path, key_map: dict[str, str] | None = None):
        self.file = GGUFFile(path)
        self.key_map = key_map or {}

    def _k(self, key: str) -> str:
        return self.key_map.get(key, key)

    def has_blocks(self, key: str) -> bool:
        return self.file.ggml_type(self._k(key)) in _BLOCK

    def blocks(self, key: str) -> tuple[np.ndarray, int, int, int]:
        k = self._k(key)
        n, kk = self.file.shape(k)
        return self.file.raw(k).reshape(n, -1), self.file.ggml_type(k), n, kk

    def dense(self, key: str) -> np.ndarray:
        return self.file.dense(self._k(key))


class SyntheticQuant:
    """Random-init weights generated on the device: matmul weights as GGUF blocks
    (nibbles / int8 uniform, d = |N(0, scale_sigma)|), 1-D norms = 1, embeddings N(0, 0.02)."""

    def __init__(self, fmt: int, device, seed: int = 0, scale_sigma: float = 0.01):
        self.fmt, self.device, self.scale_sigma = fmt, torch.device(device), scale_sigma
        self.gen = torch.Generator(device=self.device)
        self.gen.manual_seed(seed)
        self.shapes: dict[str, tuple[int, ...]] = {}

    def register(self, key: str, shape: tuple[int, ...]) -> None:
        self.shapes[key] = tuple(int(s) for s in shape)

    def has_blocks(self, key: str) -> bool:
        return len(self.shapes[key]) == 2 and not key.endswith("embed_tokens.weight")

    def blocks_device(self, key: str) -> tuple[torch.Tensor, int, int, int]:
        n, k = self.shapes[key]
        nb = k // QK
        if self.fmt == GGML_Q4_0:
            qs = torch.randint(0, 256, (n, nb, 16), dtype=torch.uint8, device=self.device, generator=self.gen)
        else:
            qs = torch.randint(0, 256, (n, nb, 32), dtype=torch.uint8, device=self.device, generator=self.gen)
        d = torch.randn((n, nb), device=self.device, generator=self.gen).abs_().mul_(self.scale_sigma).to(torch.float16)
        raw = torch.cat([d.view(torch.uint8).view(n, nb, 2), qs], dim=2)
        return raw.reshape(-1).contiguous(), self.fmt, n, k

    def dense_device(self, key: str, dtype: torch.dtype) -> torch.Tensor:
        shape = self.shapes[key]
        if len(shape) == 1:
            return torch.ones(shape, dtype=dtype, device=self.device)
        return (torch.randn(shape, device=self.device, generator=self.gen) * 0.02).to(dtype)


# ----------------------------------------------------------- weight store -----
_FMT_OF = {"q4_0": GGML_Q4_0, "q8_0": GGML_Q8_0}


class HipWeightStore:
    """Device copies of a graph's weights, loaded once and shared by forked runtimes."""

    def __init__(self, source, specs: dict, *, device, dense_dtype: torch.dtype, quant: str | None = None):
        self.source = source
        self.specs = specs
        self.device = torch.device(device)
        self.dense_dtype = dense_dtype
        self.quant = (quant or "").lower() or None
        self._dense: dict[str, torch.Tensor] = {}
        self._packed: dict[tuple[str, ...], Any] = {}
        if isinstance(source, SyntheticQuant):
            for name, spec in specs.items():
                source.register(spec.key, tuple(spec.tensor_type.shape))

    # -- dense tensors (norms, embeddings, dense matmul weights) --
    def dense(self, name: str, dtype: torch.dtype | None = None) -> torch.Tensor:
        dtype = dtype or self.dense_dtype
        key = (name, dtype)
        if key not in self._dense:
            spec = self.specs[name]
            if isinstance(self.source, SyntheticQuant):
                t = self.source.dense_device(spec.key, dtype)
            else:
                arr = np.array(self.source.dense(spec.key), copy=True, order="C")
                bits = row_bits(self.quant)
                if bits and arr.ndim == 2:
                    # the reference's --quant int4/int8 store hands every 2-D weight out packed and dequantized,
                    # dense ones (the token embedding) included (cacheir/runtime/cpu.py:28-37)
                    arr = unpack_rows(*pack_rows(arr.astype(np.float32), bits), bits, arr.shape[1])
                t = torch.from_numpy(arr).to(self.device).to(dtype)
            self._dense[key] = t.contiguous()
        return self._dense[key]

    def is_blocked(self, names: tuple[str, ...]) -> bool:
        """True when `names` run on the quantized MFMA GEMM (GGUF blocks or the reference's row packing)."""
        keys = [self.specs[n].key for n in names]
        if self.quant in _FMT_OF:
            return True
        if row_bits(self.quant):
            # the tiled layout holds whole 128-column quads; a row-packed weight of another width runs dense
            return all(self._cols(n) % 128 == 0 for n in names)
        return all(self.source.has_blocks(k) for k in keys)

    def _cols(self, name: str) -> int:
        return int(self.specs[name].tensor_type.shape[1])

    def _row_packed(self, names: tuple[str, ...], interleave: bool = False) -> "kernels.QWeight":
        """Per-row asymmetric int4/int8 packing of the concatenated rows of `names` (each row keeps its own scale and
        zero point, exactly as the reference packs each matrix); `interleave` pairs 16-row tiles of two weights."""
        bits = row_bits(self.quant)
        parts = [pack_rows(np.asarray(self.source.dense(self.specs[n].key), dtype=np.float32), bits) for n in names]
        k = int(self.specs[names[0]].tensor_type.shape[1])
        if interleave:
            rows = parts[0][0].shape[0]
            def il(a, b):
                return np.stack([a.reshape(rows // 16, 16, -1), b.reshape(rows // 16, 16, -1)], axis=1).reshape(2 * rows, -1)
            packed = il(parts[0][0], parts[1][0])
            scales = il(parts[0][1][:, None], parts[1][1][:, None]).reshape(-1)
            zps = il(parts[0][2][:, None], parts[1][2][:, None]).reshape(-1)
        else:
            packed = np.concatenate([p[0] for p in parts])
            scales = np.concatenate([p[1] for p in parts])
            zps = np.concatenate([p[2] for p in parts])
        dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(self.device)
        return kernels.QWeight.from_rows(dev(packed), dev(scales), dev(zps), bits, packed.shape[0], k)

    # -- matmul weights: one QWeight (or dense [n, k] tensor) for the concatenation of `names` --
    def matmul_weight(self, names: tuple[str, ...]):
        if names in self._packed:
            return self._packed[names]
        if row_bits(self.quant) and self.is_blocked(names):
            self._packed[names] = self._row_packed(names)
            return self._packed[names]
        if row_bits(self.quant):
            # k is not a multiple of 128 (e.g. the tiny model's ffn 688): the reference's own packed values,
            # dequantized exactly ((q - zero_point) * scale in fp32, as its runtime does at load), on the fp32 GEMM
            bits = row_bits(self.quant)
            dense = [unpack_rows(*pack_rows(np.asarray(self.source.dense(self.specs[n].key), np.float32), bits), bits,
                                 self._cols(n)) for n in names]
            self._packed[names] = torch.from_numpy(np.ascontiguousarray(np.concatenate(dense))).to(self.device)
            return self._packed[names]
        if self.is_blocked(names):
            parts, fmt, k = [], None, None
            for n in names:
                b, f, rows, kk = self._blocks(n)
                if fmt is not None and (f != fmt or kk != k):
                    raise ValueError(f"cannot fuse {names}: mixed block formats or widths")
                fmt, k = f, kk
                parts.append(b)
            cat = torch.cat([p.reshape(-1) for p in parts]).contiguous()
            n_total = sum(self._rows(n) for n in names)
            w = kernels.QWeight.from_blocks(cat, CIR_Q4_0 if fmt == GGML_Q4_0 else CIR_Q8_0, n_total, k)
            del cat, parts
        else:
            w = torch.cat([self.dense(n, torch.float32) for n in names], dim=0).contiguous()
        self._packed[names] = w
        return w

    def swiglu_weight(self, gate: str, up: str) -> "kernels.QWeight":
        """Gate and up block weights as one tiled weight with their 16-row tiles interleaved (gate c, up c, ...),
        the layout ``cir_qgemm_swiglu`` reads."""
        key = (gate, up, "swiglu")
        if key not in self._packed and row_bits(self.quant):
            self._packed[key] = self._row_packed((gate, up), interleave=True)
        if key not in self._packed:
            (gb, gf, rows, k), (ub, uf, rows_u, ku) = self._blocks(gate), self._blocks(up)
            if gf != uf or k != ku or rows != rows_u:
                raise ValueError(f"cannot pair {gate} and {up}: shapes or block formats differ")
            inter = kernels.interleave_gate_up(gb.reshape(rows, -1), ub.reshape(rows, -1), rows)
            self._packed[key] = kernels.QWeight.from_blocks(inter.reshape(-1), CIR_Q4_0 if gf == GGML_Q4_0 else CIR_Q8_0,
                                                            2 * rows, k)
            del gb, ub, inter
        return self._packed[key]

    def _rows(self, name: str) -> int:
        return int(self.specs[name].tensor_type.shape[0])

    def _blocks(self, name: str) -> tuple[torch.Tensor, int, int, int]:
        key = self.specs[name].key
        if isinstance(self.source, SyntheticQuant):
            return self.source.blocks_device(key)
        if self.source.has_blocks(key):
            raw, t, n, k = self.source.blocks(key)
            return torch.from_numpy(np.ascontiguousarray(raw).reshape(-1)).to(self.device), t, n, k
        dense = np.asarray(self.source.dense(key), dtype=np.float32)
        fmt = _FMT_OF[self.quant]
        raw = quantize_q4_0(dense) if fmt == GGML_Q4_0 else quantize_q8_0(dense)
        return torch.from_numpy(raw.reshape(-1)).to(self.device), fmt, dense.shape[0], dense.shape[1]

    def nbytes(self) -> int:
        total = sum(t.numel() * t.element_size() for t in self._dense.values())
        for w in self._packed.values():
            total += w.nbytes if isinstance(w, kernels.QWeight) else w.numel() * w.element_size()
        return total
