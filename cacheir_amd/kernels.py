"""Torch-tensor wrappers over the C ABI, with host-side shape/dtype/bounds checks.

Every wrapper checks on the host that operand shapes, dtypes, devices and
contiguity match what the kernel and its grid assume before anything is launched;
violations raise ``ValueError``/``TypeError`` (mirroring the reference runtime's
error types, ``cacheir/runtime/cuda.py:551-561``).  Page tables can additionally be
range-checked against the pool (``check_tables=True``; costs a device sync).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from cacheir_amd import hip
from cacheir_amd.hip import CIR_F16, CIR_F32, CIR_Q4_0, CIR_Q8_0

QK = 32
BLOCK_BYTES = {CIR_Q4_0: 18, CIR_Q8_0: 34}
FMT_NAMES = {"q4_0": CIR_Q4_0, "q8_0": CIR_Q8_0}


def _req(cond: bool, msg: str, exc=ValueError) -> None:
    if not cond:
        raise exc(msg)


def _cuda(t: torch.Tensor, name: str, rows_only: bool = False) -> None:
    """GPU tensor check; ``rows_only`` accepts a 2-D view whose rows are contiguous (any row stride)."""
    _req(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor", TypeError)
    _req(t.is_cuda, f"{name} must be on the GPU")
    if rows_only:
        _req(t.dim() == 2 and t.stride(1) == 1, f"{name} rows must be contiguous")
    else:
        _req(t.is_contiguous(), f"{name} must be contiguous")


# ------------------------------------------------------------------ attention --
def attention_workspace(rows: int, num_heads: int, head_dim: int, max_context: int, device) -> torch.Tensor:
    n = hip.size_call("cir_paged_attention_workspace_bytes", rows, num_heads, head_dim, max_context)
    # holds split partials O and (max, sum), each written before it is read: no clearing needed
    return torch.empty(max(n, 4), dtype=torch.uint8, device=device)


def _check_pool(q, k_pool, v_pool, page_table, seq_lens, num_heads, check_tables):
    for t, n in ((q, "q"), (k_pool, "k_pool"), (v_pool, "v_pool"), (page_table, "page_table"), (seq_lens, "seq_lens")):
        _cuda(t, n)
    _req(k_pool.dtype == v_pool.dtype == q.dtype, "q, k_pool and v_pool must share a dtype", TypeError)
    _req(k_pool.dim() == 4 and v_pool.shape == k_pool.shape, "pools must be [slots, kv_heads, page_size, head_dim]")
    _req(page_table.dtype == torch.int32 and seq_lens.dtype == torch.int32, "page_table/seq_lens must be int32", TypeError)
    slots, kvh, psize, hd = k_pool.shape
    _req(num_heads % kvh == 0, f"num_heads {num_heads} must be a multiple of kv heads {kvh}")
    if check_tables and page_table.numel():
        _req(int(page_table.min()) >= 0 and int(page_table.max()) < slots, "page_table has slots outside the pool")
        _req(int(seq_lens.max()) <= page_table.shape[1] * psize, "seq_lens exceed the page table capacity")
    return slots, kvh, psize, hd


def paged_decode_attention(q, k_pool, v_pool, page_table, seq_lens, *, scale: float | None = None,
                           out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                           check_tables: bool = False) -> torch.Tensor:
    """q ``[B, Hq, D]`` -> out ``[B, Hq, D]`` over the paged context (decode, one query per sequence)."""
    _req(q.dim() == 3, "q must be [batch, num_heads, head_dim]")
    batch, num_heads, head_dim = q.shape
    _, kvh, psize, hd = _check_pool(q, k_pool, v_pool, page_table, seq_lens, num_heads, check_tables)
    _req(hd == head_dim and page_table.shape[0] == batch and seq_lens.shape == (batch,), "shape mismatch")
    max_pages = page_table.shape[1]
    out = torch.empty_like(q) if out is None else out
    _cuda(out, "out")
    _req(out.shape == q.shape and out.dtype == q.dtype, "out must match q")
    if workspace is None:
        workspace = attention_workspace(batch, num_heads, head_dim, max_pages * psize, q.device)
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    hip.call("cir_paged_decode_attention", q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), page_table.data_ptr(),
             seq_lens.data_ptr(), out.data_ptr(), workspace.data_ptr(), workspace.numel(), batch, num_heads, kvh,
             head_dim, psize, max_pages, float(scale), hip.dtype_code(q.dtype), hip.stream_handle())
    return out


def paged_decode_attention_noalloc(q, k_pool, v_pool, page_table, seq_lens, *, scale: float | None = None,
                                   out: torch.Tensor | None = None) -> torch.Tensor:
    """``paged_decode_attention`` through ``cir_paged_decode_attention_noalloc``: the split partials go to the
    library's static per-GPU scratch (no workspace; calls overlapping on one GPU race).  ``out`` must be given by
    callers that cannot allocate."""
    _req(q.dim() == 3, "q must be [batch, num_heads, head_dim]")
    batch, num_heads, head_dim = q.shape
    _, kvh, psize, hd = _check_pool(q, k_pool, v_pool, page_table, seq_lens, num_heads, False)
    _req(hd == head_dim and page_table.shape[0] == batch and seq_lens.shape == (batch,), "shape mismatch")
    out = torch.empty_like(q) if out is None else out
    _cuda(out, "out")
    _req(out.shape == q.shape and out.dtype == q.dtype, "out must match q")
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    hip.call("cir_paged_decode_attention_noalloc", q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
             page_table.data_ptr(), seq_lens.data_ptr(), out.data_ptr(), batch, num_heads, kvh, head_dim, psize,
             page_table.shape[1], float(scale), hip.dtype_code(q.dtype), hip.stream_handle())
    return out


def paged_decode_attention_qkv(part, inv_freq, positions, k_pool, v_pool, page_table, seq_lens, *, num_heads: int,
                               scale: float | None = None, out: torch.Tensor | None = None,
                               workspace: torch.Tensor | None = None, check_tables: bool = False) -> torch.Tensor:
    """Decode attention fed by the QKV projection's fp32 partials ``[splits, B, (Hq + 2 Hkv) D]``: RoPE, the KV
    append of the new token and attention in one launch (fp16 pools, head_dim 128). Returns out ``[B, Hq, D]``."""
    _cuda(part, "part")
    _req(part.dtype == torch.float32 and part.dim() == 3, "part must be float32 [splits, batch, n]", TypeError)
    splits, batch, n = part.shape
    _req(k_pool.dtype == torch.float16, "the fused QKV attention needs float16 pools", TypeError)
    _, kvh, psize, hd = _check_pool(k_pool, k_pool, v_pool, page_table, seq_lens, num_heads, check_tables)
    _req(n == (num_heads + 2 * kvh) * hd, "qkv partial width must be (num_heads + 2 kv_heads) * head_dim")
    _req(page_table.shape[0] == batch and seq_lens.shape == (batch,), "shape mismatch")
    _cuda(positions, "positions")
    _cuda(inv_freq, "inv_freq")
    _req(positions.dtype == torch.int32 and positions.numel() == batch, "positions must be int32 [batch]", TypeError)
    _req(inv_freq.dtype == torch.float32 and inv_freq.numel() == hd // 2, "inv_freq must be float32 [D/2]", TypeError)
    max_pages = page_table.shape[1]
    if out is None:
        out = torch.empty((batch, num_heads, hd), dtype=k_pool.dtype, device=k_pool.device)
    _cuda(out, "out")
    _req(out.shape == (batch, num_heads, hd) and out.dtype == k_pool.dtype, "out must be [batch, num_heads, head_dim]")
    if workspace is None:
        workspace = attention_workspace(batch, num_heads, hd, max_pages * psize, k_pool.device)
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    hip.call("cir_paged_decode_attention_qkv", part.data_ptr(), splits, inv_freq.data_ptr(), positions.data_ptr(),
             k_pool.data_ptr(), v_pool.data_ptr(), page_table.data_ptr(), seq_lens.data_ptr(), out.data_ptr(),
             workspace.data_ptr(), workspace.numel(), batch, num_heads, kvh, hd, psize, max_pages, float(scale),
             hip.stream_handle())
    return out


def paged_prefill_attention(q, k_pool, v_pool, page_table, seq_lens, q_len: int, *, scale: float | None = None,
                            out=None, workspace=None, check_tables: bool = False) -> torch.Tensor:
    """q ``[B*q_len, Hq, D]``; ``seq_lens`` are lengths after appending the q_len tokens (causal)."""
    _req(q.dim() == 3 and q_len >= 1 and q.shape[0] % q_len == 0, "q must be [batch*q_len, num_heads, head_dim]")
    rows, num_heads, head_dim = q.shape
    batch = rows // q_len
    _, kvh, psize, hd = _check_pool(q, k_pool, v_pool, page_table, seq_lens, num_heads, check_tables)
    _req(hd == head_dim and page_table.shape[0] == batch and seq_lens.shape == (batch,), "shape mismatch")
    max_pages = page_table.shape[1]
    out = torch.empty_like(q) if out is None else out
    if workspace is None:
        workspace = attention_workspace(rows, num_heads, head_dim, max_pages * psize, q.device)
    scale = 1.0 / math.sqrt(head_dim) if scale is None else scale
    hip.call("cir_paged_prefill_attention", q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), page_table.data_ptr(),
             seq_lens.data_ptr(), out.data_ptr(), workspace.data_ptr(), workspace.numel(), batch, q_len, num_heads, kvh,
             head_dim, psize, max_pages, float(scale), hip.dtype_code(q.dtype), hip.stream_handle())
    return out


# -------------------------------------------------------------- block weights --
@dataclass
class QWeight:
    """A Q4_0/Q8_0 (or per-row asymmetric int4/int8) weight ``W[n, k]`` kept on the device in the tiled layout."""

    tiled: torch.Tensor  # uint8
    fmt: int
    n: int
    k: int

    @property
    def shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @property
    def nbytes(self) -> int:
        return self.tiled.numel()

    @classmethod
    def from_rows(cls, packed: torch.Tensor, scales: torch.Tensor, zero_points: torch.Tensor, bits: int, n: int,
                  k: int) -> "QWeight":
        """Repack the reference's per-row asymmetric packing (uint8 codes ``[n, ceil(k/2)]`` for 4 bit or
        ``[n, k]`` for 8 bit, fp32 scales ``[n]``, int32 zero points ``[n]``, on the GPU) into the tiled layout."""
        for t, name in ((packed, "packed"), (scales, "scales"), (zero_points, "zero_points")):
            _cuda(t, name)
        _req(bits in (4, 8), f"bits must be 4 or 8 (got {bits})")
        _req(k % 128 == 0, f"k={k} must be a multiple of 128 for the tiled GEMM")
        row_bytes = (k + 1) // 2 if bits == 4 else k
        _req(packed.dtype == torch.uint8 and packed.numel() == n * row_bytes, "packed codes must be uint8 [n, row_bytes]")
        _req(scales.dtype == torch.float32 and scales.numel() == n, "scales must be float32 [n]", TypeError)
        _req(zero_points.dtype == torch.int32 and zero_points.numel() == n, "zero_points must be int32 [n]", TypeError)
        fmt = hip.CIR_I4_ROW if bits == 4 else hip.CIR_I8_ROW
        size = hip.size_call("cir_qweight_tiled_bytes", fmt, n, k)
        tiled = torch.empty(size, dtype=torch.uint8, device=packed.device)
        hip.call("cir_qweight_repack_rows", packed.data_ptr(), scales.data_ptr(), zero_points.data_ptr(),
                 tiled.data_ptr(), fmt, n, k, hip.stream_handle())
        return cls(tiled, fmt, n, k)

    @classmethod
    def from_blocks(cls, blocks: torch.Tensor, fmt: int, n: int, k: int) -> "QWeight":
        """Repack GGUF blocks (uint8, ``n * k/32 * block_bytes``, on the GPU) into the tiled layout."""
        _cuda(blocks, "blocks")
        _req(fmt in BLOCK_BYTES, f"unsupported block format {fmt}")
        _req(k % 128 == 0, f"k={k} must be a multiple of 128 for the tiled GEMM")
        _req(blocks.dtype == torch.uint8 and blocks.numel() == n * (k // QK) * BLOCK_BYTES[fmt],
             "blocks must be uint8 with n*k/32*block_bytes elements")
        size = hip.size_call("cir_qweight_tiled_bytes", fmt, n, k)
        tiled = torch.empty(size, dtype=torch.uint8, device=blocks.device)
        hip.call("cir_qweight_repack", blocks.data_ptr(), tiled.data_ptr(), fmt, n, k, hip.stream_handle())
        return cls(tiled, fmt, n, k)


def dequant_blocks(blocks: torch.Tensor, fmt: int, n: int, k: int) -> torch.Tensor:
    _cuda(blocks, "blocks")
    _req(blocks.numel() == n * (k // QK) * BLOCK_BYTES[fmt], "block byte count mismatch")
    out = torch.empty((n, k), dtype=torch.float32, device=blocks.device)
    hip.call("cir_dequant", blocks.data_ptr(), 0, fmt, out.data_ptr(), n, k, hip.stream_handle())
    return out


def dequant_tiled(w: QWeight) -> torch.Tensor:
    out = torch.empty((w.n, w.k), dtype=torch.float32, device=w.tiled.device)
    hip.call("cir_dequant", w.tiled.data_ptr(), 1, w.fmt, out.data_ptr(), w.n, w.k, hip.stream_handle())
    return out


def paged_decode_splits(batch: int, num_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                        max_pages: int, kv_dtype: torch.dtype) -> int:
    """Context splits the decode attention uses at these sizes (``cir_paged_decode_splits``)."""
    return hip.load().cir_paged_decode_splits(batch, num_heads, num_kv_heads, head_dim, page_size, max_pages,
                                              hip.dtype_code(kv_dtype))


def paged_decode_attention_qkv_parts(part, inv_freq, positions, k_pool, v_pool, page_table, seq_lens, *,
                                     num_heads: int, workspace: torch.Tensor, scale: float | None = None) -> int:
    """``paged_decode_attention_qkv`` without the merge: the split partials stay in ``workspace`` (O
    ``[B, Hq, S, D]`` fp32 at its start, (max, sum) ``[B, Hq, S, 2]`` after it) for ``qgemm_attn``.
    Returns S (> 1 is required)."""
    _cuda(part, "part")
    _req(part.dtype == torch.float32 and part.dim() == 3, "part must be float32 [splits, batch, n]", TypeError)
    splits, batch, n = part.shape
    _req(k_pool.dtype == torch.float16, "the fused QKV attention needs float16 pools", TypeError)
    _, kvh, psize, hd = _check_pool(k_pool, k_pool, v_pool, page_table, seq_lens, num_heads, False)
    _req(n == (num_heads + 2 * kvh) * hd, "qkv partial width must be (num_heads + 2 kv_heads) * head_dim")
    _req(page_table.shape[0] == batch and seq_lens.shape == (batch,), "shape mismatch")
    _cuda(positions, "positions")
    _cuda(inv_freq, "inv_freq")
    _cuda(workspace, "workspace")
    max_pages = page_table.shape[1]
    S = paged_decode_splits(batch, num_heads, kvh, hd, psize, max_pages, k_pool.dtype)
    _req(S > 1, "the unmerged decode attention needs more than one context split")
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    hip.call("cir_paged_decode_attention_qkv_parts", part.data_ptr(), splits, inv_freq.data_ptr(),
             positions.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), page_table.data_ptr(), seq_lens.data_ptr(),
             workspace.data_ptr(), workspace.numel() * workspace.element_size(), batch, num_heads, kvh, hd, psize,
             max_pages, float(scale), hip.stream_handle())
    return S


def qgemm_attn(workspace: torch.Tensor, attn_splits: int, num_heads: int, w: QWeight, m: int,
               splits: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 partials ``[splits, m, n]`` of ``merge(attention partials) @ W^T`` (``cir_qgemm_attn``): the attention
    output of ``m`` rows, merged from ``workspace`` as ``paged_decode_attention_qkv_parts`` left it, is the input."""
    _cuda(workspace, "workspace")
    _req(w.k == num_heads * 128, "the O projection's k must be num_heads * 128")
    head_dim = 128
    o_floats = m * num_heads * attn_splits * head_dim
    _req(workspace.numel() * workspace.element_size() >= 4 * (o_floats + m * num_heads * attn_splits * 2),
         "workspace smaller than the attention partials")
    splits = choose_splits(m, w.n, w.k) if splits is None else splits
    if out is None:
        out = torch.empty((splits, m, w.n), dtype=torch.float32, device=workspace.device)
    _req(out.numel() >= splits * m * w.n and out.dtype == torch.float32, "partial buffer too small")
    base = workspace.data_ptr()
    hip.call("cir_qgemm_attn", base, base + 4 * o_floats, attn_splits, num_heads, w.tiled.data_ptr(), w.fmt,
             out.data_ptr(), m, w.n, w.k, splits, hip.stream_handle())
    return out.view(-1)[: splits * m * w.n].view(splits, m, w.n)


def gemm_plan(op: int, fmt: int, m: int, n: int, k: int, splits: int = 1) -> str:
    """Name of the kernel the library runs for this GEMM (``cir_qgemm_plan``; op = ``hip.GEMM_*``)."""
    return hip.load().cir_qgemm_plan(op, fmt, m, n, k, splits).decode()


def choose_splits(m: int, n: int, k: int) -> int:
    """k-split the library tunes ``cir_qgemm`` for at this shape (``cir_qgemm_splits``)."""
    s = hip.load().cir_qgemm_splits(m, n, k)
    _req(s > 0, f"no k-split for shape m={m} n={n} k={k} (k must be a positive multiple of 128)")
    return s


def qgemm_partial(x: torch.Tensor, w: QWeight, splits: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 partials ``[splits, m, n]`` of ``x[m, k] @ W[n, k]^T`` (x fp16, rows contiguous, any row stride)."""
    _cuda(x, "x", rows_only=True)
    _req(x.dtype == torch.float16, "qgemm activations must be float16", TypeError)
    _req(x.dim() == 2 and x.shape[1] == w.k, f"x must be [m, {w.k}]")
    _req(x.stride(1) == 1 and x.stride(0) >= w.k, "x rows must be contiguous (row stride >= k)")
    m = x.shape[0]
    splits = choose_splits(m, w.n, w.k) if splits is None else splits
    if out is None:
        out = torch.empty((splits, m, w.n), dtype=torch.float32, device=x.device)
    _req(out.numel() >= splits * m * w.n and out.dtype == torch.float32, "partial buffer too small")
    hip.call("cir_qgemm", x.data_ptr(), x.stride(0), w.tiled.data_ptr(), w.fmt, out.data_ptr(), m, w.n, w.k, splits,
             hip.stream_handle())
    return out.view(-1)[: splits * m * w.n].view(splits, m, w.n)


def interleave_gate_up(gate_blocks: torch.Tensor, up_blocks: torch.Tensor, rows: int) -> torch.Tensor:
    """GGUF block rows of gate and up ([rows, row_bytes] each, uint8) -> [2*rows, row_bytes] in the order
    gate 16c..16c+15, up 16c..16c+15, c = 0, 1, ... (the tile pairing ``cir_qgemm_swiglu`` reads)."""
    _req(rows % 16 == 0, "gate/up rows must be a multiple of 16")
    g = gate_blocks.reshape(rows // 16, 1, 16, -1)
    u = up_blocks.reshape(rows // 16, 1, 16, -1)
    return torch.cat([g, u], dim=1).reshape(2 * rows, -1).contiguous()


def qgemm_swiglu(x: torch.Tensor, w: QWeight, out_dtype: torch.dtype = torch.float16, out=None) -> torch.Tensor:
    """``silu(x @ gate^T) * (x @ up^T)`` from the interleaved gate|up tiled weight (``interleave_gate_up``)."""
    _cuda(x, "x", rows_only=True)
    _req(x.dtype == torch.float16, "qgemm activations must be float16", TypeError)
    _req(x.dim() == 2 and x.shape[1] == w.k and w.n % 32 == 0, f"x must be [m, {w.k}] and n a multiple of 32")
    m, inter = x.shape[0], w.n // 2
    if out is None:
        out = torch.empty((m, inter), dtype=out_dtype, device=x.device)
    _req(out.shape == (m, inter) and out.is_contiguous(), "out must be [m, n/2] contiguous")
    hip.call("cir_qgemm_swiglu", x.data_ptr(), x.stride(0), w.tiled.data_ptr(), w.fmt, out.data_ptr(),
             hip.dtype_code(out.dtype), m, inter, w.k, hip.stream_handle())
    return out


def qgemm_argmax_workspace(m: int, n: int, device) -> torch.Tensor:
    return torch.empty(max(hip.size_call("cir_qgemm_argmax_workspace_bytes", m, n), 4), dtype=torch.uint8,
                       device=device)


def qgemm_argmax(x: torch.Tensor, w: QWeight, out=None, workspace=None) -> torch.Tensor:
    """Greedy ids ``argmax_j (x @ W^T)[r, j]`` without storing the logits (first index on ties, NaN as the
    maximum); equal to ``argmax(qgemm_partial(x, w, splits=1)[0])``."""
    _cuda(x, "x", rows_only=True)
    _req(x.dtype == torch.float16, "qgemm activations must be float16", TypeError)
    _req(x.dim() == 2 and x.shape[1] == w.k, f"x must be [m, {w.k}]")
    m = x.shape[0]
    if out is None:
        out = torch.empty(m, dtype=torch.int64, device=x.device)
    _req(out.dtype == torch.int64 and out.numel() == m and out.is_contiguous(), "out must be int64 [m]", TypeError)
    if workspace is None:
        workspace = qgemm_argmax_workspace(m, w.n, x.device)
    hip.call("cir_qgemm_argmax", x.data_ptr(), x.stride(0), w.tiled.data_ptr(), w.fmt, out.data_ptr(),
             workspace.data_ptr(), workspace.numel() * workspace.element_size(), m, w.n, w.k, hip.stream_handle())
    return out


def gemm_f32_partial(x: torch.Tensor, w: torch.Tensor, splits: int = 1, out=None) -> torch.Tensor:
    _cuda(x, "x")
    _cuda(w, "w")
    _req(x.dtype == torch.float32 and w.dtype == torch.float32, "gemm_f32 needs float32 x and w", TypeError)
    _req(x.dim() == 2 and w.dim() == 2 and x.shape[1] == w.shape[1], "x [m,k] and w [n,k] required")
    m, k = x.shape
    n = w.shape[0]
    if out is None:
        out = torch.empty((splits, m, n), dtype=torch.float32, device=x.device)
    hip.call("cir_gemm_f32", x.data_ptr(), k, w.data_ptr(), out.data_ptr(), m, n, k, splits, hip.stream_handle())
    return out.view(-1)[: splits * m * n].view(splits, m, n)


# ------------------------------------------------------------------ epilogues --
def epilogue_store(part: torch.Tensor, out_dtype: torch.dtype, residual: torch.Tensor | None = None, out=None):
    splits, m, n = part.shape
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=part.device)
    if residual is not None:
        _cuda(residual, "residual")
        _req(residual.numel() == m * n and residual.dtype == out.dtype, "residual must match the output")
    hip.call("cir_epilogue_store", part.data_ptr(), splits, hip.ptr(residual), out.data_ptr(), hip.dtype_code(out.dtype),
             m, n, hip.stream_handle())
    return out


def epilogue_residual_rmsnorm(part: torch.Tensor, residual: torch.Tensor, norm_w: torch.Tensor, eps: float,
                              h_out: torch.Tensor, xn_out: torch.Tensor):
    """h_out = residual + sum(part) (fp32); xn_out = RMSNorm(h_out) * norm_w (GEMM input dtype)."""
    splits, m, n = part.shape
    for t, nm in ((residual, "residual"), (h_out, "h_out"), (xn_out, "xn_out"), (norm_w, "norm_w")):
        _cuda(t, nm)
    _req(residual.dtype == torch.float32 and h_out.dtype == torch.float32, "residual/h_out must be float32", TypeError)
    _req(residual.numel() == m * n and h_out.numel() == m * n and xn_out.numel() == m * n and norm_w.numel() == n,
         "residual_rmsnorm shape mismatch")
    hip.call("cir_epilogue_residual_rmsnorm", part.data_ptr(), splits, residual.data_ptr(), h_out.data_ptr(),
             norm_w.data_ptr(), hip.dtype_code(norm_w.dtype), float(eps), xn_out.data_ptr(),
             hip.dtype_code(xn_out.dtype), m, n, hip.stream_handle())
    return h_out, xn_out


def epilogue_swiglu(part: torch.Tensor, out_dtype: torch.dtype, out=None):
    splits, m, n2 = part.shape
    _req(n2 % 2 == 0, "swiglu partials need gate|up columns")
    inter = n2 // 2
    if out is None:
        out = torch.empty((m, inter), dtype=out_dtype, device=part.device)
    hip.call("cir_epilogue_swiglu", part.data_ptr(), splits, out.data_ptr(), hip.dtype_code(out.dtype), m, inter,
             hip.stream_handle())
    return out


def epilogue_qkv_rope_append(part, inv_freq, positions, page_table, q_out, k_pool, v_pool, *, batch: int, q_len: int,
                             num_heads: int, num_kv_heads: int, head_dim: int) -> torch.Tensor:
    splits, rows, n = part.shape
    _req(rows == batch * q_len and n == (num_heads + 2 * num_kv_heads) * head_dim, "qkv partial shape mismatch")
    _req(positions.dtype == torch.int32 and positions.numel() == batch, "positions must be int32 [batch]")
    _req(page_table.dtype == torch.int32 and page_table.shape[0] == batch, "page_table must be int32 [batch, pages]")
    _req(k_pool.shape[1:] == (num_kv_heads, k_pool.shape[2], head_dim), "pool shape mismatch")
    _req(inv_freq.numel() == head_dim // 2 and inv_freq.dtype == torch.float32, "inv_freq must be float32 [D/2]")
    hip.call("cir_epilogue_qkv_rope_append", part.data_ptr(), splits, inv_freq.data_ptr(), positions.data_ptr(),
             page_table.data_ptr(), page_table.shape[1], q_out.data_ptr(), hip.dtype_code(q_out.dtype),
             k_pool.data_ptr(), v_pool.data_ptr(), hip.dtype_code(k_pool.dtype), batch, q_len, num_heads,
             num_kv_heads, head_dim, k_pool.shape[2], hip.stream_handle())
    return q_out


# ---------------------------------------------------------------- row kernels --
def embedding(ids: torch.Tensor, table: torch.Tensor, out_dtype: torch.dtype, out=None) -> torch.Tensor:
    _cuda(ids, "ids")
    _cuda(table, "table")
    _req(ids.dtype == torch.int64, "ids must be int64", TypeError)
    rows = ids.numel()
    vocab, hidden = table.shape
    if out is None:
        out = torch.empty((rows, hidden), dtype=out_dtype, device=table.device)
    hip.call("cir_embedding", ids.data_ptr(), table.data_ptr(), hip.dtype_code(table.dtype), out.data_ptr(),
             hip.dtype_code(out.dtype), rows, hidden, vocab, hip.stream_handle())
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out_dtype: torch.dtype, out=None) -> torch.Tensor:
    _cuda(x, "x")
    _cuda(w, "w")
    hidden = x.shape[-1]
    _req(w.numel() == hidden, "norm weight size mismatch")
    rows = x.numel() // hidden
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    hip.call("cir_rmsnorm", x.data_ptr(), hip.dtype_code(x.dtype), w.data_ptr(), hip.dtype_code(w.dtype),
             out.data_ptr(), hip.dtype_code(out.dtype), rows, hidden, float(eps), hip.stream_handle())
    return out


def add(a: torch.Tensor, b: torch.Tensor, out=None) -> torch.Tensor:
    _cuda(a, "a")
    _cuda(b, "b")
    _req(a.shape == b.shape and a.dtype == b.dtype, "add operands must match")
    out = torch.empty_like(a) if out is None else out
    hip.call("cir_add", a.data_ptr(), b.data_ptr(), out.data_ptr(), hip.dtype_code(a.dtype), a.numel(),
             hip.stream_handle())
    return out


def cast(x: torch.Tensor, dtype: torch.dtype, out=None) -> torch.Tensor:
    _cuda(x, "x")
    out = torch.empty(x.shape, dtype=dtype, device=x.device) if out is None else out
    _req(out.numel() == x.numel(), "cast: size mismatch")
    hip.call("cir_cast", x.data_ptr(), hip.dtype_code(x.dtype), out.data_ptr(), hip.dtype_code(out.dtype), x.numel(),
             hip.stream_handle())
    return out


def argmax(logits: torch.Tensor, out=None) -> torch.Tensor:
    _cuda(logits, "logits")
    _req(logits.dtype == torch.float32 and logits.dim() == 2, "logits must be float32 [rows, vocab]")
    rows, vocab = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    hip.call("cir_argmax", logits.data_ptr(), vocab, out.data_ptr(), rows, vocab, hip.stream_handle())
    return out


def stream_read(buf: torch.Tensor, workgroups: int, threads: int, layout: int, out: torch.Tensor,
                side: torch.Tensor | None = None, side_ratio: int = 0) -> None:
    """Read every byte of ``buf`` (``cir_stream_read``; read-bandwidth calibration, not on the decode path), with
    ``side_ratio`` 16-byte reads of the L2-resident ``side`` per 8 of ``buf``."""
    _cuda(buf, "buf")
    _cuda(out, "out")
    sp, sb = 0, 0
    if side is not None:
        _cuda(side, "side")
        sp, sb = side.data_ptr(), side.numel() * side.element_size()
    hip.call("cir_stream_read", buf.data_ptr(), buf.numel() * buf.element_size(), int(workgroups), int(threads),
             int(layout), sp, sb, int(side_ratio), out.data_ptr(), hip.stream_handle())
