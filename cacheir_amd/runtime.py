"""``HipRuntime``: the ROCm backend's artifact runtime for CacheIR decode graphs.

Duck-typed to the reference ``CudaRuntime`` (``cacheir/runtime/cuda.py:430-1263``)
so the scheduler, benchmark and server can drive it unchanged:
``run(input_ids, mode=, reset_kv=)``, ``run_decode_batch(sessions, token_ids)``,
``run_prefill_batch(sessions, batches)``, ``prefill_tokens``, ``generate``,
``generate_ids``, ``fork()``, ``synchronize()``, ``cache_stats()`` and the
attributes ``artifact, tokenizer, prefix_cache, kv_cache, kv_allocator,
supports_variable_prefill_batch``.  Error types follow the reference
(``ValueError`` / ``TypeError`` / ``NotImplementedError`` / ``RuntimeError``,
``cuda.py:551-561,777,531-536``).

Execution: each (mode, batch, tokens-per-sequence, page-table width) gets a
``StepPlan`` -- the lowered graph translated once into a list of C-ABI launches
over static device buffers.  The host only fills the token ids, positions and page
table per step; a plan can be captured into a HIP graph and replayed
(``cacheir/backends/cuda_graphs.py:38-55`` names exactly these static inputs).
Fusions done at plan time (semantics unchanged):
* ``fused_rmsnorm_qkv_rope``: RMSNorm -> one GEMM over Q|K|V -> epilogue that
  applies interleaved RoPE at the pre-append position and writes K/V straight into
  the page pool, i.e. the append the attention node would do (``cpu.py:239-241,352``);
* ``matmul`` whose only consumer is a residual ``add``: the add runs in the GEMM
  epilogue;
* ``fused_swiglu``: one GEMM over gate|up, SiLU-mul in the epilogue.
There is no CPU fallback anywhere on this path.
"""
from __future__ import annotations

import itertools
import json
from collections import OrderedDict
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable

import numpy as np
import torch

from cacheir_amd import hip, kernels
from cacheir_amd.artifact import CompileArtifact
from cacheir_amd.ir import Graph, Node
from cacheir_amd.kv import HipKVPageAllocator, HipPagedKVCache
from cacheir_amd.weights import GGUFSource, HipWeightStore, NpzDir, SyntheticQuant, row_bits

_QKV_OPS = {"fused_rmsnorm_qkv_rope", "quantized_fused_rmsnorm_qkv_rope"}
_SWIGLU_OPS = {"fused_swiglu", "quantized_fused_swiglu"}
_MATMUL_OPS = {"matmul", "quantized_matmul"}
_ATTN_OPS = {"paged_attention_decode", "paged_attention_prefill", "grouped_query_attention"}
_GGUF_KEYS = {"model.embed_tokens.weight": "token_embd.weight", "model.norm.weight": "output_norm.weight",
              "lm_head.weight": "output.weight"}
_GGUF_LAYER_KEYS = {"input_layernorm.weight": "attn_norm.weight", "self_attn.q_proj.weight": "attn_q.weight",
                    "self_attn.k_proj.weight": "attn_k.weight", "self_attn.v_proj.weight": "attn_v.weight",
                    "self_attn.o_proj.weight": "attn_output.weight",
                    "post_attention_layernorm.weight": "ffn_norm.weight", "mlp.gate_proj.weight": "ffn_gate.weight",
                    "mlp.up_proj.weight": "ffn_up.weight", "mlp.down_proj.weight": "ffn_down.weight"}


def hip_runtime_available() -> bool:
    return bool(torch.cuda.is_available() and hip.LIB_PATH.exists())


def gguf_key_map(num_layers: int) -> dict[str, str]:
    """HF weight names -> GGUF tensor names (the mapping of ``cacheir/compiler.py:85-107``)."""
    m = dict(_GGUF_KEYS)
    for layer in range(num_layers):
        for hf, gg in _GGUF_LAYER_KEYS.items():
            m[f"model.layers.{layer}.{hf}"] = f"blk.{layer}.{gg}"
    return m


def rope_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """``1 / theta ** (arange(0, D/2, float32) * 2 / D)`` evaluated in float32 as ``cpu.py:330`` does."""
    return (1.0 / (theta ** (np.arange(0, head_dim // 2, dtype=np.float32) * 2.0 / head_dim))).astype(np.float32)


class ByteTokenizer:
    """Byte tokenizer with the reference's encode/decode rules (``cacheir/runtime/tokenizer.py:7-23``)."""

    def __init__(self, vocab_size: int):
        self.vocab_size = max(1, int(vocab_size))

    def encode(self, text: str) -> list[int]:
        if not isinstance(text, str):
            raise TypeError("encode expects a string prompt")
        return [b % self.vocab_size for b in (text.encode("utf-8") or b"\x00")]

    def decode(self, ids: Iterable[int]) -> str:
        return "".join(chr(v) if 32 <= v <= 126 else f"<{v}>" for v in (int(i) % self.vocab_size for i in ids))


@dataclass
class PrefixPages:
    """A cached prefix: the slots holding its K/V (one reference held by the cache) and its length."""

    allocator: HipKVPageAllocator
    slots: list[int]
    tokens: int

    def release(self) -> None:
        self.allocator.release(self.slots)
        self.slots = []


class PrefixCache:
    """LRU map ``token prefix -> pages`` (``cacheir/runtime/kv_cache.py:262-307`` semantics).

    The reference stores host snapshots of a prefix's KV and copies them back into a
    new session.  Here an entry holds a reference to the prefix's device pages and a
    hit aliases them into the new session's page table (``HipPagedKVCache.alias_prefix``):
    no copy, and sequences that share a prompt prefix read the same pages."""

    def __init__(self, capacity: int = 8):
        self.capacity = max(1, int(capacity))
        self._entries: OrderedDict[tuple[int, ...], Any] = OrderedDict()
        self.hits = self.misses = self.evictions = 0

    def put(self, token_ids, snapshot) -> None:
        key = tuple(int(t) for t in token_ids)
        old = self._entries.pop(key, None)
        if old is not None and hasattr(old, "release"):
            old.release()
        self._entries[key] = snapshot
        while len(self._entries) > self.capacity:
            _, ev = self._entries.popitem(last=False)
            if hasattr(ev, "release"):
                ev.release()
            self.evictions += 1

    def longest_prefix(self, token_ids):
        query = tuple(int(t) for t in token_ids)
        best, value = (), None
        for key, snap in self._entries.items():
            if len(key) > len(best) and query[: len(key)] == key:
                best, value = key, snap
        if value is not None:
            self._entries.move_to_end(best)
            self.hits += 1
        else:
            self.misses += 1
        return best, value

    def clear(self) -> None:
        for v in self._entries.values():
            if hasattr(v, "release"):
                v.release()
        self._entries.clear()

    def stats(self) -> dict[str, int]:
        return {"capacity": self.capacity, "entries": len(self._entries), "hits": self.hits, "misses": self.misses,
                "evictions": self.evictions}


# ============================================================================ plan ==
class StepPlan:
    """One graph translated into C-ABI launches over static buffers."""

    def __init__(self, rt: "HipRuntime", mode: str, batch: int, q_len: int, max_pages: int):
        self.rt, self.mode, self.batch, self.q_len, self.max_pages = rt, mode, batch, q_len, max_pages
        self.generation = rt.kv_allocator.generation
        dev = rt.device
        self.rows = rows = batch * q_len
        # The step inputs live in one int32 device buffer (ids as int64 pairs, positions, seq_lens, page table)
        # filled from one pinned host buffer by one copy per step; the launches below read these views, so a
        # captured graph replays with whatever the last copy wrote.
        self._in_pos = 2 * rows
        self._in_len = self._in_pos + batch
        self._in_pt = self._in_len + batch
        total = self._in_pt + batch * max_pages
        self._in_dev = torch.zeros(total, dtype=torch.int32, device=dev)
        self._in_host = torch.zeros(total, dtype=torch.int32, pin_memory=True)
        self._in_np = self._in_host.numpy()
        self._in_copied = torch.cuda.Event()
        self._in_pending = False
        self.ids = self._in_dev[: 2 * rows].view(torch.int64)
        self.positions = self._in_dev[self._in_pos: self._in_len]
        self.seq_lens = self._in_dev[self._in_len: self._in_pt]
        self.page_table = self._in_dev[self._in_pt:].view(batch, max_pages)
        self.launches: list = []
        self.graph_obj: torch.cuda.CUDAGraph | None = None
        self.graphs: dict[str, torch.cuda.CUDAGraph] = {}  # "logits" / "greedy" -> captured step
        self.replays = 0
        self._head: tuple | None = None  # (x, lm_head weight, workspace) when the greedy head can be fused
        self._head_at = 0
        self._gemm_need = 1
        self._logits_swappable = False  # the logits GEMM writes ``self.logits`` as found at launch
        self._build(rt.artifact.graph(mode))
        self.gemm_ws = torch.empty(self._gemm_need, dtype=torch.float32, device=dev)
        attn_need = kernels.hip.size_call("cir_paged_attention_workspace_bytes", rows, rt.config.num_attention_heads,
                                          rt.config.head_dim, max_pages * rt.kv_allocator.page_size)
        # split partials of the attention (and of the O projection's merge at batch <= 8): every launch writes
        # what it later reads, so the buffer needs no clearing
        self.attn_ws = torch.empty(max(attn_need, 4), dtype=torch.uint8, device=dev)

    # ------------------------------------------------------------------ build --
    def _fuse_qkv_into_attention(self, users, k_pool: torch.Tensor, head_dim: int) -> bool:
        """Decode steps whose q feeds only decode attention over fp16 pages (head_dim 128) run the QKV
        epilogue inside the attention kernel (``cir_paged_decode_attention_qkv``)."""
        cfg = self.rt.config
        return (self.q_len == 1 and bool(users) and all(u.op == "paged_attention_decode" for u in users)
                and k_pool.dtype == torch.float16 and self.rt.dtype == torch.float16 and head_dim == 128
                and k_pool.shape[2] % 16 == 0 and cfg.num_attention_heads // cfg.num_key_value_heads <= 8)

    def _build(self, graph: Graph) -> None:
        rt, rows = self.rt, self.rows
        consumers = graph.consumers()
        env: dict[str, Any] = {}
        skip: set[int] = set()
        normed: dict[tuple[str, str], torch.Tensor] = {}  # (value, norm weight) -> RMSNorm already computed
        self.logits_name = graph.outputs[0]

        def gemm_dtype(weight) -> torch.dtype:
            return torch.float16 if isinstance(weight, kernels.QWeight) else torch.float32

        def input_dtype_for(value: str) -> torch.dtype | None:
            """The dtype the first matmul-family consumer of ``value`` wants, if any."""
            for c in consumers.get(value, []):
                # decided from the weight format, without packing a weight the plan may never use
                if c.op in _MATMUL_OPS:
                    return torch.float16 if rt.weights.is_blocked((c.inputs[1],)) else torch.float32
                if c.op in _SWIGLU_OPS:
                    return torch.float16 if rt.weights.is_blocked((c.inputs[1], c.inputs[2])) else torch.float32
            return None

        def buf(n: int, dtype: torch.dtype) -> torch.Tensor:
            return torch.empty((rows, n), dtype=dtype, device=rt.device)

        def as_dtype(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
            if t.dtype == dtype:
                return t
            out = torch.empty(t.shape, dtype=dtype, device=t.device)
            self.launches.append(lambda t=t, out=out: kernels.cast(t, out.dtype, out=out))
            return out

        def gemm(x, weight) -> tuple[Any, int, int]:
            """Queue the GEMM into the shared workspace; returns (partials getter, splits, n).  ``x`` may be the
            marker of split attention partials left in the attention workspace (merged by the GEMV)."""
            if isinstance(x, tuple) and x[0] == "attn-parts":
                _, S, heads = x
                n, k = weight.n, weight.k
                splits = kernels.choose_splits(rows, n, k)
                self._gemm_need = max(self._gemm_need, splits * rows * n)
                self.launches.append(lambda w=weight, s=splits, S=S, h=heads: kernels.qgemm_attn(
                    self.attn_ws, S, h, w, rows, splits=s, out=self.gemm_ws))
                rt._count("rocm.attn_merge_qgemv")
                rt._record_gemm_plan(hip.GEMM_ATTN_MERGE, weight, rows, splits)
                part = lambda s=splits, n=n: self.gemm_ws[: s * rows * n].view(s, rows, n)
                return part, splits, n
            if isinstance(weight, kernels.QWeight):
                n, k = weight.n, weight.k
                splits = kernels.choose_splits(rows, n, k)
                x = as_dtype(x, torch.float16)
                self._gemm_need = max(self._gemm_need, splits * rows * n)
                self.launches.append(lambda x=x, w=weight, s=splits: kernels.qgemm_partial(x, w, splits=s,
                                                                                           out=self.gemm_ws))
                rt._count("rocm.qgemm_blocks")
                rt._record_gemm_plan(hip.GEMM_PARTIALS, weight, rows, splits)
            else:
                n, k = weight.shape
                splits = 1
                x = as_dtype(x, torch.float32)
                self._gemm_need = max(self._gemm_need, rows * n)
                self.launches.append(lambda x=x, w=weight: kernels.gemm_f32_partial(x, w, splits=1, out=self.gemm_ws))
                rt._count("rocm.gemm_f32")
            part = lambda s=splits, n=n: self.gemm_ws[: s * rows * n].view(s, rows, n)
            return part, splits, n

        for idx, node in enumerate(graph.nodes):
            if idx in skip:
                continue
            op, ins, outs, attrs = node.op, node.inputs, node.outputs, node.attrs
            if op == "token_embedding":
                table = rt.weights.dense(ins[1], rt.dense_dtype)
                out = buf(table.shape[1], torch.float32)
                self.launches.append(lambda t=table, o=out: kernels.embedding(self.ids, t, torch.float32, out=o))
                env[outs[0]] = out
            elif op in _QKV_OPS:
                layer = int(attrs.get("layer", 0))
                x = env[ins[0]]
                W = rt.weights.matmul_weight(tuple(ins[2:5]))
                xn = normed.get((ins[0], ins[1]))
                if xn is None or xn.dtype != gemm_dtype(W):
                    w_norm = rt.weights.dense(ins[1], rt.dense_dtype)
                    xn = buf(x.shape[1], gemm_dtype(W))
                    eps = float(attrs.get("eps", 1e-6))
                    self.launches.append(lambda x=x, w=w_norm, o=xn, e=eps: kernels.rmsnorm(x, w, e, o.dtype, out=o))
                part, _, _ = gemm(xn, W)
                cfg = rt.config
                hd = int(attrs.get("head_dim", cfg.head_dim))
                inv = rt.inv_freq(hd, float(attrs.get("rope_theta", cfg.rope_theta)))
                kp, vp = rt.kv_allocator.layer_pools(layer)
                if self._fuse_qkv_into_attention(consumers.get(outs[0], []), kp, hd):
                    # RoPE + KV append happen inside the decode attention kernel that consumes q
                    env[outs[0]] = ("qkv-partials", part, inv, layer)
                    env[outs[1]], env[outs[2]] = ("kv-appended", layer), ("kv-appended", layer)
                    rt._count("rocm.rmsnorm_qkv")
                    continue
                q_out = buf(cfg.num_attention_heads * hd, rt.dtype)
                self.launches.append(lambda part=part, inv=inv, q=q_out, kp=kp, vp=vp, hd=hd:
                                     kernels.epilogue_qkv_rope_append(
                                         part(), inv, self.positions, self.page_table, q, kp, vp, batch=self.batch,
                                         q_len=self.q_len, num_heads=cfg.num_attention_heads,
                                         num_kv_heads=cfg.num_key_value_heads, head_dim=hd))
                rt._count("rocm.rmsnorm_qkv_rope_kv_append")
                env[outs[0]], env[outs[1]], env[outs[2]] = q_out, ("kv-appended", layer), ("kv-appended", layer)
            elif op in _ATTN_OPS:
                layer = int(attrs.get("layer", 0))
                if env.get(ins[1]) != ("kv-appended", layer) or env.get(ins[2]) != ("kv-appended", layer):
                    raise NotImplementedError(
                        f"{node.name}: attention whose K/V are not produced by fused_rmsnorm_qkv_rope of layer {layer}")
                heads, hd = int(attrs["num_heads"]), int(attrs["head_dim"])
                out = buf(heads * hd, rt.dtype)
                kp, vp = rt.kv_allocator.layer_pools(layer)
                qin = env[ins[0]]
                if isinstance(qin, tuple) and qin[0] == "qkv-partials" and self._merge_into_o(
                        consumers.get(outs[0], []), outs[0], graph, heads, hd, kp):
                    # the split partials stay in the workspace; the O projection's GEMV merges them
                    _, part, inv, _ = qin
                    S = kernels.paged_decode_splits(self.batch, heads, kp.shape[1], hd, kp.shape[2], self.max_pages,
                                                    kp.dtype)
                    def attn_parts(part=part, inv=inv, kp=kp, vp=vp, h=heads, S=S):
                        got = kernels.paged_decode_attention_qkv_parts(
                            part(), inv, self.positions, kp, vp, self.page_table, self.seq_lens, num_heads=h,
                            workspace=self.attn_ws)
                        if got != S:  # the O projection below reads the workspace laid out for S splits
                            raise RuntimeError(f"decode attention used {got} context splits, the plan expects {S}")

                    self.launches.append(attn_parts)
                    rt._count("rocm.rope_kv_append_paged_attention_decode_parts")
                    env[outs[0]] = ("attn-parts", S, heads)
                    continue
                if isinstance(qin, tuple) and qin[0] == "qkv-partials":
                    _, part, inv, _ = qin
                    ov = out.view(rows, heads, hd)
                    self.launches.append(lambda part=part, inv=inv, ov=ov, kp=kp, vp=vp, h=heads:
                                         kernels.paged_decode_attention_qkv(
                                             part(), inv, self.positions, kp, vp, self.page_table, self.seq_lens,
                                             num_heads=h, out=ov, workspace=self.attn_ws))
                    rt._count("rocm.rope_kv_append_paged_attention_decode")
                    env[outs[0]] = out
                    continue
                q = as_dtype(qin, rt.dtype)
                decode = op == "paged_attention_decode" and self.q_len == 1
                qv, ov = q.view(rows, heads, hd), out.view(rows, heads, hd)
                if decode:
                    self.launches.append(lambda qv=qv, ov=ov, kp=kp, vp=vp: kernels.paged_decode_attention(
                        qv, kp, vp, self.page_table, self.seq_lens, out=ov, workspace=self.attn_ws))
                else:
                    self.launches.append(lambda qv=qv, ov=ov, kp=kp, vp=vp: kernels.paged_prefill_attention(
                        qv, kp, vp, self.page_table, self.seq_lens, self.q_len, out=ov, workspace=self.attn_ws))
                rt._count("rocm.paged_attention_decode" if decode else "rocm.paged_attention_prefill")
                env[outs[0]] = out
            elif op in _MATMUL_OPS:
                W = rt.weights.matmul_weight((ins[1],))
                if outs[0] == self.logits_name and isinstance(W, kernels.QWeight):
                    # greedy steps may replace this GEMM + store by the fused head (cir_qgemm_argmax)
                    x16 = as_dtype(env[ins[0]], torch.float16)
                    self._head_at = len(self.launches)
                    self._head = (x16, W, kernels.qgemm_argmax_workspace(rows, W.n, rt.device))
                    rt._record_gemm_plan(hip.GEMM_ARGMAX, W, rows, 1)
                    env[ins[0]] = x16
                users = consumers.get(outs[0], [])
                fuse = (len(users) == 1 and users[0].op == "add" and outs[0] in users[0].inputs
                        and outs[0] not in graph.outputs)
                if (not fuse and isinstance(W, kernels.QWeight) and not isinstance(env[ins[0]], tuple)
                        and kernels.choose_splits(rows, W.n, W.k) == 1):
                    # one k-split: the GEMM's fp32 partial plane is the output itself (the store epilogue would
                    # copy it bit for bit).  The logits GEMM writes whichever buffer ``self.logits`` holds at
                    # launch, so an eager plan can hand its logits to the caller (``take_logits``).
                    x = as_dtype(env[ins[0]], torch.float16)
                    out = buf(W.n, torch.float32)
                    is_logits = outs[0] == self.logits_name
                    self.launches.append(lambda x=x, w=W, o=out, lg=is_logits: kernels.qgemm_partial(
                        x, w, splits=1, out=self.logits if lg else o))
                    self._logits_swappable |= is_logits
                    rt._count("rocm.qgemm_blocks")
                    rt._record_gemm_plan(hip.GEMM_PARTIALS, W, rows, 1)
                    env[outs[0]] = out
                    continue
                part, _, n = gemm(env[ins[0]], W)
                if fuse:
                    add = users[0]
                    other = add.inputs[1] if add.inputs[0] == outs[0] else add.inputs[0]
                    resid = as_dtype(env[other], torch.float32)
                    out = buf(n, torch.float32)
                    env[add.outputs[0]] = out
                    skip.add(graph.nodes.index(add))
                    norm = self._normalizer(consumers.get(add.outputs[0], []), add.outputs[0])
                    if norm is not None:
                        # residual add and the RMSNorm that reads its result in one kernel
                        nw_name = norm.inputs[1]
                        nw = rt.weights.dense(nw_name, rt.dense_dtype)
                        if norm.op == "rms_norm":
                            xdt = input_dtype_for(norm.outputs[0]) or torch.float32
                        else:
                            xdt = gemm_dtype(rt.weights.matmul_weight(tuple(norm.inputs[2:5])))
                        xn = buf(n, xdt)
                        eps = float(norm.attrs.get("eps", 1e-6))
                        self.launches.append(lambda part=part, r=resid, o=out, nw=nw, e=eps, xn=xn:
                                             kernels.epilogue_residual_rmsnorm(part(), r, nw, e, o, xn))
                        normed[(add.outputs[0], nw_name)] = xn
                        if norm.op == "rms_norm":
                            env[norm.outputs[0]] = xn
                            skip.add(graph.nodes.index(norm))
                    else:
                        self.launches.append(lambda part=part, r=resid, o=out: kernels.epilogue_store(
                            part(), o.dtype, residual=r, out=o))
                else:
                    out = buf(n, torch.float32)
                    self.launches.append(lambda part=part, o=out: kernels.epilogue_store(part(), o.dtype, out=o))
                    env[outs[0]] = out
            elif op == "add":
                a, b = as_dtype(env[ins[0]], torch.float32), as_dtype(env[ins[1]], torch.float32)
                out = buf(a.shape[1], torch.float32)
                self.launches.append(lambda a=a, b=b, o=out: kernels.add(a, b, out=o))
                env[outs[0]] = out
            elif op == "rms_norm":
                x = env[ins[0]]
                w = rt.weights.dense(ins[1], rt.dense_dtype)
                odt = input_dtype_for(outs[0]) or torch.float32
                out = buf(x.shape[1], odt)
                eps = float(attrs.get("eps", 1e-6))
                self.launches.append(lambda x=x, w=w, o=out, e=eps: kernels.rmsnorm(x, w, e, o.dtype, out=o))
                env[outs[0]] = out
            elif op in _SWIGLU_OPS:
                odt = input_dtype_for(outs[0]) or torch.float32
                inter = rt.weights._rows(ins[1])
                if rt.weights.is_blocked((ins[1], ins[2])) and inter % 16 == 0:
                    # gate|up GEMM with the SwiGLU applied in registers (interleaved gate/up tiles)
                    W = rt.weights.swiglu_weight(ins[1], ins[2])
                    x = as_dtype(env[ins[0]], torch.float16)
                    out = buf(inter, odt)
                    self.launches.append(lambda x=x, w=W, o=out: kernels.qgemm_swiglu(x, w, o.dtype, out=o))
                    rt._count("rocm.qgemm_swiglu")
                    rt._record_gemm_plan(hip.GEMM_SWIGLU, W, rows, 1)
                    env[outs[0]] = out
                    continue
                W = rt.weights.matmul_weight((ins[1], ins[2]))
                part, _, n2 = gemm(env[ins[0]], W)
                out = buf(n2 // 2, odt)
                self.launches.append(lambda part=part, o=out: kernels.epilogue_swiglu(part(), o.dtype, out=o))
                rt._count("rocm.swiglu_epilogue")
                env[outs[0]] = out
            else:
                raise NotImplementedError(f"HIP runtime does not implement op {op}")
        logits = env[self.logits_name]
        if not isinstance(logits, torch.Tensor):
            raise NotImplementedError("graph output is not a tensor value")
        self.logits = logits
        self.next_ids = torch.zeros(rows, dtype=torch.int64, device=rt.device)

    def _merge_into_o(self, users: list[Node], value: str, graph: Graph, heads: int, head_dim: int,
                      k_pool: torch.Tensor) -> bool:
        """At batch <= 8 a decode attention that splits its context leaves the partials for the O projection's
        GEMV to merge (``cir_qgemm_attn``) when that projection, a Q4_0/Q8_0 matmul, is the only reader."""
        if self.rows > 8 or head_dim != 128 or len(users) != 1 or users[0].op not in _MATMUL_OPS:
            return False
        if value in graph.outputs or users[0].inputs[0] != value:
            return False
        if not self.rt.weights.is_blocked((users[0].inputs[1],)):
            return False
        w = self.rt.weights.matmul_weight((users[0].inputs[1],))
        if not isinstance(w, kernels.QWeight) or w.fmt not in (hip.CIR_Q4_0, hip.CIR_Q8_0) or w.k != heads * 128:
            return False
        S = kernels.paged_decode_splits(self.batch, heads, k_pool.shape[1], head_dim, k_pool.shape[2],
                                        self.max_pages, k_pool.dtype)
        splits = kernels.choose_splits(self.rows, w.n, w.k)
        return 1 < S <= 8 and self.rows * (w.k // 128 // splits) <= 256

    @staticmethod
    def _normalizer(users: list[Node], value: str) -> Node | None:
        """The single RMSNorm (plain or inside a fused QKV node) that reads ``value``, if any."""
        found = [u for u in users if (u.op == "rms_norm" or u.op in _QKV_OPS) and u.inputs[0] == value]
        return found[0] if len(found) == 1 else None

    # ------------------------------------------------------------------ run ----
    def set_inputs(self, ids: np.ndarray, page_rows: np.ndarray, positions: np.ndarray) -> None:
        """Stage the step inputs in the pinned buffer and copy them to the device buffer (one async copy, stream
        ordered before the step).  Waits first for the previous copy to have left the pinned buffer."""
        if self._in_pending:
            self._in_copied.synchronize()
        h, B, rows = self._in_np, self.batch, self.rows
        h[: 2 * rows].view(np.int64)[:] = np.asarray(ids, dtype=np.int64).reshape(-1)
        pos = np.asarray(positions, dtype=np.int32).reshape(-1)
        h[self._in_pos: self._in_len] = pos
        h[self._in_len: self._in_pt] = pos + np.int32(self.q_len)
        table = h[self._in_pt:].reshape(B, self.max_pages)
        if isinstance(page_rows, np.ndarray) and page_rows.ndim == 2:
            table[:] = page_rows
        else:  # one int32 row of slots per sequence, zero-padded to the plan's width
            table[:] = 0
            for b, r in enumerate(page_rows):
                table[b, : len(r)] = r
        self._in_dev.copy_(self._in_host, non_blocking=True)
        self._in_copied.record()
        self._in_pending = True

    def launch(self) -> None:
        for fn in self.launches:
            fn()

    def launch_with_argmax(self) -> None:
        self.launch()
        kernels.argmax(self.logits, out=self.next_ids)

    def launch_greedy(self) -> None:
        """The step up to the final norm, then the LM head fused with the argmax: next_ids is set, the logits
        buffer is not written.  Falls back to ``launch_with_argmax`` for a dense (fp32) head."""
        if self._head is None:
            self.launch_with_argmax()
            return
        for fn in self.launches[: self._head_at]:
            fn()
        x, w, ws = self._head
        kernels.qgemm_argmax(x, w, out=self.next_ids, workspace=ws)

    def take_logits(self) -> torch.Tensor:
        """The logits of the step just launched, for the caller to keep.  A plan that has never been captured
        and whose logits GEMM reads ``self.logits`` at launch hands that buffer over and writes its next step
        into a fresh one (no copy); a captured plan writes a fixed address, so its logits are copied."""
        if self.graph_obj is not None or self.graphs or not self._logits_swappable:
            return self.logits.clone()
        out = self.logits
        self.logits = torch.empty(out.shape, dtype=out.dtype, device=out.device)
        return out

    def capture(self, with_argmax: bool = True, greedy: bool = False) -> torch.cuda.CUDAGraph:
        """Capture the step into a HIP graph (after one eager warm-up on a side stream).  ``greedy`` captures
        ``launch_greedy`` (ids only); otherwise the logits, plus the argmax when ``with_argmax``."""
        body = self.launch_greedy if greedy else (self.launch_with_argmax if with_argmax else self.launch)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            body()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            body()
        self.graph_obj = g
        return g

    def replay(self) -> None:
        if self.graph_obj is None:
            raise RuntimeError("plan has not been captured")
        self.graph_obj.replay()

    def run_graph(self, kind: str) -> None:
        """The step as a HIP graph replay: ``"logits"`` (the logits buffer) or ``"greedy"`` (next_ids through the
        fused head).  Captured on first use: the capture's eager warm-up on a side stream computes this step
        (capturing itself runs nothing); later calls replay the graph over the inputs ``set_inputs`` copied.
        The static inputs are those of ``cacheir/backends/cuda_graphs.py:38-55``: ids, page table, lengths."""
        g = self.graphs.get(kind)
        if g is None:
            self.graphs[kind] = self.capture(with_argmax=False, greedy=(kind == "greedy"))
            self.rt._count("rocm.graph_capture")
        else:
            g.replay()
            self.replays += 1


# ========================================================================= runtime ==
class HipRuntime:
    """Execute compiled CacheIR graphs on an MI355X through the cacheir_amd HIP kernels.

    Decode steps (``run`` in decode mode, ``run_decode_batch``, ``decode_greedy``) replay a HIP graph of the
    step captured once per (batch, page-table width, pool generation); only the inputs are copied per step
    (``use_graphs=False`` launches the same kernels one by one instead).  Prefill launches eagerly."""

    supports_variable_prefill_batch = True

    def __init__(self, artifact: CompileArtifact | str | Path, *, device: str = "cuda", dtype: str | None = "auto",
                 weights: HipWeightStore | None = None, source=None, tokenizer=None,
                 prefix_cache: PrefixCache | None = None, kv_allocator: HipKVPageAllocator | None = None,
                 kv_capacity_pages: int = 64, memory_limit_mb: float | None = None, use_graphs: bool = True,
                 max_plans: int = 16, _plans: OrderedDict | None = None, _inv_freq: dict | None = None,
                 _gemm_plans: OrderedDict | None = None):
        if not torch.cuda.is_available():
            raise RuntimeError("HipRuntime requested a GPU, but torch.cuda.is_available() is false")
        hip.load()  # no CPU fallback: fail here if the kernel library is missing
        self.artifact = CompileArtifact.load(artifact) if isinstance(artifact, (str, Path)) else artifact
        self.config = self.artifact.config
        self.device = torch.device(device)
        graph = self.artifact.graph("decode")
        quant = (self.artifact.quant or "").lower() or None
        if weights is None:
            source = source if source is not None else self._open_source()
            blocked = (quant in {"q4_0", "q8_0"} or row_bits(quant) is not None
                       or isinstance(source, (GGUFSource, SyntheticQuant)))
            self.dtype = self._select_dtype(dtype, blocked)
            dense_dtype = torch.float16 if self.dtype == torch.float16 else torch.float32
            weights = HipWeightStore(source, graph.weights, device=self.device, dense_dtype=dense_dtype, quant=quant)
        else:
            self.dtype = self._select_dtype(dtype, weights.dense_dtype == torch.float16)
        self.weights = weights
        self.dense_dtype = weights.dense_dtype
        self.tokenizer = tokenizer or ByteTokenizer(self.config.vocab_size)
        page_size = int(graph.attrs.get("execution_hints", {}).get("page_size", 16))
        self.kv_allocator = kv_allocator or HipKVPageAllocator(
            num_layers=self.config.num_layers, kv_heads=self.config.num_key_value_heads, head_dim=self.config.head_dim,
            page_size=page_size, dtype=self.dtype, device=self.device, capacity_pages=kv_capacity_pages)
        if self.kv_allocator.dtype != self.dtype:
            raise ValueError("kv_allocator dtype differs from the runtime dtype")
        self.kv_cache = HipPagedKVCache(self.kv_allocator)
        self._extra_rows: list[HipPagedKVCache] = []  # rows 1.. of a multi-row run([B, S]) batch
        self.prefix_cache = prefix_cache or PrefixCache(capacity=8)
        self.memory_limit_mb = memory_limit_mb
        self.use_graphs = bool(use_graphs)
        # step plans, least recently used first; at most max_plans are kept (each owns its static buffers and up
        # to two captured graphs), shared with every fork
        self.max_plans = max(1, int(max_plans))
        self._plans: OrderedDict = _plans if _plans is not None else OrderedDict()
        self.plan_evictions = 0
        self._inv_freq: dict = _inv_freq if _inv_freq is not None else {}
        self.kernel_counts: OrderedDict[str, int] = OrderedDict()
        self.gemm_plans: OrderedDict[str, str] = _gemm_plans if _gemm_plans is not None else OrderedDict()
        self.oom_recoveries = 0

    # ------------------------------------------------------------- helpers --
    def _open_source(self):
        path = Path(self.artifact.model_path)
        if path.suffix == ".gguf":
            return GGUFSource(path, gguf_key_map(self.config.num_layers))
        if path.is_dir() or path.suffix == ".npz":
            return NpzDir(path)
        raise FileNotFoundError(f"no weights found for model_path {str(path)!r}; pass source= or weights=")

    def _select_dtype(self, name: str | None, blocked: bool) -> torch.dtype:
        if name in (None, "auto"):
            half = blocked or str(self.config.dtype).lower() in {"float16", "fp16", "bfloat16", "bf16"}
            return torch.float16 if half else torch.float32
        table = {"float16": torch.float16, "fp16": torch.float16, "float32": torch.float32, "fp32": torch.float32}
        if name.lower() not in table:
            raise ValueError(f"Unsupported HIP runtime dtype {name!r} (float16 or float32)")
        return table[name.lower()]

    def _count(self, name: str) -> None:
        self.kernel_counts[name] = self.kernel_counts.get(name, 0) + 1

    def _record_gemm_plan(self, op: int, w: "kernels.QWeight", m: int, splits: int) -> None:
        """``gemm_plans`` entry for a projection, keyed as the reference keys them (``cuda.py:956-974``):
        ``(m, k)x(n, k)`` -> the kernel the library runs and its k-split."""
        n = w.n
        kernel = kernels.gemm_plan(op, w.fmt, m, n, w.k, splits)
        tag = {hip.GEMM_SWIGLU: "swiglu:", hip.GEMM_ARGMAX: "argmax:", hip.GEMM_ATTN_MERGE: "attn_merge:"}.get(op, "")
        self.gemm_plans[f"{tag}{(m, w.k)}x{(n, w.k)}"] = f"rocm.{kernel} splits={splits}"

    def inv_freq(self, head_dim: int, theta: float) -> torch.Tensor:
        key = (head_dim, float(theta))
        if key not in self._inv_freq:
            self._inv_freq[key] = torch.from_numpy(rope_inv_freq(head_dim, theta)).to(self.device)
        return self._inv_freq[key]

    def plan(self, mode: str, batch: int, q_len: int, max_pages: int) -> StepPlan:
        """The step plan for this shape, built on first use (or after the pool was re-based).  The cache keeps the
        ``max_plans`` most recently used plans: a scheduler whose batch size changes every round would otherwise
        accumulate one plan, its buffers and its graphs per shape it ever ran."""
        key = (mode, batch, q_len, max_pages)
        plan = self._plans.get(key)
        if plan is None or plan.generation != self.kv_allocator.generation:
            self._plans.pop(key, None)
            while len(self._plans) >= self.max_plans:
                self._plans.popitem(last=False)
                self.plan_evictions += 1
            plan = StepPlan(self, mode, batch, q_len, max_pages)
            self._plans[key] = plan
        else:
            self._plans.move_to_end(key)
        return plan

    @staticmethod
    def _bucket(pages: int) -> int:
        b = 4
        while b < pages:
            b *= 2
        return b

    def _enforce_memory_limit(self) -> None:
        if self.memory_limit_mb is None:
            return
        mb = torch.cuda.memory_allocated(self.device) / (1024.0 * 1024.0)
        if mb > float(self.memory_limit_mb):
            self._recover_from_oom()
            raise RuntimeError(f"CacheIR HIP memory limit exceeded: {mb:.1f} MB allocated, limit "
                               f"{float(self.memory_limit_mb):.1f} MB")

    def _recover_from_oom(self) -> None:
        self.oom_recoveries += 1
        self._clear_rows()
        self._plans.clear()
        torch.cuda.empty_cache()

    def _clear_rows(self) -> None:
        self.kv_cache.clear()
        for c in self._extra_rows:
            c.clear()
        self._extra_rows = []

    def _row_caches(self, rows: int) -> list[HipPagedKVCache]:
        """The KV caches of a ``run`` over ``rows`` sequences: ``kv_cache`` holds row 0, further rows get caches of
        their own on the shared pool.  The row count may change only while every row is empty."""
        caches = [self.kv_cache] + self._extra_rows
        if len(caches) != rows:
            if any(c.tokens for c in caches):
                raise ValueError(f"input has {rows} rows but the session's KV cache holds {len(caches)}; "
                                 "prefill with reset_kv to change the batch")
            for c in self._extra_rows:
                c.clear()
            self._extra_rows = [HipPagedKVCache(self.kv_allocator) for _ in range(rows - 1)]
            caches = [self.kv_cache] + self._extra_rows
        elif len({c.tokens for c in caches}) > 1:
            raise ValueError("the rows of a run([B, S]) batch hold different lengths")
        return caches

    # -------------------------------------------------------------- API -----
    @classmethod
    def available(cls) -> bool:
        return hip_runtime_available()

    def fork(self) -> "HipRuntime":
        """New session sharing artifact, weights, tokenizer, prefix cache, plans and the KV allocator."""
        return HipRuntime(self.artifact, device=str(self.device), dtype=self._dtype_name(), weights=self.weights,
                          tokenizer=self.tokenizer, prefix_cache=self.prefix_cache, kv_allocator=self.kv_allocator,
                          memory_limit_mb=self.memory_limit_mb, use_graphs=self.use_graphs,
                          max_plans=self.max_plans, _plans=self._plans,
                          _inv_freq=self._inv_freq, _gemm_plans=self.gemm_plans)

    def _dtype_name(self) -> str:
        return "float16" if self.dtype == torch.float16 else "float32"

    def _prepare(self, caches: list[HipPagedKVCache], ids: np.ndarray, mode: str) -> "StepPlan":
        """Reserve and map the KV pages the step writes, and load the step inputs into its plan."""
        batch, q_len = ids.shape
        if ids.size and (int(ids.min()) < 0 or int(ids.max()) >= self.config.vocab_size):
            bad = int(ids.min()) if int(ids.min()) < 0 else int(ids.max())
            # the reference's embedding lookup raises IndexError (cpu.py:223-224)
            raise IndexError(f"token id {bad} is out of range for vocabulary size {self.config.vocab_size}")
        P = self.kv_allocator.page_size
        need_pages = sum(max(0, -(-(c.tokens + q_len) // P) - len(c.slots)) for c in caches)
        self.kv_allocator.reserve(need_pages)  # grow (and re-base pools) before any plan is built
        positions = np.fromiter((c.tokens for c in caches), dtype=np.int32, count=batch)
        for c in caches:
            c.ensure_capacity(c.tokens + q_len)
        max_pages = self._bucket(max(len(c.slots) for c in caches))
        rows = [c.slot_array() for c in caches]
        self._enforce_memory_limit()
        try:
            plan = self.plan(mode, batch, q_len, max_pages)
            plan.set_inputs(ids, rows, positions)
        except torch.cuda.OutOfMemoryError as exc:
            self._recover_from_oom()
            raise RuntimeError("CacheIR HIP runtime recovered from an out-of-memory condition; "
                               "retry with a smaller batch/context") from exc
        return plan

    def _step(self, caches: list[HipPagedKVCache], ids: np.ndarray, mode: str, greedy: bool = False) -> StepPlan:
        """One step over ``caches``: a graph replay for decode (when ``use_graphs``), eager launches otherwise.
        ``greedy`` runs the fused LM head + argmax (``plan.next_ids``) instead of writing the logits."""
        q_len = ids.shape[1]
        plan = self._prepare(caches, ids, mode)
        try:
            if self.use_graphs and mode == "decode":
                plan.run_graph("greedy" if greedy else "logits")
            elif greedy:
                plan.launch_greedy()
            else:
                plan.launch()
        except torch.cuda.OutOfMemoryError as exc:
            self._recover_from_oom()
            raise RuntimeError("CacheIR HIP runtime recovered from an out-of-memory condition; "
                               "retry with a smaller batch/context") from exc
        for c in caches:
            c.tokens += q_len
        return plan

    def _execute(self, caches: list[HipPagedKVCache], ids: np.ndarray, mode: str) -> torch.Tensor:
        batch, q_len = ids.shape
        plan = self._step(caches, ids, mode)
        return plan.take_logits().view(batch, q_len, -1)

    def run(self, input_ids, *, mode: str = "prefill", reset_kv: bool | None = None) -> torch.Tensor:
        """``cuda.py:508-539``: ``input_ids`` ``[S]`` or ``[B, S]`` -> logits ``[B, S, V]``.  A ``[B, S]`` batch is
        B sequences of this session, each with its own pages (prefill them together, then decode ``[B, 1]``)."""
        if reset_kv is None:
            reset_kv = mode == "prefill"
        ids = np.asarray(input_ids, dtype=np.int64)
        if ids.ndim == 1:
            ids = ids[None, :]
        if ids.ndim != 2 or ids.shape[0] < 1 or ids.shape[1] < 1:
            raise ValueError("HipRuntime.run takes token ids [seq] or [batch, seq]")
        if mode == "decode" and ids.shape[1] != 1:
            raise ValueError("decode mode takes exactly one token per step")
        if mode == "prefill" and reset_kv:
            self._clear_rows()
        return self._execute(self._row_caches(ids.shape[0]), ids, mode)

    def _check_sessions(self, sessions) -> None:
        if not sessions:
            raise ValueError("batch requires at least one session")
        for s in sessions:
            if not isinstance(s, HipRuntime):
                raise TypeError("only HipRuntime sessions can be batched")
            if s.artifact is not self.artifact and s.artifact.to_dict() != self.artifact.to_dict():
                raise ValueError("all HIP sessions must use the same CacheIR artifact")
            if s.device != self.device:
                raise ValueError("all HIP sessions must use the same device")
            if s.kv_allocator is not self.kv_allocator:
                raise ValueError("all HIP sessions must share one KV allocator (create them with fork())")
            if s._extra_rows:
                raise ValueError("a session holding a multi-row run([B, S]) batch cannot join a session batch")

    def run_decode_batch(self, sessions: list["HipRuntime"], token_ids) -> torch.Tensor:
        """One decode token for several sessions in one step -> logits ``[B, 1, V]`` (``cuda.py:541-582``)."""
        if not sessions:
            raise ValueError("run_decode_batch requires at least one session")
        if len(sessions) != len(token_ids):
            raise ValueError("sessions and token_ids must have the same length")
        self._check_sessions(sessions)
        ids = np.array([[int(t)] for t in token_ids], dtype=np.int64)
        self._count("cacheir.rocm_decode_batch_graph")
        return self._execute([s.kv_cache for s in sessions], ids, "decode")

    def run_prefill_batch(self, sessions: list["HipRuntime"], token_id_batches: list[list[int]]) -> torch.Tensor:
        """Prefill several sessions -> logits ``[B, max_len, V]`` (rows past a prompt's end are zero)."""
        if not sessions:
            raise ValueError("run_prefill_batch requires at least one session")
        if len(sessions) != len(token_id_batches):
            raise ValueError("sessions and token_id_batches must have the same length")
        lens = [len(t) for t in token_id_batches]
        if any(n <= 0 for n in lens):
            raise ValueError("run_prefill_batch requires non-empty token batches")
        self._check_sessions(sessions)
        for s in sessions:
            s._clear_rows()
        self._count("cacheir.rocm_prefill_batch_graph")
        caches = [s.kv_cache for s in sessions]
        if len(set(lens)) == 1:
            return self._execute(caches, np.array(token_id_batches, dtype=np.int64), "prefill")
        return self._prefill_padded(caches, token_id_batches)

    def _prefill_padded(self, caches: list[HipPagedKVCache], batches: list[list[int]]) -> torch.Tensor:
        """A variable-length prefill as one pass over the batch padded to the longest prompt (the reference pads
        too, ``cuda.py:607-629``).  Row b's padding tokens sit at positions len_b.. past its prompt: their K/V go
        to offsets past len_b of its last page (overwritten by its next decode appends, never read below its
        length) or, past that page, to one padding page that only padding rows read; the causal mask keeps every
        prompt token's attention inside its own prompt.  Each session ends holding exactly its prompt, and the
        logits of padding positions are returned as zeros."""
        lens = [len(t) for t in batches]
        B, L, P = len(caches), max(lens), self.kv_allocator.page_size
        ids = np.zeros((B, L), dtype=np.int64)
        for b, toks in enumerate(batches):
            ids[b, : len(toks)] = toks
        real = np.concatenate([np.asarray(t, dtype=np.int64) for t in batches])
        if int(real.min()) < 0 or int(real.max()) >= self.config.vocab_size:
            bad = int(real.min()) if int(real.min()) < 0 else int(real.max())
            raise IndexError(f"token id {bad} is out of range for vocabulary size {self.config.vocab_size}")
        width = -(-L // P)
        self.kv_allocator.reserve(sum(-(-n // P) for n in lens) + 1)
        pad_slot = self.kv_allocator.allocate("prefill-padding")
        try:
            for c, n in zip(caches, lens):
                c.ensure_capacity(c.tokens + n)
            max_pages = self._bucket(width)
            rows = np.zeros((B, max_pages), dtype=np.int32)
            for b, c in enumerate(caches):
                own = c.slot_array()
                rows[b, : len(own)] = own
                rows[b, len(own): width] = pad_slot
            positions = np.fromiter((c.tokens for c in caches), dtype=np.int32, count=B)
            self._enforce_memory_limit()
            try:
                plan = self.plan("prefill", B, L, max_pages)
                plan.set_inputs(ids, rows, positions)
                plan.launch()
            except torch.cuda.OutOfMemoryError as exc:
                self._recover_from_oom()
                raise RuntimeError("CacheIR HIP runtime recovered from an out-of-memory condition; "
                                   "retry with fewer or shorter prompts") from exc
        finally:
            # stream ordered: a later user of the slot writes it only after this step's padding writes
            self.kv_allocator.release([pad_slot])
        for c, n in zip(caches, lens):
            c.tokens += n
        out = plan.take_logits().view(B, L, -1)
        for b, n in enumerate(lens):
            if n < L:
                out[b, n:] = 0
        self._count("rocm.prefill_padded_batch")
        return out

    def prefill_tokens(self, token_ids, *, use_prefix_cache: bool = False, remember_prefix: bool = False):
        """``cpu.py:140-165``: with ``use_prefix_cache`` the longest cached prefix of ``token_ids`` is reused
        (its pages aliased, not copied) and only the rest is prefilled; returns (logits of the prefilled
        tokens, the reused prefix)."""
        ids = [int(t) for t in token_ids]
        reused: tuple[int, ...] = ()
        if use_prefix_cache and ids:
            prefix, pages = self.prefix_cache.longest_prefix(ids)
            if pages is not None and 0 < len(prefix) < len(ids) and pages.allocator is self.kv_allocator:
                self._clear_rows()
                self.kv_cache.alias_prefix(pages.slots, len(prefix))
                reused = tuple(prefix)
                logits = self.run([ids[len(prefix):]], mode="prefill", reset_kv=False)
            else:
                logits = self.run([ids], mode="prefill", reset_kv=True)
        else:
            logits = self.run([ids], mode="prefill", reset_kv=True)
        if remember_prefix and ids:
            self.remember_prefix(ids)
        return logits, reused

    def remember_prefix(self, token_ids) -> None:
        """Cache this session's pages as the KV of ``token_ids`` (the tokens it holds now)."""
        ids = [int(t) for t in token_ids]
        if len(ids) != self.kv_cache.tokens:
            raise ValueError(f"remember_prefix: the session holds {self.kv_cache.tokens} tokens, not {len(ids)}")
        pages = -(-len(ids) // self.kv_allocator.page_size)
        slots = list(self.kv_cache.slots[:pages])
        self.kv_allocator.share(slots)
        self.prefix_cache.put(ids, PrefixPages(self.kv_allocator, slots, len(ids)))

    def load_longest_prefix(self, token_ids) -> tuple[int, ...]:
        """``cuda.py:677-681``: make the longest cached prefix of ``token_ids`` this session's KV (its pages aliased,
        not copied, replacing what the session held) and return it; ``()`` when no cached prefix matches."""
        prefix, pages = self.prefix_cache.longest_prefix([int(t) for t in token_ids])
        if pages is None:
            return ()
        if pages.allocator is not self.kv_allocator:
            raise ValueError("the cached prefix lives in another KV allocator (share one through fork())")
        self._clear_rows()
        self.kv_cache.alias_prefix(pages.slots, len(prefix))
        return tuple(prefix)

    def decode_greedy(self, sessions: list["HipRuntime"], token_ids) -> list[int]:
        """One decode step for ``sessions`` (one token each) returning the greedy next ids instead of logits
        (``run_decode_batch`` + argmax of scheduler.py:535-543, with the LM head and argmax fused)."""
        if len(sessions) != len(token_ids):
            raise ValueError("sessions and token_ids must have the same length")
        self._check_sessions(sessions)
        ids = np.asarray(token_ids, dtype=np.int64).reshape(len(sessions), 1)
        plan = self._step([s.kv_cache for s in sessions], ids, "decode", greedy=True)
        return [int(v) % self.config.vocab_size for v in plan.next_ids.cpu().tolist()]

    def generate_ids(self, prompt_ids, max_new_tokens: int = 16) -> list[int]:
        logits = self.run([list(prompt_ids)], mode="prefill", reset_kv=True)
        out = []
        if max_new_tokens <= 0:
            return out
        nxt = int(torch.argmax(logits[0, -1]).item()) % self.config.vocab_size
        out.append(nxt)
        for _ in range(max_new_tokens - 1):
            nxt = self.decode_greedy([self], [nxt])[0]
            out.append(nxt)
        return out

    def generate(self, prompt: str, *, max_new_tokens: int = 16, use_prefix_cache: bool = False,
                 remember_prefix: bool = True):
        ids = self.tokenizer.encode(prompt)
        logits, _ = self.prefill_tokens(ids, use_prefix_cache=use_prefix_cache,
                                        remember_prefix=remember_prefix and use_prefix_cache)
        for _ in range(max_new_tokens):
            nxt = int(torch.argmax(logits[0, -1]).item()) % self.config.vocab_size
            yield self.tokenizer.decode([nxt])
            logits = self.run([[nxt]], mode="decode")

    def synchronize(self) -> None:
        torch.cuda.synchronize(self.device)

    def cache_stats(self) -> dict[str, object]:
        stats = self.kv_cache.stats()
        stats["prefix_cache"] = self.prefix_cache.stats()
        stats["kernel_counts"] = dict(self.kernel_counts)
        stats["gemm_plans"] = dict(self.gemm_plans)
        stats["step_graphs"] = {
            f"{mode}:b{batch}:q{q_len}:p{pages}": {"captured": sorted(plan.graphs), "replays": plan.replays,
                                                  "launches": len(plan.launches)}
            for (mode, batch, q_len, pages), plan in self._plans.items() if plan.graphs}
        stats["step_plans"] = {"cached": len(self._plans), "max": self.max_plans, "evictions": self.plan_evictions}
        stats["oom_recoveries"] = self.oom_recoveries
        stats["memory_limit_mb"] = self.memory_limit_mb
        stats["weight_bytes"] = self.weights.nbytes()
        return stats
