"""NumPy graph runtime restating CacheIR's CPU ``Runtime`` (test infrastructure only).

* ``create_tiny_weights`` follows ``cacheir/importers/tiny.py:23,40-60``: one
  ``np.random.default_rng(seed)`` stream drawn in the order embed, lm_head, then per
  layer q, k, v, o, gate, up, down (``N(0,1)*0.02`` cast to float32); norms are ones.
* ``OracleRuntime.run`` follows ``cacheir/runtime/cpu.py:111-140`` (graph walk over
  nodes, env of values) with the op table of ``cpu.py:221-282``; the KV cache is the
  contiguous per-layer cache of ``kv_cache.py:66-79``; RoPE offset is the layer's
  length before the append (``cpu.py:314-317``).
* ``generate_ids`` follows ``cpu.py:167-184`` on token ids (no tokenizer).
* ``decode_batch`` runs each session's decode separately and stacks the logits,
  which is what the reference scheduler does when it cannot batch
  (``scheduler.py:445-454,559-565``).

Weights are given as a dict ``value name -> float32 array`` (GGUF Q4_0/Q8_0 weights
already decoded to float32 as ``gguf.py`` does at load).

Rows of one batch may hold different lengths (a ragged decode batch, as a scheduler
forms from sessions at different positions): ``keys[layer]`` / ``values[layer]`` are
then lists of per-row ``[T_b, Hkv, D]`` arrays.  Each row's RoPE offset is its own
length (``ops.rope_offsets``, ``cuda.py:1084-1102``) and its attention runs over its own
cache; the matmuls run over the whole batch.  Row ``b`` gives what a session holding
only that row computes (pinned against ``decode_batch`` in the CPU tests).

``OracleRuntime(..., fp16_storage=True)`` rounds values to float16 where a float16
backend stores them (every matmul input, i.e. the normalised activations, the
attention output and the SwiGLU output; q, k and v after RoPE, k and v as they enter
the cache) and computes everything else in float32 as above.  It is the reference for
an fp16 backend at the step level: in a randomly initialised network the attention
softmax amplifies those storage roundings to ~1e-3 of the logits' scale, which the
fp32 path cannot tell from a kernel error.  It restates no other arithmetic; it is
pinned by the fp32 path (``fp16_storage=False`` gives the same results bit for bit as
before) plus the points it rounds.
"""
from __future__ import annotations

import numpy as np

from oracle import ops


def create_tiny_weights(*, seed: int, vocab_size: int, hidden_size: int, intermediate_size: int,
                        num_layers: int, num_attention_heads: int, num_key_value_heads: int) -> dict[str, np.ndarray]:
    """``tiny.py:40-60`` draw order; keys are the HF names the graph's WeightSpecs point at."""
    rng = np.random.default_rng(seed)

    def normal(shape, scale=0.02):
        return (rng.standard_normal(shape) * scale).astype(np.float32)

    w = {
        "model.embed_tokens.weight": normal((vocab_size, hidden_size)),
        "model.norm.weight": np.ones((hidden_size,), dtype=np.float32),
        "lm_head.weight": normal((vocab_size, hidden_size)),
    }
    head_dim = hidden_size // num_attention_heads
    kv_dim = num_key_value_heads * head_dim
    for layer in range(num_layers):
        p = f"model.layers.{layer}"
        w[f"{p}.input_layernorm.weight"] = np.ones((hidden_size,), dtype=np.float32)
        w[f"{p}.self_attn.q_proj.weight"] = normal((hidden_size, hidden_size))
        w[f"{p}.self_attn.k_proj.weight"] = normal((kv_dim, hidden_size))
        w[f"{p}.self_attn.v_proj.weight"] = normal((kv_dim, hidden_size))
        w[f"{p}.self_attn.o_proj.weight"] = normal((hidden_size, hidden_size))
        w[f"{p}.post_attention_layernorm.weight"] = np.ones((hidden_size,), dtype=np.float32)
        w[f"{p}.mlp.gate_proj.weight"] = normal((intermediate_size, hidden_size))
        w[f"{p}.mlp.up_proj.weight"] = normal((intermediate_size, hidden_size))
        w[f"{p}.mlp.down_proj.weight"] = normal((hidden_size, intermediate_size))
    return w


class OracleRuntime:
    """One session: a compiled-graph dict per mode, weights by HF key, and a contiguous KV cache."""

    def __init__(self, graphs: dict[str, dict], weights_by_key: dict[str, np.ndarray], vocab_size: int,
                 fp16_storage: bool = False):
        self.graphs = graphs
        self.vocab_size = vocab_size
        self.fp16_storage = fp16_storage
        self.keys: dict[int, np.ndarray] = {}
        self.values: dict[int, np.ndarray] = {}
        self.weights = {}
        for graph in graphs.values():
            for name, spec in graph["weights"].items():
                self.weights[name] = np.asarray(weights_by_key[spec["key"]], dtype=np.float32)

    def fork(self) -> "OracleRuntime":
        other = OracleRuntime.__new__(OracleRuntime)
        other.graphs, other.vocab_size, other.weights = self.graphs, self.vocab_size, self.weights
        other.fp16_storage = self.fp16_storage
        other.keys, other.values = {}, {}
        return other

    def kv_length(self, layer: int) -> int:
        if isinstance(self.keys.get(layer), list):
            raise ValueError(f"the rows of layer {layer}'s cache hold different lengths (a ragged cache)")
        return int(self.keys[layer].shape[1]) if layer in self.keys else 0

    def _rope(self, x: np.ndarray, layer: int, hd: int, theta: float) -> np.ndarray:
        """RoPE at the layer's cache length: one offset for a uniform cache, one per row for a ragged one."""
        kk = self.keys.get(layer)
        if isinstance(kk, list):
            return ops.rope_offsets(x, hd, theta, [len(r) for r in kk])
        return ops.rope_one(x, hd, theta, self.kv_length(layer))

    def run(self, input_ids, *, mode: str = "prefill", reset_kv: bool | None = None) -> np.ndarray:
        graph = self.graphs[mode]
        if reset_kv is None:
            reset_kv = mode == "prefill"
        if mode == "prefill" and reset_kv:
            self.keys.clear()
            self.values.clear()
        ids = np.asarray(input_ids, dtype=np.int64)
        if ids.ndim == 1:
            ids = ids[None, :]
        env: dict[str, np.ndarray] = {"input_ids": ids}
        env.update(self.weights)
        for node in graph["nodes"]:
            outs = self._execute(node, env, mode)
            for name, value in zip(node["outputs"], outs):
                env[name] = value
        return env[graph["outputs"][0]]

    def _append(self, layer: int, k: np.ndarray, v: np.ndarray):
        if layer not in self.keys:
            self.keys[layer], self.values[layer] = k.copy(), v.copy()
        else:
            self.keys[layer] = np.concatenate([self.keys[layer], k], axis=1)
            self.values[layer] = np.concatenate([self.values[layer], v], axis=1)
        return self.keys[layer], self.values[layer]

    def _st(self, x: np.ndarray) -> np.ndarray:
        """A value as a float16 backend stores it (identity unless ``fp16_storage``)."""
        return x.astype(np.float16).astype(np.float32) if self.fp16_storage else x

    def _execute(self, node: dict, env: dict, mode: str) -> list[np.ndarray]:
        op, ins, attrs = node["op"], node["inputs"], node["attrs"]
        st = self._st
        if op == "token_embedding":
            return [env[ins[1]][env[ins[0]]]]
        if op == "rms_norm":
            return [ops.rms_norm(env[ins[0]], env[ins[1]], float(attrs.get("eps", 1e-6)))]
        if op in {"matmul", "quantized_matmul"}:
            return [ops.matmul(st(env[ins[0]]), env[ins[1]])]
        if op == "qkv_projection":
            x = st(env[ins[0]])
            return [ops.matmul(x, env[ins[1]]), ops.matmul(x, env[ins[2]]), ops.matmul(x, env[ins[3]])]
        if op in {"fused_rmsnorm_qkv_rope", "quantized_fused_rmsnorm_qkv_rope"}:
            x = st(ops.rms_norm(env[ins[0]], env[ins[1]], float(attrs.get("eps", 1e-6))))
            q, k, v = ops.matmul(x, env[ins[2]]), ops.matmul(x, env[ins[3]]), ops.matmul(x, env[ins[4]])
            layer = int(attrs.get("layer", 0))
            hd, theta = int(attrs["head_dim"]), float(attrs.get("rope_theta", 10000.0))
            return [st(self._rope(q, layer, hd, theta)), st(self._rope(k, layer, hd, theta)), st(v)]
        if op == "rope":
            layer = int(attrs.get("layer", 0))
            hd, theta = int(attrs["head_dim"]), float(attrs.get("rope_theta", 10000.0))
            return [self._rope(env[ins[0]], layer, hd, theta), self._rope(env[ins[1]], layer, hd, theta)]
        if op in {"paged_attention_prefill", "paged_attention_decode", "grouped_query_attention"}:
            q, k, v = env[ins[0]], env[ins[1]], env[ins[2]]
            layer = int(attrs.get("layer", 0))
            heads, kvh, hd = int(attrs["num_heads"]), int(attrs["num_kv_heads"]), int(attrs["head_dim"])
            b, s, _ = q.shape
            k4, v4 = k.reshape(b, k.shape[1], kvh, hd), v.reshape(b, v.shape[1], kvh, hd)
            if isinstance(self.keys.get(layer), list):  # ragged: each row over its own cache
                outs = []
                for r in range(b):
                    self.keys[layer][r] = np.concatenate([self.keys[layer][r], k4[r]], axis=0)
                    self.values[layer][r] = np.concatenate([self.values[layer][r], v4[r]], axis=0)
                    outs.append(ops.attention(q[r: r + 1].reshape(1, s, heads, hd), self.keys[layer][r][None],
                                              self.values[layer][r][None], heads, kvh, hd,
                                              causal=(mode == "prefill")))
                return [np.concatenate(outs, axis=0)]
            kh, vh = self._append(layer, k4, v4)
            return [ops.attention(q.reshape(b, s, heads, hd), kh, vh, heads, kvh, hd, causal=(mode == "prefill"))]
        if op == "add":
            return [env[ins[0]] + env[ins[1]]]
        if op == "silu":
            return [ops.silu(env[ins[0]])]
        if op == "elementwise_mul":
            return [env[ins[0]] * env[ins[1]]]
        if op in {"fused_swiglu", "quantized_fused_swiglu"}:
            x = st(env[ins[0]])
            return [ops.silu_mul(ops.matmul(x, env[ins[1]]), ops.matmul(x, env[ins[2]]))]
        raise NotImplementedError(f"oracle runtime does not implement op {op}")


def generate_ids(rt: OracleRuntime, prompt_ids: list[int], max_new_tokens: int) -> tuple[list[int], np.ndarray]:
    """``cpu.py:175-184`` on ids; returns the greedy ids and the last logits row seen."""
    logits = rt.run([list(prompt_ids)], mode="prefill", reset_kv=True)
    out = []
    for _ in range(max_new_tokens):
        nxt = int(np.argmax(logits[0, -1])) % rt.vocab_size
        out.append(nxt)
        logits = rt.run([[nxt]], mode="decode")
    return out, logits


def decode_batch(sessions: list[OracleRuntime], token_ids: list[int]) -> np.ndarray:
    """Sequential per-session decode, stacked ``[B, 1, V]``."""
    return np.concatenate([s.run([[int(t)]], mode="decode") for s, t in zip(sessions, token_ids)], axis=0)


def direct_generate(w: dict[str, np.ndarray], *, num_layers: int, num_heads: int, num_kv_heads: int, eps: float,
                    theta: float, vocab: int, prompt_ids: list[int], max_new_tokens: int) -> tuple[list[int], list[np.ndarray]]:
    """Llama decoder written out directly (no graph): the per-layer sequence of
    ``cacheir/importers/hf.py:196-266`` with the op semantics of ``cpu.py:221-377``.

    Used to pin the graph builder's wiring: graph-driven and direct generation must
    agree.  Returns the greedy ids and the logits row of every step.
    """
    hidden = w["model.embed_tokens.weight"].shape[1]
    hd = hidden // num_heads
    cache_k: dict[int, np.ndarray] = {}
    cache_v: dict[int, np.ndarray] = {}

    def forward(ids: np.ndarray, causal: bool) -> np.ndarray:
        x = w["model.embed_tokens.weight"][ids]
        for layer in range(num_layers):
            p = f"model.layers.{layer}"
            h = ops.rms_norm(x, w[f"{p}.input_layernorm.weight"], eps)
            q = ops.matmul(h, w[f"{p}.self_attn.q_proj.weight"])
            k = ops.matmul(h, w[f"{p}.self_attn.k_proj.weight"])
            v = ops.matmul(h, w[f"{p}.self_attn.v_proj.weight"])
            off = cache_k[layer].shape[1] if layer in cache_k else 0
            q, k = ops.rope_one(q, hd, theta, off), ops.rope_one(k, hd, theta, off)
            b, s, _ = q.shape
            kh, vh = k.reshape(b, s, num_kv_heads, hd), v.reshape(b, s, num_kv_heads, hd)
            cache_k[layer] = kh if layer not in cache_k else np.concatenate([cache_k[layer], kh], axis=1)
            cache_v[layer] = vh if layer not in cache_v else np.concatenate([cache_v[layer], vh], axis=1)
            a = ops.attention(q.reshape(b, s, num_heads, hd), cache_k[layer], cache_v[layer], num_heads, num_kv_heads,
                              hd, causal=causal)
            x = x + ops.matmul(a, w[f"{p}.self_attn.o_proj.weight"])
            h = ops.rms_norm(x, w[f"{p}.post_attention_layernorm.weight"], eps)
            g = ops.silu_mul(ops.matmul(h, w[f"{p}.mlp.gate_proj.weight"]), ops.matmul(h, w[f"{p}.mlp.up_proj.weight"]))
            x = x + ops.matmul(g, w[f"{p}.mlp.down_proj.weight"])
        x = ops.rms_norm(x, w["model.norm.weight"], eps)
        return ops.matmul(x, w["lm_head.weight"])

    logits = forward(np.asarray([prompt_ids], dtype=np.int64), causal=True)
    rows, out = [], []
    for _ in range(max_new_tokens):
        rows.append(logits[0, -1].copy())
        nxt = int(np.argmax(logits[0, -1])) % vocab
        out.append(nxt)
        logits = forward(np.asarray([[nxt]], dtype=np.int64), causal=False)
    return out, rows
