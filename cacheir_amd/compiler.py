"""Lowered decode/prefill graphs for the ``rocm`` target.

``build_graph`` emits the graph CacheIR's pipeline produces for a Llama/Mistral/Qwen
decoder (``cacheir/compiler.py:114-132``): the logical graph of
``cacheir/importers/hf.py:171-268`` after QKV + RMSNorm + RoPE fusion
(``passes/transformer.py:124-226``), SwiGLU fusion (``transformer.py:229-281``),
decode/prefill specialisation (``transformer.py:284-304``), layout conversion
(``transformer.py:307-329``), quantisation lowering (``transformer.py:332-353``),
hardware hints with ``page_size`` 16 for decode (``transformer.py:391-424``), kernel
selection (``transformer.py:356-388``) and execution planning
(``transformer.py:427-450``).  Node names, value names, op names and the attributes
the runtime reads (``layer, eps, head_dim, rope_theta, num_heads, num_kv_heads,
page_size``) match the reference so artifacts are interchangeable.

``RocmKernelSelection`` is the backend's entry in the kernel-selection pass: it
assigns ``rocm.*`` kernel names (the reference assigns ``triton.*`` for cuda and
``cpu.*`` otherwise, ``transformer.py:370-388``) and can retarget a graph compiled by
the reference for any target.

Quant names: ``q4_0`` / ``q8_0`` mean GGUF block weights kept packed on the device;
``int4*`` / ``int8`` are the reference's per-row asymmetric formats
(``cacheir/quantization.py:63-71``).
"""
from __future__ import annotations

from cacheir_amd.artifact import CompileArtifact, ModelConfig
from cacheir_amd.ir import Graph, Node, TensorType, WeightSpec

#: op -> ROCm kernel name (the rocm row of the kernel-selection table).
ROCM_KERNELS = {
    "token_embedding": "embedding_gather",
    "rms_norm": "rms_norm",
    "matmul": "gemm",
    "quantized_matmul": "qgemm_blocks",
    "fused_rmsnorm_qkv_rope": "fused_rmsnorm_qkv_rope_kv_append",
    "quantized_fused_rmsnorm_qkv_rope": "qgemm_rmsnorm_qkv_rope_kv_append",
    "paged_attention_prefill": "paged_attention_prefill",
    "paged_attention_decode": "paged_attention_decode",
    "fused_swiglu": "fused_swiglu",
    "quantized_fused_swiglu": "qgemm_swiglu",
    "add": "residual_add",
    "silu": "silu",
    "elementwise_mul": "elementwise_mul",
    "softmax": "softmax",
}

_MATMUL_FAMILY = {"matmul", "quantized_matmul", "qkv_projection", "fused_rmsnorm_qkv_rope",
                  "quantized_fused_rmsnorm_qkv_rope", "fused_swiglu", "quantized_fused_swiglu"}


def weight_layout_for(quant: str | None) -> str:
    q = (quant or "").lower()
    if q in {"q4_0", "q8_0"}:
        return f"{q}_blocks"
    if q:
        return "row_asymmetric_packed"
    return "row_major_out_in"


class RocmKernelSelection:
    """Kernel selection + hardware hints + schedule for the ``rocm`` target (in place)."""

    name = "rocm_kernel_selection"

    def __init__(self, quant: str | None = None, page_size: int = 16):
        self.quant = quant
        self.page_size = page_size

    def run(self, graph: Graph) -> Graph:
        layout = weight_layout_for(self.quant)
        graph.target = "rocm"
        hints = dict(graph.attrs.get("execution_hints", {}))
        hints.update({"target": "rocm", "mode": graph.mode, "page_size": self.page_size,
                      "prefer_fused_decode_attention": graph.mode == "decode", "low_vram_mode": False})
        graph.attrs["execution_hints"] = hints
        graph.attrs["kernel_target"] = "rocm"
        for idx, node in enumerate(graph.nodes):
            if node.op in _MATMUL_FAMILY:
                node.attrs["weight_layout"] = layout
                node.attrs["activation_layout"] = "bsh"
            if node.op in {"paged_attention_decode", "paged_attention_prefill"}:
                node.attrs["page_size"] = self.page_size
                node.attrs["low_vram_mode"] = False
            node.attrs["kernel"] = f"rocm.{ROCM_KERNELS.get(node.op, node.op)}"
            node.attrs["schedule_index"] = idx
        return graph


def build_graph(config: ModelConfig, mode: str = "decode", *, quant: str | None = None,
                weight_dtype: str | None = None) -> Graph:
    """Lowered graph for ``mode`` in {"decode", "prefill"} (see module docstring)."""
    if mode not in {"decode", "prefill"}:
        raise ValueError(f"unknown mode {mode!r}")
    h, i, kv = config.hidden_size, config.intermediate_size, config.kv_dim
    dtype = weight_dtype or config.dtype
    g = Graph(name=f"{config.architecture}_{mode}", mode=mode, target="rocm")
    g.attrs["model_config"] = config.to_dict()
    g.attrs["execution_mode"] = mode
    g.attrs["kv_cache"] = {"policy": "paged", "compiled_with_graph": True, "decode_token_granularity": mode == "decode"}
    ids_type = TensorType(("batch", "seq"), "int64")
    g.inputs["input_ids"] = ids_type
    g.values["input_ids"] = ids_type
    act = TensorType(("batch", "seq", h), dtype)
    qflag = quant if quant else None

    def weight(name: str, key: str, shape: tuple, q: bool = False) -> None:
        spec = WeightSpec(key, TensorType(shape, dtype), quant=None, file=None)
        g.weights[name] = spec
        g.values[name] = spec.tensor_type

    def node(op: str, ins: list[str], outs: list[str], attrs: dict, name: str) -> None:
        if qflag and op in {"matmul", "fused_rmsnorm_qkv_rope", "fused_swiglu"}:
            op = "quantized_" + op
            attrs = dict(attrs, quant=qflag)
        g.nodes.append(Node(op, ins, outs, attrs, name))

    weight("tok_embeddings", "model.embed_tokens.weight", (config.vocab_size, h))
    weight("final_norm_w", "model.norm.weight", (h,))
    lm_key = "model.embed_tokens.weight" if config.tie_word_embeddings else "lm_head.weight"
    weight("lm_head_w", lm_key, (config.vocab_size, h))
    node("token_embedding", ["input_ids", "tok_embeddings"], ["hidden_0"], {}, "embed")
    hidden = "hidden_0"
    for layer in range(config.num_layers):
        p, ln = f"model.layers.{layer}", f"layer{layer}"
        weight(f"{ln}_attn_norm_w", f"{p}.input_layernorm.weight", (h,))
        weight(f"{ln}_q_w", f"{p}.self_attn.q_proj.weight", (h, h))
        weight(f"{ln}_k_w", f"{p}.self_attn.k_proj.weight", (kv, h))
        weight(f"{ln}_v_w", f"{p}.self_attn.v_proj.weight", (kv, h))
        weight(f"{ln}_o_w", f"{p}.self_attn.o_proj.weight", (h, h))
        weight(f"{ln}_mlp_norm_w", f"{p}.post_attention_layernorm.weight", (h,))
        weight(f"{ln}_gate_w", f"{p}.mlp.gate_proj.weight", (i, h))
        weight(f"{ln}_up_w", f"{p}.mlp.up_proj.weight", (i, h))
        weight(f"{ln}_down_w", f"{p}.mlp.down_proj.weight", (h, i))
        node("fused_rmsnorm_qkv_rope",
             [hidden, f"{ln}_attn_norm_w", f"{ln}_q_w", f"{ln}_k_w", f"{ln}_v_w"],
             [f"{ln}_q_rope", f"{ln}_k_rope", f"{ln}_v"],
             {"layer": layer, "eps": config.rms_norm_eps, "head_dim": config.head_dim,
              "rope_theta": config.rope_theta, "cost_class": "elementwise_or_fused"},
             f"{ln}.fused_rmsnorm_qkv_rope")
        attn_op = "paged_attention_decode" if mode == "decode" else "paged_attention_prefill"
        node(attn_op, [f"{ln}_q_rope", f"{ln}_k_rope", f"{ln}_v"], [f"{ln}_attn"],
             {"layer": layer, "num_heads": config.num_attention_heads, "num_kv_heads": config.num_key_value_heads,
              "head_dim": config.head_dim, "kv_cache": "paged", "mode": mode, "kv_cache_policy": "append_only_pages",
              "cost_class": "kv_bandwidth_bound" if mode == "decode" else "mixed_attention"},
             f"{ln}.attention")
        node("matmul", [f"{ln}_attn", f"{ln}_o_w"], [f"{ln}_attn_out"],
             {"layer": layer, "projection": "o", "cost_class": "compute_bound"}, f"{ln}.o_proj")
        node("add", [hidden, f"{ln}_attn_out"], [f"{ln}_post_attn"],
             {"layer": layer, "kind": "residual", "cost_class": "elementwise_or_fused"}, f"{ln}.attn_residual")
        node("rms_norm", [f"{ln}_post_attn", f"{ln}_mlp_norm_w"], [f"{ln}_mlp_norm"],
             {"eps": config.rms_norm_eps, "layer": layer, "cost_class": "elementwise_or_fused"}, f"{ln}.mlp_norm")
        node("fused_swiglu", [f"{ln}_mlp_norm", f"{ln}_gate_w", f"{ln}_up_w"], [f"{ln}_gated"],
             {"layer": layer, "cost_class": "elementwise_or_fused"}, f"{ln}.fused_swiglu")
        node("matmul", [f"{ln}_gated", f"{ln}_down_w"], [f"{ln}_down"],
             {"layer": layer, "projection": "down", "cost_class": "compute_bound"}, f"{ln}.down_proj")
        node("add", [f"{ln}_post_attn", f"{ln}_down"], [f"{ln}_post_mlp"],
             {"layer": layer, "kind": "residual", "cost_class": "elementwise_or_fused"}, f"{ln}.mlp_residual")
        hidden = f"{ln}_post_mlp"
    node("rms_norm", [hidden, "final_norm_w"], ["final_hidden"],
         {"eps": config.rms_norm_eps, "cost_class": "elementwise_or_fused"}, "final_norm")
    node("matmul", ["final_hidden", "lm_head_w"], ["logits"],
         {"projection": "lm_head", "cost_class": "compute_bound"}, "lm_head")
    g.outputs = ["logits"]
    for n in g.nodes:
        for out in n.outputs:
            g.values.setdefault(out, act)
    g.values["logits"] = TensorType(("batch", "seq", config.vocab_size), dtype)
    return RocmKernelSelection(quant=quant).run(g)


def compile_config(config: ModelConfig, *, quant: str | None = None, model_path: str = "",
                   modes=("prefill", "decode"), weight_dtype: str | None = None) -> CompileArtifact:
    """Artifact with one lowered graph per mode (the ``compile_model`` product, ``compiler.py:135-181``)."""
    graphs = {m: build_graph(config, m, quant=quant, weight_dtype=weight_dtype) for m in modes}
    return CompileArtifact(target="rocm", quant=quant, model_path=model_path, config=config, graphs=graphs,
                           metadata={"compiler": "CacheIR", "backend": "cacheir_amd", "modes": list(modes)})


def retarget(artifact: CompileArtifact) -> CompileArtifact:
    """Apply ``RocmKernelSelection`` to every graph of an artifact compiled for another target."""
    for g in artifact.graphs.values():
        RocmKernelSelection(quant=artifact.quant).run(g)
    artifact.target = "rocm"
    return artifact
