"""Model config and compile artifact in CacheIR's JSON layout.

``ModelConfig`` mirrors ``cacheir/importers/hf.py:11-56`` (fields, HF-config key
aliases, ``head_dim = hidden // heads``).  ``CompileArtifact`` mirrors
``cacheir/runtime/artifact.py:13-57,109-114`` (``{version, created_at, target, quant,
model_path, config, graphs{mode: graph}, pass_traces, metadata}``).  Field names are
kept identical so artifacts written by the reference compiler load unchanged.
"""
from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

from cacheir_amd.ir import Graph


@dataclass
class ModelConfig:
    architecture: str
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    vocab_size: int
    max_position_embeddings: int = 2048
    rope_theta: float = 10000.0
    rms_norm_eps: float = 1e-6
    dtype: str = "float32"
    tie_word_embeddings: bool = False
    quantization: str | None = None

    @property
    def head_dim(self) -> int:
        if self.hidden_size % self.num_attention_heads:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        return self.hidden_size // self.num_attention_heads

    @property
    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> "ModelConfig":
        heads = int(d.get("num_attention_heads", d.get("n_head", 0)))
        q = d.get("quantization_config", d.get("quantization"))
        if isinstance(q, dict):
            q = str(q.get("quant_method") or q.get("load_in_4bit") or q.get("bits") or "quantized")
        return cls(
            architecture=d.get("architecture") or (d.get("architectures") or ["Unknown"])[0],
            hidden_size=int(d["hidden_size"]),
            intermediate_size=int(d.get("intermediate_size", d.get("ffn_hidden_size", int(d["hidden_size"]) * 4))),
            num_layers=int(d.get("num_layers", d.get("num_hidden_layers", d.get("n_layer", 0)))),
            num_attention_heads=heads,
            num_key_value_heads=int(d.get("num_key_value_heads", heads)),
            vocab_size=int(d["vocab_size"]),
            max_position_embeddings=int(d.get("max_position_embeddings", d.get("seq_length", 2048))),
            rope_theta=float(d.get("rope_theta", d.get("rope_freq_base", 10000.0))),
            rms_norm_eps=float(d.get("rms_norm_eps", d.get("layer_norm_epsilon", 1e-6))),
            dtype=str(d.get("torch_dtype", d.get("dtype", "float32"))).replace("torch.", ""),
            tie_word_embeddings=bool(d.get("tie_word_embeddings", False)),
            quantization=(str(q) if q else None),
        )


@dataclass
class CompileArtifact:
    target: str
    quant: str | None
    model_path: str
    config: ModelConfig
    graphs: dict[str, Graph]
    pass_traces: dict[str, list[dict[str, Any]]] = field(default_factory=dict)
    version: str = "0.1"
    created_at: str = field(default_factory=lambda: datetime.now(timezone.utc).isoformat())
    metadata: dict[str, Any] = field(default_factory=dict)

    def graph(self, mode: str = "decode") -> Graph:
        if mode in self.graphs:
            return self.graphs[mode]
        if self.graphs:
            return next(iter(self.graphs.values()))
        raise KeyError("artifact has no graphs")

    def to_dict(self) -> dict[str, Any]:
        return {
            "version": self.version, "created_at": self.created_at, "target": self.target, "quant": self.quant,
            "model_path": self.model_path, "config": self.config.to_dict(),
            "graphs": {m: g.to_dict() for m, g in self.graphs.items()},
            "pass_traces": self.pass_traces, "metadata": self.metadata,
        }

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> "CompileArtifact":
        return cls(
            target=d.get("target", "cpu"), quant=d.get("quant"), model_path=d.get("model_path", ""),
            config=ModelConfig.from_dict(d["config"]),
            graphs={m: Graph.from_dict(g) for m, g in d.get("graphs", {}).items()},
            pass_traces={m: list(t) for m, t in d.get("pass_traces", {}).items()},
            version=d.get("version", "0.1"), created_at=d.get("created_at", ""), metadata=dict(d.get("metadata", {})),
        )

    def save(self, path: str | Path) -> Path:
        out = Path(path)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(self.to_dict(), indent=2), encoding="utf-8")
        return out

    @classmethod
    def load(cls, path: str | Path) -> "CompileArtifact":
        p = Path(path)
        if p.is_dir():
            p = p / "artifact.json"
        return cls.from_dict(json.loads(p.read_text(encoding="utf-8")))
