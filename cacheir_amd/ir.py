"""CacheIR graph schema as consumed by the ROCm backend.

The JSON layout is CacheIR's own (``cacheir/ir.py:28-139`` for TensorType,
WeightSpec and Node; ``cacheir/ir.py:262-289`` for ``Graph.to_dict/from_dict``):
a graph is ``{name, mode, target, inputs, outputs, nodes, values, weights,
constants, attrs}``; a node is ``{op, inputs, outputs, attrs, name, side_effect}``;
a weight is ``{key, tensor_type, quant, file}``; a tensor type is
``{shape, dtype, layout}``.  The backend must read artifacts written by the
reference compiler unchanged, so the field names and nesting are kept identical.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any


@dataclass(frozen=True)
class TensorType:
    shape: tuple
    dtype: str = "float32"
    layout: str = "row_major"

    def to_dict(self) -> dict[str, Any]:
        return {"shape": list(self.shape), "dtype": self.dtype, "layout": self.layout}

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> "TensorType":
        return cls(tuple(d["shape"]), d.get("dtype", "float32"), d.get("layout", "row_major"))


@dataclass
class WeightSpec:
    key: str
    tensor_type: TensorType
    quant: str | None = None
    file: str | None = None

    def to_dict(self) -> dict[str, Any]:
        return {"key": self.key, "tensor_type": self.tensor_type.to_dict(), "quant": self.quant, "file": self.file}

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> "WeightSpec":
        return cls(d["key"], TensorType.from_dict(d["tensor_type"]), d.get("quant"), d.get("file"))


@dataclass
class Node:
    op: str
    inputs: list[str]
    outputs: list[str]
    attrs: dict[str, Any] = field(default_factory=dict)
    name: str | None = None
    side_effect: bool = False

    def to_dict(self) -> dict[str, Any]:
        return {"op": self.op, "inputs": list(self.inputs), "outputs": list(self.outputs),
                "attrs": self.attrs, "name": self.name, "side_effect": self.side_effect}

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> "Node":
        return cls(d["op"], list(d.get("inputs", [])), list(d.get("outputs", [])), dict(d.get("attrs", {})),
                   d.get("name"), bool(d.get("side_effect", False)))


@dataclass
class Graph:
    name: str
    mode: str = "logical"
    target: str = "cpu"
    inputs: dict[str, TensorType] = field(default_factory=dict)
    outputs: list[str] = field(default_factory=list)
    nodes: list[Node] = field(default_factory=list)
    values: dict[str, TensorType] = field(default_factory=dict)
    weights: dict[str, WeightSpec] = field(default_factory=dict)
    constants: dict[str, Any] = field(default_factory=dict)
    attrs: dict[str, Any] = field(default_factory=dict)

    def to_dict(self) -> dict[str, Any]:
        return {
            "name": self.name, "mode": self.mode, "target": self.target,
            "inputs": {k: v.to_dict() for k, v in self.inputs.items()},
            "outputs": list(self.outputs),
            "nodes": [n.to_dict() for n in self.nodes],
            "values": {k: v.to_dict() for k, v in self.values.items()},
            "weights": {k: v.to_dict() for k, v in self.weights.items()},
            "constants": self.constants, "attrs": self.attrs,
        }

    @classmethod
    def from_dict(cls, d: dict[str, Any]) -> "Graph":
        return cls(
            name=d["name"], mode=d.get("mode", "logical"), target=d.get("target", "cpu"),
            inputs={k: TensorType.from_dict(v) for k, v in d.get("inputs", {}).items()},
            outputs=list(d.get("outputs", [])),
            nodes=[Node.from_dict(n) for n in d.get("nodes", [])],
            values={k: TensorType.from_dict(v) for k, v in d.get("values", {}).items()},
            weights={k: WeightSpec.from_dict(v) for k, v in d.get("weights", {}).items()},
            constants=dict(d.get("constants", {})), attrs=dict(d.get("attrs", {})),
        )

    def producers(self) -> dict[str, Node]:
        return {out: n for n in self.nodes for out in n.outputs}

    def consumers(self) -> dict[str, list[Node]]:
        table: dict[str, list[Node]] = {}
        for n in self.nodes:
            for i in n.inputs:
                table.setdefault(i, []).append(n)
        return table
