"""cacheir_amd: an MI355X (gfx950) decode-step backend for CacheIR.

Public entry points mirror the reference's (``cacheir/runtime/__init__.py:10-24``):
``create_runtime(artifact, backend="rocm")`` returns a :class:`HipRuntime`;
``compile_config`` / ``build_graph`` produce lowered graphs for the ``rocm``
target; ``RocmKernelSelection`` retargets graphs compiled by the reference.
"""
from __future__ import annotations

from pathlib import Path

from cacheir_amd.artifact import CompileArtifact, ModelConfig
from cacheir_amd.compiler import RocmKernelSelection, build_graph, compile_config, retarget
from cacheir_amd.registry import Backend, BackendRegistry, default_registry, rocm_backend

__version__ = "0.1.0"


def create_runtime(artifact: CompileArtifact | str | Path, *, backend: str = "auto", **kwargs):
    """``backend`` "rocm" (or "auto") returns a HipRuntime; this package ships no CPU runtime."""
    loaded = CompileArtifact.load(artifact) if isinstance(artifact, (str, Path)) else artifact
    if backend not in {"auto", "rocm", "hip"}:
        raise ValueError(f"Unknown CacheIR runtime backend {backend!r} for cacheir_amd (use 'rocm')")
    from cacheir_amd.runtime import HipRuntime

    return HipRuntime(loaded, **kwargs)


def __getattr__(name):
    if name in {"HipRuntime", "StepPlan"}:
        from cacheir_amd import runtime

        return getattr(runtime, name)
    raise AttributeError(name)


__all__ = ["Backend", "BackendRegistry", "CompileArtifact", "HipRuntime", "ModelConfig", "RocmKernelSelection",
           "build_graph", "compile_config", "create_runtime", "default_registry", "retarget", "rocm_backend"]
