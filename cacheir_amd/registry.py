"""Backend registry entry for the ROCm target.

Mirrors ``cacheir/backends/registry.py:6-67`` (``Backend(name, devices, kernels,
notes)`` in a name-keyed registry).  ``register_into(registry)`` adds the entry to
any object with a ``register(backend)`` method, e.g. the reference's
``BackendRegistry``.
"""
from __future__ import annotations

from dataclasses import dataclass

from cacheir_amd.compiler import ROCM_KERNELS


@dataclass(frozen=True)
class Backend:
    name: str
    devices: tuple[str, ...]
    kernels: tuple[str, ...]
    notes: str = ""


class BackendRegistry:
    def __init__(self) -> None:
        self._backends: dict[str, Backend] = {}

    def register(self, backend: Backend) -> None:
        self._backends[backend.name] = backend

    def get(self, name: str) -> Backend:
        return self._backends[name]

    def names(self) -> list[str]:
        return sorted(self._backends)


def rocm_backend() -> Backend:
    return Backend(
        name="rocm",
        devices=("gfx950", "mi355x"),
        kernels=tuple(sorted(set(ROCM_KERNELS.values()))),
        notes="Hand-written HIP kernels for CDNA4 behind a C ABI (libcacheir_hip.so): MFMA paged decode attention, "
              "Q4_0/Q8_0 dequant-fused MFMA GEMM, RMSNorm+QKV+RoPE+KV-append and SwiGLU epilogues, HIP-graph "
              "decode steps.",
    )


def register_into(registry) -> None:
    registry.register(rocm_backend())


def default_registry() -> BackendRegistry:
    reg = BackendRegistry()
    register_into(reg)
    return reg
