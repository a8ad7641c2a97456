"""Artifacts written by the reference's compile_model, run by this backend (GPU).

The path a CacheIR user takes: ``CompileArtifact.load`` of the reference's JSON, ``retarget`` to rocm,
``create_runtime(..., backend="rocm")`` (cacheir/runtime/__init__.py:10-24 with the rocm branch added), then the
reference's greedy loop (cacheir/runtime/cpu.py:167-184).  ``model_path`` points at a directory holding the tiny
model's weights, which ``create_tiny_weights`` reproduces bit for bit (tests/test_reference_fixture.py).

* quant None, fp32: the 32 greedy ids equal those the reference's NumPy backend produced
  (tests/golden/reference_tiny.json).
* quant int4_awq (the reference packs every linear weight per row, quantization.py:96-139; this backend runs the
  packed codes on the MFMA GEMM with fp16 activations): teacher-forced on the reference's ids, the argmax equals
  the reference's id at every step whose reference top-2 margin exceeds 0.01 (28 of the 32 steps; fp16
  activations move these logits by ~1e-3).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import cacheir_amd
from oracle.runtime import create_tiny_weights

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name: str, tmp_path: Path):
    d = json.loads((GOLDEN / name).read_text())
    fixture = d.pop("fixture", None)
    c = json.loads((GOLDEN / "reference_tiny.json").read_text())["config"]
    model = tmp_path / "tiny"
    model.mkdir()
    np.savez(model / "weights.npz", **create_tiny_weights(**c))
    d["model_path"] = str(model)
    path = tmp_path / "artifact.json"
    path.write_text(json.dumps(d))
    art = cacheir_amd.retarget(cacheir_amd.CompileArtifact.load(path))
    return art, fixture


def test_reference_artifact_fp32_greedy_ids(tmp_path, device):
    art, _ = _load("reference_artifact_tiny.json", tmp_path)
    rt = cacheir_amd.create_runtime(art, backend="rocm", dtype="float32")
    ref = json.loads((GOLDEN / "reference_tiny.json").read_text())
    logits = rt.run([ref["prompt"]], mode="prefill")
    ids = []
    for _ in range(32):
        nxt = int(torch.argmax(logits[0, -1]).item()) % art.config.vocab_size
        ids.append(nxt)
        logits = rt.run([[nxt]], mode="decode")
    assert ids == ref["greedy_ids"]
    assert rt.cache_stats()["kernel_counts"].get("rocm.graph_capture", 0) >= 1  # the decode steps replayed a graph


def test_reference_artifact_int4_awq_teacher_forced(tmp_path, device):
    art, fx = _load("reference_artifact_tiny_int4_awq.json", tmp_path)
    rt = cacheir_amd.create_runtime(art, backend="rocm")
    assert rt.dtype == torch.float16
    logits = rt.run([fx["prompt"]], mode="prefill")
    checked = 0
    for step, (want, margin) in enumerate(zip(fx["greedy_ids"], fx["top2_margins"])):
        got = int(torch.argmax(logits[0, -1]).item())
        if margin > 0.01:
            assert got == want, f"step {step}: {got} != {want} (reference margin {margin:.4f})"
            checked += 1
        logits = rt.run([[want]], mode="decode")
    assert checked >= 28
    assert rt.kernel_counts.get("rocm.qgemm_swiglu", 0) > 0
