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
* quant None on a GGUF file (``compile_model("x.gguf")``: the config from GGUF metadata, weight specs keyed by
  GGUF tensor names, cacheir/compiler.py:40-107; ``tests/golden/tiny_gguf.py`` rebuilds the file, checked by its
  SHA-256), Q4_0 and Q8_0: the blocks load packed straight from the file, every step's logits are within the fp16
  bound 2e-3 + 1e-2|ref| of the oracle run on the decoded blocks (the fp16-storage oracle sits at 42-48% of
  that bound on this model), and teacher-forced on the reference's ids the argmax equals the reference's id at
  every step whose reference margin exceeds 0.01 (26 of 32 steps for Q4_0, 31 for Q8_0).
"""
import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import cacheir_amd
from oracle.runtime import OracleRuntime, create_tiny_weights

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import tiny_gguf  # noqa: E402


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


def _close16(got, ref, what):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    ratio = (np.abs(got - ref) / (2e-3 + 1e-2 * np.abs(ref))).max()
    assert ratio <= 1.0, f"{what}: worst |d| / (2e-3 + 1e-2|ref|) = {ratio:.3f}"
    return ratio


@pytest.mark.parametrize("fmt,min_checked", [("q4_0", 26), ("q8_0", 31)])
def test_reference_gguf_artifact_teacher_forced(tmp_path, device, fmt, min_checked):
    d = json.loads((GOLDEN / f"reference_artifact_tiny_gguf_{fmt}.json").read_text())
    fx = d.pop("fixture")
    gguf = tmp_path / f"tiny_{fmt}.gguf"
    assert tiny_gguf.write_tiny_gguf(gguf, fmt) == fx["gguf_sha256"]
    d["model_path"] = str(gguf)
    path = tmp_path / "artifact.json"
    path.write_text(json.dumps(d))
    art = cacheir_amd.retarget(cacheir_amd.CompileArtifact.load(path))
    rt = cacheir_amd.create_runtime(art, backend="rocm")
    assert rt.dtype == torch.float16
    orc = OracleRuntime({m: art.graph(m).to_dict() for m in ("prefill", "decode")}, tiny_gguf.decoded_weights(fmt),
                        art.config.vocab_size)
    logits = rt.run([fx["prompt"]], mode="prefill")
    worst = _close16(logits.cpu().numpy(), orc.run([fx["prompt"]], mode="prefill"), "prefill")
    checked = 0
    for step, (want, margin) in enumerate(zip(fx["greedy_ids"], fx["top2_margins"])):
        got = int(torch.argmax(logits[0, -1]).item())
        if margin > 0.01:
            assert got == want, f"step {step}: {got} != {want} (reference margin {margin:.4f})"
            checked += 1
        logits = rt.run([[want]], mode="decode")
        worst = max(worst, _close16(logits.cpu().numpy(), orc.run([[want]], mode="decode"), f"decode step {step}"))
    print(f"{fmt}: {checked} ids checked, worst logit error {worst:.3f} of the fp16 bound")
    assert checked >= min_checked
    counts = rt.cache_stats()["kernel_counts"]
    assert counts.get("rocm.qgemm_blocks", 0) > 0 and counts.get("rocm.qgemm_swiglu", 0) > 0
    assert counts.get("rocm.graph_capture", 0) >= 1
