"""Writes the reference compiler's artifacts and packing vectors used as boundary fixtures.

* ``reference_artifact_tiny.json`` / ``reference_artifact_tiny_int4_awq.json``: the artifact JSON that
  the reference's ``compile_model`` (cacheir/compiler.py:135-181, saved by cacheir/runtime/artifact.py:109-114)
  writes for BASELINE config 1's tiny model (cacheir/importers/tiny.py:9-70, seed 0), target "cpu", with quant
  None and with ``int4_awq``.  ``model_path`` is blanked (the tests point it at a directory holding the same
  weights, which the oracle's ``create_tiny_weights`` reproduces bit for bit) and ``pass_traces`` keeps each
  mode's first two entries.  The int4_awq file also records
  the reference NumPy backend's 32 greedy ids for the config-1 prompt (cacheir/runtime/cpu.py:111-184) and each
  step's top-2 margin.
* ``reference_pack.json``: ``pack_quantized_weight`` (cacheir/quantization.py:63-139) for 4 and 8 bits on a
  fixed 7 x 37 matrix (odd width: the last byte of each 4-bit row holds one nibble) whose rows include exact
  halves, so np.round's half-to-even rule decides zero points and codes; packed bytes, scales, zero points and
  ``dequantize_packed_weight``'s output.
* ``reference_artifact_tiny_gguf_q4_0.json`` / ``..._q8_0.json``: the artifact ``compile_model`` writes for the
  tiny model stored as a GGUF file (``tiny_gguf.py``: Q4_0 or Q8_0 linear weights, F16 embedding, F32 norms,
  ``llama.*`` metadata), i.e. the config built from GGUF metadata (cacheir/compiler.py:40-63) and weight specs
  keyed by GGUF tensor names (compiler.py:66-107).  Each also records the GGUF file's SHA-256 and the reference
  NumPy backend's 32 greedy ids and top-2 margins on it (the blocks decoded by GGUFReader.read_tensor,
  cacheir/runtime/cpu.py:60-68, then the greedy loop of cpu.py:167-184).

Only this script reads /root/reference; it runs with the working directory outside this repository (the
reference's native-extension search path then finds nothing and its NumPy branches run).

Run (in a container that has /root/reference): python tests/golden/make_reference_artifacts.py
"""
import json
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

sys.dont_write_bytecode = True  # importing the reference must leave no __pycache__ in its tree
HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))  # the repo root: oracle/ and tests/golden/tiny_gguf.py
sys.path.insert(0, str(HERE))
import tiny_gguf  # noqa: E402

REF = Path(os.environ.get("CACHEIR_REFERENCE", "/root/reference"))
CFG = dict(seed=0, vocab_size=1024, hidden_size=256, intermediate_size=688, num_layers=2, num_attention_heads=4,
           num_key_value_heads=2)


def pack_matrix() -> np.ndarray:
    rng = np.random.default_rng(11)
    w = rng.standard_normal((7, 37)).astype(np.float32)
    # row 0: min -1.25, max 6.25 -> 4-bit scale 0.5, -min/scale = 2.5 (zero point by half-to-even: 2)
    w[0] = np.linspace(-1.25, 6.25, 37, dtype=np.float32)
    w[0, 5] = 0.25  # 0.25 / 0.5 + 2 = 2.5 -> code 2
    # row 1: min -0.75, max 0.75 -> scale 0.1, -min/scale = 7.5 (-> 8); codes at x.5 both ways
    w[1] = np.linspace(-0.75, 0.75, 37, dtype=np.float32)
    # row 2: constant row (scale clamps to 1e-8)
    w[2] = 0.5
    return w


def greedy(rt, prompt: list[int], steps: int = 32) -> tuple[list[int], list[float]]:
    """cpu.py:167-184 on the reference Runtime ``rt``: ids and each step's top-2 margin."""
    logits = rt.run([prompt], mode="prefill")
    ids, margins = [], []
    for _ in range(steps):
        last = np.asarray(logits[0, -1], dtype=np.float64)
        top = np.sort(last)[-2:]
        nxt = int(np.argmax(last)) % 1024
        ids.append(nxt)
        margins.append(float(top[1] - top[0]))
        logits = rt.run([[nxt]], mode="decode")
    return ids, margins


def main() -> None:
    with tempfile.TemporaryDirectory() as tmp:
        os.chdir(tmp)
        sys.path.insert(0, str(REF))
        from cacheir import Runtime, compile_model  # reference package
        from cacheir.importers import create_tiny_model
        from cacheir.quantization import dequantize_packed_weight, pack_quantized_weight

        model = create_tiny_model(Path(tmp) / "tiny", **CFG)
        prompt = np.random.default_rng(1).integers(0, 1024, 16).tolist()
        for quant, name in ((None, "reference_artifact_tiny.json"), ("int4_awq", "reference_artifact_tiny_int4_awq.json")):
            art = compile_model(model, target="cpu", quant=quant, mode=["prefill", "decode"], max_seq=256)
            d = art.to_dict()
            d["model_path"] = ""
            # the per-pass graph snapshots (~0.5 MB, read by no runtime) are cut to each mode's first two entries
            d["pass_traces"] = {m: list(t)[:2] for m, t in d["pass_traces"].items()}
            if quant:
                ids, margins = greedy(Runtime(art), prompt)
                d["fixture"] = {"prompt": prompt, "greedy_ids": ids, "top2_margins": margins}
            (HERE / name).write_text(json.dumps(d, indent=1) + "\n", encoding="utf-8")
            print(f"wrote {name}")

        for fmt in ("q4_0", "q8_0"):
            gguf = Path(tmp) / f"tiny_{fmt}.gguf"
            sha = tiny_gguf.write_tiny_gguf(gguf, fmt)
            art = compile_model(gguf, target="cpu", mode=["prefill", "decode"], max_seq=256)
            ids, margins = greedy(Runtime(art), prompt)
            d = art.to_dict()
            d["model_path"] = ""
            d["pass_traces"] = {m: list(t)[:2] for m, t in d["pass_traces"].items()}
            d["fixture"] = {"prompt": prompt, "greedy_ids": ids, "top2_margins": margins, "gguf_sha256": sha}
            name = f"reference_artifact_tiny_gguf_{fmt}.json"
            (HERE / name).write_text(json.dumps(d, indent=1) + "\n", encoding="utf-8")
            print(f"wrote {name}")

        w = pack_matrix()
        out = {"weight": w.tolist()}
        for bits, quant in ((4, "int4_awq"), (8, "int8")):
            p = pack_quantized_weight(w, quant)
            assert p.bits == bits
            out[str(bits)] = {
                "packed_hex": p.packed_values.tobytes().hex(), "packed_shape": list(p.packed_values.shape),
                "scales": p.scales.tolist(), "zero_points": p.zero_points.tolist(),
                "dequant": dequantize_packed_weight(p).tolist(),
            }
        (HERE / "reference_pack.json").write_text(json.dumps(out, indent=1) + "\n", encoding="utf-8")
        print("wrote reference_pack.json")


if __name__ == "__main__":
    main()
