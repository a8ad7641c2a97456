"""Writes tests/golden/reference_tiny.json from the reference's own NumPy backend.

BASELINE config 1 (tiny Llama decoder, seed 0; batch 1; 16-token prompt
np.random.default_rng(1).integers(0, 1024, 16); 32 greedy tokens) run through the
reference: cacheir/importers/tiny.py:9-70 (create_tiny_model), cacheir/compiler.py:135
(compile_model, target "cpu"), cacheir/runtime/cpu.py:111-138 (Runtime.run) with the
greedy loop of cpu.py:167-184 (argmax of the last logits, then one decode step).

Nothing in the reference's tests fixes these ids or the tiny weights, so they are
recorded here as vectors: the greedy ids, each step's top-2 margin, the sum and
sum of squares of every weight array (pins the seeded draw order of our
oracle's restatement), the decode graph's op sequence, and the last step's top-8
logits.  Only this script reads /root/reference; it runs with the working directory
outside this repository so the reference's native-extension search path
(cacheir/backends/native.py) finds nothing and its pure-NumPy branches run.

Run (in a container that has /root/reference): python tests/golden/make_reference_tiny.py
"""
import json
import os
import sys
import tempfile
from pathlib import Path

import numpy as np

sys.dont_write_bytecode = True  # importing the reference must leave no __pycache__ in its tree

REF = Path(os.environ.get("CACHEIR_REFERENCE", "/root/reference"))
OUT = Path(__file__).resolve().parent / "reference_tiny.json"
CFG = dict(seed=0, vocab_size=1024, hidden_size=256, intermediate_size=688, num_layers=2, num_attention_heads=4,
           num_key_value_heads=2)


def main() -> None:
    with tempfile.TemporaryDirectory() as tmp:
        os.chdir(tmp)
        sys.path.insert(0, str(REF))
        from cacheir import Runtime, compile_model  # reference package
        from cacheir.importers import create_tiny_model

        model = create_tiny_model(Path(tmp) / "tiny", **CFG)
        weights = np.load(Path(model) / "weights.npz")
        checks = {k: [float(np.sum(weights[k], dtype=np.float64)), float(np.sum(np.square(weights[k], dtype=np.float64)))]
                  for k in sorted(weights.files)}
        art = compile_model(model, target="cpu", mode=["prefill", "decode"], max_seq=256)
        rt = Runtime(art)
        prompt = np.random.default_rng(1).integers(0, 1024, 16).tolist()
        logits = rt.run([prompt], mode="prefill")
        ids, margins = [], []
        for _ in range(32):
            last = np.asarray(logits[0, -1], dtype=np.float64)
            top = np.sort(last)[-2:]
            nxt = int(np.argmax(last)) % 1024
            ids.append(nxt)
            margins.append(float(top[1] - top[0]))
            logits = rt.run([[nxt]], mode="decode")
        last = np.asarray(logits[0, -1], dtype=np.float64)
        order = np.argsort(-last)[:8]
        decode_ops = [n.op for n in art.graph("decode").nodes]
        fixture = {
            "config": CFG,
            "prompt": prompt,
            "greedy_ids": ids,
            "top2_margins": margins,
            "weight_sum_and_sumsq": checks,
            "decode_ops": decode_ops,
            "final_top8": {"ids": order.tolist(), "logits": last[order].tolist()},
        }
    OUT.write_text(json.dumps(fixture, indent=1) + "\n", encoding="utf-8")
    print(f"wrote {OUT}: greedy {ids[:8]}... min margin {min(margins):.4g}")


if __name__ == "__main__":
    main()
