"""Writes tests/golden/tiny_greedy.json: BASELINE config 1 through the NumPy oracle.

Tiny Llama decoder: 2 layers, hidden 256, 4 query / 2 KV heads, head_dim 64,
SwiGLU ffn 688, vocab 1024, RMSNorm eps 1e-5, RoPE theta 10000, fp32 weights
N(0, 0.02) drawn as cacheir/importers/tiny.py:40-60 does with seed 0; batch 1,
16-token prompt = np.random.default_rng(1).integers(0, 1024, 16); greedy decode of
32 tokens; KV page size 16.

The ids come from the oracle's graph-driven runtime (oracle/runtime.py) and are
cross-checked here against the oracle's direct (graph-free) forward.  Also stored:
each step's top-2 logit margin, so a reader can see how close any argmax is.
Run: python tests/golden/make_tiny_greedy.py
"""
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from cacheir_amd.artifact import ModelConfig  # noqa: E402
from cacheir_amd.compiler import compile_config  # noqa: E402
from oracle.runtime import OracleRuntime, create_tiny_weights, direct_generate, generate_ids  # noqa: E402

CFG = dict(seed=0, vocab_size=1024, hidden_size=256, intermediate_size=688, num_layers=2, num_attention_heads=4,
           num_key_value_heads=2)


def tiny_config() -> ModelConfig:
    return ModelConfig(architecture="CacheIRTinyForCausalLM", hidden_size=256, intermediate_size=688, num_layers=2,
                       num_attention_heads=4, num_key_value_heads=2, vocab_size=1024, max_position_embeddings=256,
                       rope_theta=10000.0, rms_norm_eps=1e-5, dtype="float32")


def main() -> None:
    weights = create_tiny_weights(**CFG)
    prompt = np.random.default_rng(1).integers(0, 1024, 16).tolist()
    art = compile_config(tiny_config())
    graphs = {m: g.to_dict() for m, g in art.graphs.items()}
    rt = OracleRuntime(graphs, weights, 1024)
    ids, _ = generate_ids(rt, prompt, 32)
    direct_ids, rows = direct_generate(weights, num_layers=2, num_heads=4, num_kv_heads=2, eps=1e-5, theta=10000.0,
                                       vocab=1024, prompt_ids=prompt, max_new_tokens=32)
    assert ids == direct_ids, (ids, direct_ids)
    margins = []
    for r in rows:
        top = np.sort(r)[-2:]
        margins.append(float(top[1] - top[0]))
    out = {"config": CFG, "prompt_ids": prompt, "greedy_ids": ids, "top2_margins": margins,
           "first_step_logits_head": [float(v) for v in rows[0][:16]]}
    Path(__file__).with_name("tiny_greedy.json").write_text(json.dumps(out, indent=1))
    print("greedy", ids)
    print("min margin", min(margins))


if __name__ == "__main__":
    main()
