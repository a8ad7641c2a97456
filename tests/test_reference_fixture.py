"""The oracle and the graph builder against vectors written by the reference's own
NumPy backend (tests/golden/reference_tiny.json, made by
tests/golden/make_reference_tiny.py from cacheir/importers/tiny.py,
cacheir/compiler.py:135 and cacheir/runtime/cpu.py:111-184)."""
import json
from pathlib import Path

import numpy as np

from cacheir_amd.artifact import ModelConfig
from cacheir_amd.compiler import compile_config
from oracle.runtime import OracleRuntime, create_tiny_weights, generate_ids

FX = json.loads((Path(__file__).resolve().parent / "golden" / "reference_tiny.json").read_text())


def tiny_config() -> ModelConfig:
    c = FX["config"]
    return ModelConfig(architecture="CacheIRTinyForCausalLM", hidden_size=c["hidden_size"],
                       intermediate_size=c["intermediate_size"], num_layers=c["num_layers"],
                       num_attention_heads=c["num_attention_heads"], num_key_value_heads=c["num_key_value_heads"],
                       vocab_size=c["vocab_size"], max_position_embeddings=256, rope_theta=10000.0,
                       rms_norm_eps=1e-5, dtype="float32")


def test_tiny_weights_bit_identical_to_reference():
    w = create_tiny_weights(**FX["config"])
    assert sorted(w) == sorted(FX["weight_sum_and_sumsq"])
    for k, (s, q) in FX["weight_sum_and_sumsq"].items():
        assert float(np.sum(w[k], dtype=np.float64)) == s, k
        assert float(np.sum(np.square(w[k], dtype=np.float64))) == q, k


def test_decode_graph_ops_match_reference():
    art = compile_config(tiny_config())
    assert [n.op for n in art.graph("decode").nodes] == FX["decode_ops"]


def test_oracle_greedy_ids_match_reference_numpy_backend():
    art = compile_config(tiny_config())
    w = create_tiny_weights(**FX["config"])
    rt = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, w, FX["config"]["vocab_size"])
    ids, last = generate_ids(rt, FX["prompt"], 32)
    assert ids == FX["greedy_ids"]
    top = FX["final_top8"]
    np.testing.assert_allclose(np.asarray(last, np.float64)[0, -1][top["ids"]], top["logits"], rtol=1e-5, atol=1e-5)


def test_oracle_ragged_batch_decode_equals_per_session_decode():
    """A ragged batch (rows at different positions, each with its own cache) in one oracle pass gives each row what
    that row's own session computes: RoPE at the row's length, attention over the row's cache only."""
    from oracle.runtime import decode_batch

    art = compile_config(tiny_config())
    w = create_tiny_weights(**FX["config"])
    graphs = {m: g.to_dict() for m, g in art.graphs.items()}
    vocab = FX["config"]["vocab_size"]
    rng = np.random.default_rng(11)
    for fp16_storage in (False, True):
        base = OracleRuntime(graphs, w, vocab, fp16_storage=fp16_storage)
        sessions = []
        for n in (3, 17, 9, 30):
            s = base.fork()
            s.run([rng.integers(0, vocab, n).tolist()], mode="prefill")
            sessions.append(s)
        batch = base.fork()
        layers = sorted(sessions[0].keys)
        for layer in layers:
            batch.keys[layer] = [s.keys[layer][0].copy() for s in sessions]
            batch.values[layer] = [s.values[layer][0].copy() for s in sessions]
        toks = rng.integers(0, vocab, len(sessions)).tolist()
        got = batch.run(np.asarray(toks)[:, None], mode="decode")
        want = decode_batch(sessions, toks)
        # batched and one-row matmuls sum in different orders: fp32 rounding apart, and with fp16 storage that
        # can flip a stored value by one fp16 ulp (~2.4e-4 relative), which the next layer carries on
        tol = dict(rtol=1e-2, atol=2e-3) if fp16_storage else dict(rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(got, want, **tol)
        for layer in layers:
            assert [len(r) for r in batch.keys[layer]] == [s.keys[layer].shape[1] for s in sessions]
            for r, s in zip(batch.values[layer], sessions):
                np.testing.assert_allclose(r, s.values[layer][0], **tol)
