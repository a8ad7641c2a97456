"""The drop-in boundary against files the reference itself wrote (tests/golden/make_reference_artifacts.py).

* ``reference_pack.json``: the reference's ``pack_quantized_weight`` / ``dequantize_packed_weight``
  (cacheir/quantization.py:63-139) on a 7 x 37 matrix with exact halves.  The weight store's ``pack_rows`` (what
  HipRuntime packs for ``--quant int4_awq / int8``) and the oracle's restatement must give the same bytes, scales
  and zero points, and the oracle's dequant the same floats -- so a swapped nibble order or a round-half-up zero
  point fails here.
* ``reference_artifact_tiny*.json``: artifacts written by the reference's ``compile_model`` (target "cpu", quant
  None and int4_awq).  They load into ``CompileArtifact``, ``retarget`` moves every node to a ``rocm.*`` kernel,
  and their decode/prefill graphs have exactly the node list, op names, value names and weight keys that
  ``compile_config`` builds -- the graph HipRuntime executes.  (Running them on the GPU is
  tests/test_reference_artifacts_gpu.py.)
* ``reference_artifact_tiny_gguf_{q4_0,q8_0}.json``: what ``compile_model`` writes for a GGUF file (config from
  GGUF metadata, cacheir/compiler.py:40-63; weight specs keyed by GGUF tensor names, compiler.py:66-107), with
  the reference NumPy backend's greedy ids on it.  The file ``tests/golden/tiny_gguf.py`` builds must be the
  file the reference ran (SHA-256); this backend's GGUF reader returns every tensor the specs name, in the
  shape they state, with the blocks' bytes as stored; and the oracle run on the decoded blocks reproduces all
  32 of the reference's ids.
"""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

from cacheir_amd import CompileArtifact, retarget
from cacheir_amd.compiler import compile_config
from cacheir_amd.weights import GGUFFile, pack_rows, unpack_rows
from oracle import quant as oq
from oracle.runtime import OracleRuntime

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import tiny_gguf  # noqa: E402
PACK = json.loads((GOLDEN / "reference_pack.json").read_text())


@pytest.mark.parametrize("bits", [4, 8])
def test_row_packing_equals_the_reference_bytes(bits):
    w = np.asarray(PACK["weight"], dtype=np.float32)
    ref = PACK[str(bits)]
    ref_packed = np.frombuffer(bytes.fromhex(ref["packed_hex"]), dtype=np.uint8).reshape(ref["packed_shape"])
    ref_scales = np.asarray(ref["scales"], dtype=np.float32)
    ref_zps = np.asarray(ref["zero_points"], dtype=np.int32)
    packed, scales, zps = pack_rows(w, bits)
    assert packed.shape == tuple(ref["packed_shape"]) and np.array_equal(packed, ref_packed)
    assert np.array_equal(scales, ref_scales) and np.array_equal(zps, ref_zps)
    # the weight store's own dequant (used for widths the tiled GEMM cannot hold) gives the reference's floats
    assert np.array_equal(unpack_rows(packed, scales, zps, bits, w.shape[1]), np.asarray(ref["dequant"], np.float32))
    o = oq.asymmetric_pack(w, bits)
    assert np.array_equal(o["packed_values"], ref_packed)
    assert np.array_equal(o["scales"], ref_scales) and np.array_equal(o["zero_points"], ref_zps)
    assert np.array_equal(oq.asymmetric_dequant(o), np.asarray(ref["dequant"], dtype=np.float32))
    if bits == 4:
        # the half-to-even rows: zero point 2 (not 3) for -min/scale = 2.5; column 5 (high nibble of byte 2, odd
        # columns go high) holds code 2 for 0.25/0.5 + 2 = 2.5
        assert ref_zps[0] == 2 and (ref_packed[0, 2] >> 4) == 2
        assert w.shape[1] % 2 == 1 and np.all(ref_packed[:, -1] >> 4 == 0)  # odd width: last high nibble empty


def _reference_artifact(name: str) -> CompileArtifact:
    return CompileArtifact.from_dict(json.loads((GOLDEN / name).read_text()))


@pytest.mark.parametrize("name,quant", [("reference_artifact_tiny.json", None),
                                        ("reference_artifact_tiny_int4_awq.json", "int4_awq")])
def test_reference_artifact_retargets_to_the_graph_the_runtime_runs(name, quant):
    art = _reference_artifact(name)
    assert art.target == "cpu" and art.quant == quant
    ours = compile_config(art.config, quant=quant)
    retarget(art)
    assert art.target == "rocm"
    for mode in ("prefill", "decode"):
        g, o = art.graph(mode), ours.graph(mode)
        assert [n.op for n in g.nodes] == [n.op for n in o.nodes]
        assert [n.name for n in g.nodes] == [n.name for n in o.nodes]
        assert [(n.inputs, n.outputs) for n in g.nodes] == [(n.inputs, n.outputs) for n in o.nodes]
        assert list(g.inputs) == list(o.inputs) and list(g.outputs) == list(o.outputs)
        assert {k: s.key for k, s in g.weights.items()} == {k: s.key for k, s in o.weights.items()}
        assert all(n.attrs["kernel"].startswith("rocm.") for n in g.nodes)
        assert [n.attrs["kernel"] for n in g.nodes] == [n.attrs["kernel"] for n in o.nodes]
        for n, m in zip(g.nodes, o.nodes):  # the attrs the runtime reads
            for key in ("layer", "eps", "head_dim", "rope_theta", "num_heads", "num_kv_heads"):
                if key in m.attrs:
                    assert n.attrs.get(key) == m.attrs[key], (n.name, key)
        assert g.attrs["execution_hints"]["page_size"] == 16


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_reference_gguf_artifact_loads_and_the_oracle_reproduces_its_ids(fmt, tmp_path):
    d = json.loads((GOLDEN / f"reference_artifact_tiny_gguf_{fmt}.json").read_text())
    fx = d.pop("fixture")
    path = tmp_path / f"tiny_{fmt}.gguf"
    assert tiny_gguf.write_tiny_gguf(path, fmt) == fx["gguf_sha256"]
    art = CompileArtifact.from_dict(d)
    assert art.quant is None and art.config.quantization == "gguf" and art.config.dtype == "float16"
    assert art.config.hidden_size == tiny_gguf.CFG["hidden_size"] and art.config.num_layers == 2
    retarget(art)
    assert art.target == "rocm"
    f = GGUFFile(path)
    code = oq.GGML_TYPE_Q4_0 if fmt == "q4_0" else oq.GGML_TYPE_Q8_0
    for mode in ("prefill", "decode"):
        g = art.graph(mode)
        assert all(n.attrs["kernel"].startswith("rocm.") for n in g.nodes)
        for name, spec in g.weights.items():
            assert spec.key in f.tensors, (name, spec.key)
            assert f.shape(spec.key) == tuple(spec.tensor_type.shape), spec.key
            if len(spec.tensor_type.shape) == 2 and spec.key != "token_embd.weight":
                assert f.ggml_type(spec.key) == code  # the blocks load packed, as stored
    w = tiny_gguf.decoded_weights(fmt)
    orc = OracleRuntime({m: art.graph(m).to_dict() for m in ("prefill", "decode")}, w, art.config.vocab_size)
    logits = orc.run([fx["prompt"]], mode="prefill")
    ids = []
    for want in fx["greedy_ids"]:  # teacher forced, so one early flip cannot hide the rest
        ids.append(int(np.argmax(logits[0, -1])))
        logits = orc.run([[want]], mode="decode")
    assert ids == fx["greedy_ids"]
