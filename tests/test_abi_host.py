"""CPU-only checks of the C-ABI library and the host-side logic (no GPU calls)."""
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from cacheir_amd import hip
from cacheir_amd.artifact import ModelConfig
from cacheir_amd.compiler import ROCM_KERNELS, build_graph, compile_config
from cacheir_amd.weights import GGML_Q4_0, GGML_Q8_0, quantize_q4_0, quantize_q8_0
from oracle import quant

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "cacheir_hip.h"


def declared_symbols() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(cir_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_bound_entry_points():
    syms = declared_symbols()
    assert len(syms) >= 20
    assert syms == set(hip._SIGNATURES), syms ^ set(hip._SIGNATURES)


@pytest.mark.skipif(not hip.library_path().exists(), reason="libcacheir_hip.so not built (python -m cacheir_amd.build)")
def test_library_exports_every_declared_symbol():
    nm = shutil.which("nm") or "/opt/rocm/llvm/bin/llvm-nm"
    out = subprocess.run([nm, "-D", "--defined-only", str(hip.library_path())], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\b(cir_[a-z0-9_]+)\b", out))
    missing = declared_symbols() - exported
    assert not missing, f"declared in {HEADER.name} but not exported: {sorted(missing)}"


@pytest.mark.skipif(not hip.library_path().exists(), reason="libcacheir_hip.so not built")
def test_library_loads_and_reports_version_without_a_gpu():
    lib = hip.load()
    assert lib.cir_version().decode().startswith("cacheir_amd")
    # size queries are pure host arithmetic
    assert lib.cir_qweight_tiled_bytes(hip.CIR_Q4_0, 64, 256) == 64 * 256 // 32 * 18
    assert lib.cir_qweight_tiled_bytes(hip.CIR_Q8_0, 64, 256) == 64 * 256 // 32 * 34
    assert lib.cir_qweight_tiled_bytes(hip.CIR_Q4_0, 64, 100) == 0  # k must be a multiple of 128
    assert lib.cir_paged_attention_workspace_bytes(0, 8, 128, 2048) == 0
    assert lib.cir_paged_attention_workspace_bytes(2, 8, 128, 2048) > 0


def llama(layers=3, **kw):
    base = dict(architecture="LlamaForCausalLM", hidden_size=256, intermediate_size=512, num_layers=layers,
                num_attention_heads=8, num_key_value_heads=2, vocab_size=1000, rope_theta=10000.0, rms_norm_eps=1e-5,
                dtype="float16")
    base.update(kw)
    return ModelConfig(**base)


@pytest.mark.parametrize("mode", ["decode", "prefill"])
@pytest.mark.parametrize("quant_name", [None, "q4_0"])
def test_graph_structure(mode, quant_name):
    cfg = llama()
    g = build_graph(cfg, mode, quant=quant_name)
    ops = [n.op for n in g.nodes]
    qp = "quantized_" if quant_name else ""  # the reference's op names for quantized graphs
    assert len(ops) == 1 + 8 * cfg.num_layers + 2
    assert ops[0] == "token_embedding" and ops[-2:] == ["rms_norm", qp + "matmul"]
    attn = "paged_attention_decode" if mode == "decode" else "paged_attention_prefill"
    assert ops.count(attn) == cfg.num_layers and ops.count(qp + "fused_swiglu") == cfg.num_layers
    assert ops.count(qp + "fused_rmsnorm_qkv_rope") == cfg.num_layers and ops.count("add") == 2 * cfg.num_layers
    assert g.attrs["execution_hints"]["page_size"] == 16
    for n in g.nodes:
        assert n.attrs["kernel"] == "rocm." + ROCM_KERNELS[n.op]
        if n.op.endswith("fused_rmsnorm_qkv_rope"):
            assert n.attrs["head_dim"] == 32 and n.attrs["rope_theta"] == 10000.0
    # every weight input names a weight spec
    for n in g.nodes:
        for v in n.inputs:
            assert v in g.weights or v in g.values or v == "input_ids" or any(v in m.outputs for m in g.nodes)


def test_artifact_roundtrip(tmp_path):
    art = compile_config(llama(layers=2), quant="q8_0")
    path = tmp_path / "a.json"
    art.save(path)
    from cacheir_amd.artifact import CompileArtifact

    back = CompileArtifact.load(path)
    assert back.target == "rocm" and back.quant == "q8_0"
    assert [n.op for n in back.graph("decode").nodes] == [n.op for n in art.graph("decode").nodes]


@pytest.mark.parametrize("fmt", [GGML_Q4_0, GGML_Q8_0])
def test_host_quantizer_matches_oracle_decode(fmt):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 256)).astype(np.float32)
    raw = quantize_q4_0(w) if fmt == GGML_Q4_0 else quantize_q8_0(w)
    blocks = raw.reshape(16, -1)
    dec = quant.decode_q4_0(blocks, 256) if fmt == GGML_Q4_0 else quant.decode_q8_0(blocks, 256)
    amax = np.abs(w.reshape(16, -1, 32)).max(-1, keepdims=True)
    step = (amax / (8 if fmt == GGML_Q4_0 else 127)).repeat(32, -1).reshape(w.shape)
    # Q4_0 (d = signed max / -8) clips the far end of the range to 7 steps: error <= one step;
    # Q8_0 rounds to nearest: half a step, plus the fp16 rounding of d times |q| <= 127.
    bound = step * 1.001 if fmt == GGML_Q4_0 else step * (0.5 + 127 * 2.0 ** -11)
    assert np.all(np.abs(dec - w) <= bound + 1e-7)
    # the largest-magnitude value of each block is reproduced up to the fp16 rounding of d
    i = np.abs(w.reshape(16, -1, 32)).argmax(-1)
    wm = np.take_along_axis(w.reshape(16, -1, 32), i[..., None], -1)
    dm = np.take_along_axis(dec.reshape(16, -1, 32), i[..., None], -1)
    np.testing.assert_allclose(dm, wm, rtol=2.0 ** -10)
