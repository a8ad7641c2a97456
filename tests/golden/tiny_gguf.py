"""The tiny GGUF model of the reference-artifact fixtures: a tiny Llama decoder drawn as BASELINE config 1's
(``create_tiny_weights``, seed 0) but at shapes the block formats and the fp16 MFMA kernels take (hidden 512,
ffn 1024: k a multiple of 128; 4 query / 2 KV heads of head_dim 128), in one GGUF v3 file, every linear weight (q/k/v/o, gate/up/down and the LM head) as Q4_0 or Q8_0 blocks, the token embedding
as F16 and the norms as F32, with the ``llama.*`` metadata the reference's ``_config_from_gguf`` reads
(cacheir/compiler.py:40-63) and tensor names from its ``_gguf_key_map`` (compiler.py:85-107).

The bytes are a pure function of this file and the oracle's ``create_tiny_weights`` (the reference's
``create_tiny_model`` draw, tests/test_reference_fixture.py), so the fixture script and the GPU test
build the same file; the fixture records its SHA-256 and the test checks it before use.

Quantizers (block of 32 along k, one fp16 scale d):
* Q8_0: d = amax / 127, q = clip(rint(w / d), -127, 127).
* Q4_0: d = m / -8 for the signed value m of largest magnitude, nibble = clip(floor(w / d + 8.5), 0, 15).
Both are the GGML quantizers' published rules; any deterministic rule would do, since parity is checked on
whatever blocks the file holds.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np

from oracle import quant as oq
from oracle.runtime import create_tiny_weights

CFG = dict(seed=0, vocab_size=1024, hidden_size=512, intermediate_size=1024, num_layers=2, num_attention_heads=4,
           num_key_value_heads=2)
EPS = 1e-5
THETA = 10000.0

_TOP = {"model.embed_tokens.weight": "token_embd.weight", "model.norm.weight": "output_norm.weight",
        "lm_head.weight": "output.weight"}
_LAYER = {"input_layernorm.weight": "attn_norm.weight", "self_attn.q_proj.weight": "attn_q.weight",
          "self_attn.k_proj.weight": "attn_k.weight", "self_attn.v_proj.weight": "attn_v.weight",
          "self_attn.o_proj.weight": "attn_output.weight", "post_attention_layernorm.weight": "ffn_norm.weight",
          "mlp.gate_proj.weight": "ffn_gate.weight", "mlp.up_proj.weight": "ffn_up.weight",
          "mlp.down_proj.weight": "ffn_down.weight"}


def gguf_name(hf: str) -> str:
    if hf in _TOP:
        return _TOP[hf]
    parts = hf.split(".")  # model.layers.<i>.<rest>
    return f"blk.{parts[2]}.{_LAYER['.'.join(parts[3:])]}"


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    n, k = w.shape
    b = w.astype(np.float32).reshape(n, k // 32, 32)
    d = (np.abs(b).max(axis=2) / np.float32(127.0)).astype(np.float16)
    df = d.astype(np.float32)
    inv = np.divide(1.0, df, out=np.zeros_like(df), where=df > 0)
    q = np.clip(np.rint(b * inv[..., None]), -127, 127).astype(np.int8)
    return oq.encode_q8_0(q.reshape(n, k), d)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    n, k = w.shape
    b = w.astype(np.float32).reshape(n, k // 32, 32)
    m = np.take_along_axis(b, np.abs(b).argmax(axis=2)[..., None], axis=2)[..., 0]
    d = (m / np.float32(-8.0)).astype(np.float16)
    df = d.astype(np.float32)
    inv = np.divide(1.0, df, out=np.zeros_like(df), where=df != 0)
    nib = np.clip(np.floor(b * inv[..., None] + np.float32(8.5)), 0, 15).astype(np.uint8)
    return oq.encode_q4_0(nib.reshape(n, k), d)


def write_tiny_gguf(path: str | Path, fmt: str) -> str:
    """Write the tiny model as a GGUF file with ``fmt`` ("q4_0" / "q8_0") linear weights; returns its SHA-256."""
    w = create_tiny_weights(**CFG)
    qfn, code = (quantize_q4_0, oq.GGML_TYPE_Q4_0) if fmt == "q4_0" else (quantize_q8_0, oq.GGML_TYPE_Q8_0)
    tensors = []
    for key in sorted(w):
        arr = w[key]
        dims = tuple(reversed(arr.shape))  # GGUF lists the contiguous (in) dimension first
        if key == "model.embed_tokens.weight":
            tensors.append((gguf_name(key), oq.GGML_TYPE_F16, dims, arr.astype(np.float16).tobytes()))
        elif arr.ndim == 2:
            tensors.append((gguf_name(key), code, dims, qfn(arr).tobytes()))
        else:
            tensors.append((gguf_name(key), oq.GGML_TYPE_F32, dims, arr.astype(np.float32).tobytes()))
    c = CFG
    meta = {
        "general.architecture": "llama",
        "llama.embedding_length": c["hidden_size"],
        "llama.feed_forward_length": c["intermediate_size"],
        "llama.block_count": c["num_layers"],
        "llama.attention.head_count": c["num_attention_heads"],
        "llama.attention.head_count_kv": c["num_key_value_heads"],
        "llama.vocab_size": c["vocab_size"],
        "llama.context_length": 256,
        "llama.rope.freq_base": THETA,
        "llama.attention.layer_norm_rms_epsilon": EPS,
    }
    oq.write_gguf(path, tensors, meta)
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def decoded_weights(fmt: str) -> dict[str, np.ndarray]:
    """The file's tensors as the reference's GGUFReader.read_tensor returns them (gguf.py:192-211), keyed by GGUF
    name: blocks decoded to float32 (the oracle's restatement of gguf.py:273-310), F16 widened, F32 as is."""
    w = create_tiny_weights(**CFG)
    qfn, dec = (quantize_q4_0, oq.decode_q4_0) if fmt == "q4_0" else (quantize_q8_0, oq.decode_q8_0)
    out = {}
    for key, arr in w.items():
        if key == "model.embed_tokens.weight":
            out[gguf_name(key)] = arr.astype(np.float16).astype(np.float32)
        elif arr.ndim == 2:
            out[gguf_name(key)] = dec(qfn(arr), arr.shape[1])
        else:
            out[gguf_name(key)] = arr.astype(np.float32)
    return out
