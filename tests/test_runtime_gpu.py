"""End-to-end HipRuntime parity against the NumPy oracle (GPU).

* BASELINE config 1 (tiny fp32 model): greedy ids identical to the committed
  oracle fixture; every step's logits within 1e-4 (the reference's own GPU parity
  tolerance, tests/test_runtime.py:62).
* Batched decode over ragged sessions equals sequential decode (the invariant of
  tests/test_scheduler.py:146-183).
* A Q4_0 model (MFMA GEMM + MFMA attention, fp16 activations): logits within the
  fp16 bound |d| <= 2e-3 + 1e-2|ref| of the oracle run on the decoded blocks, and the
  same model loaded from a GGUF file gives bit-identical logits.
* A captured HIP graph replays the eager step exactly, several times, with eager
  work in between.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from cacheir_amd.artifact import ModelConfig
from cacheir_amd.compiler import compile_config
from oracle import quant as oq
from oracle.runtime import OracleRuntime, create_tiny_weights, generate_ids

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).with_name("golden")


def tiny_config(**kw) -> ModelConfig:
    base = dict(architecture="CacheIRTinyForCausalLM", hidden_size=256, intermediate_size=688, num_layers=2,
                num_attention_heads=4, num_key_value_heads=2, vocab_size=1024, max_position_embeddings=256,
                rope_theta=10000.0, rms_norm_eps=1e-5, dtype="float32")
    base.update(kw)
    return ModelConfig(**base)


def write_model(path: Path, cfg: ModelConfig, weights: dict) -> Path:
    path.mkdir(parents=True, exist_ok=True)
    np.savez(path / "weights.npz", **weights)
    (path / "config.json").write_text(json.dumps({"hidden_size": cfg.hidden_size}))
    return path


def close16(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = np.abs(got - ref) - (2e-3 + 1e-2 * np.abs(ref))
    assert np.all(err <= 0), f"max violation {err.max():.3e}"


@pytest.fixture(scope="module")
def tiny(tmp_path_factory, device):
    fx = json.loads((GOLDEN / "tiny_greedy.json").read_text())
    w = create_tiny_weights(**fx["config"])
    cfg = tiny_config()
    path = write_model(tmp_path_factory.mktemp("tiny"), cfg, w)
    art = compile_config(cfg, model_path=str(path))
    return fx, w, cfg, art


def test_tiny_model_greedy_identical_fp32(tiny):
    from cacheir_amd.runtime import HipRuntime

    fx, w, cfg, art = tiny
    rt = HipRuntime(art, dtype="float32")
    orc = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, w, cfg.vocab_size)
    prompt = fx["prompt_ids"]
    logits = rt.run([prompt], mode="prefill")
    ref = orc.run([prompt], mode="prefill")
    np.testing.assert_allclose(logits.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    ids = []
    for _ in range(32):
        nxt = int(torch.argmax(logits[0, -1]).item())
        ids.append(nxt)
        logits = rt.run([[nxt]], mode="decode")
        ref = orc.run([[nxt]], mode="decode")
        np.testing.assert_allclose(logits.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    assert ids == fx["greedy_ids"]
    # the same ids the reference's own NumPy backend produced (make_reference_tiny.py)
    ref_fx = json.loads((GOLDEN / "reference_tiny.json").read_text())
    assert ref_fx["prompt"] == prompt and ids == ref_fx["greedy_ids"]
    assert rt.kv_cache.tokens == 16 + 32
    stats = rt.cache_stats()
    assert stats["kernel_counts"]


def test_tiny_model_fp16_agreement(tiny):
    """fp16 weights, activations and KV: the prefill logits within the fp16 bound of the fp32 oracle, then
    teacher-forced on the reference NumPy backend's 32 greedy ids (tests/golden/reference_tiny.json): the argmax
    equals the reference's id at every step whose reference top-2 margin exceeds 0.01 (29 of the 32; fp16 storage
    alone moves this model's logits by at most 1.25e-3, measured with the oracle's fp16-storage variant)."""
    from cacheir_amd.runtime import HipRuntime

    fx, w, cfg, art = tiny
    ref = json.loads((GOLDEN / "reference_tiny.json").read_text())
    assert ref["prompt"] == fx["prompt_ids"]
    rt = HipRuntime(art, dtype="float16")
    orc = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, w, cfg.vocab_size)
    logits = rt.run([ref["prompt"]], mode="prefill")
    close16(logits.cpu().numpy(), orc.run([ref["prompt"]], mode="prefill"))
    checked = agree = 0
    for step, (want, margin) in enumerate(zip(ref["greedy_ids"], ref["top2_margins"])):
        got = int(torch.argmax(logits[0, -1]).item())
        agree += got == want
        if margin > 0.01:
            assert got == want, f"step {step}: {got} != {want} (reference margin {margin:.4f})"
            checked += 1
        logits = rt.run([[want]], mode="decode")
    print(f"fp16 teacher-forced agreement {agree}/32, {checked} steps asserted")
    assert checked == 29


def test_batched_decode_equals_sequential(tiny):
    from cacheir_amd.runtime import HipRuntime

    fx, w, cfg, art = tiny
    base = HipRuntime(art, dtype="float32")
    prompts = [[1, 2, 3], list(range(40, 60)), [7] * 17, list(range(100, 133))]
    batch = [base.fork() for _ in prompts]
    seq = [base.fork() for _ in prompts]
    first = []
    for s, p in zip(batch, prompts):
        first.append(int(torch.argmax(s.run([p], mode="prefill")[0, -1])))
    for s, p in zip(seq, prompts):
        s.run([p], mode="prefill")
    toks = list(first)
    for _ in range(5):
        blog = base.run_decode_batch(batch, toks).cpu().numpy()
        slog = np.concatenate([s.run([[t]], mode="decode").cpu().numpy() for s, t in zip(seq, toks)], axis=0)
        np.testing.assert_allclose(blog, slog, rtol=1e-5, atol=1e-5)
        toks = [int(np.argmax(r[-1])) for r in blog]
    # pages of forked sessions are disjoint slots in one shared pool
    slots = [set(s.kv_cache.slots) for s in batch + seq]
    assert sum(len(x) for x in slots) == len(set().union(*slots))


def test_batch_validation_errors(tiny):
    from cacheir_amd.runtime import HipRuntime

    _, _, _, art = tiny
    rt = HipRuntime(art, dtype="float32")
    with pytest.raises(ValueError):
        rt.run_decode_batch([], [])
    with pytest.raises(ValueError):
        rt.run_decode_batch([rt], [1, 2])
    with pytest.raises(TypeError):
        rt.run_decode_batch([object()], [1])
    other = HipRuntime(art, dtype="float32")  # separate allocator
    with pytest.raises(ValueError):
        rt.run_decode_batch([rt, other], [1, 1])
    # token ids outside the vocabulary raise IndexError on the host, as the reference's table lookup does, and
    # leave the session untouched (the device embedding would otherwise clamp them)
    vocab = art.config.vocab_size
    rt.run([1, 2, 3], mode="prefill")
    held = rt.kv_cache.tokens
    for bad in (vocab, -1):
        with pytest.raises(IndexError):
            rt.run([[bad]], mode="decode")
        with pytest.raises(IndexError):
            rt.run_decode_batch([rt], [bad])
        with pytest.raises(IndexError):
            rt.decode_greedy([rt], [bad])
    with pytest.raises(IndexError):
        rt.run([5, vocab + 7, 6], mode="prefill", reset_kv=False)
    assert rt.kv_cache.tokens == held
    rt.run([[vocab - 1]], mode="decode")  # the largest id is fine
    assert rt.kv_cache.tokens == held + 1


def _q4_model(tmp: Path, fmt: str):
    """A small Q4_0/Q8_0 model whose shapes hit the MFMA paths (head_dim 128, k % 128 == 0)."""
    from cacheir_amd.weights import quantize_q4_0, quantize_q8_0

    cfg = tiny_config(hidden_size=256, intermediate_size=512, num_attention_heads=2, num_key_value_heads=1,
                      vocab_size=512, dtype="float16")
    w = create_tiny_weights(seed=3, vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2,
                            num_attention_heads=2, num_key_value_heads=1)
    qfn = quantize_q4_0 if fmt == "q4_0" else quantize_q8_0
    dec = oq.decode_q4_0 if fmt == "q4_0" else oq.decode_q8_0
    blocks, decoded = {}, dict(w)
    for k, v in w.items():
        if v.ndim == 2 and "embed" not in k:
            blocks[k] = qfn(v)
            decoded[k] = dec(blocks[k], v.shape[1])
    # norms/embeddings are fp16 in the device copy; give the oracle the same values
    for k, v in w.items():
        if k not in blocks:
            decoded[k] = v.astype(np.float16).astype(np.float32)
    return cfg, w, blocks, decoded


@pytest.mark.parametrize("fmt", ["q4_0", "q8_0"])
def test_block_quant_model_matches_oracle_and_gguf(tmp_path, device, fmt):
    from cacheir_amd.runtime import HipRuntime, gguf_key_map

    cfg, w, blocks, decoded = _q4_model(tmp_path, fmt)
    path = write_model(tmp_path / "m", cfg, w)
    art = compile_config(cfg, quant=fmt, model_path=str(path))
    rt = HipRuntime(art)
    assert rt.dtype == torch.float16
    orc = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, decoded, cfg.vocab_size)
    prompt = list(range(5, 25))
    got = rt.run([prompt], mode="prefill").cpu().numpy()
    close16(got, orc.run([prompt], mode="prefill"))
    tok = int(np.argmax(got[0, -1]))
    for _ in range(4):
        g = rt.run([[tok]], mode="decode").cpu().numpy()
        close16(g, orc.run([[tok]], mode="decode"))
        tok = int(np.argmax(g[0, -1]))

    # The same blocks in a GGUF file load packed and give identical logits.
    km = gguf_key_map(cfg.num_layers)
    t_code = oq.GGML_TYPE_Q4_0 if fmt == "q4_0" else oq.GGML_TYPE_Q8_0
    tensors = []
    for key, arr in w.items():
        if key in blocks:
            tensors.append((km[key], t_code, tuple(reversed(arr.shape)), blocks[key].tobytes()))
        else:
            tensors.append((km[key], oq.GGML_TYPE_F32, tuple(reversed(arr.shape)), arr.astype(np.float32).tobytes()))
    gguf = tmp_path / "m.gguf"
    oq.write_gguf(gguf, tensors, {"general.architecture": "llama"})
    art2 = compile_config(cfg, quant=None, model_path=str(gguf))
    rt2 = HipRuntime(art2)
    got2 = rt2.run([prompt], mode="prefill").cpu().numpy()
    assert np.array_equal(got2, got)


@pytest.mark.parametrize("use_graphs", [False, True])
def test_prefill_hands_its_logits_buffer_to_the_caller(tmp_path, device, use_graphs):
    """A prefill whose LM head runs as one k-split writes the logits straight from the GEMM and returns the plan's
    buffer itself (no store epilogue, no copy); the plan writes its next call into a fresh buffer, so an earlier
    result is never overwritten, and the same prompt again gives the same bits.  Decode at batch 1 (two k-splits)
    and captured decode plans copy their logits out, so those results stay the caller's too."""
    from cacheir_amd import kernels
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    art = compile_config(cfg, quant="q4_0", model_path=str(write_model(tmp_path / "m", cfg, w)))
    rt = HipRuntime(art, use_graphs=use_graphs)
    orc = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, decoded, cfg.vocab_size)
    p1, p2 = list(range(5, 25)), list(range(30, 50))  # 20 tokens each: one plan
    assert kernels.choose_splits(len(p1), cfg.vocab_size, cfg.hidden_size) == 1
    a = rt.run([p1], mode="prefill")
    a_host = a.cpu().numpy().copy()
    close16(a_host, orc.run([p1], mode="prefill"))
    plan = rt._plans[("prefill", 1, len(p1), rt._bucket(len(rt.kv_cache.slots)))]
    assert plan._logits_swappable
    fresh = plan.logits.data_ptr()
    b = rt.run([p2], mode="prefill")
    assert b.data_ptr() == fresh != a.data_ptr()
    assert np.array_equal(a.cpu().numpy(), a_host)
    close16(b.cpu().numpy(), orc.run([p2], mode="prefill"))
    c = rt.run([p1], mode="prefill")
    assert np.array_equal(c.cpu().numpy(), a_host)
    orc.run([p1], mode="prefill")  # the oracle's cache now holds p1, as the runtime's does
    d1 = rt.run([[7]], mode="decode")
    d1_host = d1.cpu().numpy().copy()
    close16(d1_host, orc.run([[7]], mode="decode"))
    d2 = rt.run([[8]], mode="decode")
    assert d2.data_ptr() != d1.data_ptr()
    assert np.array_equal(d1.cpu().numpy(), d1_host)
    close16(d2.cpu().numpy(), orc.run([[8]], mode="decode"))


def test_graph_capture_replays_eager(tmp_path, device):
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    art = compile_config(cfg, quant="q4_0", model_path=str(write_model(tmp_path / "g", cfg, w)))
    base = HipRuntime(art)
    sessions = [base.fork() for _ in range(3)]
    for i, s in enumerate(sessions):
        s.run([list(range(3 + i, 20 + 3 * i))], mode="prefill")
    eager = base.run_decode_batch(sessions, [4, 5, 6]).cpu().numpy()
    # roll the sessions back one token and replay the same step through a captured graph
    for s in sessions:
        s.kv_cache.tokens -= 1
    plan = base.plan("decode", 3, 1, base._bucket(max(len(s.kv_cache.slots) for s in sessions)))
    rows = np.zeros((3, plan.max_pages), np.int32)
    for b, s in enumerate(sessions):
        rows[b, : len(s.kv_cache.slots)] = s.kv_cache.slots
    plan.set_inputs(np.array([[4], [5], [6]]), rows, np.array([s.kv_cache.tokens for s in sessions]))
    plan.capture(with_argmax=True)
    for _ in range(3):
        plan.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(plan.logits.view(3, 1, -1).cpu().numpy(), eager)
        assert plan.next_ids.cpu().tolist() == [int(np.argmax(r[-1])) for r in eager]
        _ = torch.ones(1024, device=device).sum().item()  # eager work between replays


def test_prefix_cache_aliases_pages_with_copy_on_write(tmp_path, device):
    """prefill_tokens(use_prefix_cache=True) reuses a cached prefix by aliasing its pages: the reusing session
    matches a session that prefilled everything, and the prefix owner is untouched by the reuser's writes
    (its partially filled last prefix page is copied before the reuser appends)."""
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    path = write_model(tmp_path / "m", cfg, w)
    art = compile_config(cfg, quant="q4_0", model_path=str(path))
    owner = HipRuntime(art)
    prefix = list(range(3, 23))          # 20 tokens: one full page + 4 tokens of the second
    suffix = [40, 41, 42, 43, 44, 45, 46]
    owner.prefill_tokens(prefix, remember_prefix=True)
    reuser, full, fresh = owner.fork(), owner.fork(), owner.fork()
    logits_r, reused = reuser.prefill_tokens(prefix + suffix, use_prefix_cache=True)
    assert reused == tuple(prefix) and logits_r.shape[1] == len(suffix)
    assert reuser.kv_cache.slots[0] == owner.kv_cache.slots[0]          # full page aliased
    assert reuser.kv_cache.slots[1] != owner.kv_cache.slots[1]          # partial page copied on write
    logits_f, _ = full.prefill_tokens(prefix + suffix)
    close16(logits_r.cpu().numpy(), logits_f[:, len(prefix):].cpu().numpy())
    tr, tf = int(torch.argmax(logits_r[0, -1])), int(torch.argmax(logits_f[0, -1]))
    for _ in range(3):
        lr, lf = reuser.run([[tr]], mode="decode"), full.run([[tf]], mode="decode")
        close16(lr.cpu().numpy(), lf.cpu().numpy())
        tr, tf = int(torch.argmax(lr[0, -1])), int(torch.argmax(lf[0, -1]))
    # the owner continues exactly like a session that never shared its pages
    fresh.prefill_tokens(prefix)
    for tok in (7, 8):
        assert torch.equal(owner.run([[tok]], mode="decode"), fresh.run([[tok]], mode="decode"))
    st = owner.kv_allocator.stats()
    assert st["shared_pages"] >= 1 and st["copied_pages"] >= 1


def test_ragged_prefill_batch_is_one_padded_pass(tiny):
    """run_prefill_batch over prompts of different lengths runs one padded pass (cuda.py:584-629): each row's
    logits at its own positions match a prefill of that prompt alone, padding positions are zero, every session
    holds exactly its prompt, and decoding on from the batch equals decoding on from the separate prefills (the
    padding's K/V writes reached no page a session reads)."""
    from cacheir_amd.runtime import HipRuntime

    fx, w, cfg, art = tiny
    base = HipRuntime(art, dtype="float32")
    prompts = [[5, 6, 7], list(range(40, 77)), [9] * 16, list(range(100, 117))]  # 3, 37, 16, 17 tokens
    batch = [base.fork() for _ in prompts]
    alone = [base.fork() for _ in prompts]
    out = base.run_prefill_batch(batch, prompts).cpu().numpy()
    L = max(len(p) for p in prompts)
    assert out.shape == (len(prompts), L, cfg.vocab_size)
    assert base.kernel_counts.get("rocm.prefill_padded_batch") == 1
    for b, (s, p) in enumerate(zip(alone, prompts)):
        ref = s.run([p], mode="prefill").cpu().numpy()[0]
        np.testing.assert_allclose(out[b, : len(p)], ref, rtol=1e-4, atol=1e-4)
        assert np.all(out[b, len(p):] == 0)
        assert batch[b].kv_cache.tokens == len(p) and len(batch[b].kv_cache.slots) == -(-len(p) // 16)
    toks = [int(np.argmax(out[b, len(p) - 1])) for b, p in enumerate(prompts)]
    for _ in range(3):
        got = base.run_decode_batch(batch, toks).cpu().numpy()
        ref = base.run_decode_batch(alone, toks).cpu().numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
        toks = [int(np.argmax(r[-1])) for r in got]
    # the padding page went back to the pool: only the sessions' own pages are resident
    held = sum(len(s.kv_cache.slots) for s in batch + alone) + len(base.kv_cache.slots)
    assert base.kv_allocator.stats()["resident_pages"] == held


def test_load_longest_prefix_and_plan_eviction(tmp_path, device):
    """load_longest_prefix (cuda.py:677-681) makes the longest cached prefix the session's KV (aliased pages); a
    session continuing from it equals one that prefilled the prefix itself.  The step-plan cache keeps at most
    max_plans plans (least recently used evicted), and an evicted shape still runs correctly when it returns."""
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    art = compile_config(cfg, quant="q4_0", model_path=str(write_model(tmp_path / "m", cfg, w)))
    owner = HipRuntime(art, max_plans=3)
    prefix = list(range(3, 35))  # 32 tokens: two full pages
    owner.prefill_tokens(prefix, remember_prefix=True)
    user, full = owner.fork(), owner.fork()
    assert user.load_longest_prefix(prefix + [50, 51]) == tuple(prefix)
    assert user.kv_cache.tokens == len(prefix) and user.kv_cache.slots == owner.kv_cache.slots[:2]
    assert user.load_longest_prefix([999]) == () and user.kv_cache.tokens == len(prefix)
    full.prefill_tokens(prefix)
    for tok in (50, 51, 52):
        assert torch.equal(user.run([[tok]], mode="decode"), full.run([[tok]], mode="decode"))
    # plans: decode at batch 1 (already cached), then batches 2, 3, 4 -> the oldest shapes are evicted
    sessions = [owner.fork() for _ in range(4)]
    for s in sessions:
        s.prefill_tokens(prefix)
    first = owner.run_decode_batch(sessions[:2], [60, 61]).cpu().numpy()
    for n in (3, 4, 1):
        owner.run_decode_batch(sessions[:n], [62] * n)
    st = owner.cache_stats()["step_plans"]
    assert st["cached"] <= 3 and st["evictions"] >= 1
    for s in sessions[:2]:  # the batch-2 plan was evicted; rebuild it over the same inputs (the same positions)
        s.kv_cache.tokens = len(prefix)
    again = owner.run_decode_batch(sessions[:2], [60, 61]).cpu().numpy()
    assert np.array_equal(first, again)


@pytest.mark.parametrize("quant_name", ["int4_awq", "int8"])
def test_reference_row_packed_model_matches_oracle(tmp_path, device, quant_name):
    """An artifact compiled with the reference's own --quant int4_awq / int8 (per-row asymmetric packing,
    quantization.py:96-139) runs on the MFMA GEMM: logits match the oracle on the dequantized weights."""
    from cacheir_amd.runtime import HipRuntime

    cfg = tiny_config(hidden_size=256, intermediate_size=512, num_attention_heads=2, num_key_value_heads=1,
                      vocab_size=512, dtype="float16")
    w = create_tiny_weights(seed=5, vocab_size=512, hidden_size=256, intermediate_size=512, num_layers=2,
                            num_attention_heads=2, num_key_value_heads=1)
    bits = 4 if "4" in quant_name else 8
    decoded = {}
    for k, v in w.items():
        if v.ndim == 2:  # every 2-D weight, the embedding table too (cacheir/runtime/cpu.py:28-37)
            decoded[k] = oq.asymmetric_dequant(oq.asymmetric_pack(v, bits))
            if "embed" in k:  # held as fp16 on the device, like every dense weight of an fp16 runtime
                decoded[k] = decoded[k].astype(np.float16).astype(np.float32)
        else:
            decoded[k] = v.astype(np.float16).astype(np.float32)
    path = write_model(tmp_path / "m", cfg, w)
    art = compile_config(cfg, quant=quant_name, model_path=str(path))
    rt = HipRuntime(art)
    assert rt.dtype == torch.float16
    orc = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, decoded, cfg.vocab_size)
    prompt = list(range(7, 26))
    got = rt.run([prompt], mode="prefill").cpu().numpy()
    close16(got, orc.run([prompt], mode="prefill"))
    tok = int(np.argmax(got[0, -1]))
    for _ in range(3):
        g = rt.run([[tok]], mode="decode").cpu().numpy()
        close16(g, orc.run([[tok]], mode="decode"))
        tok = int(np.argmax(g[0, -1]))
    assert rt.kernel_counts.get("rocm.qgemm_swiglu", 0) > 0


def test_greedy_step_fuses_head_and_argmax(tmp_path, device):
    """decode_greedy (LM head fused with the argmax, no logits written) returns the greedy ids of
    run_decode_batch's logits, and a captured greedy graph replays them; generate_ids (which decodes through
    decode_greedy) matches the reference tiny-model ids computed from logits."""
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    art = compile_config(cfg, quant="q4_0", model_path=str(write_model(tmp_path / "g", cfg, w)))
    base = HipRuntime(art)
    sessions = [base.fork() for _ in range(3)]
    for i, s in enumerate(sessions):
        s.run([list(range(3 + i, 20 + 3 * i))], mode="prefill")
    logits = base.run_decode_batch(sessions, [4, 5, 6]).cpu().numpy()
    want = [int(np.argmax(r[-1])) % cfg.vocab_size for r in logits]
    for s in sessions:
        s.kv_cache.tokens -= 1
    assert base.decode_greedy(sessions, [4, 5, 6]) == want
    for s in sessions:
        s.kv_cache.tokens -= 1
    plan = base.plan("decode", 3, 1, base._bucket(max(len(s.kv_cache.slots) for s in sessions)))
    assert plan._head is not None
    rows = np.zeros((3, plan.max_pages), np.int32)
    for b, s in enumerate(sessions):
        rows[b, : len(s.kv_cache.slots)] = s.kv_cache.slots
    plan.set_inputs(np.array([[4], [5], [6]]), rows, np.array([s.kv_cache.tokens for s in sessions]))
    plan.capture(greedy=True)
    for _ in range(3):
        plan.next_ids.zero_()
        plan.replay()
        torch.cuda.synchronize()
        assert plan.next_ids.cpu().tolist() == want
        _ = torch.ones(1024, device=device).sum().item()  # eager work between replays
    # generate_ids: first id from the prefill logits, the rest through decode_greedy
    prompt = list(range(5, 21))
    fresh = HipRuntime(art)
    got = fresh.generate_ids(prompt, max_new_tokens=6)
    ref_rt = HipRuntime(art)
    lg = ref_rt.run([prompt], mode="prefill", reset_kv=True)
    ref = []
    for _ in range(6):
        nxt = int(torch.argmax(lg[0, -1]).item()) % cfg.vocab_size
        ref.append(nxt)
        lg = ref_rt.run([[nxt]], mode="decode")
    assert got == ref


def test_decode_steps_replay_a_graph_equal_to_eager_launches(tmp_path, device):
    """run_decode_batch and decode_greedy replay one captured HIP graph per (batch, page-table width): 8
    consecutive steps over sessions whose positions cross page boundaries (and the page-table bucket 4 -> 8)
    give logits and ids bitwise equal to the same steps launched kernel by kernel."""
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    art = compile_config(cfg, quant="q4_0", model_path=str(write_model(tmp_path / "m", cfg, w)))
    prompts = [list(range(3, 15)), list(range(20, 82)), [9] * 5]  # 12, 62, 5 tokens: pages 16, 64 are crossed
    runs = {}
    for use_graphs in (False, True):
        base = HipRuntime(art, use_graphs=use_graphs)
        sessions = [base.fork() for _ in prompts]
        toks = [int(torch.argmax(s.run([p], mode="prefill")[0, -1])) for s, p in zip(sessions, prompts)]
        logits, greedy = [], []
        for step in range(8):
            lg = base.run_decode_batch(sessions, toks)
            logits.append(lg.cpu())
            toks = [int(v) for v in lg[:, 0].argmax(dim=1).cpu()]
            if step % 3 == 2:  # a greedy step in between: ids only
                toks = base.decode_greedy(sessions, toks)
                greedy.append(list(toks))
        runs[use_graphs] = (logits, greedy, base.cache_stats())
    (le, ge, se), (lg_, gg, sg) = runs[False], runs[True]
    for a, b in zip(le, lg_):
        assert torch.equal(a, b)
    assert ge == gg
    assert "rocm.graph_capture" not in se["kernel_counts"] and not se["step_graphs"]
    assert sg["kernel_counts"]["rocm.graph_capture"] >= 3  # logits + greedy at page width 4, logits at 8
    assert sum(e["replays"] for e in sg["step_graphs"].values()) >= 5


def test_run_takes_a_batch_of_rows(tmp_path, device):
    """run([B, S]) (cuda.py:508-539): B sequences of one session, each on pages of its own; prefill then decode
    [B, 1] against the oracle, which runs the same [B, S] batch (cpu.py:111-140)."""
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q8_0")
    art = compile_config(cfg, quant="q8_0", model_path=str(write_model(tmp_path / "m", cfg, w)))
    rt = HipRuntime(art)
    orc = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, decoded, cfg.vocab_size)
    ids = [list(range(5, 23)), list(range(40, 58)), [7] * 18]
    got = rt.run(ids, mode="prefill").cpu().numpy()
    assert got.shape == (3, 18, cfg.vocab_size)
    close16(got, orc.run(ids, mode="prefill"))
    for _ in range(3):
        nxt = [[int(np.argmax(r[-1]))] for r in got]
        got = rt.run(nxt, mode="decode").cpu().numpy()
        close16(got, orc.run(nxt, mode="decode"))
    assert rt.kv_cache.tokens == 21 and all(c.tokens == 21 for c in rt._extra_rows)
    with pytest.raises(ValueError):
        rt.run([[1], [2]], mode="decode")  # the session holds 3 rows
    # a new prefill with reset_kv may change the row count
    one = rt.run([list(range(5, 23))], mode="prefill").cpu().numpy()
    np.testing.assert_array_equal(one[0], rt.fork().run([list(range(5, 23))], mode="prefill").cpu().numpy()[0])


@pytest.mark.parametrize("batch", [1, 4])
def test_long_context_decode_merges_attention_in_the_o_projection(tmp_path, device, batch):
    """At batch <= 8 with contexts past 256 tokens the decode attention splits its context and the O projection
    merges the split partials while staging its input (cir_paged_decode_attention_qkv_parts + cir_qgemm_attn):
    logits of that path against the oracle, over 300+ token prompts."""
    from cacheir_amd.runtime import HipRuntime

    cfg, w, blocks, decoded = _q4_model(tmp_path, "q4_0")
    art = compile_config(cfg, quant="q4_0", model_path=str(write_model(tmp_path / "m", cfg, w)))
    base = HipRuntime(art, kv_capacity_pages=256)
    rng = np.random.default_rng(batch)
    prompts = [rng.integers(0, cfg.vocab_size, 300 + 37 * b).tolist() for b in range(batch)]
    sessions = [base.fork() for _ in range(batch)]
    oracles = []
    toks = []
    for s, p in zip(sessions, prompts):
        lg = s.run([p], mode="prefill")
        o = OracleRuntime({m: g.to_dict() for m, g in art.graphs.items()}, decoded, cfg.vocab_size)
        close16(lg.cpu().numpy()[:, -1], o.run([p], mode="prefill")[:, -1])
        oracles.append(o)
        toks.append(int(torch.argmax(lg[0, -1])))
    for _ in range(3):
        got = base.run_decode_batch(sessions, toks).cpu().numpy()
        ref = np.concatenate([o.run([[t]], mode="decode") for o, t in zip(oracles, toks)], axis=0)
        close16(got, ref)
        toks = [int(np.argmax(r[-1])) for r in got]
    counts = base.cache_stats()["kernel_counts"]
    assert counts.get("rocm.attn_merge_qgemv", 0) > 0
    assert counts.get("rocm.rope_kv_append_paged_attention_decode_parts", 0) > 0
    plans = base.cache_stats()["gemm_plans"]
    assert any(k.startswith("attn_merge:") for k in plans), plans
