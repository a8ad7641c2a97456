"""CPU-only checks of the C-ABI library and the host-side logic (no GPU calls)."""
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import torch
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


@pytest.mark.skipif(not hip.library_path().exists(), reason="libcacheir_hip.so not built")
def test_gemm_planner_splits_and_kernels_without_a_gpu():
    """The planner's choices are host arithmetic: the large-m kernel takes k-splits that need not divide k/128
    (none empty), the m <= 32 kernel only divisors."""
    from cacheir_amd import kernels

    q8, q4, P = hip.CIR_Q8_0, hip.CIR_Q4_0, hip.GEMM_PARTIALS
    # Qwen2-7B down at m = 128: 148 quads over 9 splits (17 each, the last 12), one round of 252 workgroups
    assert kernels.choose_splits(128, 3584, 18944) == 9
    assert kernels.gemm_plan(P, q8, 128, 3584, 18944, 9) == "qgemm_xl_kernel<MT=8>"
    # its O (28 quads) stays on the small kernel, whose splits must divide k/128
    assert kernels.gemm_plan(P, q8, 128, 3584, 3584, 2).startswith("qgemm_xs_kernel")
    assert kernels.gemm_plan(P, q8, 128, 3584, 3584, 3) == "invalid"
    # QKV keeps 7 splits of 4 quads (36 column groups)
    assert kernels.choose_splits(128, 4608, 3584) == 7
    # 64 quads over 9 splits would leave the last empty; over 10 the last holds one quad
    assert kernels.gemm_plan(P, q8, 128, 100, 8192, 9) == "invalid"
    assert kernels.gemm_plan(P, q8, 128, 100, 8192, 10) == "qgemm_xl_kernel<MT=8>"
    # a 2048-token prefill fills the CUs with row blocks alone: large-m kernel, one split, for every projection
    for n, k in ((6144, 4096), (4096, 4096), (4096, 14336), (128256, 4096)):
        assert kernels.choose_splits(2048, n, k) == 1
        assert kernels.gemm_plan(P, q4, 2048, n, k, 1) == "qgemm_xl_kernel<MT=8>", (n, k)
    assert kernels.gemm_plan(hip.GEMM_SWIGLU, q4, 2048, 28672, 4096, 1) == "qgemm_xl_kernel<MT=8,EPI=swiglu>"
    # decode at m = 32 is untouched: divisor splits on the small kernel
    assert kernels.gemm_plan(P, q4, 32, 4096, 14336, 8).startswith("qgemm_xs_kernel")
    assert kernels.gemm_plan(P, q4, 32, 4096, 14336, 9) == "invalid"


@pytest.mark.skipif(not hip.library_path().exists(), reason="libcacheir_hip.so not built")
def test_default_splits_are_always_accepted():
    """Whatever k-split the library proposes for a shape, its own launch accepts (no empty last split): the
    Qwen2.5-3B down (n 2048, k 11008: 86 quads) at m = 64 once got 16 splits, which start split 15 past the end."""
    from cacheir_amd import kernels

    ns = (128, 896, 1536, 2048, 3584, 4096, 4608, 8960, 11008, 14336, 18944, 37888)
    ks = (128, 512, 896 // 128 * 128, 1536, 2048, 3584, 8960, 11008, 14336, 18944)
    bad = []
    for fmt in (hip.CIR_Q4_0, hip.CIR_Q8_0):
        for m in (1, 8, 16, 32, 33, 48, 64, 65, 96, 128, 200, 512):
            for n in ns:
                for k in ks:
                    s = kernels.choose_splits(m, n, k)
                    if kernels.gemm_plan(hip.GEMM_PARTIALS, fmt, m, n, k, s) == "invalid":
                        bad.append((fmt, m, n, k, s))
    assert not bad, bad[:10]
    assert kernels.choose_splits(64, 2048, 11008) == 15  # 15 splits of 6 quads, the last 2
    assert kernels.gemm_plan(hip.GEMM_PARTIALS, hip.CIR_Q8_0, 64, 2048, 11008, 15) != "invalid"


def _llvm_tool(name: str):
    for cand in (Path("/opt/rocm/llvm/bin") / name, shutil.which(name)):
        if cand and Path(cand).exists():
            return str(cand)
    return None


@pytest.mark.skipif(not hip.library_path().exists(), reason="libcacheir_hip.so not built")
@pytest.mark.skipif(_llvm_tool("llvm-objcopy") is None or _llvm_tool("llvm-readelf") is None,
                    reason="LLVM binutils not available")
def test_no_kernel_spills_to_scratch(tmp_path):
    """Every kernel in the built library keeps its values in registers: the gfx950 code objects' metadata gives a
    private segment of 0 bytes for every kernel (a spill to scratch turns a register access into a memory round
    trip and has cost 1.5x on a kernel here).  Reads the library's own device code: the .hip_fatbin section holds
    one clang offload bundle per source file; each bundle's gfx950 entry is an ELF code object whose notes list
    the kernels."""
    import struct

    fat = tmp_path / "fatbin.bin"
    subprocess.run([_llvm_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={fat}", str(hip.library_path()),
                    str(tmp_path / "lib_copy.so")], check=True, capture_output=True)
    data = fat.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts, i = [], data.find(magic)
    while i >= 0:
        starts.append(i)
        i = data.find(magic, i + 1)
    assert starts, "no offload bundle in .hip_fatbin"
    kernels_seen, spills = 0, []
    for b, start in enumerate(starts):
        pos = start + len(magic)
        (entries,) = struct.unpack_from("<Q", data, pos)
        pos += 8
        for _ in range(entries):
            off, size, tlen = struct.unpack_from("<QQQ", data, pos)
            pos += 24
            triple = data[pos:pos + tlen].decode()
            pos += tlen
            if "gfx950" not in triple:
                continue
            obj = tmp_path / f"co{b}.o"
            obj.write_bytes(data[start + off:start + off + size])
            notes = subprocess.run([_llvm_tool("llvm-readelf"), "--notes", str(obj)], check=True,
                                   capture_output=True, text=True).stdout
            name = None
            for line in notes.splitlines():
                line = line.strip()
                if line.startswith(".name:"):
                    name = line.split(":", 1)[1].strip()
                elif line.startswith(".private_segment_fixed_size:"):
                    kernels_seen += 1
                    if int(line.split(":", 1)[1]) != 0:
                        spills.append((name, int(line.split(":", 1)[1])))
    assert kernels_seen >= 100, f"only {kernels_seen} kernels found in the code objects"
    assert not spills, spills[:10]


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


# ------------------------------------------------------------------ KV pages (host logic, CPU tensors) --
def _alloc(pages=4):
    from cacheir_amd.kv import HipKVPageAllocator

    return HipKVPageAllocator(num_layers=2, kv_heads=1, head_dim=4, page_size=4, dtype=torch.float32, device="cpu",
                              capacity_pages=pages)


def test_kv_pages_refcount_alias_and_copy_on_write():
    from cacheir_amd.kv import HipPagedKVCache

    a = _alloc()
    src = HipPagedKVCache(a)
    src.ensure_capacity(6)  # 2 pages, the second half full
    src.tokens = 6
    for i, slot in enumerate(src.slots):
        a.k[:, slot] = float(i + 1)
        a.v[:, slot] = float(-(i + 1))
    dst = HipPagedKVCache(a)
    dst.alias_prefix(src.slots, 6)
    assert dst.slots == src.slots and dst.tokens == 6
    assert all(a.refcount(s) == 2 for s in src.slots)
    # dst appends token 6: it lands in page 1, still shared -> copied; page 0 stays aliased
    dst.ensure_capacity(7)
    assert dst.slots[0] == src.slots[0] and dst.slots[1] != src.slots[1]
    assert a.refcount(src.slots[0]) == 2 and a.refcount(src.slots[1]) == 1 and a.refcount(dst.slots[1]) == 1
    assert torch.equal(a.k[:, dst.slots[1]], a.k[:, src.slots[1]]) and a.copied_pages == 1
    a.k[:, dst.slots[1], :, 2] = 99.0  # the writer's copy changes, the source page does not
    assert float(a.k[0, src.slots[1], 0, 2, 0]) == 2.0
    # a page-aligned prefix needs no copy: new tokens go to new pages
    dst2 = HipPagedKVCache(a)
    dst2.alias_prefix(src.slots, 4)
    dst2.ensure_capacity(5)
    assert dst2.slots[0] == src.slots[0] and len(dst2.slots) == 2 and dst2.slots[1] not in src.slots
    # releasing every user frees the pages
    before = a.free_pages
    for c in (dst, dst2, src):
        c.clear()
    assert a.stats()["resident_pages"] == 0 and a.free_pages == before + 4


def test_kv_lanes_keep_a_batch_page_major():
    """Sessions of equal length hold page i side by side (stripe i), whether they allocate one after another or a
    page at a time; a dry lane borrows from the fullest one before the pool grows; released slots are reused lowest
    stripe first."""
    from cacheir_amd.kv import HipKVPageAllocator, HipPagedKVCache

    L, B, pages = 5, 4, 6
    a = HipKVPageAllocator(num_layers=1, kv_heads=1, head_dim=4, page_size=4, dtype=torch.float32, device="cpu",
                           capacity_pages=L * pages, lanes=L)
    assert a.capacity == L * pages and a.free_pages == L * pages
    one_by_one = [HipPagedKVCache(a) for _ in range(B)]
    for c in one_by_one:
        c.ensure_capacity(4 * pages)
    lanes = [c.lane for c in one_by_one]
    assert lanes == list(range(B))
    for c in one_by_one:
        assert c.slots == [i * L + c.lane for i in range(pages)]
    for c in one_by_one:
        c.clear()
    assert a.free_pages == L * pages
    # a page at a time (decode appends): the same placement
    stepped = [HipPagedKVCache(a, lane=b) for b in range(B)]
    for t in range(1, 4 * pages + 1):
        for c in stepped:
            c.ensure_capacity(t)
    for c in stepped:
        assert c.slots == [i * L + c.lane for i in range(pages)]
    # lane 4 holds 6 free slots; lanes 0-3 none: a session in lane 0 borrows lane 4's before the pool grows
    extra = HipPagedKVCache(a, lane=0)
    extra.ensure_capacity(4 * 3)
    assert extra.slots == [4, 9, 14] and a.pool_grows == 1
    extra.ensure_capacity(4 * 6)
    assert a.pool_grows == 1 and a.free_pages == 0
    extra.ensure_capacity(4 * 7)  # nothing free anywhere: the pool doubles in whole stripes
    assert a.pool_grows == 2 and a.capacity == 2 * L * pages and a.capacity % L == 0
    assert extra.slots[-1] == L * pages  # lane 0's first new stripe
    stepped[2].clear()
    again = HipPagedKVCache(a, lane=2)
    again.ensure_capacity(4 * 2)
    assert again.slots == [2, 2 + L]
    used = [s for c in stepped + [extra, again] for s in c.slots]
    assert len(used) == len(set(used)) and all(a.refcount(s) == 1 for s in used)


def test_kv_allocator_random_sequences_keep_invariants():
    """Random mixes of sessions growing, copying on write, aliasing prefixes and releasing pages, over several lane
    counts: no slot is held twice, the free count and the per-lane free heaps always account for every slot, refcounts
    equal the number of page tables (and cache holds) using a slot, and capacity stays a whole number of stripes."""
    import numpy as np

    from cacheir_amd.kv import HipKVPageAllocator, HipPagedKVCache

    for lanes, seed in ((1, 0), (3, 1), (5, 2), (33, 3)):
        rng = np.random.default_rng(seed)
        a = HipKVPageAllocator(num_layers=1, kv_heads=1, head_dim=4, page_size=4, dtype=torch.float32, device="cpu",
                               capacity_pages=7, lanes=lanes)
        caches: list[HipPagedKVCache] = []
        held: list[list[int]] = []  # extra references (a prefix cache would hold)
        for _ in range(400):
            op = rng.integers(0, 6)
            if op == 0 or not caches:
                caches.append(HipPagedKVCache(a))
            c = caches[int(rng.integers(0, len(caches)))]
            if op in (0, 1):
                c.ensure_capacity(c.tokens + int(rng.integers(1, 20)))
                c.tokens = len(c.slots) * 4 - int(rng.integers(0, 4))
            elif op == 2 and c.tokens:
                src = caches[int(rng.integers(0, len(caches)))]
                if src is not c and src.tokens:
                    n = int(rng.integers(1, src.tokens + 1))
                    c.alias_prefix(list(src.slots), n)
            elif op == 3 and c.tokens:
                a.share(list(c.slots))
                held.append(list(c.slots))
            elif op == 4 and held:
                a.release(held.pop(int(rng.integers(0, len(held)))))
            elif op == 5:
                c.clear()
            # invariants
            uses: dict[int, int] = {}
            for cc in caches:
                for sl in cc.slots:
                    uses[sl] = uses.get(sl, 0) + 1
            for h in held:
                for sl in h:
                    uses[sl] = uses.get(sl, 0) + 1
            assert all(a.refcount(sl) == n for sl, n in uses.items())
            assert a.stats()["resident_pages"] == len(uses)
            free = [sl for heap in a._lane_free for sl in heap]
            assert len(free) == len(set(free)) == a.free_pages
            assert not set(free) & set(uses)
            assert len(free) + len(uses) == a.capacity and a.capacity % lanes == 0
            for ln, heap in enumerate(a._lane_free):  # each lane's free slots: its own, in min-heap order
                assert all(sl % lanes == ln for sl in heap)
                assert all(heap[(i - 1) // 2] <= heap[i] for i in range(1, len(heap)))


def test_prefix_cache_holds_and_releases_pages():
    from cacheir_amd.kv import HipPagedKVCache
    from cacheir_amd.runtime import PrefixCache, PrefixPages

    a = _alloc()
    s = HipPagedKVCache(a)
    s.ensure_capacity(8)
    s.tokens = 8
    pc = PrefixCache(capacity=1)
    a.share(s.slots)
    pc.put(list(range(8)), PrefixPages(a, list(s.slots), 8))
    s.clear()  # the cache still holds the pages
    assert a.stats()["resident_pages"] == 2
    key, pages = pc.longest_prefix(list(range(10)))
    assert key == tuple(range(8)) and pages.tokens == 8 and pc.hits == 1
    assert pc.longest_prefix([5, 6])[1] is None and pc.misses == 1
    s2 = HipPagedKVCache(a)
    s2.ensure_capacity(4)
    s2.tokens = 4
    a.share(s2.slots)
    pc.put([1, 2, 3, 4], PrefixPages(a, list(s2.slots), 4))  # evicts the first entry (capacity 1)
    assert pc.evictions == 1 and a.stats()["resident_pages"] == 1
    pc.clear()
    s2.clear()
    assert a.stats()["resident_pages"] == 0


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("cols", [256, 257])
def test_row_packer_matches_reference_restatement(bits, cols):
    """cacheir_amd.weights.pack_rows (product) == oracle.quant.asymmetric_pack (the restatement pinned to the
    reference's own case), bit for bit, incl. an odd column count and rows of one sign."""
    from cacheir_amd.weights import pack_rows, row_bits

    rng = np.random.default_rng(bits * 1000 + cols)
    w = rng.standard_normal((24, cols)).astype(np.float32)
    w[3] = np.abs(w[3]) + 0.5     # all positive: zero point below 0
    w[5] = -np.abs(w[5]) - 0.5    # all negative: zero point above qmax
    w[7] = 0.25                   # constant row: scale floor 1e-8
    packed, scales, zps = pack_rows(w, bits)
    ref = quant.asymmetric_pack(w, bits)
    assert np.array_equal(packed, ref["packed_values"])
    assert np.array_equal(scales, ref["scales"]) and np.array_equal(zps, ref["zero_points"])
    assert row_bits("int4_awq") == 4 and row_bits("gptq") == 4 and row_bits("int8") == 8 and row_bits("q4_0") is None
