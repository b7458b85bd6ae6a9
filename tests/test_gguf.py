"""The GGUF writer and reader (freemoe_amd/gguf.py), CPU only.

Round trips through this package's own reader, and, where oracle/_ref is
built, conformance with the reference's parser and adapters: the native
freemoe-tiny-v1 layout and the llama-family Mixtral layout at the benchmark
shapes (hidden 4096 / ffn 14336 / 8 experts Q4_0 and Q8_0; hidden 2048 / ffn
768 / 128 experts top-8 Q4_K; Q4_K gate/up with Q8_0 down), written sparse so
that full-size files cost no disk. The reference's manifest must accept each
file and place every expert's three projections exactly where this package's
reader takes them from.
"""
import tempfile
from pathlib import Path

import numpy as np
import pytest

import fmoracle as fo
from freemoe_amd import gguf
from freemoe_amd import workloads as wl
from golden import engine_models as em

needs_ref = pytest.mark.skipif(not fo.ref_available(), reason="oracle/_ref not built (needs the FreeMoe tree)")


def test_fnv1a64_known_values():
    # the published FNV-1a 64 test vectors
    assert gguf.fnv1a64(b"") == 0xCBF29CE484222325
    assert gguf.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert gguf.fnv1a64(b"foobar") == 0x85944171F73967E8


def test_metadata_and_tensors_round_trip(tmp_path):
    g = gguf.GGUFFile(alignment=64)
    g.add("a.u8", gguf.UINT8, 7)
    g.add("a.i32", gguf.INT32, -5)
    g.add("a.f32", gguf.FLOAT32, 1.5)
    g.add("a.f64", gguf.FLOAT64, -2.25)
    g.add("a.bool", gguf.BOOL, True)
    g.add("a.str", gguf.STRING, "héllo")
    g.add("a.u64s", gguf.ARRAY, (gguf.UINT64, [1, 2 ** 63, 3]))
    g.add("a.strs", gguf.ARRAY, (gguf.STRING, ["x", "", "yz"]))
    q = wl.matrix(wl.Q4_K, np.random.default_rng(1), 3, 512)
    f = np.arange(10, dtype=np.float32)
    g.add_tensor("t.q4k", [512, 3], gguf.Q4_K, q)
    g.add_tensor("t.f32", [10], gguf.F32, f)
    size = g.write(tmp_path / "x.gguf")
    assert size == (tmp_path / "x.gguf").stat().st_size
    r = gguf.read(tmp_path / "x.gguf")
    md = r.metadata
    assert md["a.u8"] == (gguf.UINT8, 7) and md["a.i32"] == (gguf.INT32, -5)
    assert md["a.f32"] == (gguf.FLOAT32, 1.5) and md["a.f64"] == (gguf.FLOAT64, -2.25)
    assert md["a.bool"] == (gguf.BOOL, True) and md["a.str"] == (gguf.STRING, "héllo")
    assert md["a.u64s"] == (gguf.ARRAY, (gguf.UINT64, [1, 2 ** 63, 3]))
    assert md["a.strs"] == (gguf.ARRAY, (gguf.STRING, ["x", "", "yz"]))
    assert r.tensors["t.q4k"].offset % 64 == 0 and r.tensors["t.f32"].offset % 64 == 0
    assert np.array_equal(r.tensor_bytes("t.q4k"), q.ravel())
    assert np.array_equal(r.tensor_bytes("t.f32").view(np.float32), f)


def test_tensor_size_checks():
    g = gguf.GGUFFile()
    with pytest.raises(ValueError):
        g.add_tensor("bad", [100, 2], gguf.Q4_0, b"\0" * 72)  # 100 is not whole 32-element blocks
    with pytest.raises(ValueError):
        g.add_tensor("short", [32, 2], gguf.Q8_0, b"\0" * 67)


def test_native_layer_loads_back_unchanged(tmp_path):
    """moe_layer() on a written native checkpoint gives back the layer's bytes."""
    m = em.build("q4_k_router_q8_0_top4")
    em.write(m, tmp_path / "m.gguf")
    r = gguf.read(tmp_path / "m.gguf")
    for li, lw in enumerate(m.layers):
        got = gguf.moe_layer(r, li)
        assert (got.hidden, got.ffn, got.experts, got.top_k) == (lw.hidden, lw.ffn, lw.experts, lw.top_k)
        assert (got.gate_type, got.down_type, got.router_type) == (lw.gate_type, lw.down_type, lw.router_type)
        assert got.weights_norm and got.rms_eps == lw.rms_eps
        assert np.array_equal(got.norm_weight, lw.norm_weight)
        assert np.array_equal(got.router_bytes, lw.router_bytes)
        for a, b in ((got.gate, lw.gate), (got.up, lw.up), (got.down, lw.down)):
            assert all(np.array_equal(x, y) for x, y in zip(a, b))


SHAPES = {
    # name: (hidden, ffn, experts, top_k, gate/up type, down type, per-expert slot bytes)
    "mixtral_q4_0": (4096, 14336, 8, 2, gguf.Q4_0, gguf.Q4_0, 99_090_432),
    "mixtral_q8_0": (4096, 14336, 8, 2, gguf.Q8_0, gguf.Q8_0, 187_170_816),
    "finegrained_q4_k": (2048, 768, 128, 8, gguf.Q4_K, gguf.Q4_K, 2_654_208),
    "mixed_q4_k_q8_0": (2048, 768, 16, 2, gguf.Q4_K, gguf.Q8_0, 2 * 768 * 8 * 144 + 2048 * 24 * 34),
}


@needs_ref
@pytest.mark.parametrize("name", list(SHAPES))
def test_mixtral_llama_layout_accepted_by_reference_adapter(tmp_path, name):
    H, F, E, K, gt, dt, slot = SHAPES[name]
    layers = 2
    g = gguf.mixtral_llama(hidden=H, ffn=F, layers=layers, heads=32, kv_heads=8, experts=E, top_k=K,
                           vocab=32000, expert_type=gt, down_type=dt)
    path = tmp_path / f"{name}.gguf"
    g.write(path, sparse=True)
    m = fo.ref_manifest(path)
    assert (m["layers"], m["experts"], m["top_k"], m["hidden"]) == (layers, E, K, H)
    assert m["records"] == layers * E and m["slot_bytes"] == slot
    r = gguf.read(path)
    for i, (l, e) in enumerate(m["who"]):
        sl = r.expert_slices(int(l), int(e))
        for j, key in enumerate(("gate", "up", "down")):
            arr, t = sl[key]
            off = arr.ctypes.data - r.data.ctypes.data
            assert (off, arr.nbytes, t) == tuple(int(v) for v in m["extents"][i, j]), (l, e, key)
    # the loader reads the router and the routing options the way the adapter does
    lw = gguf.moe_layer(r, 1)
    assert (lw.hidden, lw.ffn, lw.experts, lw.top_k, lw.weights_norm) == (H, F, E, K, True)
    assert (lw.gate_type, lw.down_type) == (gt, dt)


@needs_ref
def test_native_layout_at_mixtral_shape_accepted_by_reference_adapter(tmp_path):
    """The freemoe-tiny-v1 layout at hidden 4096 / ffn 14336 / 8 experts Q4_0
    (checksums as placeholders: the manifest does not read expert bytes)."""
    H, F, E, K = 4096, 14336, 8, 2
    g = gguf.native_sparse(hidden=H, ffn=F, heads=32, experts=E, top_k=K, layers=1, expert_type=gguf.Q4_0)
    path = tmp_path / "native.gguf"
    g.write(path, sparse=True)
    m = fo.ref_manifest(path)
    assert (m["experts"], m["top_k"], m["hidden"], m["records"]) == (E, K, H, E)
    assert m["slot_bytes"] == 99_090_432


REF_FIXTURES = ["moe-fm", "quant-moe-q4_0", "quant-moe-q8_0", "quant-moe-q4_k", "quant-moe-q6_k",
                "quant-expert-fused", "quant-expert-separate"]
FIXTURE_DIR = Path(__file__).resolve().parent / "golden" / "freemoe_reference"


@pytest.mark.parametrize("name", REF_FIXTURES)
def test_reference_fixtures_load(name):
    """FreeMoe's own conformance checkpoints (Q6_K experts and router, Q4_K
    gate/up with Q6_K down as separate or fused gate_up tensors) read into
    LayerWeights with the types and routing options their adapters give."""
    r = gguf.read(FIXTURE_DIR / f"{name}.gguf")
    lw = gguf.moe_layer(r, 0)
    want = {
        "moe-fm": (gguf.F32, gguf.F32, gguf.F32, True),
        "quant-moe-q4_0": (gguf.Q4_0, gguf.Q4_0, gguf.Q4_0, True),
        "quant-moe-q8_0": (gguf.Q8_0, gguf.Q8_0, gguf.Q8_0, True),
        "quant-moe-q4_k": (gguf.Q4_K, gguf.Q4_K, gguf.Q4_K, True),
        "quant-moe-q6_k": (gguf.Q6_K, gguf.Q6_K, gguf.Q6_K, True),
        # qwen3moe files without the key: renormalisation off (gguf.cpp:1445)
        "quant-expert-fused": (gguf.Q4_K, gguf.Q6_K, gguf.F32, False),
        "quant-expert-separate": (gguf.Q4_K, gguf.Q6_K, gguf.F32, False),
    }[name]
    assert (lw.gate_type, lw.down_type, lw.router_type, lw.weights_norm) == want
    assert lw.router_bias is None and lw.weights_scale == 1.0


@needs_ref
@pytest.mark.parametrize("name", REF_FIXTURES)
def test_reference_fixture_slices_match_the_adapter(name):
    """Every expert's gate / up / down slice sits at the offset, size and type
    of the reference manifest's extents (the fused file's gate and up halves
    included)."""
    path = FIXTURE_DIR / f"{name}.gguf"
    m = fo.ref_manifest(path)
    r = gguf.read(path)
    assert m["records"] > 0
    for i, (l, e) in enumerate(m["who"]):
        sl = r.expert_slices(int(l), int(e))
        for j, key in enumerate(("gate", "up", "down")):
            arr, t = sl[key]
            off = arr.ctypes.data - r.data.ctypes.data
            assert (off, arr.nbytes, t) == tuple(int(v) for v in m["extents"][i, j]), (name, l, e, key)


def _llama_with(tmp_path, extra_tensor=None, arch="llama", **kw):
    H, F, E, K = 64, 64, 4, 2
    g = gguf.mixtral_llama(hidden=H, ffn=F, layers=1, heads=4, kv_heads=4, experts=E, top_k=K, vocab=300,
                           expert_type=gguf.Q8_0, arch=arch, **kw)
    if extra_tensor is not None:
        g.add_tensor(f"blk.0.{extra_tensor}", [E], gguf.F32)
    path = tmp_path / "x.gguf"
    g.write(path, sparse=True)
    return gguf.read(path)


@pytest.mark.parametrize("extra", ["ffn_exp_probs_b.bias", "ffn_gate_exps.bias", "ffn_gate_inp_shexp.weight"])
def test_reader_refuses_blocks_it_does_not_run(tmp_path, extra):
    with pytest.raises(NotImplementedError):
        gguf.moe_layer(_llama_with(tmp_path, extra), 0)


@pytest.mark.parametrize("arch", ["gemma2", "gpt-oss", "glm4-moe", "smallthinker"])
def test_reader_refuses_other_block_families(tmp_path, arch):
    with pytest.raises(NotImplementedError):
        gguf.moe_layer(_llama_with(tmp_path, arch=arch), 0)


def test_reader_routing_options(tmp_path):
    r = _llama_with(tmp_path, router_bias=True, weights_norm=False, weights_scale=2.5)
    lw = gguf.moe_layer(r, 0)
    assert lw.router_bias is not None and lw.router_bias.shape == (4,)
    assert (lw.weights_norm, lw.weights_scale, lw.epsilon_additive) == (False, 2.5, False)
    # families whose renormalisation the architecture fixes (gguf.cpp:2046-2058)
    assert gguf.moe_layer(_llama_with(tmp_path, arch="dbrx", weights_norm=False), 0).weights_norm
    assert not gguf.moe_layer(_llama_with(tmp_path, arch="deepseek", weights_norm=True), 0).weights_norm
    assert gguf.moe_layer(_llama_with(tmp_path, arch="maple", weights_scale=3.0), 0).weights_scale == 1.0
    ds = gguf.moe_layer(_llama_with(tmp_path, arch="deepseek41"), 0)
    assert (ds.epsilon_additive, ds.weights_epsilon) == (True, 1e-20)


def test_reader_refuses_unknown_block_types():
    t = gguf.Tensor("blk.0.x", [32, 4], 99, None)
    with pytest.raises(ValueError, match="block type 99"):
        t.nbytes()
