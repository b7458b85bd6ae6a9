"""The oracle against the reference's own compiled kernels: bit for bit, through
the committed goldens (always) and live through oracle/_ref (where built)."""
from pathlib import Path

import numpy as np
import pytest

import fmoracle as fo
from freemoe_amd import workloads as wl
from golden.make_goldens import KERNEL_CASES, LAYER_CASES, host_layer, kernel_inputs, weights_digest

GOLDEN = Path(__file__).resolve().parent / "golden"


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def kernels():
    return np.load(GOLDEN / "ref_kernels.npz")


@pytest.fixture(scope="module")
def layers():
    return np.load(GOLDEN / "ref_layers.npz")


@pytest.mark.parametrize("i", range(len(KERNEL_CASES)))
@pytest.mark.parametrize("isa", [fo.ISA_SCALAR, fo.ISA_AVX2])
def test_gemv_matches_reference_golden(kernels, i, isa):
    t, o, n = KERNEL_CASES[i]
    assert list(kernels[f"k{i}_shape"]) == [t, o, n]
    w, x = kernel_inputs(i, t, o, n)
    got = fo.gemv(t, w, x, o, n, isa)
    assert np.array_equal(bits(got), bits(kernels[f"k{i}_isa{isa}_y"]))


@pytest.mark.parametrize("name", list(LAYER_CASES))
def test_layer_matches_reference_golden(layers, name):
    H, F, E, K, t, T, seed, zm = (int(v) for v in layers[f"{name}_meta"])
    lw = wl.make_layer(H, F, E, K, t, seed, zipf_s=None if zm < 0 else zm / 1000)
    assert weights_digest(lw) == bytes(layers[f"{name}_digest"]).hex(), "workload generator drifted"
    x = wl.inputs(H, T, seed + 1)
    out, ids, w = host_layer(lw).forward_batch(x, fo.ISA_AVX2)
    assert np.array_equal(ids, layers[f"{name}_ids"])
    assert np.array_equal(bits(w), bits(layers[f"{name}_weights"]))
    assert np.array_equal(bits(out), bits(layers[f"{name}_out"]))


# ------------------------------------------------------- live, where built --

@pytest.mark.parametrize("type_id", [0, 2, 8, 12, 14])
@pytest.mark.parametrize("isa", [fo.ISA_SCALAR, fo.ISA_AVX2])
def test_gemv_bitwise_vs_live_reference(ref_lib, type_id, isa):
    rng = np.random.default_rng(type_id * 7 + isa)
    bs = fo.GEOMETRY[type_id][0]
    for in_dim in sorted({bs * 2, bs * 8, 4096, bs * 24}):
        for out_dim in (1, 13):
            w = wl.matrix(type_id, rng, out_dim, in_dim, sigma=0.03, f32_sigma=0.3)
            x = rng.standard_normal(in_dim, dtype=np.float32) * np.float32(3.0)
            got = fo.gemv(type_id, w, x, out_dim, in_dim, isa)
            for threads in (1, 4):
                want = fo.ref_gemv(type_id, w, x, out_dim, in_dim, isa, threads)
                assert np.array_equal(bits(got), bits(want)), (in_dim, out_dim, threads)


@pytest.mark.parametrize("type_id", [0, 2, 8, 12, 14])
@pytest.mark.parametrize("isa", [fo.ISA_SCALAR, fo.ISA_AVX2])
def test_gemm_bitwise_vs_live_reference(ref_lib, type_id, isa):
    """gemm_quant (the batched product): the oracle's dequantise-then-dot
    against the reference's own gemm_quant, bit for bit, over F32 tails, block
    multiples and token counts around the 32-token tile."""
    rng = np.random.default_rng(100 + type_id * 7 + isa)
    bs = fo.GEOMETRY[type_id][0]
    dims = [7, 24, 25, 300, 1031] if type_id == 0 else sorted({bs, bs * 3, bs * 9, 2304})
    for in_dim in dims:
        for out_dim, tokens in ((1, 1), (13, 33), (40, 5)):
            w = wl.matrix(type_id, rng, out_dim, in_dim, sigma=0.03, f32_sigma=0.3)
            x = rng.standard_normal((tokens, in_dim), dtype=np.float32) * np.float32(3.0)
            got = fo.gemm(type_id, w, x, out_dim, in_dim, isa)
            for threads in (1, 2):
                want = fo.ref_gemm(type_id, w, x, out_dim, in_dim, isa, threads)
                assert np.array_equal(bits(got), bits(want)), (in_dim, out_dim, tokens, threads)


def test_f32_tails_bitwise_vs_live_reference(ref_lib):
    rng = np.random.default_rng(3)
    for n in [1, 7, 8, 9, 15, 16, 17, 23, 24, 25, 31, 33, 4103]:
        w = rng.standard_normal((3, n), dtype=np.float32)
        x = rng.standard_normal(n, dtype=np.float32)
        for isa in (fo.ISA_SCALAR, fo.ISA_AVX2):
            got = fo.gemv(0, w.view(np.uint8), x, 3, n, isa)
            want = fo.ref_gemv(0, w.view(np.uint8), x, 3, n, isa)
            assert np.array_equal(bits(got), bits(want)), (n, isa)


def test_dequant_bitwise_vs_live_reference(ref_lib):
    import ctypes
    rng = np.random.default_rng(11)
    for t in (2, 8, 12, 14):
        bs, bb = fo.GEOMETRY[t]
        raw = wl.matrix(t, rng, 64, bs, sigma=0.5)
        d = 208 if t == 14 else 0  # the f16 scale's offset (Q6_K stores it last)
        # subnormal, zero, negative and large scales
        raw[0, d:d + 2] = [1, 0]
        raw[1, d:d + 2] = [0, 0]
        raw[2, d:d + 2] = np.frombuffer(np.float16(-2.5).tobytes(), np.uint8)
        raw[3, d:d + 2] = np.frombuffer(np.float16(60000).tobytes(), np.uint8)
        got = fo.dequantize(t, raw, 64 * bs).reshape(64, bs)
        for r in range(64):
            want = np.empty(bs, np.float32)
            blk = np.ascontiguousarray(raw[r])
            assert fo.ref().fmr_dequantize_block(t, blk.ctypes.data_as(ctypes.c_void_p),
                                                  want.ctypes.data_as(ctypes.c_void_p)) == 0
            assert np.array_equal(bits(got[r]), bits(want))


@pytest.mark.parametrize("name", ["q4_0", "q4_k_zipf"])
def test_layer_bitwise_vs_live_reference_threaded(ref_lib, name):
    H, F, E, K, t, T, z = LAYER_CASES[name]
    lw = wl.make_layer(H, F, E, K, t, 5, zipf_s=z)
    x = wl.inputs(H, T, 6)
    hl = host_layer(lw)
    a = hl.forward_batch(x, fo.ISA_AVX2)
    b = hl.ref_forward_batch(x, fo.ISA_AVX2, threads=4)
    for u, v in zip(a, b):
        assert np.array_equal(np.asarray(u).view(np.uint32), np.asarray(v).view(np.uint32))
