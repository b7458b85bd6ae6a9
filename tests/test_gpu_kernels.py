"""libfmx kernels on the GPU against the oracle: packing byte for byte,
dequantisation and matvec bit for bit (the reference's AVX2 lane order)."""
import numpy as np
import pytest

import fmoracle as fo
import packing_ref
from freemoe_amd import fmx
from freemoe_amd import workloads as wl

pytestmark = pytest.mark.gpu


def dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def same_floats(got, want):
    """Bitwise, except that any NaN matches any NaN."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    n1, n2 = np.isnan(got), np.isnan(want)
    return np.array_equal(n1, n2) and np.array_equal(bits(got[~n1]), bits(want[~n2]))


@pytest.mark.parametrize("t,rows,cols", [(2, 5, 96), (2, 33, 4096), (2, 7, 14336), (8, 5, 160), (8, 9, 4096),
                                         (12, 4, 768), (12, 17, 2048), (0, 3, 40), (14, 6, 512)])
def test_pack_matches_layout(gpu, t, rows, cols):
    import torch
    raw = wl.matrix(t, np.random.default_rng(rows + cols), rows, cols)
    out = torch.zeros(fmx.packed_bytes(t, rows, cols), dtype=torch.uint8, device=gpu)
    fmx.call("fmx_pack", t, dev(raw, gpu).data_ptr(), out.data_ptr(), rows, cols, fmx.stream_handle())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), packing_ref.pack(t, raw, rows, cols))


@pytest.mark.parametrize("t", [0, 2, 8, 12, 14])
def test_dequant_bitwise(gpu, t):
    import torch
    bs, bb = wl.GEOMETRY[t]
    rng = np.random.default_rng(t)
    raw = wl.matrix(t, rng, 1, bs * 257, sigma=0.3)
    n = bs * 257
    out = torch.empty(n, dtype=torch.float32, device=gpu)
    fmx.call("fmx_dequantize", t, dev(raw, gpu).data_ptr(), out.data_ptr(), n, fmx.stream_handle())
    torch.cuda.synchronize()
    assert same_floats(out.cpu().numpy(), fo.dequantize(t, raw, n))


def test_dequant_every_half_scale(gpu):
    """All 65536 f16 scale encodings (subnormals, infinities, NaNs) through Q8_0
    and, as d and dmin, through Q4_K."""
    import torch
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    q8 = np.zeros((65536, 34), np.uint8)
    q8[:, 0:2] = h.view(np.uint8).reshape(-1, 2)
    q8[:, 2:] = np.array([1, 0xFF, 127, 0x81, 3, 0, 64, 0xC0] * 4, np.uint8)
    out = torch.empty(65536 * 32, dtype=torch.float32, device=gpu)
    fmx.call("fmx_dequantize", 8, dev(q8, gpu).data_ptr(), out.data_ptr(), 65536 * 32, fmx.stream_handle())
    torch.cuda.synchronize()
    assert same_floats(out.cpu().numpy(), fo.dequantize(8, q8, 65536 * 32))
    qk = np.frombuffer(np.random.default_rng(1).bytes(4096 * 144), np.uint8).reshape(4096, 144).copy()
    sel = h[np.random.default_rng(2).integers(0, 65536, 8192)]
    qk[:, 0:4] = sel.view(np.uint8).reshape(4096, 4)
    out = torch.empty(4096 * 256, dtype=torch.float32, device=gpu)
    fmx.call("fmx_dequantize", 12, dev(qk, gpu).data_ptr(), out.data_ptr(), 4096 * 256, fmx.stream_handle())
    torch.cuda.synchronize()
    assert same_floats(out.cpu().numpy(), fo.dequantize(12, qk, 4096 * 256))


MATVEC_CASES = [
    (0, 37, 512), (0, 5, 24), (0, 5, 40), (0, 3, 4103), (0, 1000, 4096),
    (2, 37, 512), (2, 11, 96), (2, 6, 4096), (2, 1000, 4096), (2, 513, 14336),
    (8, 37, 512), (8, 11, 96), (8, 6, 4096), (8, 1000, 4096), (8, 300, 14336),
    (12, 37, 512), (12, 6, 2048), (12, 768, 2048), (12, 2048, 768),
    # Q6_K: one lane group per row (fewer than 8 blocks), blocks split over
    # four (fewer than 8192 rows) or two lane groups per row
    (14, 37, 256), (14, 9, 2048), (14, 300, 14336), (14, 8193, 512), (14, 4095, 4096), (14, 8200, 2048),
]


@pytest.mark.parametrize("t,rows,cols", MATVEC_CASES)
def test_matvec_bitwise_vs_oracle(gpu, t, rows, cols):
    import torch
    rng = np.random.default_rng(rows * 31 + cols)
    raw = wl.matrix(t, rng, rows, cols, sigma=0.02, f32_sigma=0.1)
    x = rng.standard_normal(cols, dtype=np.float32)
    packed = torch.empty(fmx.packed_bytes(t, rows, cols), dtype=torch.uint8, device=gpu)
    fmx.call("fmx_pack", t, dev(raw, gpu).data_ptr(), packed.data_ptr(), rows, cols, fmx.stream_handle())
    y = torch.empty(rows, dtype=torch.float32, device=gpu)
    xd = dev(x, gpu)
    fmx.call("fmx_matvec", t, packed.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, cols, fmx.stream_handle())
    torch.cuda.synchronize()
    want = fo.gemv(t, raw, x, rows, cols, fo.ISA_AVX2)
    got = y.cpu().numpy()
    assert np.array_equal(bits(got), bits(want)), f"max diff {np.abs(got - want).max()}"


GEMM_CASES = [(0, 7, 13, 33), (0, 25, 40, 5), (0, 1031, 17, 70), (2, 32, 1, 1), (2, 4096, 40, 33),
              (8, 96, 300, 100), (8, 2304, 16, 32), (12, 256, 13, 9), (12, 2048, 33, 65), (14, 256, 17, 33),
              (14, 1024, 40, 5)]


@pytest.mark.parametrize("t,in_dim,out_dim,tokens", GEMM_CASES)
def test_gemm_quant_bitwise(gpu, t, in_dim, out_dim, tokens):
    """The batched product (gemm_quant) bit for bit against the oracle and,
    where it is built, the reference's own gemm_quant: F32 rows with 8-wide
    and scalar tails, every block type, token counts around the 32-token
    tile, rows around the 16-row tile."""
    import torch
    rng = np.random.default_rng(in_dim * 31 + out_dim + t)
    w = wl.matrix(t, rng, out_dim, in_dim, sigma=0.03, f32_sigma=0.3)
    x = rng.standard_normal((tokens, in_dim), dtype=np.float32) * np.float32(3.0)
    y = torch.full((tokens, out_dim), float("nan"), dtype=torch.float32, device=gpu)
    wd, xd = dev(w, gpu), dev(x, gpu)  # held: a temporary's memory would be reused by the next
    fmx.call("fmx_gemm_quant", t, wd.data_ptr(), xd.data_ptr(), y.data_ptr(), tokens, out_dim, in_dim,
             fmx.stream_handle())
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert same_floats(got, fo.gemm(t, w, x, out_dim, in_dim))
    if fo.REF_PATH.exists():
        assert same_floats(got, fo.ref_gemm(t, w, x, out_dim, in_dim))


def test_gemm_quant_errors(gpu):
    """The reference's argument checks: a zero dimension is a no-op, a row that
    is not whole blocks is SHAPE_MISMATCH, an unknown type UNSUPPORTED."""
    import torch
    lib = fmx.lib()
    x = torch.zeros(64, dtype=torch.float32, device=gpu)
    y = torch.zeros(64, dtype=torch.float32, device=gpu)
    w = torch.zeros(4096, dtype=torch.uint8, device=gpu)
    assert lib.fmx_gemm_quant(8, w.data_ptr(), x.data_ptr(), y.data_ptr(), 0, 4, 32, None) == 0
    assert lib.fmx_gemm_quant(8, w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 4, 48, None) == 3
    assert lib.fmx_gemm_quant(77, w.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 4, 32, None) == 2
    assert lib.fmx_gemm_quant(8, None, x.data_ptr(), y.data_ptr(), 1, 4, 32, None) == 1
