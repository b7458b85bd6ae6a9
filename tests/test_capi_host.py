"""libfmx.so on the host: it loads without a GPU, exports every function
include/fmx.h declares, and its host-only calls (geometry, packed sizes, status
names, fault state) behave; the packed layout is a pure permutation of the raw
GGUF bytes."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import packing_ref
from freemoe_amd import fmx
from freemoe_amd import workloads as wl

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    text = (ROOT / "include" / "fmx.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fmx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = fmx.lib()
    names = declared_functions()
    assert len(names) >= 25
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) <= set(fmx._SIGNATURES), "binding is missing a declared function"


def test_abi_version_and_status_names():
    lib = fmx.lib()
    assert lib.fmx_abi_version() == 1
    assert lib.fmx_status_name(0) == b"OK"
    assert lib.fmx_status_name(2) == b"UNSUPPORTED_QUANTISATION"
    assert lib.fmx_status_name(7) == b"FENCE_TIMEOUT"
    assert lib.fmx_status_name(8) == b"DEVICE_LOSS"


def test_status_word_mapping():
    """fmx_moe_status_of maps a device error word as fmx_moe_status does: an
    expert id out of range wins (INVALID_ARGUMENT), else a non-finite score
    (INTERNAL_ERROR)."""
    lib = fmx.lib()
    assert lib.fmx_moe_status_of(0) == 0
    assert lib.fmx_moe_status_of(1) == 4
    assert lib.fmx_moe_status_of(2) == 1
    assert lib.fmx_moe_status_of(3) == 1
    assert lib.fmx_moe_status_copy(None, None, None) == 1


def test_geometry_matches_reference_table():
    lib = fmx.lib()
    for t, (bs, bb) in {0: (1, 4), 2: (32, 18), 8: (32, 34), 12: (256, 144)}.items():
        a, b = ctypes.c_uint32(), ctypes.c_uint32()
        assert lib.fmx_quant_geometry(t, ctypes.byref(a), ctypes.byref(b)) == 0
        assert (a.value, b.value) == (bs, bb)
    a, b = ctypes.c_uint32(), ctypes.c_uint32()
    assert lib.fmx_quant_geometry(3, ctypes.byref(a), ctypes.byref(b)) == 2


@pytest.mark.parametrize("t,rows,cols", [(2, 7, 96), (2, 14336, 4096), (2, 4096, 14336), (8, 5, 160),
                                         (8, 4096, 14336), (12, 3, 768), (12, 768, 2048), (0, 3, 5)])
def test_packed_size_agrees_with_layout(t, rows, cols):
    assert fmx.packed_bytes(t, rows, cols) == packing_ref.pack(t, np.zeros((rows, wl.row_bytes(t, cols)), np.uint8),
                                                               rows, cols).size


def test_packed_size_rejects_bad_shapes():
    assert fmx.lib().fmx_packed_bytes(2, 4, 33) == 0
    assert fmx.lib().fmx_packed_bytes(5, 4, 32) == 0
    assert fmx.lib().fmx_packed_bytes(2, 0, 32) == 0


@pytest.mark.parametrize("t,rows,cols", [(2, 5, 96), (2, 9, 512), (8, 5, 160), (8, 3, 512), (12, 4, 768)])
def test_packed_layout_is_a_permutation(t, rows, cols):
    raw = wl.matrix(t, np.random.default_rng(rows * cols), rows, cols)
    packed = packing_ref.pack(t, raw, rows, cols)
    assert np.array_equal(packing_ref.unpack(t, packed, rows, cols), raw)


def test_fault_injection_is_host_side():
    lib = fmx.lib()
    assert lib.fmx_inject_fault(fmx.FAULT_TRANSFER) == 0
    fence = ctypes.c_void_p()
    buf = (ctypes.c_uint8 * 4)()
    # a transfer fault fails the upload before any HIP call
    assert lib.fmx_upload(ctypes.c_void_p(1), buf, 4, None, ctypes.byref(fence)) == 6
    assert lib.fmx_inject_fault(fmx.FAULT_DEVICE_LOSS) == 0
    assert lib.fmx_upload(ctypes.c_void_p(1), buf, 4, None, ctypes.byref(fence)) == 8
    assert lib.fmx_matvec(2, None, None, None, 4, 32, None) == 8
    assert lib.fmx_inject_fault(fmx.FAULT_FENCE_TIMEOUT) == 0
    assert lib.fmx_fence_wait(ctypes.c_void_p(1), 10) == 7
    # the timeout fires once and clears itself, as the reference's CPU backend
    assert lib.fmx_inject_fault(99) == 1
    assert lib.fmx_clear_faults() == 0


def test_argument_checks_run_before_any_launch():
    lib = fmx.lib()
    assert lib.fmx_matvec(2, None, None, None, 4, 33, None) == 3   # not whole blocks
    assert lib.fmx_matvec(3, None, None, None, 4, 32, None) == 2   # unsupported type
    assert lib.fmx_matvec(2, None, None, None, 4, 32, None) == 1   # null pointers
    assert lib.fmx_matvec(2, None, None, None, 0, 32, None) == 0   # empty product is a no-op
    desc = fmx.MoELayer()
    assert lib.fmx_moe_workspace_bytes(ctypes.byref(desc), 1) == 0
    assert lib.fmx_moe_decode(ctypes.byref(desc), None, None, 1, None, None, None, 0, None) == 1
    desc.hidden, desc.ffn, desc.experts, desc.top_k = 64, 128, 4, 5   # top_k > experts
    assert lib.fmx_moe_decode(ctypes.byref(desc), None, None, 1, None, None, None, 0, None) == 1
    assert lib.fmx_moe_bucket(None, 4, 2, 300, None, None, None, None, 0, None) == 1  # > 256 experts


def test_decode_static_refuses_oversized_layers():
    """fmx_moe_decode_static checks its fixed workspace on the host, before
    anything is launched: a layer whose one-token decode workspace exceeds
    FMX_STATIC_SCRATCH_BYTES (4 MiB) is refused with SHAPE_MISMATCH."""
    import ctypes
    import numpy as np
    from freemoe_amd import fmx
    lib = fmx.lib()
    buf = np.zeros(64, np.float32)  # any non-null, 16-byte aligned address; never read
    p = buf.ctypes.data + (-buf.ctypes.data) % 16
    layer = fmx.MoELayer(16384, 40000, 32, 32, 0, 1e-5, 0.0, 0, p, 0, 1, 0, 6.103515625e-5, 1.0, 2, 2, 2, p, p, p)
    assert lib.fmx_moe_workspace_bytes(ctypes.byref(layer), 1) > (4 << 20)
    rc = lib.fmx_moe_decode_static(ctypes.byref(layer), p, p, 1, p, p, 0, None)
    assert rc == 3  # FMX_ERR_SHAPE_MISMATCH


def test_route_checks_its_workspace_before_launching():
    """fmx_moe_route with a block-type router and no caller's h runs one token
    at a time through the workspace's h: a workspace too small for that is
    refused with INVALID_ARGUMENT before any kernel is launched (here, with no
    GPU, a launch would fail with another status)."""
    lib = fmx.lib()
    buf = np.zeros(4096, np.float32)
    p = buf.ctypes.data + (-buf.ctypes.data) % 256
    H, E, K = 256, 8, 2
    layer = fmx.MoELayer(H, 512, E, K, 0, 1e-5, 0.0, wl.Q4_0, p, 0, 1, 0, 6.103515625e-5, 1.0, 2, 2, 2, p, p, p)
    need = lib.fmx_moe_workspace_bytes(ctypes.byref(layer), 3)
    assert need > 256
    rc = lib.fmx_moe_route(ctypes.byref(layer), p, 3, None, p, p, p, p, 256, None)
    assert rc == 1


def test_attention_decode_refuses_shapes_before_launch():
    """fmx_attention_decode checks its shape on the host: positions beyond
    8192, a head width that is not a multiple of 4, heads not a multiple of
    the kv heads are SHAPE_MISMATCH, a null pointer INVALID_ARGUMENT, all
    before anything is launched."""
    lib = fmx.lib()
    buf = np.zeros(64, np.float32)
    p = buf.ctypes.data + (-buf.ctypes.data) % 16
    # positions beyond 8192, head_dim not a multiple of 4, heads not a multiple of kv_heads
    assert lib.fmx_attention_decode(p, p, 256, 128, 4, 4, 32, 8193, 0.5, p, p, 256, None) == 3
    assert lib.fmx_attention_decode(p, p, 256, 128, 4, 4, 30, 8, 0.5, p, p, 256, None) == 3
    assert lib.fmx_attention_decode(p, p, 256, 128, 6, 4, 32, 8, 0.5, p, p, 256, None) == 3
    assert lib.fmx_attention_decode(None, p, 256, 128, 4, 4, 32, 8, 0.5, p, p, 256, None) == 1
