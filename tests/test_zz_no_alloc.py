"""fmx_moe_decode_static (the decode entry point that allocates nothing: its
workspace is a device array inside libfmx) against fmx_moe_decode, bit for
bit, through the C ABI: two calls in a row, the second with a smaller layer
and fewer tokens, and the error word it reports."""
import ctypes

import numpy as np
import pytest

from freemoe_amd import fmx
from freemoe_amd import workloads as wl
from freemoe_amd.device import DeviceLayer

pytestmark = pytest.mark.gpu


def bits(t):
    return np.ascontiguousarray(t.detach().cpu().numpy()).view(np.uint32)


def decode_static(dl, x):
    import torch
    t, K = x.shape[0], dl.w.top_k
    out = torch.empty_like(x)
    ids = torch.empty((t, K), dtype=torch.int32, device=x.device)
    wts = torch.empty((t, K), dtype=torch.float32, device=x.device)
    status = torch.full((1,), 0xFFFF, dtype=torch.int32, device=x.device)
    fmx.call("fmx_moe_decode_static", ctypes.byref(dl.desc), x.data_ptr(), out.data_ptr(), t, ids.data_ptr(),
             wts.data_ptr(), status.data_ptr(), fmx.stream_handle())
    return out, ids, wts, status


CALLS = [
    # (hidden, ffn, experts, top_k, type, tokens): the second is smaller
    (1024, 2048, 8, 2, wl.Q8_0, 12),
    (256, 512, 4, 2, wl.Q4_0, 5),
]


def test_decode_static_matches_decode(gpu):
    import torch
    for i, (H, F, E, K, t, T) in enumerate(CALLS):
        lw = wl.make_layer(H, F, E, K, t, 300 + i)
        x = torch.from_numpy(wl.inputs(H, T, 310 + i)).to(gpu)
        dl = DeviceLayer(lw, gpu)
        want_out, want_ids, want_w = dl.decode(x)
        out, ids, w, status = decode_static(dl, x)
        torch.cuda.synchronize()
        assert dl.status() == 0
        assert int(status.item()) == 0, f"call {i}"
        assert np.array_equal(bits(out), bits(want_out)), f"call {i}"
        assert torch.equal(ids, want_ids), f"call {i}"
        assert np.array_equal(bits(w), bits(want_w)), f"call {i}"


def test_decode_static_reports_nonfinite_scores(gpu):
    import torch
    lw = wl.make_layer(64, 128, 4, 2, wl.F32, 3)
    dl = DeviceLayer(lw, gpu)
    x = wl.inputs(64, 3, 4)
    x[1, 5] = np.inf
    out, ids, w, status = decode_static(dl, torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert int(status.item()) == 1  # bit 0: a non-finite router score
    assert (ids.cpu().numpy() < 4).all()
