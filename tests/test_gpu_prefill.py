"""The batched (prefill) MoE layer on the GPU against the oracle.

Routing (ids, weights) must be bit-identical to the reference's per-token
routing. The expert FFN runs as grouped GEMMs on bf16 MFMA, so the layer's
FFN contribution (out - x) is checked against the oracle's within 2e-2
relative, both as a norm ratio and as max-abs over the largest reference
value. Shapes the GEMMs do not tile run the decode kernels and stay
bit-identical."""
import numpy as np
import pytest

from freemoe_amd import workloads as wl
from freemoe_amd.device import DeviceLayer
from golden.make_goldens import host_layer

pytestmark = pytest.mark.gpu

REL_TOL = 2e-2  # bf16 operands, f32 accumulation

CASES = {
    # name: (hidden, ffn, experts, top_k, type, tokens, zipf)
    "q8_0": (256, 512, 4, 2, wl.Q8_0, 64, None),
    "q4_0": (512, 512, 4, 2, wl.Q4_0, 100, None),
    "q4_k_zipf": (512, 256, 8, 4, wl.Q4_K, 96, 1.2),
    "q8_0_tiles_over_256_rows": (256, 256, 2, 1, wl.Q8_0, 700, None),
    "q8_0_ragged_top8": (256, 256, 16, 8, wl.Q8_0, 40, 1.2),
}


def to_np(t):
    return t.detach().cpu().numpy()


def check_prefill(gpu, lw, x):
    import torch
    dl = DeviceLayer(lw, gpu)
    out, ids, w = dl.prefill(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.prefill_status() == 0
    want_out, want_ids, want_w = host_layer(lw).forward_batch(x)
    assert np.array_equal(to_np(ids).astype(np.uint32), want_ids)
    assert np.array_equal(to_np(w).view(np.uint32), want_w.view(np.uint32))
    got = to_np(out).astype(np.float64) - x
    ref = want_out.astype(np.float64) - x
    err = got - ref
    norm_ratio = np.linalg.norm(err) / np.linalg.norm(ref)
    max_ratio = np.abs(err).max() / np.abs(ref).max()
    assert norm_ratio <= REL_TOL, norm_ratio
    assert max_ratio <= REL_TOL, max_ratio
    return norm_ratio, max_ratio


@pytest.mark.parametrize("name", list(CASES))
def test_prefill_vs_oracle(gpu, name):
    H, F, E, K, t, T, z = CASES[name]
    lw = wl.make_layer(H, F, E, K, t, 41, zipf_s=z)
    x = wl.inputs(H, T, 42)
    check_prefill(gpu, lw, x)


def test_prefill_mixtral_shape_q8_0(gpu):
    """The prefill benchmark layer at full size (hidden 4096, ffn 14336, 8
    experts, top-2, Q8_0), 48 tokens."""
    lw = wl.make_layer(4096, 14336, 8, 2, wl.Q8_0, 1234)
    x = wl.inputs(4096, 48, 1235)
    check_prefill(gpu, lw, x)


def test_prefill_untiled_shape_runs_decode_kernels(gpu):
    """F32 experts have no GEMM path: prefill runs the decode kernels and stays
    bit-identical to the reference."""
    import torch
    lw = wl.make_layer(64, 128, 4, 2, wl.F32, 5)
    x = wl.inputs(64, 24, 6)
    dl = DeviceLayer(lw, gpu)
    out, ids, w = dl.prefill(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    want_out, want_ids, _ = host_layer(lw).forward_batch(x)
    assert np.array_equal(to_np(ids).astype(np.uint32), want_ids)
    assert np.abs(to_np(out).astype(np.float64) - want_out).max() <= 1e-4


def test_prefill_matches_decode_routing(gpu):
    """Prefill and decode route every token identically."""
    import torch
    lw = wl.make_layer(256, 512, 8, 2, wl.Q8_0, 7)
    x = torch.from_numpy(wl.inputs(256, 32, 8)).to(gpu)
    dl = DeviceLayer(lw, gpu)
    _, ids_p, w_p = dl.prefill(x)
    _, ids_d, w_d = dl.decode(x)
    torch.cuda.synchronize()
    assert torch.equal(ids_p, ids_d)
    assert torch.equal(w_p, w_d)
