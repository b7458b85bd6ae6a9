"""The batched (prefill) MoE layer on the GPU against the oracle.

Routing (ids, weights) must be bit-identical to the reference's per-token
routing. The expert FFN runs as grouped GEMMs on bf16 MFMA, so the layer's
FFN contribution (out - x) is checked against the oracle's within 2e-2
relative, both as a norm ratio and as max-abs over the largest reference
value. Shapes the GEMMs do not tile (F32 experts) run the decode kernels and stay
bit-identical."""
import os

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
    # more than 16 experts: the single-split down GEMM and the 16 x 32 router
    # tiles
    "q8_0_32_experts": (256, 256, 32, 4, wl.Q8_0, 300, None),
    "q4_0_24_experts_zipf": (512, 256, 24, 3, wl.Q4_0, 200, 1.2),
    # 256 experts (the bucketing's maximum), top-8
    "q8_0_256_experts_top8": (1024, 128, 256, 8, wl.Q8_0, 100, 1.2),
    # raw Q6_K blocks (identity K order, unaligned 16-byte loads)
    "q6_k": (256, 512, 4, 2, wl.Q6_K, 64, None),
    "q6_k_six_row_blocks": (1024, 1024, 4, 2, wl.Q6_K, 380, None),
}

# the oracle runs the reference's per-token loop; large cases split it over
# host threads (each token's result does not depend on the split)
ORACLE_THREADS = max(1, min(16, os.cpu_count() or 1))


def to_np(t):
    return t.detach().cpu().numpy()


def check_prefill(gpu, lw, x):
    import torch
    dl = DeviceLayer(lw, gpu)
    out, ids, w = dl.prefill(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.prefill_status() == 0
    want_out, want_ids, want_w = host_layer(lw).forward_batch(x, threads=ORACLE_THREADS)
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


def test_prefill_mixtral_q8_0_512_tokens(gpu):
    """The prefill benchmark workload itself: hidden 4096, ffn 14336, 8 experts,
    top-2, Q8_0, 512 tokens, so each expert's row tiles hold about 128 pairs
    (4 or more 32-row blocks)."""
    lw, x = wl.workload("mixtral-q8_0")
    norm_ratio, max_ratio = check_prefill(gpu, lw, x)
    print(f"mixtral q8_0 512 tokens: norm ratio {norm_ratio:.3e}, max ratio {max_ratio:.3e}")


def test_prefill_finegrained_q4_k_2048_tokens(gpu):
    """The fine-grained prefill workload itself (hidden 2048, ffn 768, 128
    experts, top-8, Q4_K, Zipf(1.2) router bias, 2048 tokens): the
    single-split down GEMM, bucketing over eight 256-token chunks, and experts
    with no pair, one pair and more than one 192-pair row tile."""
    lw, x = wl.workload("finegrained")
    norm_ratio, max_ratio = check_prefill(gpu, lw, x)
    print(f"finegrained q4_k 2048 tokens: norm ratio {norm_ratio:.3e}, max ratio {max_ratio:.3e}")


@pytest.mark.parametrize("tokens", [1, 255, 256, 257, 1500])
def test_prefill_every_token_on_the_same_experts(gpu, tokens):
    """A router bias that sends every token to experts 0 and 1: two experts
    with all the pairs (up to 8 full 192-row tiles and a partial one each),
    six with none, token counts on both sides of the bucketing's 256-token
    chunks. Routing bit for bit, the FFN within the prefill tolerance."""
    lw = wl.make_layer(256, 256, 8, 2, wl.Q8_0, 81)
    bias = np.zeros(8, np.float32)
    bias[:2] = 40.0
    lw.router_bias = bias
    x = wl.inputs(256, tokens, 82)
    check_prefill(gpu, lw, x)


def test_prefill_mixed_block_types(gpu):
    """Gate/up and down in different block types (Q4_K gate/up with Q8_0 down,
    Q8_0 gate/up with Q4_0 down, Q4_K gate/up with Q6_K down as in FreeMoe's
    mixed checkpoints, Q6_K gate/up with Q8_0 down)."""
    for seed, (gt, dt) in enumerate(((wl.Q4_K, wl.Q8_0), (wl.Q8_0, wl.Q4_0), (wl.Q4_K, wl.Q6_K),
                                     (wl.Q6_K, wl.Q8_0))):
        lw = wl.make_layer(512, 512, 8, 2, gt, 60 + seed, down_type=dt)
        x = wl.inputs(512, 80, 70 + seed)
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


def test_prefill_timed_matches_prefill(gpu):
    """The instrumented prefill (events recorded by the GEMM launches) gives
    the plain prefill's outputs bit for bit and positive GEMM times; a shape
    the GEMMs do not tile is refused with FMX_ERR_SHAPE_MISMATCH."""
    import torch
    from freemoe_amd import fmx
    lw = wl.make_layer(256, 512, 8, 2, wl.Q8_0, 61)
    x = torch.from_numpy(wl.inputs(256, 40, 62)).to(gpu)
    dl = DeviceLayer(lw, gpu)
    out1, ids1, w1 = dl.prefill(x)
    out1, ids1, w1 = out1.clone(), ids1.clone(), w1.clone()
    ms = []
    out2, ids2, w2 = dl.prefill(x, kernel_ms=ms)
    torch.cuda.synchronize()
    assert dl.prefill_status() == 0
    assert torch.equal(out1.view(torch.int32), out2.view(torch.int32))
    assert torch.equal(ids1, ids2) and torch.equal(w1, w2)
    assert len(ms) == 2 and all(v > 0.0 for v in ms)
    f32 = DeviceLayer(wl.make_layer(64, 128, 4, 2, wl.F32, 5), gpu)
    with pytest.raises(fmx.FmxError):
        f32.prefill(torch.from_numpy(wl.inputs(64, 4, 6)).to(gpu), kernel_ms=[])
