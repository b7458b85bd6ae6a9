"""The synthetic workloads hold the cases the GPU tests rely on (CPU only)."""
import numpy as np

from freemoe_amd import workloads as wl
from golden.make_goldens import host_layer


def test_finegrained_1100_token_routing_histogram():
    """The 1100-token fine-grained prefill case (hidden 2048, 128 experts,
    top-8, Q4_K, Zipf(1.2) router bias, seed 41) holds empty experts, 1-pair
    experts and experts of more than 192 pairs (more than one row tile), by
    the oracle's routing."""
    lw = wl.make_layer(2048, 768, 128, 8, wl.Q4_K, 41, zipf_s=1.2)
    x = wl.inputs(2048, 1100, 42)
    hl = host_layer(lw)
    ids = np.array([hl.route(x[i])[3] for i in range(x.shape[0])])
    c = np.bincount(ids.ravel(), minlength=128)
    assert (c == 0).sum() > 0 and (c == 1).sum() > 0 and (c > 192).sum() > 0


def test_mixed_types_and_block_router():
    """make_layer keeps gate/up and down types apart and builds a block-type
    router whose rows have the router's row bytes."""
    lw = wl.make_layer(256, 128, 4, 2, wl.Q4_K, 3, down_type=wl.Q8_0, router_type=wl.Q4_0)
    assert lw.gate_type == wl.Q4_K and lw.up_type == wl.Q4_K and lw.down_type == wl.Q8_0
    assert lw.gate[0].shape == (128, wl.row_bytes(wl.Q4_K, 256))
    assert lw.down[0].shape == (256, wl.row_bytes(wl.Q8_0, 128))
    assert lw.router_bytes.shape == (4, wl.row_bytes(wl.Q4_0, 256))
