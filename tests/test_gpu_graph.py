"""Decode captured in a HIP graph (the capture a serving loop makes around a
batch-1 step): every replay must equal the eager launches bit for bit. The
capture holds only kernels (the error word is cleared by a kernel, not a
memset), and the replays alternate with eager decodes of other inputs, so a
node that only works on its first replay, or that reads state an eager call
left behind, shows up as a mismatch."""
import numpy as np
import pytest

from freemoe_amd import workloads as wl
from freemoe_amd.device import DeviceLayer

pytestmark = pytest.mark.gpu


def bits(t):
    return np.ascontiguousarray(t.detach().cpu().numpy()).view(np.uint32)


@pytest.mark.parametrize("type_id,down_type", [(wl.Q4_0, wl.Q4_0), (wl.Q4_K, wl.Q4_K), (wl.Q8_0, wl.Q6_K)],
                         ids=["q4_0", "q4_k", "q8_0_down_q6_k"])
def test_decode_graph_replays_match_eager(gpu, type_id, down_type):
    import torch
    lw = wl.make_layer(1024, 2048, 8, 2, type_id, 61, down_type=down_type)
    x = torch.from_numpy(wl.inputs(1024, 16, 62)).to(gpu)
    other = torch.from_numpy(wl.inputs(1024, 16, 63)).to(gpu)
    dl = DeviceLayer(lw, gpu)
    dl.ensure_workspace(16)
    want_out, want_ids, want_w = dl.decode(x)
    torch.cuda.synchronize()
    want = (bits(want_out), bits(want_ids), bits(want_w))

    out = torch.empty_like(x)
    ids = torch.empty_like(want_ids)
    w = torch.empty_like(want_w)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dl.decode(x, out, ids, w)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dl.decode(x, out, ids, w)
    torch.cuda.synchronize()
    for replay in range(3):
        out.fill_(0.0)
        ids.fill_(-1)
        w.fill_(0.0)
        graph.replay()
        torch.cuda.synchronize()
        got = (bits(out), bits(ids), bits(w))
        for name, g, e in zip(("out", "ids", "weights"), got, want):
            assert np.array_equal(g, e), f"replay {replay}: {name} differs from the eager decode"
        dl.decode(other)  # eager work between replays, through the same workspace
        torch.cuda.synchronize()
    assert dl.status() == 0


def test_prefill_graph_replays_match_eager(gpu):
    """The batched layer (routing, bucketing, bf16 rows, grouped GEMMs, combine)
    captured likewise: the GEMMs accumulate in a fixed order and the
    bucketing places pairs by rank, so replays equal the eager pass bit for
    bit."""
    import torch
    lw = wl.make_layer(1024, 2048, 8, 2, wl.Q8_0, 71)
    x = torch.from_numpy(wl.inputs(1024, 256, 72)).to(gpu)
    other = torch.from_numpy(wl.inputs(1024, 256, 73)).to(gpu)
    dl = DeviceLayer(lw, gpu)
    want_out, want_ids, want_w = dl.prefill(x)
    torch.cuda.synchronize()
    want = (bits(want_out), bits(want_ids), bits(want_w))
    out = torch.empty_like(x)
    ids = torch.empty_like(want_ids)
    w = torch.empty_like(want_w)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        dl.prefill(x, out, ids, w)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dl.prefill(x, out, ids, w)
    torch.cuda.synchronize()
    for replay in range(3):
        out.fill_(0.0)
        ids.fill_(-1)
        w.fill_(0.0)
        graph.replay()
        torch.cuda.synchronize()
        got = (bits(out), bits(ids), bits(w))
        for name, g, e in zip(("out", "ids", "weights"), got, want):
            assert np.array_equal(g, e), f"replay {replay}: {name} differs from the eager prefill"
        dl.prefill(other)
        torch.cuda.synchronize()
    assert dl.prefill_status() == 0
