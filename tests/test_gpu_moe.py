"""The MoE layer on the GPU against the oracle: routing bit for bit, whole
decode layers (bit for bit where libm exp agrees, 1e-4 max-abs always),
bucketing exactly, device-side error reporting."""
import numpy as np
import pytest

import fmoracle as fo
from freemoe_amd import fmx
from freemoe_amd import workloads as wl
from freemoe_amd.device import DeviceLayer
from golden.make_goldens import host_layer

pytestmark = pytest.mark.gpu

ROUTE_CASES = {
    # name: (hidden, ffn, experts, top_k, type, tokens, zipf)
    "tiny_f32": (64, 128, 4, 2, wl.F32, 64, None),
    "mixtral_router": (4096, 256, 8, 2, wl.Q4_0, 200, None),
    "finegrained_router": (2048, 256, 128, 8, wl.Q4_K, 128, 1.2),
    "odd_hidden": (200, 64, 5, 3, wl.F32, 40, None),
    # the batched router's tile shapes: 2 tokens x 16 rows (9-16 experts),
    # 16 x 32 (more), with partial token and row tiles and a 4-element tail
    "sixteen_experts_odd_tokens": (256, 64, 16, 4, wl.F32, 37, None),
    "twelve_experts": (128, 64, 12, 3, wl.F32, 21, None),
    "forty_experts_partial_tiles": (260, 64, 40, 6, wl.F32, 45, 1.2),
    # 16 x 32 tiles over a chain length (328 / 16 = 20 steps) that leaves a
    # partial LDS tile of 4 steps after a whole one, and an 8-element tail
    "twenty_experts_partial_steps": (328, 64, 20, 4, wl.F32, 37, None),
    # 256 experts, top-8, hidden 7168 (a DeepSeek-V3-sized router): hidden
    # beyond 4096 takes the 1024-thread RMSNorm and routing kernels
    "256_experts_hidden_7168": (7168, 32, 256, 8, wl.Q4_0, 24, 1.2),
}


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def to_np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("name", list(ROUTE_CASES))
def test_route_bitwise(gpu, name):
    import torch
    H, F, E, K, t, T, z = ROUTE_CASES[name]
    lw = wl.make_layer(H, F, E, K, t, 21, zipf_s=z)
    x = wl.inputs(H, T, 22) * np.float32(2.5)
    dl = DeviceLayer(lw, gpu)
    h, logits, ids, w = dl.route(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.status() == 0
    hl = host_layer(lw)
    for i in range(T):
        hh, lg, pr, ii, ww = hl.route(x[i])
        assert np.array_equal(bits(to_np(h[i])), bits(hh)), f"h token {i}"
        assert np.array_equal(bits(to_np(logits[i])), bits(lg)), f"logits token {i}"
        assert np.array_equal(to_np(ids[i]).astype(np.uint32), ii), f"ids token {i}"
        assert np.array_equal(bits(to_np(w[i])), bits(ww)), f"weights token {i}"


DECODE_CASES = {
    "tiny_f32": (64, 128, 4, 2, wl.F32, 24, None),
    "q4_0": (256, 512, 4, 2, wl.Q4_0, 12, None),
    "q4_0_partial_chunks": (96, 160, 3, 2, wl.Q4_0, 6, None),
    "q8_0": (256, 512, 4, 2, wl.Q8_0, 12, None),
    "q4_k": (512, 256, 8, 4, wl.Q4_K, 8, None),
    "q4_k_top8_zipf": (256, 768, 16, 8, wl.Q4_K, 8, 1.2),
    "256_experts_top8_hidden_7168": (7168, 64, 256, 8, wl.Q4_0, 4, 1.2),
    # the largest top-k the boundary takes (32: every expert chosen) and 16
    "q4_0_top32_all_experts": (256, 256, 32, 32, wl.Q4_0, 4, None),
    "q8_0_top16": (512, 512, 24, 16, wl.Q8_0, 4, 1.2),
    # Mixtral-shaped Q4_K: the 16-lane down kernel's whole prefetch rings
    # (56 super-blocks per row) besides its tail
    "q4_k_mixtral_shape": (4096, 14336, 8, 2, wl.Q4_K, 3, None),
    # top-1 (all 32 row slots of a 16-lane down workgroup on one rank), top-3
    # (10 rows per rank and workgroup: two idle slots, and hidden 224 leaves
    # the last workgroup's rows partly unused), rows long enough for the down
    # kernels' whole prefetch rings
    "q4_0_top3_hidden_224": (224, 4096, 4, 3, wl.Q4_0, 3, None),
    "q4_0_top1": (256, 4096, 4, 1, wl.Q4_0, 3, None),
    "q4_k_top1": (256, 4096, 4, 1, wl.Q4_K, 3, None),
}


def check_layer(gpu, lw, x):
    import torch
    dl = DeviceLayer(lw, gpu)
    out, ids, w = dl.decode(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.status() == 0
    want_out, want_ids, want_w = host_layer(lw).forward_batch(x)
    got_out = to_np(out)
    assert np.array_equal(to_np(ids).astype(np.uint32), want_ids)
    assert np.array_equal(bits(to_np(w)), bits(want_w))
    diff = np.abs(got_out.astype(np.float64) - want_out)
    # the layer's fp32 bar; beyond it the kernels reproduce the reference's
    # arithmetic, so outputs are expected bit for bit unless the device and
    # host exp() differ in a last bit that survives rounding to float
    assert diff.max() <= 1e-4, diff.max()
    mismatched = np.count_nonzero(bits(got_out) != bits(want_out))
    assert mismatched <= max(1, got_out.size // 1000), mismatched
    return mismatched


@pytest.mark.parametrize("name", list(DECODE_CASES))
def test_decode_layer_vs_oracle(gpu, name):
    H, F, E, K, t, T, z = DECODE_CASES[name]
    lw = wl.make_layer(H, F, E, K, t, 31, zipf_s=z)
    x = wl.inputs(H, T, 32)
    assert check_layer(gpu, lw, x) == 0


def test_decode_mixtral_shape_q4_0(gpu):
    """The benchmark layer at full size (hidden 4096, ffn 14336, 8 experts,
    top-2, Q4_0), a few tokens."""
    lw = wl.make_layer(4096, 14336, 8, 2, wl.Q4_0, 1234)
    x = wl.inputs(4096, 6, 1235)
    assert check_layer(gpu, lw, x) == 0


def test_route_and_decode_at_rmsnorm_near_ties(gpu):
    """Tokens whose RMSNorm output lies within 2e-15 of a float midpoint
    (tests/near_ties.py): the device's parallel sum cannot settle those, and
    the in-order sum it falls back to must give the oracle's h, logits, ids
    and weights bit for bit, on the batched route and on the decode layer."""
    import torch
    import near_ties as nt
    lw = wl.make_layer(4096, 256, 8, 2, wl.Q4_0, 21)
    X = wl.inputs(4096, 6, 23) * np.float32(2.5)
    x = np.stack([nt.craft(X[t], lw.norm_weight, lw.rms_eps)[0] for t in range(len(X))])
    dl = DeviceLayer(lw, gpu)
    xd = torch.from_numpy(x).to(gpu)
    h, logits, ids, w = dl.route(xd)
    torch.cuda.synchronize()
    assert dl.status() == 0
    hl = host_layer(lw)
    for i in range(len(x)):
        hh, lg, pr, ii, ww = hl.route(x[i])
        assert np.array_equal(bits(to_np(h[i])), bits(hh)), f"h token {i}"
        assert np.array_equal(bits(to_np(logits[i])), bits(lg)), f"logits token {i}"
        assert np.array_equal(to_np(ids[i]).astype(np.uint32), ii), f"ids token {i}"
        assert np.array_equal(bits(to_np(w[i])), bits(ww)), f"weights token {i}"
    assert check_layer(gpu, lw, x) == 0


@pytest.mark.parametrize("kind", ["halves", "wide", "zeros", "hidden_2048"])
def test_rmsnorm_in_order_sum_across_inputs(gpu, kind):
    """The in-order fallback on near-tie tokens built from different inputs:
    multiples of 1/2 (their squares' running sum meets many exact rounding
    ties), values spread over 2^-40 .. 2^40, a token that is mostly zeros,
    and hidden 2048. h, logits, ids and weights bit for bit on the batched
    route and the decode layer."""
    import torch
    import near_ties as nt
    H = 2048 if kind == "hidden_2048" else 4096
    lw = wl.make_layer(H, 256, 8, 2, wl.Q4_0, 31)
    rng = np.random.default_rng(37)
    base = []
    for t in range(4):
        if kind == "halves":
            v = rng.integers(-6, 7, H).astype(np.float32) * np.float32(0.5)
        elif kind == "wide":
            v = (rng.standard_normal(H) * np.exp2(rng.uniform(-40, 40, H))).astype(np.float32)
        elif kind == "zeros":
            v = np.zeros(H, np.float32)
            v[rng.integers(0, H, 1500)] = rng.standard_normal(1500).astype(np.float32)
        else:
            v = rng.standard_normal(H).astype(np.float32) * np.float32(2.0)
        # the crafted element moves the sum of squares: the largest for wide
        v[-1] = np.abs(v).max() if kind == "wide" else np.float32(1.5)
        base.append(v)
    x = np.stack([nt.craft(v, lw.norm_weight, lw.rms_eps)[0] for v in base])
    dl = DeviceLayer(lw, gpu)
    h, logits, ids, w = dl.route(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.status() == 0
    hl = host_layer(lw)
    for i in range(len(x)):
        hh, lg, pr, ii, ww = hl.route(x[i])
        assert np.array_equal(bits(to_np(h[i])), bits(hh)), f"h token {i}"
        assert np.array_equal(bits(to_np(logits[i])), bits(lg)), f"logits token {i}"
        assert np.array_equal(to_np(ids[i]).astype(np.uint32), ii), f"ids token {i}"
        assert np.array_equal(bits(to_np(w[i])), bits(ww)), f"weights token {i}"
    assert check_layer(gpu, lw, x) == 0


def replay_inputs(kind, T, H, rng):
    """T tokens of hidden H whose squares' in-order sum exercises the
    workgroup replay: plain normals, values with three fraction bits and with
    random trailing zero bits (their squares' sums meet exact rounding ties),
    values spread over 2^-40 .. 2^40 (the sum changes binade often) and a
    first half of zeros (the sum stays 0 for a while)."""
    v = rng.standard_normal((T, H)).astype(np.float32)
    if kind == "three_fraction_bits":
        v = np.round(v * 8) / np.float32(8)
    elif kind == "trailing_zeros":
        b = v.view(np.uint32) & ~((np.uint32(1) << rng.integers(0, 24, (T, H)).astype(np.uint32)) - np.uint32(1))
        v = b.view(np.float32)
    elif kind == "wide":
        v = (v * np.exp2(rng.uniform(-40, 40, (T, H)))).astype(np.float32)
    elif kind == "leading_zeros":
        v[:, : H // 2] = 0.0
    return np.ascontiguousarray(v, dtype=np.float32)


def near_midpoint_tokens(x, lw):
    """Tokens with an element whose in-order x*scale*gain lies within the
    device certificate's tolerance of a float midpoint: the device cannot
    settle those by its parallel sum, so they take the in-order replay."""
    import near_ties as nt
    H = x.shape[1]
    rel = 0.6e-16 * (H + 32) + 2e-15
    near = []
    for t in range(x.shape[0]):
        yd = nt.in_order_rmsnorm_double(x[t], lw.norm_weight, lw.rms_eps)
        if (nt.midpoint_distance(yd) <= rel).any():
            near.append(t)
    return near


@pytest.mark.parametrize("kind", ["normal", "three_fraction_bits", "trailing_zeros", "wide", "leading_zeros"])
@pytest.mark.parametrize("H", [2048, 4096, 8192])
def test_rmsnorm_in_order_replay_many_tokens(gpu, kind, H):
    """The in-order sum of squares, replayed by the whole workgroup (binade by
    binade) where the parallel sum cannot be certified: h bit for bit against
    the oracle's RMSNorm for every token of a 1024-token batch (the batched
    RMSNorm kernel, 0.4-10% of whose tokens lie near a float midpoint) and
    for single-token routes (the decode routing kernel) of up to 48 of the
    near tokens and 8 others."""
    import torch
    lw = wl.make_layer(H, 256, 8, 2, wl.Q4_0, 51)
    rng = np.random.default_rng(H + len(kind))
    x = replay_inputs(kind, 1024, H, rng)
    near = near_midpoint_tokens(x, lw)
    dl = DeviceLayer(lw, gpu)
    h, _, _, _ = dl.route(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.status() == 0
    got = bits(to_np(h))
    for t in range(x.shape[0]):
        want = fo.rmsnorm(x[t], lw.norm_weight, lw.rms_eps)
        assert np.array_equal(got[t], bits(want)), f"batched h token {t}"
    for t in near[:48] + list(range(8)):
        h1, _, _, _ = dl.route(torch.from_numpy(x[t:t + 1]).to(gpu))
        torch.cuda.synchronize()
        want = fo.rmsnorm(x[t], lw.norm_weight, lw.rms_eps)
        assert np.array_equal(bits(to_np(h1[0])), bits(want)), f"single-token h token {t}"
    print(f"{kind} hidden {H}: {len(near)} of 1024 tokens near a midpoint")
    assert len(near) >= 3


def one_hot_router_layer(H, E, K, seed, logits):
    """A layer whose router row e holds one nonzero weight, at element e, so
    that expert e's logit is float(h[e] * c_e) exactly on every path; c_e is
    chosen from the oracle's h of token `x` to give about `logits`."""
    lw = wl.make_layer(H, 128, E, K, wl.Q8_0, seed)
    x = wl.inputs(H, 4, seed + 1)
    h = host_layer(lw).route(x[0])[0]
    lw.router = np.zeros((E, H), np.float32)
    lw.router[np.arange(E), np.arange(E)] = (logits / h[:E]).astype(np.float32)
    return lw, x, h


def softmax_quotients(v):
    """The reference's softmax quotients e_t / sum in double (before the
    float rounding): float max, exp in double, the sum in index order."""
    import math
    m = float(np.max(v))
    ex = np.array([math.exp(float(t) - m) for t in v])
    return ex / np.cumsum(ex)[-1]


def test_route_softmax_sum_certificate_and_in_order_sum(gpu):
    """128 experts: the softmax sum of the many-expert routing kernel is a
    certified wavefront sum. A token crafted so that one quotient lies within
    1e-14 of a float midpoint (the certificate must send it to the in-order
    sum), one whose quotients include a subnormal float (always in order), and
    plain tokens: logits, ids and weights bit for bit against the oracle on
    the batched route."""
    import torch
    import near_ties as nt
    H, E, K = 256, 128, 8
    rng = np.random.default_rng(71)
    base = rng.standard_normal(E).astype(np.float32)
    # search the last expert's logit for a quotient next to a midpoint
    lw, x, h = one_hot_router_layer(H, E, K, 73, base)
    base = (np.diag(lw.router)[:E] * h[:E]).astype(np.float32)  # the logits the kernels compute
    found = None
    for start in range(0, 400_000, 2048):
        cand = (base[-1] * (1.0 + (np.arange(start, start + 2048) * 2.0 ** -22))).astype(np.float32)
        c = (cand / h[E - 1]).astype(np.float32)
        last = (c * np.float32(h[E - 1])).astype(np.float32)  # the logit float(c * h) the kernels compute
        V = np.repeat(base[None, :], len(cand), 0)
        V[:, -1] = last
        m = V.max(axis=1, keepdims=True).astype(np.float64)
        ex = np.exp(V.astype(np.float64) - m)
        q = ex / np.cumsum(ex, axis=1)[:, -1:]
        d = nt.midpoint_distance(q.ravel()).reshape(q.shape).min(axis=1)
        i = int(np.argmin(d))
        if d[i] < 5e-15:
            found = c[i]
            break
    assert found is not None, "no near-midpoint quotient found"
    lw.router[E - 1, E - 1] = found
    logits0 = host_layer(lw).route(x[0])[1]
    dist = nt.midpoint_distance(softmax_quotients(logits0)).min()
    assert dist < 1e-14, dist
    # a second layer: one expert's logit 95 below the largest, a subnormal quotient
    sub = base.copy()
    sub[5] = base.max() - np.float32(95.0)
    lw2, x2, _ = one_hot_router_layer(H, E, K, 75, sub)
    for layer, xs in ((lw, x), (lw2, x2)):
        dl = DeviceLayer(layer, gpu)
        hd, lg, ids, w = dl.route(torch.from_numpy(xs).to(gpu))
        torch.cuda.synchronize()
        assert dl.status() == 0
        hl = host_layer(layer)
        for t in range(len(xs)):
            hh, ll, _, ii, ww = hl.route(xs[t])
            assert np.array_equal(bits(to_np(lg[t])), bits(ll)), f"logits token {t}"
            assert np.array_equal(to_np(ids[t]).astype(np.uint32), ii), f"ids token {t}"
            assert np.array_equal(bits(to_np(w[t])), bits(ww)), f"weights token {t}"


def large_value_layer(gain_log2, gate_scale_bits):
    """A Q4_0 layer whose h (or act) holds values of 2^70 .. 2^106: element 5
    of h is about 2^gain_log2 (its RMSNorm gain; x[:, 5] = 1 and the router
    ignores it), and block 0 of every gate / up row has nibble 15 at element 5
    with scale 2^-24 (gate: `gate_scale_bits`), so gate, up and act grow with
    it while every value stays finite."""
    lw = wl.make_layer(256, 256, 4, 2, wl.Q4_0, 41)
    lw.norm_weight[5] = np.float32(2.0 ** gain_log2)
    lw.router[:, 5] = 0.0
    for mats, bits16 in ((lw.gate, gate_scale_bits), (lw.up, 0x0001)):
        for m in mats:
            m[:, 0:2] = np.frombuffer(np.uint16(bits16).tobytes(), np.uint8)
            m[:, 2 + 5] = (m[:, 2 + 5] & 0xF0) | 0x0F
    x = wl.inputs(256, 4, 42)
    x[:, 5] = 1.0
    return lw, x


@pytest.mark.parametrize("case", ["h_beyond_2^100", "act_beyond_2^100", "act_beyond_2^118"])
def test_decode_large_values(gpu, case):
    """Values of magnitude 2^100 and more in h (gate/up) or in act (down),
    with every product and sum still finite: the layer must match the oracle
    bit for bit there too. The nibbles become exact integers whatever the
    activations (a scaled conversion), so activations of 2^118 and more,
    where scaling the activations by 2^9 instead would overflow, are exact as
    well (the last case)."""
    if case == "h_beyond_2^100":
        lw, x = large_value_layer(101, 0x0000)  # gate ignores element 5
    elif case == "act_beyond_2^100":
        lw, x = large_value_layer(74, 0x0001)   # act ~ 2^105
    else:
        lw, x = large_value_layer(81, 0x0001)   # act ~ 2^119
    want_out = host_layer(lw).forward_batch(x)[0]
    assert np.isfinite(want_out).all() and np.abs(want_out).max() > 2.0 ** 60
    assert check_layer(gpu, lw, x) == 0


def test_decode_reports_nonfinite_scores(gpu):
    import torch
    lw = wl.make_layer(64, 128, 4, 2, wl.F32, 3)
    dl = DeviceLayer(lw, gpu)
    x = wl.inputs(64, 3, 4)
    x[1, 5] = np.inf
    out, ids, w = dl.decode(torch.from_numpy(x).to(gpu))
    torch.cuda.synchronize()
    assert dl.status() == 4  # INTERNAL_ERROR, as the reference's softmax raises
    assert (to_np(ids) < 4).all()
    assert dl.status() == 0  # read-and-clear
    # the asynchronous read: queued with the stream, read after its
    # synchronisation, the word cleared behind it
    dl.decode(torch.from_numpy(x).to(gpu))
    word = torch.full((1,), 7, dtype=torch.int32).pin_memory()
    ws = dl.workspace
    assert fmx.lib().fmx_moe_status_copy(ws.data_ptr(), word.data_ptr(), fmx.stream_handle()) == 0
    torch.cuda.synchronize()
    assert fmx.lib().fmx_moe_status_of(int(word[0])) == 4
    assert dl.status() == 0


def test_bucket_exact_vs_oracle(gpu):
    import torch
    rng = np.random.default_rng(9)
    ws = torch.zeros(256, dtype=torch.uint8, device=gpu)
    for T, K, E in [(0, 2, 8), (1, 1, 1), (512, 2, 8), (2048, 8, 128), (3000, 4, 256), (700, 8, 16)]:
        if T:
            # Zipf-skewed choices so some experts get nothing and some get many
            p = 1.0 / np.arange(1, E + 1) ** 1.2
            ids = np.stack([rng.choice(E, K, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.uint32)
        else:
            ids = np.zeros((0, K), np.uint32)
        off = torch.empty(E + 1, dtype=torch.int32, device=gpu)
        tl = torch.empty(max(T * K, 1), dtype=torch.int32, device=gpu)
        rl = torch.empty(max(T * K, 1), dtype=torch.int32, device=gpu)
        idd = torch.from_numpy(ids.astype(np.int32)).to(gpu) if T else torch.empty(1, dtype=torch.int32, device=gpu)
        fmx.call("fmx_moe_bucket", idd.data_ptr(), T, K, E, off.data_ptr(), tl.data_ptr(), rl.data_ptr(),
                 ws.data_ptr(), ws.numel(), fmx.stream_handle())
        assert fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle()) == 0
        o, t_, r_ = fo.bucket(ids, E)
        assert np.array_equal(to_np(off).astype(np.uint32), o)
        assert np.array_equal(to_np(tl)[:T * K].astype(np.uint32), t_)
        assert np.array_equal(to_np(rl)[:T * K].astype(np.uint32), r_)


def test_bucket_rejects_out_of_range_ids(gpu):
    import torch
    ws = torch.zeros(256, dtype=torch.uint8, device=gpu)
    ids = torch.tensor([[0, 1], [2, 9]], dtype=torch.int32, device=gpu)
    off = torch.empty(5, dtype=torch.int32, device=gpu)
    tl = torch.empty(4, dtype=torch.int32, device=gpu)
    rl = torch.empty(4, dtype=torch.int32, device=gpu)
    fmx.call("fmx_moe_bucket", ids.data_ptr(), 2, 2, 4, off.data_ptr(), tl.data_ptr(), rl.data_ptr(),
             ws.data_ptr(), ws.numel(), fmx.stream_handle())
    assert fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle()) == 1


@pytest.mark.parametrize("type_id", [wl.Q4_0, wl.F32])
def test_decode_timed_matches_decode(gpu, type_id):
    """The instrumented decode (launch-recorded events) gives the plain
    decode's outputs bit for bit and positive kernel times."""
    import ctypes
    import torch
    lw = wl.make_layer(256, 512, 4, 2, type_id, 51)
    x = torch.from_numpy(wl.inputs(256, 5, 52)).to(gpu)
    dl = DeviceLayer(lw, gpu)
    out1, ids1, w1 = dl.decode(x)
    out2 = torch.empty_like(x)
    ids2 = torch.empty_like(ids1)
    w2 = torch.empty_like(w1)
    ws = dl.ensure_workspace(x.shape[0])
    ms = (ctypes.c_double * 3)()
    fmx.call("fmx_moe_decode_timed", ctypes.byref(dl.desc), x.data_ptr(), out2.data_ptr(), x.shape[0],
             ids2.data_ptr(), w2.data_ptr(), ws.data_ptr(), ws.numel(), fmx.stream_handle(), ms)
    torch.cuda.synchronize()
    assert dl.status() == 0
    assert np.array_equal(bits(to_np(out1)), bits(to_np(out2)))
    assert np.array_equal(to_np(ids1), to_np(ids2))
    assert np.array_equal(bits(to_np(w1)), bits(to_np(w2)))
    assert all(v > 0.0 for v in ms)


def check_route(gpu, lw, x):
    """The device routing (h, logits, ids, weights) against the oracle, bit for
    bit, on the batched route of all tokens and on the single-token route."""
    import torch
    dl = DeviceLayer(lw, gpu)
    xd = torch.from_numpy(x).to(gpu)
    hl = host_layer(lw)
    for rows in (slice(0, len(x)), slice(0, 1)):
        h, logits, ids, w = dl.route(xd[rows])
        torch.cuda.synchronize()
        assert dl.status() == 0
        for i in range(rows.stop):
            hh, lg, pr, ii, ww = hl.route(x[i])
            assert np.array_equal(bits(to_np(h[i])), bits(hh)), f"h token {i}"
            assert np.array_equal(bits(to_np(logits[i])), bits(lg)), f"logits token {i}"
            assert np.array_equal(to_np(ids[i]).astype(np.uint32), ii), f"ids token {i}"
            assert np.array_equal(bits(to_np(w[i])), bits(ww)), f"weights token {i}"


BLOCK_ROUTER_CASES = {
    # name: (hidden, ffn, experts, top_k, expert type, router type, tokens, zipf)
    "q4_0_router": (512, 256, 8, 2, wl.Q4_0, wl.Q4_0, 24, None),
    "q8_0_router": (256, 512, 4, 2, wl.Q8_0, wl.Q8_0, 24, None),
    "q4_k_router_40_experts": (512, 256, 40, 4, wl.Q4_K, wl.Q4_K, 20, 1.2),
    "q8_0_router_q4_0_experts": (4096, 256, 8, 2, wl.Q4_0, wl.Q8_0, 12, None),
}


@pytest.mark.parametrize("name", list(BLOCK_ROUTER_CASES))
def test_block_type_router(gpu, name):
    """A quantised router (the reference's quant fixtures quantise it): logits
    are gemv_quant row dots, bit for bit, on the route, decode and prefill
    paths."""
    H, F, E, K, t, rt, T, z = BLOCK_ROUTER_CASES[name]
    lw = wl.make_layer(H, F, E, K, t, 81, zipf_s=z, router_type=rt)
    x = wl.inputs(H, T, 82)
    check_route(gpu, lw, x)
    assert check_layer(gpu, lw, x) == 0
    import test_gpu_prefill as tp
    tp.check_prefill(gpu, lw, x)


@pytest.mark.parametrize("top_k", [2, 3, 6])
def test_decode_q6_k_rows_split_over_lane_groups(gpu, top_k):
    """Q6_K down rows of at least 8 blocks run on four 16-lane groups each
    (two past top-4; every fourth or second block, the block dots added in
    block order from LDS), the gate/up rows against h staged in LDS; top-3
    and top-6 leave row slots past the last rank unused: the layer stays bit
    for bit."""
    lw = wl.make_layer(2048, 2560, 8, top_k, wl.Q6_K, 97)
    x = wl.inputs(2048, 4, 98)
    assert check_layer(gpu, lw, x) == 0


@pytest.mark.parametrize("gate_type,down_type", [(wl.Q4_K, wl.Q8_0), (wl.Q8_0, wl.Q4_0), (wl.Q4_0, wl.Q4_K),
                                                 (wl.Q4_K, wl.Q6_K), (wl.Q6_K, wl.Q8_0), (wl.Q6_K, wl.Q6_K),
                                                 (wl.F32, wl.Q4_0)])
def test_decode_mixed_block_types(gpu, gate_type, down_type):
    """Gate/up and down of different block types (the reference runs Q4_K
    gate/up with Q6_K down, tests.cpp:1479-1544): each projection keeps its
    own row order (the lane chains; Q6_K and F32 on 16 lanes per row), the
    layer stays bit for bit, and prefill matches it: the grouped GEMMs within
    their bf16 tolerance, or, for F32 (which they do not take), the decode
    kernels within 1e-4."""
    import test_gpu_prefill as tp
    lw = wl.make_layer(512, 512, 6, 2, gate_type, 91, down_type=down_type)
    x = wl.inputs(512, 8, 92)
    assert check_layer(gpu, lw, x) == 0
    if wl.F32 in (gate_type, down_type):
        import torch
        dl = DeviceLayer(lw, gpu)
        out, ids, w = dl.prefill(torch.from_numpy(x).to(gpu))
        torch.cuda.synchronize()
        want_out, want_ids, _ = host_layer(lw).forward_batch(x)
        assert np.array_equal(to_np(ids).astype(np.uint32), want_ids)
        assert np.abs(to_np(out).astype(np.float64) - want_out).max() <= 1e-4
    else:
        tp.check_prefill(gpu, lw, x)


def test_decode_refuses_16_lane_down_past_16_ranks(gpu):
    """A Q6_K (or F32) down projection runs 16 lanes per row with 16 row slots
    per workgroup shared by the ranks: more than 16 ranks is refused with
    FMX_ERR_UNSUPPORTED_QUANTISATION before anything launches, while the same
    top-k with Q4_0 down runs (top-32 above)."""
    import torch
    from freemoe_amd import fmx
    lw = wl.make_layer(256, 256, 20, 17, wl.Q4_0, 93, down_type=wl.Q6_K)
    dl = DeviceLayer(lw, gpu)
    with pytest.raises(fmx.FmxError):
        dl.decode(torch.from_numpy(wl.inputs(256, 2, 94)).to(gpu))
    torch.cuda.synchronize()


def test_route_exact_probability_ties(gpu):
    """Router rows 1 and 4, and rows 2 and 6, are equal, so their logits and
    probabilities are equal bit for bit: the stable top-k keeps the lower index
    first (engine.cpp:395-411), on every path."""
    lw = wl.make_layer(256, 256, 8, 3, wl.Q8_0, 93)
    lw.router[4] = lw.router[1]
    lw.router[6] = lw.router[2]
    x = wl.inputs(256, 64, 94)
    hl = host_layer(lw)
    tied = 0
    for i in range(len(x)):
        _, _, pr, ii, _ = hl.route(x[i])
        assert pr[1] == pr[4] and pr[2] == pr[6]
        tied += int(1 in ii and 4 in ii) + int(2 in ii and 6 in ii)
    assert tied > 0  # some tokens select both members of a tied pair
    check_route(gpu, lw, x)
    assert check_layer(gpu, lw, x) == 0
    import test_gpu_prefill as tp
    tp.check_prefill(gpu, lw, x)


ROUTING_OPTION_CASES = {
    # zero-centred norm gains (gain = 1 + w), weights scaled
    "norm_bias_1_scale_2_5": dict(norm_bias=1.0, weights_scale=2.5),
    # den = total + epsilon instead of max(total, epsilon)
    "epsilon_additive": dict(epsilon_additive=True, weights_epsilon=0.25),
    # raw probabilities, scaled
    "no_renormalisation": dict(weights_norm=False, weights_scale=0.75),
    # epsilon above every total: den = epsilon
    "epsilon_floor": dict(weights_epsilon=1.5),
}


@pytest.mark.parametrize("name", list(ROUTING_OPTION_CASES))
def test_routing_options(gpu, name):
    """The routing options of ModelConfig (norm_bias, expert_weights_norm,
    _epsilon, _epsilon_additive, _scale; engine.cpp:723-740, 1680-1702) on the
    route, decode and prefill paths, against the oracle."""
    lw = wl.make_layer(256, 256, 8, 2, wl.Q4_0, 95)
    for k, v in ROUTING_OPTION_CASES[name].items():
        setattr(lw, k, v)
    if lw.norm_bias:
        lw.norm_weight = (lw.norm_weight - np.float32(1.0)).astype(np.float32)
    x = wl.inputs(256, 32, 96)
    check_route(gpu, lw, x)
    assert check_layer(gpu, lw, x) == 0
    import test_gpu_prefill as tp
    tp.check_prefill(gpu, lw, x)


def test_bucket_rejects_duplicate_ids(gpu):
    """A token that lists one expert twice is reported (status
    INVALID_ARGUMENT), as an out-of-range id is."""
    import torch
    ws = torch.zeros(256, dtype=torch.uint8, device=gpu)
    ids = torch.tensor([[0, 1], [2, 2], [3, 1]], dtype=torch.int32, device=gpu)
    off = torch.empty(5, dtype=torch.int32, device=gpu)
    tl = torch.empty(6, dtype=torch.int32, device=gpu)
    rl = torch.empty(6, dtype=torch.int32, device=gpu)
    fmx.call("fmx_moe_bucket", ids.data_ptr(), 3, 2, 4, off.data_ptr(), tl.data_ptr(), rl.data_ptr(),
             ws.data_ptr(), ws.numel(), fmx.stream_handle())
    assert fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle()) == 1
    # a valid table on the same workspace afterwards reports nothing
    ids = torch.tensor([[0, 1], [2, 3], [3, 1]], dtype=torch.int32, device=gpu)
    fmx.call("fmx_moe_bucket", ids.data_ptr(), 3, 2, 4, off.data_ptr(), tl.data_ptr(), rl.data_ptr(),
             ws.data_ptr(), ws.numel(), fmx.stream_handle())
    assert fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle()) == 0
