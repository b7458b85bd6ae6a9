"""Closed forms and brute force for the oracle's routing, norm, activation and
bucketing (engine.cpp:378-411, 723-740, 1680-1702; activation.hpp:33-85)."""
import itertools
import math

import numpy as np
import pytest

import fmoracle as fo
from freemoe_amd import workloads as wl
from golden.make_goldens import host_layer


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(300, dtype=np.float32)
    w = (1 + rng.standard_normal(300) * 0.1).astype(np.float32)
    eps = float(np.float32(1e-5))
    got = fo.rmsnorm(x, w, eps)
    ss = 0.0
    for v in x.astype(np.float64):
        ss += v * v
    s = 1.0 / math.sqrt(ss / 300 + eps)
    want = np.array([np.float32(float(x[i]) * s * float(np.float32(float(w[i])))) for i in range(300)])
    assert np.array_equal(got, want)
    # zero-centred weights (norm_bias = 1): gain = float(1 + w)
    got1 = fo.rmsnorm(x, w, eps, 1.0)
    want1 = np.array([np.float32(float(x[i]) * s * float(np.float32(1.0 + float(w[i])))) for i in range(300)])
    assert np.array_equal(got1, want1)
    # no weight: unit gain
    assert np.array_equal(fo.rmsnorm(x, None, eps), np.array([np.float32(float(v) * s) for v in x]))


def test_softmax_closed_form_and_errors():
    v = np.array([0.5, -1.0, 3.25, 3.25, -7.0], np.float32)
    got = fo.softmax(v)
    m = 3.25
    e = [math.exp(float(a) - m) for a in v]
    s = 0.0
    for q in e:
        s += q
    assert np.array_equal(got, np.array([np.float32(q / s) for q in e]))
    for bad in (np.nan, np.inf, -np.inf):
        with pytest.raises(fo.OracleError) as err:
            fo.softmax(np.array([0.0, bad], np.float32))
        assert err.value.status == 4  # INTERNAL_ERROR


def test_topk_stable_ties_and_edge_cases():
    s = np.array([0.1, 0.4, 0.4, 0.05, 0.4], np.float32)
    assert list(fo.topk(s, 3)) == [1, 2, 4]
    assert list(fo.topk(s, 5)) == [1, 2, 4, 0, 3]
    # -inf masks an expert out and is allowed; NaN / +inf are internal errors
    assert list(fo.topk(np.array([-np.inf, 0.2, -np.inf], np.float32), 2)) == [1, 0]
    for bad in (np.nan, np.inf):
        with pytest.raises(fo.OracleError) as err:
            fo.topk(np.array([0.1, bad, 0.3], np.float32), 1)
        assert err.value.status == 4
    # a one-element sort compares nothing, so no error
    assert list(fo.topk(np.array([np.nan], np.float32), 1)) == [0]
    with pytest.raises(fo.OracleError) as err:
        fo.topk(s, 6)
    assert err.value.status == 1  # INVALID_ARGUMENT


def test_topk_brute_force_all_small_orders():
    vals = np.array([0.25, 0.5, 0.5, 0.125], np.float32)
    for perm in itertools.permutations(range(4)):
        s = vals[list(perm)]
        order = sorted(range(4), key=lambda i: (-s[i], i))
        for k in range(5):
            assert list(fo.topk(s, k)) == order[:k]


def test_route_weights_renormalise_in_rank_order():
    lw = wl.make_layer(64, 128, 6, 3, wl.F32, 9)
    hl = host_layer(lw)
    x = wl.inputs(64, 1, 10)[0]
    h, logits, probs, ids, w = hl.route(x)
    assert np.array_equal(h, fo.rmsnorm(x, lw.norm_weight, lw.rms_eps))
    assert np.array_equal(probs, fo.softmax(logits))
    assert list(ids) == list(fo.topk(probs, 3))
    total = np.float32(0)
    for i in ids:
        total = np.float32(total + probs[i])
    den = max(float(total), 6.103515625e-5)
    assert np.array_equal(w, np.array([np.float32(float(probs[i]) / den) for i in ids]))


def test_swiglu_and_combine_closed_form():
    # one expert, top-1, weights_norm: w = 1 exactly, so out = x + down(act)
    lw = wl.make_layer(64, 128, 1, 1, wl.F32, 4)
    hl = host_layer(lw)
    x = wl.inputs(64, 1, 5)[0]
    out, ids, w, h, act = hl.forward(x)
    assert list(ids) == [0] and w[0] == np.float32(1.0)
    g = fo.gemv(0, lw.gate[0], h, 128, 64)
    u = fo.gemv(0, lw.up[0], h, 128, 64)
    want_act = np.array([np.float32(np.float32(float(a) / (1.0 + math.exp(-float(a)))) * b) for a, b in zip(g, u)])
    assert np.array_equal(act[0], want_act)
    d = fo.gemv(0, lw.down[0], want_act, 64, 128)
    assert np.array_equal(out, (x + (np.float32(0) + np.float32(1) * d)).astype(np.float32))


def test_bucket_inverts_routing_table():
    rng = np.random.default_rng(2)
    for T, K, E in [(0, 2, 4), (1, 1, 1), (50, 2, 8), (300, 8, 128), (1100, 4, 16)]:
        ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.uint32) if T else \
            np.zeros((0, K), np.uint32)
        off, tl, rl = fo.bucket(ids, E)
        assert off[0] == 0 and off[-1] == T * K
        for e in range(E):
            want = [(t, r) for t in range(T) for r in range(K) if ids[t, r] == e]
            got = list(zip(tl[off[e]:off[e + 1]], rl[off[e]:off[e + 1]]))
            assert got == want


def test_rmsnorm_in_order_at_rounding_near_ties():
    """Tokens crafted so one RMSNorm output lies within 2e-15 (relative) of a
    float midpoint: the oracle keeps the in-order double sum there, and a
    pairwise sum of the same squares rounds at least one of them the other
    way, so these tokens tell the two orders apart."""
    import near_ties as nt
    lw = wl.make_layer(4096, 256, 8, 2, wl.Q4_0, 21)
    X = wl.inputs(4096, 3, 22) * np.float32(2.5)
    flips = 0
    for t in range(3):
        x, k, d = nt.craft(X[t], lw.norm_weight, lw.rms_eps)
        assert d < 2e-15
        yd = nt.in_order_rmsnorm_double(x, lw.norm_weight, lw.rms_eps)
        got = fo.rmsnorm(x, lw.norm_weight, lw.rms_eps)
        assert np.array_equal(got, yd.astype(np.float32))
        x64 = x.astype(np.float64)
        sp = 1.0 / np.sqrt(np.sum(x64 * x64) / x.size + lw.rms_eps)
        flips += np.float32((x64[k] * sp) * np.float64(lw.norm_weight[k])) != got[k]
    assert flips >= 1
