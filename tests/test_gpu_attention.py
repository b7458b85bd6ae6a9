"""fmx_attention_decode against a NumPy restatement of FreeMoe's decode
attention loop (engine.cpp:1360-1420, engine.cpp:378-393 softmax): per head,
scores float(double dot * scale) with the dot summed in index order, the
float maximum, double exponentials summed in position order,
p = float(e / sum), values summed in double in position order. The sums are
restated with np.add.accumulate (sequential, in order). Both sides use their
own exp (the device's and NumPy's, each within an ulp), so results are
compared within 1e-6 relative and most elements are expected bit for bit."""
import numpy as np
import pytest

from freemoe_amd import fmx

pytestmark = pytest.mark.gpu


def reference(q, kv, kv_heads, head_dim, v_offset, scale):
    heads = q.shape[0] // head_dim
    group = heads // kv_heads
    P = kv.shape[0]
    out = np.empty(heads * head_dim, np.float32)
    for h in range(heads):
        kvh = h // group
        qd = q[h * head_dim:(h + 1) * head_dim].astype(np.float64)
        k = kv[:, kvh * head_dim:(kvh + 1) * head_dim].astype(np.float64)
        dots = np.add.accumulate(k * qd, axis=1)[:, -1]
        s = (dots * scale).astype(np.float32)
        m = np.float64(s.max())
        e = np.exp(s.astype(np.float64) - m)
        total = np.add.accumulate(e)[-1]
        p = (e / total).astype(np.float32)
        v = kv[:, v_offset + kvh * head_dim:v_offset + (kvh + 1) * head_dim].astype(np.float64)
        acc = np.add.accumulate(p.astype(np.float64)[:, None] * v, axis=0)[-1]
        out[h * head_dim:(h + 1) * head_dim] = acc.astype(np.float32)
    return out


CASES = {
    # name: (heads, kv_heads, head_dim, positions, row padding floats)
    "one_position": (4, 4, 64, 1, 0),
    "mha_32x128_513": (32, 32, 128, 513, 0),
    "gqa_8_of_2_300": (8, 2, 64, 300, 8),
    "long_4000": (4, 4, 128, 4000, 0),
}


@pytest.mark.parametrize("name", list(CASES))
def test_attention_decode_vs_engine_restatement(gpu, name):
    import torch
    heads, kvh, D, P, pad = CASES[name]
    rng = np.random.default_rng(hash(name) & 0xFFFF)
    kv_dim = kvh * D
    stride = 2 * kv_dim + pad
    kv = (rng.standard_normal((P, stride)) * 0.5).astype(np.float32)
    q = (rng.standard_normal(heads * D) * 0.5).astype(np.float32)
    scale = 1.0 / np.sqrt(float(D))
    want = reference(q, kv, kvh, D, kv_dim, scale)
    qd = torch.from_numpy(q).to(gpu)
    kvd = torch.from_numpy(kv).to(gpu)
    out = torch.empty(heads * D, dtype=torch.float32, device=gpu)
    ws = torch.zeros(256, dtype=torch.uint8, device=gpu)
    fmx.call("fmx_attention_decode", qd.data_ptr(), kvd.data_ptr(), stride, kv_dim, heads, kvh, D, P, scale,
             out.data_ptr(), ws.data_ptr(), 256, fmx.stream_handle())
    torch.cuda.synchronize()
    assert fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle()) == 0
    got = out.cpu().numpy()
    err = np.abs(got.astype(np.float64) - want) / np.maximum(np.abs(want).max(), 1e-30)
    assert err.max() <= 1e-6, err.max()
    same = np.mean(got.view(np.uint32) == want.view(np.uint32))
    print(f"{name}: {same:.4%} of outputs bit for bit")
    assert same >= 0.9


def test_attention_decode_reports_nonfinite_scores(gpu):
    import torch
    heads, kvh, D, P = 2, 2, 32, 5
    kv = np.zeros((P, 2 * kvh * D), np.float32)
    kv[3, 0] = np.inf
    q = np.ones(heads * D, np.float32)
    qd, kvd = torch.from_numpy(q).to(gpu), torch.from_numpy(kv).to(gpu)
    out = torch.empty(heads * D, dtype=torch.float32, device=gpu)
    ws = torch.zeros(256, dtype=torch.uint8, device=gpu)
    fmx.call("fmx_attention_decode", qd.data_ptr(), kvd.data_ptr(), 2 * kvh * D, kvh * D, heads, kvh, D, P, 0.5,
             out.data_ptr(), ws.data_ptr(), 256, fmx.stream_handle())
    assert fmx.lib().fmx_moe_status(ws.data_ptr(), fmx.stream_handle()) == 4  # FMX_ERR_INTERNAL
