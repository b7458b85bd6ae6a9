"""MoE layers loaded from GGUF checkpoints (freemoe_amd.gguf.moe_layer: the
experts' raw rows, the router bias and the routing options read where the
reference's adapters place them) into HBM slots, decoded and prefilled on the
GPU against the oracle on the arrays the files were written from, and chained
through the engine-pin checkpoints against FreeMoe's compiled fm::Engine."""
from pathlib import Path

import numpy as np
import pytest

from freemoe_amd import gguf
from freemoe_amd import workloads as wl
from freemoe_amd.device import DeviceLayer
from golden import engine_models as em
from test_gpu_moe import check_layer
from test_gpu_prefill import check_prefill

pytestmark = pytest.mark.gpu


def test_native_checkpoint_layers(gpu, tmp_path):
    m = em.build("q4_k_router_q8_0_top4")
    em.write(m, tmp_path / "m.gguf")
    r = gguf.read(tmp_path / "m.gguf")
    for li in range(len(m.layers)):
        lw = gguf.moe_layer(r, li)
        x = wl.inputs(lw.hidden, 8, 500 + li)
        assert check_layer(gpu, lw, x) == 0
        check_prefill(gpu, lw, x)


def test_llama_layout_mixed_types(gpu, tmp_path):
    """A Mixtral-style llama-family file with Q4_K gate/up, Q8_0 down and a
    Q8_0 router, its MoE tensors holding real data."""
    H, F, E, K = 512, 256, 8, 2
    src = wl.make_layer(H, F, E, K, wl.Q4_K, 77, down_type=wl.Q8_0, router_type=wl.Q8_0)
    data = {
        "blk.0.ffn_norm.weight": src.norm_weight.view(np.uint8),
        "blk.0.ffn_gate_inp.weight": src.router_bytes,
        "blk.0.ffn_gate_exps.weight": gguf.stacked(src.gate),
        "blk.0.ffn_up_exps.weight": gguf.stacked(src.up),
        "blk.0.ffn_down_exps.weight": gguf.stacked(src.down),
    }
    g = gguf.mixtral_llama(hidden=H, ffn=F, layers=1, heads=8, kv_heads=8, experts=E, top_k=K, vocab=512,
                           expert_type=wl.Q4_K, down_type=wl.Q8_0, router_type=wl.Q8_0, data=data)
    g.write(tmp_path / "mix.gguf", sparse=True)
    lw = gguf.moe_layer(gguf.read(tmp_path / "mix.gguf"), 0)
    assert (lw.gate_type, lw.down_type, lw.router_type, lw.weights_norm) == (wl.Q4_K, wl.Q8_0, wl.Q8_0, True)
    x = wl.inputs(H, 12, 78)
    assert check_layer(gpu, lw, x) == 0
    check_prefill(gpu, lw, x)


GOLDEN = Path(__file__).resolve().parent / "golden" / "engine_goldens.npz"


@pytest.mark.parametrize("name", em.ALL_CASES)
def test_gpu_layers_reproduce_the_engine(gpu, tmp_path, name):
    """Every engine-pin checkpoint (native, and llama-family files with a
    router-logit bias, expert_weights_norm on / off / absent,
    expert_weights_scale and deepseek41's additive epsilon) read back by
    gguf.moe_layer into HBM; the engine's token chain run with the GPU's
    decode as every MoE layer (the oracle only looks up embeddings and runs
    the final norm and F32 head): prompt logits, routing record and greedy
    ids bit for bit against what FreeMoe's compiled fm::Engine produced.
    Then each layer's inputs of all prompts go through the batched prefill at
    once: ids and weights bit for bit against the decode, the FFN
    contribution within 2e-2 relative."""
    import torch
    goldens = np.load(GOLDEN)
    m = em.build(name)
    em.write(m, tmp_path / "m.gguf")
    r = gguf.read(tmp_path / "m.gguf")
    dls = []
    for li, lw in enumerate(m.layers):
        got = gguf.moe_layer(r, li)
        assert (got.weights_norm, got.weights_scale, got.epsilon_additive) == \
            (lw.weights_norm, lw.weights_scale, lw.epsilon_additive)
        dls.append(DeviceLayer(got, gpu))
    seen = [[] for _ in dls]

    def gpu_layer(li, x):
        seen[li].append(np.array(x, np.float32))
        out, ids, _ = dls[li].decode(torch.from_numpy(np.array(x, np.float32)[None]).to(gpu))
        torch.cuda.synchronize()
        assert dls[li].status() == 0
        return out.cpu().numpy()[0], ids.cpu().numpy()[0].astype(np.uint32)

    for i, p in enumerate(em.prompts(name)):
        g = lambda k: goldens[f"{name}/{i}/{k}"]
        given = g("input_ids") if m.family == "llama" else None
        ids, logits, gen, routing = em.oracle_run_prompt(m, p, em.GENERATE, input_ids=given, layer_fn=gpu_layer)
        assert np.array_equal(ids, g("input_ids")), (name, i)
        assert np.array_equal(routing, g("routing")), (name, i, "routing")
        assert np.array_equal(logits.view(np.uint32), g("logits").view(np.uint32)), (name, i, "logits")
        assert np.array_equal(gen, g("generated")), (name, i, "generated")

    for li, dl in enumerate(dls):
        x = torch.from_numpy(np.stack(seen[li])).to(gpu)
        d_out, d_ids, d_w = dl.decode(x)
        p_out, p_ids, p_w = dl.prefill(x)
        torch.cuda.synchronize()
        assert dl.prefill_status() == 0
        assert torch.equal(p_ids, d_ids) and torch.equal(p_w.view(torch.int32), d_w.view(torch.int32))
        ffn_d = (d_out - x).double()
        err = float(((p_out - x).double() - ffn_d).norm() / ffn_d.norm())
        assert err < 2e-2, (name, li, err)


FIXTURE_DIR = Path(__file__).resolve().parent / "golden" / "freemoe_reference"


@pytest.mark.parametrize("name", ["quant-moe-q6_k", "quant-expert-fused", "quant-expert-separate",
                                  "quant-moe-q4_k"])
def test_reference_fixture_layers(gpu, name):
    """FreeMoe's own Q6_K and mixed Q4_K / Q6_K (separate and fused gate_up)
    checkpoints read by gguf.moe_layer: decode bit for bit and prefill within
    tolerance against the oracle."""
    r = gguf.read(FIXTURE_DIR / f"{name}.gguf")
    lw = gguf.moe_layer(r, 0)
    x = wl.inputs(lw.hidden, 10, 600)
    assert check_layer(gpu, lw, x) == 0
    check_prefill(gpu, lw, x)
