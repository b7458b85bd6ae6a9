"""MoE layers loaded from GGUF checkpoints (freemoe_amd.gguf.moe_layer: the
experts' raw rows read where the reference's adapters place them) into HBM
slots, decoded and prefilled on the GPU against the oracle on the arrays the
files were written from."""
import numpy as np
import pytest

from freemoe_amd import gguf
from freemoe_amd import workloads as wl
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
