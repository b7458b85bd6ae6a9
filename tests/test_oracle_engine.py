"""The oracle against the reference's whole fm::Engine (CPU only).

tests/golden/engine_goldens.npz holds what the compiled engine
(oracle/_ref/libfmref.so, built from the FreeMoe sources) produced on the
seeded freemoe-tiny-v1 checkpoints of tests/golden/engine_models.py, whose
attention output projections are zero. The oracle's chain (RMSNorm, router,
softmax, top-k, weights, experts, SwiGLU, combine, residual, final norm, F32
head, greedy) must reproduce the engine's prompt logits bit for bit, its
routing record and its greedy ids. Planted mistakes in the oracle's inputs
(gate and up swapped, the weights left unnormalised, the additive epsilon)
must break the match, so the goldens discriminate those functions.
"""
import copy
import tempfile
from pathlib import Path

import numpy as np
import pytest

import fmoracle as fo
from golden import engine_models as em

GOLDEN = Path(__file__).resolve().parent / "golden" / "engine_goldens.npz"


@pytest.fixture(scope="module")
def goldens():
    return np.load(GOLDEN)


def sha_of(name: str) -> str:
    with tempfile.TemporaryDirectory() as d:
        return em.write(em.build(name), Path(d) / "m.gguf")


def matches(m, name, goldens, i, prompt):
    ids, logits, gen, routing = em.oracle_run_prompt(m, prompt, em.GENERATE)
    g = lambda k: goldens[f"{name}/{i}/{k}"]
    return (np.array_equal(ids, g("input_ids")), np.array_equal(logits.view(np.uint32), g("logits").view(np.uint32)),
            np.array_equal(gen, g("generated")), np.array_equal(routing, g("routing")))


@pytest.mark.parametrize("name", list(em.CASES))
def test_checkpoint_is_the_pinned_one(goldens, name):
    """The writer regenerates the exact checkpoint the goldens were taken on."""
    assert bytes(goldens[f"{name}/sha256"]).hex() == sha_of(name)


@pytest.mark.parametrize("name", list(em.CASES))
def test_oracle_reproduces_the_compiled_engine(goldens, name):
    m = em.build(name)
    for i, p in enumerate(em.prompts(name)):
        ok = matches(m, name, goldens, i, p)
        assert ok == (True, True, True, True), (name, i, ok)


def test_goldens_cover_ties_between_ranks_and_eos_free_runs(goldens):
    """Every case generates its full GENERATE tokens and routes at least 8
    token-layer pairs per prompt."""
    for name in em.CASES:
        for i in range(len(em.PROMPT_LENGTHS)):
            assert len(goldens[f"{name}/{i}/generated"]) == em.GENERATE
            assert goldens[f"{name}/{i}/routing"].shape[0] >= 8


PLANTED = {
    # SwiGLU on the wrong operand: silu(up) * gate
    "gate_and_up_swapped": lambda lw: lw.__dict__.update(gate=lw.up, up=lw.gate),
    "weights_not_renormalised": lambda lw: setattr(lw, "weights_norm", False),
    "epsilon_added_not_floored": lambda lw: setattr(lw, "epsilon_additive", True),
}


@pytest.mark.parametrize("mistake", list(PLANTED))
def test_planted_oracle_mistakes_break_the_match(goldens, mistake):
    name = "q4_k_router_q8_0_top4"
    m = em.build(name)
    m.layers = [copy.copy(lw) for lw in m.layers]
    for lw in m.layers:
        g, u = lw.gate, lw.up
        PLANTED[mistake](lw)
        assert (lw.gate is u and lw.up is g) or mistake != "gate_and_up_swapped"
    p = em.prompts(name)[3]
    ok = matches(m, name, goldens, 3, p)
    assert not ok[1], f"{mistake}: logits still match"


@pytest.mark.skipif(not fo.ref_available(), reason="oracle/_ref not built (needs the FreeMoe tree at build time)")
@pytest.mark.parametrize("name", list(em.CASES))
def test_live_engine_matches_goldens(goldens, name):
    """The compiled engine, run now, gives the committed goldens."""
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "m.gguf"
        m = em.build(name)
        em.write(m, path)
        eng = fo.RefEngine(path, isa=fo.ISA_AVX2, threads=1, top_k=m.top_k)
        try:
            for i, p in enumerate(em.prompts(name)):
                ids, logits, gen, routing = eng.run_prompt(p, em.GENERATE)
                assert np.array_equal(ids, goldens[f"{name}/{i}/input_ids"])
                assert np.array_equal(logits.view(np.uint32), goldens[f"{name}/{i}/logits"].view(np.uint32))
                assert np.array_equal(gen, goldens[f"{name}/{i}/generated"])
                assert np.array_equal(routing, goldens[f"{name}/{i}/routing"])
        finally:
            eng.close()
