"""FreeMoe's unchanged fm::Engine with the physical-GPU backend kind served by
fm::HipBackend (oracle/_ref/engine_check, built from tests/engine_check.cpp,
the adapter, FreeMoe's sources and libfmx.so).

  * compare_reference on FreeMoe's own MoE fixture (tests/golden/
    freemoe_reference: moe-fm.gguf, 20 prompts with their logits, greedy ids and
    routing records, copied as data): every prompt within the reference's 5e-3,
    every greedy id and every routing event equal;
  * compare_reference on FreeMoe's dense fixture (dense-fm.gguf, 20 prompts):
    its prompts take the engine's batched prefill, whose projections are
    gemm_quant calls, so on HipBackend they run fmx_gemm_quant;
  * FreeMoe's block-type conformance checkpoints (quant-moe-*.gguf, every
    matrix including the router in one block type; the run of tests.cpp:
    1424-1468) on the CPU backend and on HipBackend in one process, the
    quantised projections on the device: logits bit for bit, ids equal;
  * the 8-layer Mixtral-shaped decoder (hidden 4096, Q4_0 experts, F32
    attention, written at test time): CPU and HipBackend engines bit for bit;
  * the freemoe-tiny-v1 end-to-end model (2 layers, hidden 64, 4 experts top-2,
    ffn 128, F32 ~N(0, 0.02)), 64-token seeded byte prompts and 32 greedy
    tokens, on the CPU backend and on HipBackend in one process: prompt logits
    identical bit for bit, routing records and greedy ids identical.
"""
import json
import subprocess
from pathlib import Path

import pytest

from freemoe_amd import workloads as wl

ROOT = Path(__file__).resolve().parents[1]
CHECK = ROOT / "oracle" / "_ref" / "engine_check"
FUSED = ROOT / "oracle" / "_ref" / "engine_check_fused"
FIXTURES = ROOT / "tests" / "golden" / "freemoe_reference"
DEVICE_LABELS = {"hip-gfx950", "scalar-control", "cpu-quant", "cpu-batched"}


def run(*args, timeout=600, binary=CHECK):
    if not binary.exists():
        pytest.skip(f"oracle/_ref/{binary.name} not built (needs the FreeMoe tree at build time)")
    proc = subprocess.run([str(binary), *map(str, args)], capture_output=True, text=True, timeout=timeout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return json.loads(proc.stdout.strip().splitlines()[-1])


def check_device_accounting(ops, fused=False):
    """Every projection of a GPU-backend engine ran on the device. The
    unchanged engine logs each block-type projection itself under
    "cpu-quant" (engine.cpp:363-366) and each batched product under
    "cpu-batched" (2016-2022), and the renamed call logs it again under
    HipBackend's label: the counts must be equal. No F32 product ran under a
    CPU kernel's label, and no renamed call fell back to FreeMoe's CPU kernel
    in a process without a CPU engine (that would also have raised). With
    the integration's edits the engine calls the backend itself: there are
    no cpu-* records at all."""
    labels = {k for k in ops if k not in ("hooked", "quant_records", "batch_records", "fused_layers", "fallbacks",
                                          "device_attention")}
    assert labels <= DEVICE_LABELS, labels
    assert ops["hooked"].get("gemv_quant", 0) == ops["quant_records"], ops
    assert ops["hooked"].get("gemm_quant", 0) == ops["batch_records"], ops
    if fused:
        assert ops["quant_records"] == 0 and ops["batch_records"] == 0 and not ops["hooked"], ops
        assert "cpu-quant" not in ops and "cpu-batched" not in ops, ops


def check_compare(r, prompts):
    assert r["prompts"] == prompts
    assert r["within_tolerance"] == prompts and r["token_match"] == prompts and r["routing_match"] == prompts, r
    assert r["matching_tokens"] == r["reference_tokens"] > 0


def test_unchanged_engine_compare_reference_cpu():
    """The same binary on FreeMoe's CPU backend reproduces FreeMoe's goldens
    (the baseline the GPU run is held to)."""
    r = run("compare", FIXTURES / "moe-fm.gguf", FIXTURES, 20, 16, "cpu")
    check_compare(r, 20)


@pytest.mark.gpu
def test_unchanged_engine_compare_reference_on_hip_backend(gpu):
    r = run("compare", FIXTURES / "moe-fm.gguf", FIXTURES, 20, 16, "gpu")
    print(r)
    assert r["backend"] == "hip-gfx950"
    check_compare(r, 20)
    assert r["ops"].get("hip-gfx950", 0) > 0  # the projections ran on the device
    check_device_accounting(r["ops"])
    assert r["ops"]["fallbacks"] == 0


def test_unchanged_engine_dense_compare_reference_cpu():
    """The dense fixture's goldens on FreeMoe's CPU backend (batched prefill)."""
    r = run("compare", FIXTURES / "dense-fm.gguf", FIXTURES, 20, 16, "cpu")
    check_compare(r, 20)
    assert r["ops"].get("cpu-batched", 0) > 0


@pytest.mark.gpu
def test_unchanged_engine_dense_compare_reference_on_hip_backend(gpu):
    """The dense fixture's goldens on HipBackend: the batched prefill's
    projections run fmx_gemm_quant, decode runs fmx_matvec."""
    r = run("compare", FIXTURES / "dense-fm.gguf", FIXTURES, 20, 16, "gpu")
    print(r)
    assert r["backend"] == "hip-gfx950"
    check_compare(r, 20)
    assert r["ops"].get("hip-gfx950", 0) > 0
    assert r["ops"]["hooked"].get("gemm_quant", 0) > 0  # the batched projections ran on the device
    check_device_accounting(r["ops"])
    assert r["ops"]["fallbacks"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["quant-moe-q8_0", "quant-moe-q4_0", "quant-moe-q4_k", "quant-moe-q6_k",
                                     "quant-expert-fused", "quant-expert-separate"])
def test_quantised_checkpoint_conformance_on_hip_backend(gpu, variant):
    """FreeMoe's block-type checkpoints through the unchanged engine:
    quant-moe-<type> (router, attention and experts in one block type) and
    quant-expert-{fused,separate} (Q4_K gate/up with Q6_K down experts, the
    mixed-type case of tests.cpp:1479-1544). HipBackend runs every quantised
    projection, and its prompt logits and greedy ids equal the CPU backend's
    bit for bit (the reference's own tests hold the CPU run to the F32 twin
    within 1e-4)."""
    text = "mixed experts" if variant.startswith("quant-expert") else "quantised conformance"
    r = run("prompt", FIXTURES / f"{variant}.gguf", 6, text)
    print(r)
    assert r["backends"] == ["cpu", "hip-gfx950"]
    assert r["logits"] > 0 and r["differing_logits"] == 0 and r["max_abs_diff"] == 0.0
    assert r["ids_identical"] and r["routing_identical"] and r["generated"] == 6
    assert r["gpu_ops"].get("hip-gfx950", 0) > 0
    assert r["gpu_ops"]["hooked"].get("gemv_quant", 0) > 0  # the quantised projections ran on the device
    check_device_accounting(r["gpu_ops"])


@pytest.mark.gpu
def test_tiny_model_end_to_end_cpu_and_hip_identical(gpu, tmp_path):
    path = tmp_path / "freemoe-tiny-v1.gguf"
    wl.tiny_checkpoint().write(path)
    r = run("twin", path, 4, 64, 32, 7)
    print(r)
    assert r["backends"] == ["cpu", "hip-gfx950"]
    assert r["differing_logits"] == 0 and r["max_abs_diff"] == 0.0
    assert r["routing_identical"] and r["ids_identical"]
    assert r["generated"] == 4 * 32 and r["routing_events"] == 4 * (65 + 32) * 2
    assert r["gpu_ops"].get("hip-gfx950", 0) > 0
    check_device_accounting(r["gpu_ops"])


@pytest.mark.gpu
def test_residency_refills_slots_through_hip_backend(gpu):
    """Two expert slots for moe-fm's 16 experts (2 layers x 8): residency
    refills slots through HipBackend (upload into the pinned mirror and the
    HBM twin, the event fence, the FNV-1a read-back, residency.cpp:617-723) on
    nearly every routed expert, and every prompt still matches FreeMoe's
    goldens."""
    r = run("residency", FIXTURES / "moe-fm.gguf", FIXTURES, 20, 16, 2)
    print(r)
    assert r["backend"] == "hip-gfx950" and r["slots"] == 2
    check_compare(r | {"matching_tokens": 1, "reference_tokens": 1}, 20)
    assert r["evictions"] > 100 and r["cache_misses"] > 100
    assert r["checksum_checks"] >= 2 * r["cache_misses"] and r["checksum_failures"] == 0
    assert r["transfer_failures"] == 0 and r["fence_timeouts"] == 0
    assert r["experts_executed"] == r["selected_experts"]


@pytest.fixture(scope="module")
def decoder_path(tmp_path_factory):
    """The 8-layer Mixtral-shaped decoder (engine_models.write_decoder: hidden
    4096, 32 heads of 128, ffn 14336, 8 experts top-2, Q4_0 experts, F32
    attention, seed 5; about 8.5 GB), written once for this module's tests
    and removed after them."""
    import shutil
    import sys
    import time

    sys.path.insert(0, str(ROOT / "tests" / "golden"))
    import engine_models as em

    need = 12 << 30
    tmp = tmp_path_factory.mktemp("decoder")
    base = next((d for d in (Path("/dev/shm"), tmp) if d.exists() and shutil.disk_usage(d).free > need), None)
    if base is None:
        pytest.skip("no 12 GiB of scratch space for the 8.5 GB checkpoint")
    path = base / f"fmx-decoder-{id(tmp)}.gguf"
    t0 = time.time()
    size = em.write_decoder(path)
    print(f"[decoder] checkpoint {size / 1e9:.2f} GB in {time.time() - t0:.0f}s", file=sys.__stderr__, flush=True)
    try:
        yield path
    finally:
        path.unlink(missing_ok=True)


@pytest.mark.gpu
def test_eight_layer_decoder_cpu_and_hip_identical(gpu, decoder_path):
    """The 8-layer decoder through the unchanged engine on the CPU backend and
    on HipBackend in one process (12 prompt bytes, 8 greedy tokens; the full
    256 + 256 run is the golden replay below), every expert resident: prompt
    logits bit for bit, routing records and greedy ids identical. The
    attention projections run as fmx_matvec F32, the experts and router as
    the engine's gemv_quant calls on the device."""
    r = run("twin", decoder_path, 1, 12, 8, 9, 24, 64, timeout=900)
    print(r)
    assert r["backends"] == ["cpu", "hip-gfx950"]
    assert r["logits"] > 0 and r["differing_logits"] == 0 and r["max_abs_diff"] == 0.0
    assert r["routing_identical"] and r["ids_identical"] and r["generated"] >= 1
    assert r["routing_events"] >= (12 + 1) * 8
    assert r["gpu_ops"].get("hip-gfx950", 0) > 0 and r["gpu_ops"]["hooked"].get("gemv_quant", 0) > 0
    check_device_accounting(r["gpu_ops"])


DECODER_GOLDEN = ROOT / "tests" / "golden" / "decoder_256_256.fmxg"


@pytest.mark.gpu
def test_eight_layer_decoder_256_256_fused_against_cpu_engine(gpu, decoder_path):
    """The 8-layer decoder at its stated size, 256 random prompt bytes then
    256 greedy tokens, through FreeMoe's engine with the integration's edits
    on HipBackend: every MoE block runs as one fmx_moe_decode
    (Backend::moe_layer), every token's attention as one
    fmx_attention_decode per layer over the cache rows mirrored to HBM
    (Backend::attention), the F32 attention and head projections as
    fmx_matvec. Against what FreeMoe's CPU engine produced for the same
    checkpoint and prompt (tests/golden/decoder_256_256.fmxg, made by
    tests/golden/make_decoder_golden.py; the JSON beside it pins the
    checkpoint's SHA-256): every routing record and greedy id equal, prompt
    logits within 1e-4 (the attention's exp is the device's, within an ulp of
    the host libm's, so a last bit may differ; the count is printed)."""
    import hashlib
    import sys

    meta = json.loads(DECODER_GOLDEN.with_suffix(".json").read_text())
    assert decoder_path.stat().st_size == meta["checkpoint_bytes"]
    h = hashlib.sha256()
    with open(decoder_path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    assert h.hexdigest() == meta["checkpoint_sha256"], "the decoder generator drifted from the golden's"
    print("[decoder] checkpoint matches the golden's", file=sys.__stderr__, flush=True)
    r = run("replay", decoder_path, DECODER_GOLDEN, meta["hot_gib"], meta["slots"], timeout=900, binary=FUSED)
    print(r)
    assert r["backend"] == "hip-gfx950"
    assert r["prompt_tokens"] == meta["prompt_len"] + 1
    print(f"[decoder] logits differing in any bit: {r['differing_logits']} of {r['logits']}, "
          f"max abs diff {r['max_abs_diff']}", file=sys.__stderr__, flush=True)
    assert r["logits"] > 0 and r["max_abs_diff"] <= 1e-4
    assert r["routing_identical"] and r["ids_identical"]
    assert r["routing_events"] == (r["prompt_tokens"] + r["generated"] - 1) * 8 or \
        r["routing_events"] == (r["prompt_tokens"] + r["generated"]) * 8
    ops = r["gpu_ops"]
    check_device_accounting(ops, fused=True)
    assert ops["fused_layers"] == r["routing_events"]  # every MoE block ran as one fused layer
    assert ops["device_attention"] == r["routing_events"]  # and every attention on the device


@pytest.mark.gpu
def test_fused_engine_compare_reference_on_hip_backend(gpu):
    """FreeMoe's MoE fixture (20 prompts, goldens) through the engine with the
    integration's edits: every routed block of every token is one
    Backend::moe_layer call (fmx_moe_decode)."""
    r = run("compare", FIXTURES / "moe-fm.gguf", FIXTURES, 20, 16, "gpu", binary=FUSED)
    print(r)
    assert r["backend"] == "hip-gfx950"
    check_compare(r, 20)
    check_device_accounting(r["ops"], fused=True)
    assert r["ops"]["fused_layers"] > 0 and r["ops"]["device_attention"] == r["ops"]["fused_layers"]


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["quant-moe-q8_0", "quant-moe-q4_0", "quant-moe-q4_k", "quant-moe-q6_k",
                                     "quant-expert-fused", "quant-expert-separate"])
def test_fused_engine_quantised_checkpoints(gpu, variant):
    """FreeMoe's block-type checkpoints through the edited engine: the GPU
    engine's routed blocks run fused and its attention on the device, its
    other block-type projections through HipBackend::matvec_quant under the
    engine's own op names; the CPU engine in the same process runs the
    edit's defaults (FreeMoe's kernels and loops). Greedy ids and routing
    equal, prompt logits within 1e-4 (the device attention's exp may move a
    last bit)."""
    text = "mixed experts" if variant.startswith("quant-expert") else "quantised conformance"
    r = run("prompt", FIXTURES / f"{variant}.gguf", 6, text, binary=FUSED)
    print(r)
    assert r["backends"] == ["cpu", "hip-gfx950"]
    assert r["logits"] > 0 and r["max_abs_diff"] <= 1e-4
    assert r["ids_identical"] and r["routing_identical"] and r["generated"] == 6
    check_device_accounting(r["gpu_ops"], fused=True)
    assert r["gpu_ops"]["fused_layers"] == r["routing_events"]
    assert r["gpu_ops"]["device_attention"] > 0


@pytest.mark.gpu
def test_fused_engine_residency_refills(gpu):
    """moe-fm (2 layers x 8 experts) with 8 expert slots: the fused path
    holds all 8 experts of a layer at once, so every layer change refills the
    slots through HipBackend; every prompt still matches FreeMoe's goldens
    and residency's selected / executed counts agree."""
    r = run("residency", FIXTURES / "moe-fm.gguf", FIXTURES, 20, 16, 8, binary=FUSED)
    print(r)
    assert r["backend"] == "hip-gfx950" and r["slots"] == 8
    check_compare(r | {"matching_tokens": 1, "reference_tokens": 1}, 20)
    assert r["evictions"] > 100 and r["checksum_failures"] == 0
    assert r["experts_executed"] == r["selected_experts"]
