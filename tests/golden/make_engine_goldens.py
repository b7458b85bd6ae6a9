"""Writes engine_goldens.npz: the reference's whole fm::Engine (compiled from
the FreeMoe sources into oracle/_ref/libfmref.so by oracle/Makefile) run on the
checkpoints of engine_models.py, CPU backend, AVX2 kernels, one token at a
time.

    python tests/golden/make_engine_goldens.py

Stored per case: the checkpoint's SHA-256 (the weights are regenerated from
seeds, so a drifting generator is caught instead of silently re-pinned) and,
per prompt, the engine's input ids, prompt logits, greedy ids and routing
record.
"""
from __future__ import annotations

import sys
import tempfile
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))

import engine_models as em  # noqa: E402
import fmoracle as fo  # noqa: E402

OUT = HERE / "engine_goldens.npz"


def engine_outputs(name: str, path: Path) -> dict:
    m = em.build(name)
    sha = em.write(m, path)
    eng = fo.RefEngine(path, isa=fo.ISA_AVX2, threads=1, top_k=m.top_k)
    out = {f"{name}/sha256": np.frombuffer(bytes.fromhex(sha), np.uint8)}
    try:
        for i, p in enumerate(em.prompts(name)):
            ids, logits, gen, routing = eng.run_prompt(p, em.GENERATE)
            out[f"{name}/{i}/input_ids"] = ids
            out[f"{name}/{i}/logits"] = logits
            out[f"{name}/{i}/generated"] = gen
            out[f"{name}/{i}/routing"] = routing
    finally:
        eng.close()
    return out


def main() -> None:
    if not fo.ref_available():
        raise SystemExit("oracle/_ref/libfmref.so is not built (make -C oracle ref, with the FreeMoe tree)")
    data = {}
    with tempfile.TemporaryDirectory() as d:
        for name in em.ALL_CASES:
            data.update(engine_outputs(name, Path(d) / f"{name}.gguf"))
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({len(data)} arrays)")


if __name__ == "__main__":
    main()
