"""Writes decoder_256_256.fmxg: FreeMoe's own fm::Engine (compiled from its
sources, oracle/_ref/engine_check, CPU backend, AVX2 kernels at 2 threads) on
the 8-layer Mixtral-shaped decoder of engine_models.write_decoder (hidden 4096,
32 heads of 128, 8 experts top-2, ffn 14336, Q4_0 experts, F32 attention,
seed 5): one prompt of 256 seeded random bytes (BOS + 256 tokens through the
byte tokenizer), then 256 greedy tokens. The file holds the prompt, the
engine's input ids, prompt logits, generated ids and routing record; the JSON
beside it the checkpoint's SHA-256 and size, so a drifting generator is caught
instead of silently compared.

    python tests/golden/make_decoder_golden.py [scratch directory]

The checkpoint (about 8.5 GB) is written to the scratch directory (default
/dev/shm) and removed afterwards. The CPU run takes several minutes.
"""
from __future__ import annotations

import hashlib
import json
import subprocess
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(HERE))

import engine_models as em  # noqa: E402

OUT = HERE / "decoder_256_256.fmxg"
META = HERE / "decoder_256_256.json"
PROMPT_LEN, GENERATE, PROMPT_SEED = 256, 256, 11
# hot-memory budget (GiB) and expert slots: every expert of the 8 layers resident
HOT_GIB, SLOTS = 24, 64


def sha256_file(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def main() -> None:
    check = ROOT / "oracle" / "_ref" / "engine_check"
    if not check.exists():
        raise SystemExit("oracle/_ref/engine_check is not built (make -C oracle ref, with the FreeMoe tree)")
    scratch = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/dev/shm")
    path = scratch / "fmx-decoder-golden.gguf"
    try:
        t0 = time.time()
        size = em.write_decoder(path)
        sha = sha256_file(path)
        print(f"checkpoint {size / 1e9:.2f} GB, sha256 {sha[:16]}..., {time.time() - t0:.0f}s", flush=True)
        subprocess.run([str(check), "record", str(path), "1", str(PROMPT_LEN), str(GENERATE), str(PROMPT_SEED),
                        str(OUT), str(HOT_GIB), str(SLOTS)], check=True)
        print(f"engine run done at {time.time() - t0:.0f}s", flush=True)
    finally:
        path.unlink(missing_ok=True)
    META.write_text(json.dumps({
        "checkpoint": "engine_models.write_decoder() defaults (8 layers, hidden 4096, ffn 14336, 8 experts "
                      "top-2, 32 heads, Q4_0 experts, F32 attention, seed 5)",
        "checkpoint_sha256": sha, "checkpoint_bytes": size,
        "prompt_len": PROMPT_LEN, "generate": GENERATE, "prompt_seed": PROMPT_SEED,
        "hot_gib": HOT_GIB, "slots": SLOTS,
        "engine": "FreeMoe fm::Engine, CPU backend, KernelIsa::Auto (AVX2+FMA), 2 kernel threads",
    }, indent=1) + "\n")
    print(f"wrote {OUT} and {META}")


if __name__ == "__main__":
    main()
