"""Writes ref_kernels.npz and ref_layers.npz from the reference's own kernels.

Run where oracle/_ref/libfmref.so exists (it is compiled from the FreeMoe
sources by oracle/Makefile):

    python tests/golden/make_goldens.py

Every input is regenerated from a seed; layer weights are stored only as a
SHA-256 so a drifting generator is caught instead of silently re-pinned.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path[:0] = [str(ROOT), str(ROOT / "oracle")]

import fmoracle as fo  # noqa: E402
from freemoe_amd import workloads as wl  # noqa: E402

KERNEL_CASES = [  # (type, out_dim, in_dim)
    (0, 37, 512), (0, 5, 24), (0, 5, 40), (0, 3, 4103),
    (2, 37, 512), (2, 11, 96), (2, 6, 4096),
    (8, 37, 512), (8, 11, 96), (8, 6, 4096),
    (12, 37, 512), (12, 6, 2048),
]

LAYER_CASES = {
    # name: (hidden, ffn, experts, top_k, type, tokens, zipf_s)
    "tiny_f32": (64, 128, 4, 2, wl.F32, 32, None),
    "q4_0": (256, 512, 4, 2, wl.Q4_0, 16, None),
    "q8_0": (256, 512, 4, 2, wl.Q8_0, 16, None),
    "q4_k": (512, 256, 8, 4, wl.Q4_K, 16, None),
    "q4_k_zipf": (256, 256, 16, 4, wl.Q4_K, 24, 1.2),
}


def weights_digest(lw: wl.LayerWeights) -> str:
    h = hashlib.sha256()
    for a in [lw.norm_weight, lw.router] + ([lw.router_bias] if lw.router_bias is not None else []):
        h.update(np.ascontiguousarray(a).tobytes())
    for arr in (lw.gate, lw.up, lw.down):
        for m in arr:
            h.update(m.tobytes())
    return h.hexdigest()


host_layer = fo.host_layer


def kernel_inputs(case_index: int, type_id: int, out_dim: int, in_dim: int):
    rng = np.random.default_rng(1000 + case_index)
    w = wl.matrix(type_id, rng, out_dim, in_dim, sigma=0.05, f32_sigma=0.5)
    x = rng.standard_normal(in_dim, dtype=np.float32)
    return w, x


def main() -> None:
    if not fo.ref_available():
        sys.exit("oracle/_ref/libfmref.so is not built")
    out = {}
    for i, (t, o, n) in enumerate(KERNEL_CASES):
        w, x = kernel_inputs(i, t, o, n)
        for isa in (fo.ISA_SCALAR, fo.ISA_AVX2):
            out[f"k{i}_isa{isa}_y"] = fo.ref_gemv(t, w, x, o, n, isa)
        out[f"k{i}_shape"] = np.array([t, o, n])
    np.savez_compressed(HERE / "ref_kernels.npz", **out)

    lay = {}
    for name, (H, F, E, K, t, T, z) in LAYER_CASES.items():
        seed = 77 + len(lay)
        lw = wl.make_layer(H, F, E, K, t, seed, zipf_s=z)
        x = wl.inputs(H, T, seed + 1)
        hl = host_layer(lw)
        o, ids, w = hl.ref_forward_batch(x, fo.ISA_AVX2, threads=1)
        lay[f"{name}_meta"] = np.array([H, F, E, K, t, T, seed, -1 if z is None else int(z * 1000)])
        lay[f"{name}_digest"] = np.frombuffer(bytes.fromhex(weights_digest(lw)), np.uint8)
        lay[f"{name}_out"] = o
        lay[f"{name}_ids"] = ids
        lay[f"{name}_weights"] = w
    np.savez_compressed(HERE / "ref_layers.npz", **lay)
    print("wrote", HERE / "ref_kernels.npz", HERE / "ref_layers.npz")


if __name__ == "__main__":
    main()
