"""Seeded synthetic MoE layers and inputs in raw GGUF block layout.

Shapes are the benchmark and test workloads of this path:

  tiny           hidden 64, ffn 128, 4 experts, top-2, F32 weights ~N(0, 0.02)
                 (the freemoe-tiny-v1 MoE block shape)
  mixtral-q4_0   hidden 4096, ffn 14336, 8 experts, top-2, Q4_0 experts,
                 decode at batch 1 (1000 tokens, one at a time)
  mixtral-q8_0   same layer with Q8_0 experts, prefill of 512 tokens
  finegrained    hidden 2048, ffn 768, 128 experts, top-8, Q4_K experts,
                 2048 tokens, Zipf(s=1.2) router bias

Weights: block scales d = f16(|N(0, 0.01)|) (Q4_K: d and dmin); Q4_0 nibbles
and Q4_K nibbles / 6-bit scale codes uniform; Q8_0 quants uniform in
-127..127. The F32 router is N(0, 1/hidden) so logits are ~N(0, 1); RMSNorm
gains are 1 + N(0, 0.02). Inputs x ~ N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14
GEOMETRY = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}
TYPE_NAMES = {F32: "f32", Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q6_K: "q6_k"}


def row_bytes(type_id: int, cols: int) -> int:
    bs, bb = GEOMETRY[type_id]
    if cols % bs:
        raise ValueError(f"{cols} columns is not a whole number of {TYPE_NAMES[type_id]} blocks")
    return cols // bs * bb


def _half_scales(rng: np.random.Generator, n: int, sigma: float) -> np.ndarray:
    return np.abs(rng.standard_normal(n) * sigma).astype(np.float16).view(np.uint8).reshape(n, 2)


def matrix(type_id: int, rng: np.random.Generator, rows: int, cols: int, sigma: float = 0.01,
           f32_sigma: float = 0.02) -> np.ndarray:
    """A [rows x cols] weight matrix as raw GGUF bytes, shape (rows, row_bytes)."""
    if type_id == F32:
        return (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(f32_sigma)).view(np.uint8)
    bs, bb = GEOMETRY[type_id]
    nb = rows * (cols // bs)
    if type_id == Q8_0:
        w = np.empty((nb, bb), np.uint8)
        w[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    else:
        w = np.frombuffer(rng.bytes(nb * bb), np.uint8).reshape(nb, bb).copy()
    if type_id == Q6_K:
        # ql, qh and the 16 int8 sub-block scales uniform; f16 d last
        w[:, 208:210] = _half_scales(rng, nb, sigma)
        return w.reshape(rows, -1)
    w[:, 0:2] = _half_scales(rng, nb, sigma)
    if type_id == Q4_K:
        w[:, 2:4] = _half_scales(rng, nb, sigma)
    return w.reshape(rows, -1)


@dataclass
class LayerWeights:
    hidden: int
    ffn: int
    experts: int
    top_k: int
    gate_type: int
    norm_weight: np.ndarray
    router: np.ndarray                 # F32 [experts x hidden]
    gate: list                         # per expert raw [ffn x row_bytes(hidden)]
    up: list
    down: list                         # per expert raw [hidden x row_bytes(ffn)]
    router_bias: np.ndarray | None = None
    rms_eps: float = float(np.float32(1e-5))
    weights_norm: bool = True
    seed: int = 0
    notes: dict = field(default_factory=dict)
    down_type: int | None = None       # None: gate_type
    router_type: int = F32             # the router's block type (raw rows in `router_raw`)
    router_raw: np.ndarray | None = None
    norm_bias: float = 0.0             # 1.0 for zero-centred norm gains
    epsilon_additive: bool = False     # expert_weights_epsilon_additive
    weights_epsilon: float = 6.103515625e-5
    weights_scale: float = 1.0

    def __post_init__(self):
        if self.down_type is None:
            self.down_type = self.gate_type

    @property
    def up_type(self):
        return self.gate_type

    @property
    def router_bytes(self) -> np.ndarray:
        """The router as raw GGUF rows [experts x row_bytes(hidden)]."""
        if self.router_type == F32:
            return np.ascontiguousarray(self.router).view(np.uint8)
        return self.router_raw


def make_layer(hidden: int, ffn: int, experts: int, top_k: int, type_id: int, seed: int,
               zipf_s: float | None = None, down_type: int | None = None,
               router_type: int = F32) -> LayerWeights:
    """A seeded layer; gate/up in `type_id`, down in `down_type` (default the
    same). A block-type router holds rows of quants uniform as the experts'
    with scales f16(|N(0, 1/hidden)|), so that logits keep a unit scale."""
    rng = np.random.default_rng(seed)
    norm = (1.0 + rng.standard_normal(hidden) * 0.02).astype(np.float32)
    router = (rng.standard_normal((experts, hidden)) / np.sqrt(hidden)).astype(np.float32)
    bias = None
    notes = {}
    if zipf_s is not None:
        ranks = rng.permutation(experts) + 1
        bias = (-zipf_s * np.log(ranks)).astype(np.float32)
        notes["router_bias"] = f"-{zipf_s}*ln(rank), ranks a seeded permutation of 1..{experts}"
    dt = type_id if down_type is None else down_type
    gate, up, down = [], [], []
    for _ in range(experts):
        gate.append(matrix(type_id, rng, ffn, hidden))
        up.append(matrix(type_id, rng, ffn, hidden))
        down.append(matrix(dt, rng, hidden, ffn))
    router_raw = None
    if router_type != F32:
        router_raw = matrix(router_type, np.random.default_rng(seed + 7919), experts, hidden,
                            sigma=float(1.0 / hidden))
    return LayerWeights(hidden, ffn, experts, top_k, type_id, norm, router, gate, up, down, bias,
                        seed=seed, notes=notes, down_type=dt, router_type=router_type,
                        router_raw=router_raw)


def inputs(hidden: int, tokens: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((tokens, hidden), dtype=np.float32)


WORKLOADS = {
    "tiny": dict(hidden=64, ffn=128, experts=4, top_k=2, type_id=F32, tokens=64),
    "mixtral-q4_0": dict(hidden=4096, ffn=14336, experts=8, top_k=2, type_id=Q4_0, tokens=1000),
    "mixtral-q8_0": dict(hidden=4096, ffn=14336, experts=8, top_k=2, type_id=Q8_0, tokens=512),
    "finegrained": dict(hidden=2048, ffn=768, experts=128, top_k=8, type_id=Q4_K, tokens=2048, zipf_s=1.2),
}


def workload(name: str, seed: int = 1234):
    """(LayerWeights, x[tokens x hidden]) of a named workload."""
    w = dict(WORKLOADS[name])
    tokens = w.pop("tokens")
    layer = make_layer(seed=seed, **w)
    return layer, inputs(layer.hidden, tokens, seed + 1)


def tiny_checkpoint(seed: int = 2026):
    """The freemoe-tiny-v1 end-to-end model as a GGUF file object
    (freemoe_amd.gguf): 2 layers, hidden 64, 4 heads of dim 16, 4 experts with
    top-2 routing, expert ffn 128, the 258-entry byte vocabulary, F32 weight
    matrices ~N(0, 0.02) (norm gains 1 + N(0, 0.02)), seeded."""
    from . import gguf

    H, F, E, K, L = 64, 128, 4, 2, 2
    rng = np.random.default_rng(seed)

    def n(*shape):
        return (rng.standard_normal(shape) * 0.02).astype(np.float32)

    def gain():
        return (1.0 + rng.standard_normal(H) * 0.02).astype(np.float32)

    layers = []
    for _ in range(L):
        router = n(E, H)
        gate = [n(F, H) for _ in range(E)]
        up = [n(F, H) for _ in range(E)]
        down = [n(H, F) for _ in range(E)]
        layers.append(dict(attn_norm=gain(), attn_q=n(H, H), attn_k=n(H, H), attn_v=n(H, H), attn_output=n(H, H),
                           ffn_norm=gain(), moe=gguf.MoEBlock(router, F32, gate, up, down, F32, F32)))
    vocab = dict(token_embd=n(258, H), output_norm=gain(), output=n(258, H))
    return gguf.freemoe_tiny(hidden=H, ffn=F, heads=4, experts=E, top_k=K, layers=layers, vocab_tensors=vocab,
                             seed=seed, name="freemoe-tiny-v1 synthetic")
