"""Seeded freemoe-tiny-v1 MoE checkpoints for pinning the oracle against the
reference's whole fm::Engine, and the oracle's reproduction of that engine.

Every checkpoint's attention output projections are zero, so the attention
branch adds exactly zero to the residual stream (engine.cpp:1436-1458) and
each MoE block sees the token's embedding row (layer 0) or the previous MoE
block's output. What the engine then computes per token is the oracle's own
chain: RMSNorm (ffn_norm) -> router -> softmax -> stable top-k -> weights ->
experts (gate/up, SwiGLU, down) -> rank-order combine -> residual, per layer,
then RMSNorm (output_norm) and the F32 head (engine.cpp:1825-1827), then
greedy argmax (lowest id on ties) until EOS. The goldens hold the engine's
prompt logits (bit patterns), its routing record and its greedy ids.
"""
from __future__ import annotations

import hashlib
import sys
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (ROOT, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import fmoracle as fo  # noqa: E402
from freemoe_amd import gguf  # noqa: E402
from freemoe_amd import workloads as wl  # noqa: E402

VOCAB, BOS, EOS = 258, 256, 257

CASES = {
    # name: (hidden, ffn, experts, top_k, layers, heads, expert type, router type, seed)
    "f32_two_layers": (64, 128, 4, 2, 2, 4, wl.F32, wl.F32, 11),
    "q4_0_router_q4_0": (256, 256, 8, 2, 1, 4, wl.Q4_0, wl.Q4_0, 12),
    "q8_0_hidden_1024": (1024, 64, 8, 2, 1, 8, wl.Q8_0, wl.F32, 13),
    "q4_k_router_q8_0_top4": (512, 256, 8, 4, 2, 8, wl.Q4_K, wl.Q8_0, 14),
}

PROMPT_LENGTHS = (1, 4, 9, 23)
GENERATE = 6


@dataclass
class Model:
    name: str
    hidden: int
    top_k: int
    embd: np.ndarray          # [vocab x hidden]
    output_norm: np.ndarray   # [hidden]
    head: np.ndarray          # [vocab x hidden]
    layers: list              # LayerWeights per layer
    rms_eps: float
    file: gguf.GGUFFile


def build(name: str) -> Model:
    H, F, E, K, nl, heads, et, rt, seed = CASES[name]
    rng = np.random.default_rng(seed)
    embd = rng.standard_normal((VOCAB, H), dtype=np.float32)
    head = (rng.standard_normal((VOCAB, H)) / np.sqrt(H)).astype(np.float32)
    out_norm = (1.0 + rng.standard_normal(H) * 0.02).astype(np.float32)
    layers, specs = [], []
    for i in range(nl):
        lw = wl.make_layer(H, F, E, K, et, seed * 100 + i, router_type=rt)
        layers.append(lw)
        specs.append(dict(
            attn_norm=(1.0 + rng.standard_normal(H) * 0.02).astype(np.float32),
            attn_q=(rng.standard_normal((H, H)) * 0.02).astype(np.float32),
            attn_k=(rng.standard_normal((H, H)) * 0.02).astype(np.float32),
            attn_v=(rng.standard_normal((H, H)) * 0.02).astype(np.float32),
            attn_output=np.zeros((H, H), np.float32),
            ffn_norm=lw.norm_weight,
            moe=gguf.MoEBlock(lw.router_bytes, rt, lw.gate, lw.up, lw.down, et, et)))
    f = gguf.freemoe_tiny(hidden=H, ffn=F, heads=heads, experts=E, top_k=K, layers=specs, seed=seed,
                          rms_eps=1e-5, vocab_tensors=dict(token_embd=embd, output_norm=out_norm, output=head),
                          name=f"fmx engine pin {name}")
    return Model(name, H, K, embd, out_norm, head, layers, float(np.float32(1e-5)), f)


def write(m: Model, path: Path) -> str:
    """Writes the checkpoint; returns its SHA-256."""
    m.file.write(path)
    return hashlib.sha256(path.read_bytes()).hexdigest()


def prompts(name: str) -> list[bytes]:
    rng = np.random.default_rng(CASES[name][-1] + 7)
    return [bytes(rng.integers(0, 256, n, dtype=np.uint8)) for n in PROMPT_LENGTHS]


def oracle_run_prompt(m: Model, prompt: bytes, generate: int):
    """The oracle's reproduction of Engine::run_prompt on a checkpoint of
    build(): (input ids, prompt logits, generated ids, routing rows)."""
    hls = [fo.host_layer(lw) for lw in m.layers]
    head_raw = m.head.view(np.uint8)
    routing = []

    def forward(tok: int, pos: int) -> np.ndarray:
        x = m.embd[tok].copy()
        for li, hl in enumerate(hls):
            out, ids, _, _, _ = hl.forward(x)
            routing.append([pos, li, *ids.tolist()])
            x = out
        hn = fo.rmsnorm(x, m.output_norm, m.rms_eps)
        return fo.gemv(fo.TYPE_F32, head_raw, hn, VOCAB, m.hidden)

    input_ids = [BOS] + list(prompt)
    logits = None
    for pos, tok in enumerate(input_ids):
        logits = forward(tok, pos)
    prompt_logits = logits.copy()
    generated = []
    pos = len(input_ids)
    for _ in range(generate):
        tok = int(np.argmax(logits))  # first maximum: the lowest id wins ties
        generated.append(tok)
        if tok == EOS:
            break
        logits = forward(tok, pos)
        pos += 1
    return (np.array(input_ids, np.int32), prompt_logits, np.array(generated, np.int32),
            np.array(routing, np.uint32).reshape(-1, 2 + m.top_k))


def write_decoder(path: Path, *, layers: int = 8, hidden: int = 4096, ffn: int = 14336, experts: int = 8,
                  top_k: int = 2, heads: int = 32, expert_type: int = wl.Q4_0, seed: int = 5) -> int:
    """A full-size seeded freemoe-tiny-v1 decoder (the 8-layer Mixtral-shaped
    decoder: F32 attention and router ~N(0, 0.02), norm gains 1 + N(0, 0.02),
    Q4_0 experts of the Mixtral layer's shape) written to `path`, with the
    adapter's FNV-1a expert checksums; returns the file size. About 8.5 GB at
    the default sizes; the tensors are generated in memory."""
    rng = np.random.default_rng(seed)

    def n(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))

    def gain():
        return (1.0 + rng.standard_normal(hidden, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    blocks, lay = [], []
    for _ in range(layers):
        gate = [wl.matrix(expert_type, rng, ffn, hidden) for _ in range(experts)]
        up = [wl.matrix(expert_type, rng, ffn, hidden) for _ in range(experts)]
        down = [wl.matrix(expert_type, rng, hidden, ffn) for _ in range(experts)]
        b = gguf.MoEBlock(n(experts, hidden), wl.F32, gate, up, down, expert_type, expert_type)
        blocks.append(b)
        lay.append(dict(attn_norm=gain(), attn_q=n(hidden, hidden), attn_k=n(hidden, hidden),
                        attn_v=n(hidden, hidden), attn_output=n(hidden, hidden), ffn_norm=gain(), moe=b))
    sums = [fo.fnv1a64(b.gate[e], b.up[e], b.down[e]) for b in blocks for e in range(experts)]
    vocab = dict(token_embd=n(VOCAB, hidden), output_norm=gain(), output=n(VOCAB, hidden))
    g = gguf.freemoe_tiny(hidden=hidden, ffn=ffn, heads=heads, experts=experts, top_k=top_k, layers=lay,
                          vocab_tensors=vocab, seed=seed, checksums=sums, name="fmx 8-layer decoder")
    return g.write(path)
