"""GGUF v3 writer for FreeMoe-loadable MoE checkpoints.

Writes the containers FreeMoe's parser and adapters read (src/gguf.cpp):

  * the native ``freemoe-tiny-v1`` layout (gguf.cpp:2990-3213): stacked expert
    tensors ``blk.N.ffn_{gate,up,down}_exps.weight`` of dims [in, out, experts]
    (innermost first), a per-layer ``ffn_router.weight`` [hidden, experts], the
    byte tokenizer, and one FNV-1a 64 checksum per expert payload
    (gate | up | down bytes, the slot payload residency verifies,
    residency.cpp:700-720);
  * the llama-family Mixtral layout (gguf.cpp:2860-2965): ``llama`` metadata
    keys, ``ffn_gate_inp.weight`` as the router, the same stacked experts.

Format (GGUF v3, little endian): magic ``GGUF``, version, tensor count, metadata
count; metadata as (string key, u32 value type, value); tensor infos as
(string name, u32 n_dims, u64 dims[n_dims] innermost first, u32 type, u64
offset into the data section); the data section starts at the next multiple of
``general.alignment`` and every tensor's offset is a multiple of it. Strings
are a u64 byte length followed by the bytes; arrays a u32 element type, a u64
count and the elements.

``write(..., sparse=True)`` writes headers only and extends the file to its
full size without storing the (zero) tensor bytes, for conformance checks on
full-size shapes that do not need real weights.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field
from typing import Any, Iterable

import numpy as np

# value type ids of the GGUF metadata section
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# block geometry (elements, bytes) of the tensor types written and read here
# (gguf.cpp:58-106): F32, Q4_0, Q8_0, Q4_K and Q6_K
F32, Q4_0, Q8_0, Q4_K, Q6_K = 0, 2, 8, 12, 14
GEOMETRY = {F32: (1, 4), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def geometry(type_id: int, name: str = "") -> tuple[int, int]:
    """(elements, bytes) per block of `type_id`; a type outside GEOMETRY is
    refused by name instead of failing as a missing key."""
    try:
        return GEOMETRY[type_id]
    except KeyError:
        raise ValueError(f"{name or 'tensor'}: block type {type_id} is not one of F32, Q4_0, Q8_0, Q4_K, "
                         f"Q6_K") from None

FNV64_OFFSET = 0xCBF29CE484222325
FNV64_PRIME = 0x100000001B3


def fnv1a64(data: bytes) -> int:
    """FNV-1a, 64-bit: h = (h xor byte) * prime mod 2^64 from the offset basis."""
    h = FNV64_OFFSET
    prime = FNV64_PRIME
    mask = 0xFFFFFFFFFFFFFFFF
    for b in bytes(data):
        h = ((h ^ b) * prime) & mask
    return h


def _string(s: str | bytes) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value: Any) -> bytes:
    if vtype == STRING:
        return _string(value)
    if vtype == ARRAY:
        etype, items = value
        items = list(items)
        out = [struct.pack("<IQ", etype, len(items))]
        if etype == STRING:
            out.extend(_string(s) for s in items)
        elif etype == ARRAY:
            raise ValueError("nested arrays are not written")
        else:
            out.append(np.asarray(items, dtype=np.dtype(_SCALAR[etype][1:]).newbyteorder("<")).tobytes())
        return b"".join(out)
    return struct.pack(_SCALAR[vtype], value)


@dataclass
class Tensor:
    name: str
    dims: list[int]          # innermost first, as stored
    type_id: int
    data: bytes | np.ndarray | None  # None: zeros (sparse writes only)

    def nbytes(self) -> int:
        bs, bb = geometry(self.type_id, self.name)
        n = int(np.prod(self.dims, dtype=np.int64))
        if self.dims[0] % bs:
            raise ValueError(f"{self.name}: innermost dimension {self.dims[0]} is not whole blocks of {bs}")
        return n // bs * bb


@dataclass
class GGUFFile:
    alignment: int = 32
    metadata: list[tuple[str, int, Any]] = field(default_factory=list)
    tensors: list[Tensor] = field(default_factory=list)

    def add(self, key: str, vtype: int, value: Any) -> None:
        self.metadata.append((key, vtype, value))

    def add_tensor(self, name: str, dims: Iterable[int], type_id: int, data=None) -> None:
        t = Tensor(name, [int(d) for d in dims], type_id, data)
        if data is not None:
            n = np.asarray(data).nbytes if isinstance(data, np.ndarray) else len(data)
            if n != t.nbytes():
                raise ValueError(f"{name}: {n} bytes given, dims and type need {t.nbytes()}")
        self.tensors.append(t)

    def _layout(self) -> tuple[bytes, list[int], int]:
        """Header bytes (through the alignment padding), tensor offsets, data size.
        A reader assumes 32-byte alignment unless ``general.alignment`` says
        otherwise, so any other alignment is stated in the metadata."""
        keys = {k for k, _, _ in self.metadata}
        if self.alignment != 32 and "general.alignment" not in keys:
            self.metadata.insert(0, ("general.alignment", UINT32, self.alignment))
        offsets, at = [], 0
        for t in self.tensors:
            at = (at + self.alignment - 1) // self.alignment * self.alignment
            offsets.append(at)
            at += t.nbytes()
        head = [b"GGUF", struct.pack("<IQQ", 3, len(self.tensors), len(self.metadata))]
        for key, vtype, value in self.metadata:
            head += [_string(key), struct.pack("<I", vtype), _value(vtype, value)]
        for t, off in zip(self.tensors, offsets):
            head += [_string(t.name), struct.pack("<I", len(t.dims)),
                     struct.pack(f"<{len(t.dims)}Q", *t.dims), struct.pack("<IQ", t.type_id, off)]
        h = b"".join(head)
        pad = (-len(h)) % self.alignment
        return h + b"\0" * pad, offsets, at

    def write(self, path: str | os.PathLike, sparse: bool = False) -> int:
        """Writes the file; returns its size. sparse: tensor bytes are not
        written (the file is extended to its size and reads as zeros)."""
        head, offsets, data_bytes = self._layout()
        with open(path, "wb") as f:
            f.write(head)
            base = len(head)
            for t, off in zip(self.tensors, offsets):
                if t.data is None:
                    if not sparse:
                        raise ValueError(f"{t.name} has no data (only sparse writes allow that)")
                    continue
                f.seek(base + off)
                f.write(t.data.tobytes() if isinstance(t.data, np.ndarray) else bytes(t.data))
            f.truncate(base + data_bytes)
        return base + data_bytes


# ----------------------------------------------------------- model layouts --

def byte_tokens() -> list[str]:
    """The freemoe.byte-v1 token table: 256 byte tokens, then BOS and EOS."""
    return [f"<byte_{i:02x}>" for i in range(256)] + ["<bos>", "<eos>"]


@dataclass
class MoEBlock:
    """One MoE layer's weights as raw GGUF rows (row-major [out x in] blocks):
    router [experts x row_bytes(hidden)], gate/up [ffn x row_bytes(hidden)] and
    down [hidden x row_bytes(ffn)] per expert."""
    router: np.ndarray
    router_type: int
    gate: list
    up: list
    down: list
    gate_type: int
    down_type: int


def stacked(mats: list) -> np.ndarray:
    """Experts' raw matrices stacked along the outermost axis."""
    return np.concatenate([np.ascontiguousarray(m).view(np.uint8).ravel() for m in mats])


def expert_checksums(blocks: list[MoEBlock]) -> list[int]:
    """FNV-1a 64 of each expert's slot payload, gate | up | down, layers in
    order, experts in order."""
    out = []
    for b in blocks:
        for e in range(len(b.gate)):
            payload = b"".join(np.ascontiguousarray(m).view(np.uint8).tobytes()
                               for m in (b.gate[e], b.up[e], b.down[e]))
            out.append(fnv1a64(payload))
    return out


def _native_metadata(g: GGUFFile, *, hidden, ffn, heads, layers, experts, top_k, context, rms_eps, rope_theta,
                     seed, checksums, name) -> None:
    md = [
        ("general.architecture", STRING, "freemoe-tiny"),
        ("general.name", STRING, name),
        ("general.alignment", UINT32, g.alignment),
        ("general.file_type", UINT32, 0),
        ("general.quantization_version", UINT32, 1),
        ("freemoe.adapter", STRING, "freemoe-tiny-v1"),
        ("freemoe.model_kind", STRING, "moe"),
        ("freemoe.hidden_size", UINT32, hidden),
        ("freemoe.intermediate_size", UINT32, ffn),
        ("freemoe.num_hidden_layers", UINT32, layers),
        ("freemoe.num_attention_heads", UINT32, heads),
        ("freemoe.num_key_value_heads", UINT32, heads),
        ("freemoe.head_dim", UINT32, hidden // heads),
        ("freemoe.vocab_size", UINT32, 258),
        ("freemoe.max_context_length", UINT32, context),
        ("freemoe.rms_norm_epsilon", FLOAT32, rms_eps),
        ("freemoe.rope_theta", FLOAT32, rope_theta),
        ("freemoe.rope_mode", STRING, "half"),
        ("freemoe.tokenizer_model", STRING, "freemoe.byte-v1"),
        ("freemoe.router_operation", STRING, "linear-topk-softmax-v1"),
        ("freemoe.shared_expert", BOOL, False),
        ("freemoe.expert_layout", STRING, "stacked-f32"),
        ("freemoe.expert_count", UINT32, experts),
        ("freemoe.expert_top_k", UINT32, top_k),
        ("freemoe.expert_checksums", ARRAY, (UINT64, checksums)),
        ("freemoe.seed", UINT32, seed & 0xFFFFFFFF),
        ("tokenizer.ggml.model", STRING, "freemoe.byte-v1"),
        ("tokenizer.ggml.bos_token_id", UINT32, 256),
        ("tokenizer.ggml.eos_token_id", UINT32, 257),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, byte_tokens())),
        ("tokenizer.chat_template", STRING, "raw-v1"),
    ]
    for key, vtype, value in md:
        g.add(key, vtype, value)


def freemoe_tiny(*, hidden: int, ffn: int, heads: int, vocab_tensors: dict, layers: list[dict],
                 experts: int, top_k: int, context: int = 1024, rms_eps: float = 1e-5,
                 rope_theta: float = 10000.0, seed: int = 0, checksums: list[int] | None = None,
                 name: str = "fmx synthetic moe", alignment: int = 32) -> GGUFFile:
    """A native freemoe-tiny-v1 MoE checkpoint (the adapter of
    gguf.cpp:2990-3213). vocab_tensors: token_embd, output_norm, output as F32
    arrays ([vocab x hidden], [hidden], [vocab x hidden]). layers: per layer
    attn_norm, attn_q, attn_k, attn_v, attn_output ([hidden x hidden] F32),
    ffn_norm, and `moe`, an MoEBlock. The vocabulary is the byte tokenizer's
    258 entries. The adapter needs gate, up and down of equal byte strides
    (one block type for all three, gguf.cpp:3185-3187)."""
    vocab = 258
    blocks = [l["moe"] for l in layers]
    g = GGUFFile(alignment=alignment)
    _native_metadata(g, hidden=hidden, ffn=ffn, heads=heads, layers=len(layers), experts=experts, top_k=top_k,
                     context=context, rms_eps=rms_eps, rope_theta=rope_theta, seed=seed, name=name,
                     checksums=checksums if checksums is not None else expert_checksums(blocks))

    def f32(a) -> np.ndarray:
        return np.ascontiguousarray(a, np.float32)

    g.add_tensor("token_embd.weight", [hidden, vocab], F32, f32(vocab_tensors["token_embd"]))
    for i, l in enumerate(layers):
        p = f"blk.{i}."
        g.add_tensor(p + "attn_norm.weight", [hidden], F32, f32(l["attn_norm"]))
        for nm in ("attn_q", "attn_k", "attn_v", "attn_output"):
            g.add_tensor(p + nm + ".weight", [hidden, hidden], F32, f32(l[nm]))
        g.add_tensor(p + "ffn_norm.weight", [hidden], F32, f32(l["ffn_norm"]))
        b = l["moe"]
        g.add_tensor(p + "ffn_router.weight", [hidden, experts], b.router_type,
                     np.ascontiguousarray(b.router).view(np.uint8))
        g.add_tensor(p + "ffn_gate_exps.weight", [hidden, ffn, experts], b.gate_type, stacked(b.gate))
        g.add_tensor(p + "ffn_up_exps.weight", [hidden, ffn, experts], b.gate_type, stacked(b.up))
        g.add_tensor(p + "ffn_down_exps.weight", [ffn, hidden, experts], b.down_type, stacked(b.down))
    g.add_tensor("output_norm.weight", [hidden], F32, f32(vocab_tensors["output_norm"]))
    g.add_tensor("output.weight", [hidden, vocab], F32, f32(vocab_tensors["output"]))
    return g


def native_sparse(*, hidden: int, ffn: int, heads: int, experts: int, top_k: int, layers: int, expert_type: int,
                  router_type: int = F32, context: int = 1024) -> GGUFFile:
    """The freemoe-tiny-v1 layout with no tensor data (for sparse writes at full
    size) and zero checksums: the adapter's manifest does not read expert bytes,
    but residency would reject such a file's experts when it loads them."""
    g = GGUFFile()
    _native_metadata(g, hidden=hidden, ffn=ffn, heads=heads, layers=layers, experts=experts, top_k=top_k,
                     context=context, rms_eps=1e-5, rope_theta=10000.0, seed=0, name="fmx sparse moe",
                     checksums=[0] * (layers * experts))
    g.add_tensor("token_embd.weight", [hidden, 258], F32)
    for i in range(layers):
        p = f"blk.{i}."
        g.add_tensor(p + "attn_norm.weight", [hidden], F32)
        for nm in ("attn_q", "attn_k", "attn_v", "attn_output"):
            g.add_tensor(p + nm + ".weight", [hidden, hidden], F32)
        g.add_tensor(p + "ffn_norm.weight", [hidden], F32)
        g.add_tensor(p + "ffn_router.weight", [hidden, experts], router_type)
        g.add_tensor(p + "ffn_gate_exps.weight", [hidden, ffn, experts], expert_type)
        g.add_tensor(p + "ffn_up_exps.weight", [hidden, ffn, experts], expert_type)
        g.add_tensor(p + "ffn_down_exps.weight", [ffn, hidden, experts], expert_type)
    g.add_tensor("output_norm.weight", [hidden], F32)
    g.add_tensor("output.weight", [hidden, 258], F32)
    return g


def mixtral_llama(*, hidden: int, ffn: int, layers: int, heads: int, kv_heads: int, experts: int, top_k: int,
                  vocab: int, expert_type: int, router_type: int = F32, down_type: int | None = None,
                  context: int = 4096,
                  rms_eps: float = 1e-5, rope_theta: float = 1e6, data: dict | None = None,
                  alignment: int = 32, router_bias: bool = False, weights_norm: bool | None = True,
                  weights_scale: float | None = None, arch: str = "llama") -> GGUFFile:
    """A Mixtral-style llama-family checkpoint (the vendor layout the llama
    adapter reads, gguf.cpp:2860-2965): ``llama.*`` hyper-parameters,
    ``blk.N.ffn_gate_inp.weight`` as the router and stacked
    ``ffn_{gate,up,down}_exps`` experts (down may hold another block type, as
    Q4_K gate/up with Q6_K down files do). `data` maps tensor names to raw bytes;
    a tensor without an entry is left to a sparse write. The tokenizer is a
    plain llama (SentencePiece) table of `vocab` pieces.

    Routing options, as the llama adapter reads them: `router_bias` adds an F32
    ``blk.N.ffn_gate_inp.bias`` [experts] per layer (added to the router logits
    before the softmax, gguf.cpp:1535, engine.cpp:1611-1616);
    ``llama.expert_weights_norm`` is written as `weights_norm` (None leaves
    the key out, and the adapter's default, off, applies: gguf.cpp:1445);
    ``llama.expert_weights_scale`` (F32) is written when `weights_scale` is
    given (gguf.cpp:1446). `arch` names another family that shares the llama
    block and reads the same keys under its own prefix (deepseek41, whose
    renormalisation adds 1e-20 to the sum instead of clamping it, gguf.cpp:
    1943-1947)."""
    data = data or {}
    g = GGUFFile(alignment=alignment)
    head_dim = hidden // heads
    md = [
        ("general.architecture", STRING, arch),
        ("general.name", STRING, "fmx synthetic mixtral"),
        ("general.alignment", UINT32, alignment),
        (f"{arch}.block_count", UINT32, layers),
        (f"{arch}.context_length", UINT32, context),
        (f"{arch}.embedding_length", UINT32, hidden),
        (f"{arch}.feed_forward_length", UINT32, ffn),
        (f"{arch}.attention.head_count", UINT32, heads),
        (f"{arch}.attention.head_count_kv", UINT32, kv_heads),
        (f"{arch}.attention.layer_norm_rms_epsilon", FLOAT32, rms_eps),
        (f"{arch}.rope.freq_base", FLOAT32, rope_theta),
        (f"{arch}.rope.dimension_count", UINT32, head_dim),
        (f"{arch}.expert_count", UINT32, experts),
        (f"{arch}.expert_used_count", UINT32, top_k),
        (f"{arch}.vocab_size", UINT32, vocab),
        ("tokenizer.ggml.model", STRING, "llama"),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, ["<unk>", "<s>", "</s>"] +
                                          [f"<0x{i:02X}>" for i in range(256)] +
                                          [f"tok{i}" for i in range(vocab - 259)])),
        ("tokenizer.ggml.scores", ARRAY, (FLOAT32, [0.0] * vocab)),
        ("tokenizer.ggml.token_type", ARRAY, (INT32, [2, 3, 3] + [6] * 256 + [1] * (vocab - 259))),
        ("tokenizer.ggml.bos_token_id", UINT32, 1),
        ("tokenizer.ggml.eos_token_id", UINT32, 2),
    ]
    if weights_norm is not None:
        md.append((f"{arch}.expert_weights_norm", BOOL, bool(weights_norm)))
    if weights_scale is not None:
        md.append((f"{arch}.expert_weights_scale", FLOAT32, float(weights_scale)))
    for key, vtype, value in md:
        g.add(key, vtype, value)

    def t(name, dims, type_id):
        g.add_tensor(name, dims, type_id, data.get(name))

    t("token_embd.weight", [hidden, vocab], F32)
    kv = kv_heads * head_dim
    for i in range(layers):
        p = f"blk.{i}."
        t(p + "attn_norm.weight", [hidden], F32)
        t(p + "attn_q.weight", [hidden, hidden], F32)
        t(p + "attn_k.weight", [hidden, kv], F32)
        t(p + "attn_v.weight", [hidden, kv], F32)
        t(p + "attn_output.weight", [hidden, hidden], F32)
        t(p + "ffn_norm.weight", [hidden], F32)
        t(p + "ffn_gate_inp.weight", [hidden, experts], router_type)
        if router_bias:
            t(p + "ffn_gate_inp.bias", [experts], F32)
        t(p + "ffn_gate_exps.weight", [hidden, ffn, experts], expert_type)
        t(p + "ffn_up_exps.weight", [hidden, ffn, experts], expert_type)
        t(p + "ffn_down_exps.weight", [ffn, hidden, experts], expert_type if down_type is None else down_type)
    t("output_norm.weight", [hidden], F32)
    t("output.weight", [hidden, vocab], F32)
    return g


# ----------------------------------------------------------------- reading --

@dataclass
class TensorInfo:
    name: str
    dims: list[int]
    type_id: int
    offset: int      # absolute byte offset in the file
    nbytes: int


@dataclass
class GGUFReader:
    """A GGUF v3 file's metadata and tensor table, the file memory-mapped."""
    path: str
    metadata: dict
    tensors: dict
    data: np.memmap

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        return self.data[t.offset:t.offset + t.nbytes]

    def expert_slices(self, layer: int, expert: int, router_name: str | None = None) -> dict:
        """Expert `expert` of layer `layer` in a stacked layout: gate, up and down
        as raw row-major matrices [(rows, row_bytes)], with their types. The
        expert's slice of a stacked tensor is its outermost-axis index. A fused
        ``ffn_gate_up_exps`` tensor holds each expert's gate rows, then its up
        rows (gguf.cpp:1988-2000, 2928-2958); a file with both the fused and
        the separate names is refused, as the adapter refuses it."""
        out = {}
        p = f"blk.{layer}."
        fused = self.tensors.get(p + "ffn_gate_up_exps.weight")
        if fused is not None and p + "ffn_gate_exps.weight" in self.tensors:
            raise ValueError(f"{p}: both ffn_gate_up_exps and ffn_gate_exps are present")
        for key in ("gate", "up", "down"):
            if fused is not None and key != "down":
                t = fused
                cols, rows2, experts = t.dims
                rows = rows2 // 2
                bs, bb = geometry(t.type_id, t.name)
                row_bytes = cols // bs * bb
                stride = rows * row_bytes
                if 2 * stride * experts != t.nbytes or rows2 % 2:
                    raise ValueError(f"{t.name}: fused size does not split into gate and up of {experts} experts")
                lo = t.offset + expert * 2 * stride + (stride if key == "up" else 0)
            else:
                t = self.tensors[p + f"ffn_{key}_exps.weight"]
                cols, rows, experts = t.dims
                bs, bb = geometry(t.type_id, t.name)
                row_bytes = cols // bs * bb
                stride = rows * row_bytes
                if stride * experts != t.nbytes:
                    raise ValueError(f"{t.name}: stacked size does not divide by {experts} experts")
                lo = t.offset + expert * stride
            out[key] = (self.data[lo:lo + stride].reshape(rows, row_bytes), t.type_id)
        return out


def _read_string(buf, at: int) -> tuple[str, int]:
    (n,) = struct.unpack_from("<Q", buf, at)
    at += 8
    return bytes(buf[at:at + n]).decode("utf-8"), at + n


def _read_value(buf, at: int, vtype: int):
    if vtype == STRING:
        return _read_string(buf, at)
    if vtype == ARRAY:
        etype, n = struct.unpack_from("<IQ", buf, at)
        at += 12
        if etype == STRING:
            items = []
            for _ in range(n):
                s, at = _read_string(buf, at)
                items.append(s)
            return (etype, items), at
        fmt = _SCALAR[etype]
        size = struct.calcsize(fmt)
        arr = np.frombuffer(bytes(buf[at:at + n * size]), dtype=np.dtype(fmt[1:]).newbyteorder("<"))
        return (etype, arr.tolist()), at + n * size
    fmt = _SCALAR[vtype]
    (v,) = struct.unpack_from(fmt, buf, at)
    return v, at + struct.calcsize(fmt)


def read(path: str | os.PathLike) -> GGUFReader:
    """Parses a GGUF v3 file (metadata as {key: (type, value)}, tensors with
    absolute offsets); tensor bytes stay in the memory map."""
    data = np.memmap(path, dtype=np.uint8, mode="r")
    buf = memoryview(data)
    if bytes(buf[0:4]) != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    version, n_tensors, n_kv = struct.unpack_from("<IQQ", buf, 4)
    if version != 3:
        raise ValueError(f"{path}: GGUF version {version}, expected 3")
    at = 24
    md = {}
    for _ in range(n_kv):
        key, at = _read_string(buf, at)
        (vtype,) = struct.unpack_from("<I", buf, at)
        value, at = _read_value(buf, at + 4, vtype)
        md[key] = (vtype, value)
    infos = []
    for _ in range(n_tensors):
        name, at = _read_string(buf, at)
        (nd,) = struct.unpack_from("<I", buf, at)
        dims = list(struct.unpack_from(f"<{nd}Q", buf, at + 4))
        at += 4 + 8 * nd
        type_id, off = struct.unpack_from("<IQ", buf, at)
        at += 12
        infos.append((name, dims, type_id, off))
    align = md.get("general.alignment", (UINT32, 32))[1]
    base = (at + align - 1) // align * align
    tensors = {}
    for name, dims, type_id, off in infos:
        t = Tensor(name, dims, type_id, None)
        tensors[name] = TensorInfo(name, dims, type_id, base + off, t.nbytes())
    return GGUFReader(str(path), md, tensors, data)


# Families whose router weight normalisation is fixed by the architecture, not
# by ``expert_weights_norm`` (gguf.cpp:2046-2058).
_WEIGHTS_NORM_ON = ("dbrx", "ernie4-5-moe", "maple", "minimax-m2")
_WEIGHTS_NORM_OFF = ("deepseek",)
# Families whose MoE block is not plain SwiGLU experts under softmax routing
# (GeGLU / gelu: gemma, gguf.cpp:1566-1571; relu: smallthinker, 2040-2043; the
# clamped swiglu-oai and softmax-weight gating of gpt-oss / minimax-m3,
# 1900, 1950-1956; sigmoid gating by default: glm4-moe, 1463-1469).
_OTHER_BLOCKS = ("gemma", "gemma2", "gemma3", "smallthinker", "gpt-oss", "minimax-m3", "glm4-moe")


def _opt(md: dict, arch: str, name: str, default):
    """A metadata value as the llama adapter looks it up (gguf.cpp:1035-1037,
    768-820): the first present of ``arch.name``, ``freemoe.name`` and
    ``name`` in sorted order."""
    for key in sorted({f"{arch}.{name}", f"freemoe.{name}", name}):
        if key in md:
            return md[key][1]
    return default


def moe_layer(r: GGUFReader, layer: int):
    """Layer `layer`'s MoE block of a checkpoint as workloads.LayerWeights (the
    arrays are views of the memory map): the norm gains (ffn_norm), the router
    (native ``ffn_router.weight`` or llama ``ffn_gate_inp.weight``, F32 or a
    block type) and every expert's raw gate / up / down rows.

    Routing options follow the adapters. The native layout renormalises the
    selected weights with scale 1 (gguf.cpp:3027-3028). A llama-family file
    carries them as metadata and tensors: ``expert_weights_norm`` (default
    off, gguf.cpp:1445; forced on or off for five families, 2046-2058),
    ``expert_weights_scale`` (1445-1448; fixed at 1 for maple, 2062-2064),
    the additive 1e-20 epsilon of deepseek41 (1943-1947) and an F32
    ``ffn_gate_inp.bias`` added to the logits before the softmax (1535,
    engine.cpp:1611-1616). A file whose MoE block needs anything else (another
    gating function, a selection bias, group-limited routing, shared experts,
    expert projection biases, another activation or zero-centred norms) is
    refused with NotImplementedError rather than routed differently."""
    from .workloads import LayerWeights

    md = r.metadata
    arch = md["general.architecture"][1]
    router_bias = None
    weights_scale = 1.0
    epsilon_additive, weights_epsilon = False, 6.103515625e-5
    if arch == "freemoe-tiny":
        hidden = md["freemoe.hidden_size"][1]
        ffn = md["freemoe.intermediate_size"][1]
        experts = md["freemoe.expert_count"][1]
        top_k = md["freemoe.expert_top_k"][1]
        eps = md["freemoe.rms_norm_epsilon"][1]
        weights_norm = True
        router_name = f"blk.{layer}.ffn_router.weight"
    else:
        hidden = md[f"{arch}.embedding_length"][1]
        ffn = md[f"{arch}.feed_forward_length"][1]
        experts = md[f"{arch}.expert_count"][1]
        top_k = md[f"{arch}.expert_used_count"][1]
        eps = md[f"{arch}.attention.layer_norm_rms_epsilon"][1]
        router_name = f"blk.{layer}.ffn_gate_inp.weight"
        if arch in _OTHER_BLOCKS:
            raise NotImplementedError(f"{arch}: its MoE block is not softmax-routed SwiGLU experts")
        if int(_opt(md, arch, "expert_gating_func", 0)) not in (0, 1):
            raise NotImplementedError(f"{arch}: expert_gating_func is not softmax")
        if int(_opt(md, arch, "expert_group_count", 0)) > 1:
            raise NotImplementedError(f"{arch}: group-limited routing")
        if f"{arch}.swiglu_clamp_exp" in md:
            raise NotImplementedError(f"{arch}: clamped SwiGLU")
        for tail in ("ffn_exp_probs_b.bias", "ffn_gate_exps.bias", "ffn_up_exps.bias", "ffn_down_exps.bias",
                     "ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight",
                     "ffn_gate_inp_shexp.weight"):
            if any(name.endswith(tail) for name in r.tensors):
                raise NotImplementedError(f"{arch}: the MoE block carries {tail}")
        weights_norm = bool(_opt(md, arch, "expert_weights_norm", False))
        if arch in _WEIGHTS_NORM_ON:
            weights_norm = True
        if arch in _WEIGHTS_NORM_OFF:
            weights_norm = False
        weights_scale = float(_opt(md, arch, "expert_weights_scale", 1.0))
        if not weights_scale > 0.0:
            raise ValueError(f"{arch}: expert_weights_scale must be positive")
        if arch == "maple":
            weights_scale = 1.0
        if arch == "deepseek41":
            epsilon_additive, weights_epsilon = True, 1e-20
        bias_name = f"blk.{layer}.ffn_gate_inp.bias"
        if bias_name in r.tensors:
            bt = r.tensors[bias_name]
            if bt.type_id != F32 or bt.dims != [experts]:
                raise NotImplementedError(f"{bias_name}: only an F32 [experts] router bias is read")
            router_bias = np.array(r.tensor_bytes(bias_name).view(np.float32))
    rt = r.tensors[router_name]
    bs, bb = geometry(rt.type_id, router_name)
    router_raw = r.tensor_bytes(router_name).reshape(experts, hidden // bs * bb)
    norm = r.tensor_bytes(f"blk.{layer}.ffn_norm.weight").view(np.float32)
    gate, up, down = [], [], []
    types = None
    for e in range(experts):
        sl = r.expert_slices(layer, e)
        gate.append(sl["gate"][0])
        up.append(sl["up"][0])
        down.append(sl["down"][0])
        types = (sl["gate"][1], sl["down"][1])
    router_f32 = router_raw.view(np.float32).reshape(experts, hidden) if rt.type_id == F32 else None
    return LayerWeights(hidden, ffn, experts, top_k, types[0], norm, router_f32, gate, up, down, router_bias,
                        rms_eps=float(np.float32(eps)), weights_norm=weights_norm, down_type=types[1],
                        router_type=rt.type_id, router_raw=None if rt.type_id == F32 else router_raw,
                        epsilon_additive=epsilon_additive, weights_epsilon=weights_epsilon,
                        weights_scale=weights_scale, notes={"source": r.path, "layer": layer})
