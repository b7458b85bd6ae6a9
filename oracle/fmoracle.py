"""ctypes binding of the CPU oracle (libfmoracle.so) and of oracle/_ref/libfmref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. Nothing in freemoe_amd/ imports it.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# FMORACLE_LIBRARY: another build of the C restatement (the host-sanitizer build)
ORACLE_PATH = Path(os.environ.get("FMORACLE_LIBRARY") or HERE / "libfmoracle.so")
REF_PATH = HERE / "_ref" / "libfmref.so"

ISA_SCALAR, ISA_AVX2 = 0, 1
TYPE_F32, TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 2, 8, 12, 14
GEOMETRY = {TYPE_F32: (1, 4), TYPE_Q4_0: (32, 18), TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144),
            TYPE_Q6_K: (256, 210)}


class OracleError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: status {status}")


class Layer(ctypes.Structure):
    _fields_ = [("hidden", c_uint32), ("ffn", c_uint32), ("experts", c_uint32), ("top_k", c_uint32),
                ("norm_weight", c_void_p), ("rms_eps", c_double), ("norm_bias", c_double),
                ("router_type", c_uint32), ("router", c_void_p), ("router_bias", c_void_p),
                ("weights_norm", c_int), ("epsilon_additive", c_int), ("weights_epsilon", c_double),
                ("weights_scale", c_double), ("gate_type", c_uint32), ("up_type", c_uint32),
                ("down_type", c_uint32), ("gate", c_void_p), ("up", c_void_p), ("down", c_void_p)]


def _p(a):
    return None if a is None else a.ctypes.data_as(c_void_p)


_oracle = None
_ref = None


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        lib = ctypes.CDLL(str(ORACLE_PATH))
        lib.fmo_fp16_to_f32.restype = c_float
        lib.fmo_fp16_to_f32.argtypes = [c_uint16]
        for name in ["fmo_dequantize_block", "fmo_dequantize_region", "fmo_gemv", "fmo_gemm", "fmo_rmsnorm",
                     "fmo_softmax", "fmo_topk", "fmo_route", "fmo_moe_layer", "fmo_moe_layer_batch",
                     "fmo_moe_bucket", "fmo_quant_geometry", "fmo_moe_experts"]:
            getattr(lib, name).restype = c_int
        lib.fmo_dequantize_region.argtypes = [c_uint32, c_void_p, c_void_p, c_uint64]
        lib.fmo_gemv.argtypes = [c_int, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]
        lib.fmo_gemm.argtypes = [c_int, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]
        lib.fmo_fnv1a64.restype = c_uint64
        lib.fmo_fnv1a64.argtypes = [c_uint64, c_void_p, c_uint64]
        lib.fmo_rmsnorm.argtypes = [c_void_p, c_void_p, c_uint32, c_double, c_double, c_void_p]
        lib.fmo_softmax.argtypes = [c_void_p, c_uint32, c_void_p]
        lib.fmo_topk.argtypes = [c_void_p, c_uint32, c_uint32, c_void_p]
        lib.fmo_route.argtypes = [c_int, POINTER(Layer), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_void_p]
        lib.fmo_moe_layer.argtypes = [c_int, POINTER(Layer), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p]
        lib.fmo_moe_layer_batch.argtypes = [c_int, POINTER(Layer), c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_uint32]
        lib.fmo_moe_experts.argtypes = [c_int, POINTER(Layer), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p]
        lib.fmo_moe_bucket.argtypes = [c_void_p, c_uint32, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p]
        _oracle = lib
    return _oracle


def ref_available() -> bool:
    return REF_PATH.exists()


def ref() -> ctypes.CDLL:
    """The reference's own kernels (built from the FreeMoe sources by oracle/Makefile)."""
    global _ref
    if _ref is None:
        lib = ctypes.CDLL(str(REF_PATH))
        lib.fmr_fp16_to_f32.restype = c_float
        lib.fmr_fp16_to_f32.argtypes = [c_uint16]
        lib.fmr_dequantize_block.argtypes = [c_uint32, c_void_p, c_void_p]
        lib.fmr_gemv.argtypes = [c_int, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]
        lib.fmr_gemm.argtypes = [c_int, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                 c_uint32]
        lib.fmr_moe_layer_batch.argtypes = [c_int, c_uint32, POINTER(Layer), c_void_p, c_void_p, c_void_p,
                                            c_void_p, c_uint32]
        lib.fmr_resolved_threads.restype = c_uint32
        lib.fmr_resolved_threads.argtypes = [c_uint32]
        lib.fmr_engine_open.restype = c_void_p
        lib.fmr_engine_open.argtypes = [ctypes.c_char_p, c_int, c_uint32, ctypes.c_char_p, c_uint32]
        lib.fmr_engine_close.restype = None
        lib.fmr_engine_close.argtypes = [c_void_p]
        lib.fmr_engine_prompt.restype = c_int
        lib.fmr_engine_prompt.argtypes = [c_void_p, ctypes.c_char_p, c_uint32, c_uint32,
                                          c_void_p, c_uint32, POINTER(c_uint32), c_void_p, c_uint32,
                                          POINTER(c_uint32), c_void_p, c_uint32, POINTER(c_uint32),
                                          c_void_p, c_uint32, c_uint32, POINTER(c_uint32),
                                          ctypes.c_char_p, c_uint32]
        lib.fmr_manifest_probe.restype = c_int
        lib.fmr_manifest_probe.argtypes = [ctypes.c_char_p, c_void_p, c_void_p, c_void_p, c_uint32,
                                           ctypes.c_char_p, c_uint32]
        _ref = lib
    return _ref


def ref_manifest(path, cap: int = 4096) -> dict:
    """The reference's parse_gguf + build_manifest on a checkpoint: its
    layer / expert / top-k / hidden counts, slot and fixed-weight bytes, and
    per expert record (layer, expert) and three extents (offset, bytes,
    type)."""
    info = np.zeros(9, np.uint32)
    ext = np.zeros((cap, 3, 3), np.uint64)
    who = np.zeros((cap, 2), np.uint32)
    err = ctypes.create_string_buffer(512)
    rc = ref().fmr_manifest_probe(str(path).encode(), _p(info), _p(ext), _p(who), cap, err, 512)
    if rc:
        raise OracleError(rc, f"build_manifest: {err.value.decode()}")
    n = int(info[4])
    return dict(layers=int(info[0]), experts=int(info[1]), top_k=int(info[2]), hidden=int(info[3]),
                records=n, slot_bytes=int(info[5]) | int(info[6]) << 32,
                fixed_weight_bytes=int(info[7]) | int(info[8]) << 32,
                who=who[:min(n, cap)].copy(), extents=ext[:min(n, cap)].copy())


class RefEngine:
    """The reference's own fm::Engine (compiled from the FreeMoe sources into
    libfmref) on a checkpoint, CPU backend, one token at a time."""

    def __init__(self, model_path, isa: int = ISA_AVX2, threads: int = 1, top_k: int = 2):
        err = ctypes.create_string_buffer(512)
        self.top_k = top_k
        self.h = ref().fmr_engine_open(str(model_path).encode(), isa, threads, err, 512)
        if not self.h:
            raise RuntimeError(f"fm::Engine could not open {model_path}: {err.value.decode()}")

    def close(self):
        if self.h:
            ref().fmr_engine_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def run_prompt(self, prompt: bytes, generate: int, vocab_cap: int = 1 << 16):
        """(input_ids, prefill logits, generated ids, routing rows
        [position, layer, ids...]) of Engine::run_prompt."""
        cap = len(prompt) + 2
        ids = np.empty(cap, np.int32)
        logits = np.empty(vocab_cap, np.float32)
        gen = np.empty(max(generate, 1), np.int32)
        rcap = 64 * (cap + generate)
        routing = np.empty((rcap, 2 + self.top_k), np.uint32)
        n_in, n_v, n_g, n_r = c_uint32(), c_uint32(), c_uint32(), c_uint32()
        err = ctypes.create_string_buffer(512)
        rc = ref().fmr_engine_prompt(self.h, prompt, len(prompt), generate, _p(ids), cap, ctypes.byref(n_in),
                                     _p(logits), vocab_cap, ctypes.byref(n_v), _p(gen), max(generate, 1),
                                     ctypes.byref(n_g), _p(routing), rcap, self.top_k, ctypes.byref(n_r),
                                     err, 512)
        if rc:
            raise OracleError(rc, f"fm::Engine::run_prompt: {err.value.decode()}")
        return (ids[:n_in.value].copy(), logits[:n_v.value].copy(), gen[:n_g.value].copy(),
                routing[:n_r.value].copy())


def check(rc: int, where: str) -> None:
    if rc != 0:
        raise OracleError(rc, where)


# ----------------------------------------------------------------- kernels --

def fp16_to_f32(h: int) -> float:
    return oracle().fmo_fp16_to_f32(h)


def dequantize(type_id: int, raw: np.ndarray, count: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    check(oracle().fmo_dequantize_region(type_id, _p(raw), _p(out), count), "fmo_dequantize_region")
    return out


def gemv(type_id: int, w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int, isa: int = ISA_AVX2) -> np.ndarray:
    y = np.empty(out_dim, np.float32)
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    check(oracle().fmo_gemv(isa, type_id, _p(w), _p(x), _p(y), out_dim, in_dim), "fmo_gemv")
    return y


def ref_gemv(type_id: int, w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int, isa: int = ISA_AVX2,
             threads: int = 1) -> np.ndarray:
    y = np.empty(out_dim, np.float32)
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x, dtype=np.float32)
    check(ref().fmr_gemv(isa, threads, type_id, _p(w), _p(x), _p(y), out_dim, in_dim), "fmr_gemv")
    return y


def fnv1a64(*parts) -> int:
    """FNV-1a 64 over the concatenated bytes of `parts` (arrays or bytes)."""
    h = 14695981039346656037
    for p in parts:
        a = np.ascontiguousarray(np.frombuffer(p, np.uint8) if isinstance(p, (bytes, bytearray)) else p)
        h = oracle().fmo_fnv1a64(h, _p(a.view(np.uint8)), a.nbytes)
    return h


def gemm(type_id: int, w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int, isa: int = ISA_AVX2) -> np.ndarray:
    """gemm_quant: x [tokens x in_dim] -> y [tokens x out_dim]."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    y = np.empty((x.shape[0], out_dim), np.float32)
    w = np.ascontiguousarray(w)
    check(oracle().fmo_gemm(isa, type_id, _p(w), _p(x), _p(y), x.shape[0], out_dim, in_dim), "fmo_gemm")
    return y


def ref_gemm(type_id: int, w: np.ndarray, x: np.ndarray, out_dim: int, in_dim: int, isa: int = ISA_AVX2,
             threads: int = 1) -> np.ndarray:
    """The reference's own gemm_quant."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    y = np.empty((x.shape[0], out_dim), np.float32)
    w = np.ascontiguousarray(w)
    check(ref().fmr_gemm(isa, threads, type_id, _p(w), _p(x), _p(y), x.shape[0], out_dim, in_dim), "fmr_gemm")
    return y


def rmsnorm(x: np.ndarray, w, eps: float, norm_bias: float = 0.0) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    check(oracle().fmo_rmsnorm(_p(x), _p(w), x.size, eps, norm_bias, _p(y)), "fmo_rmsnorm")
    return y


def softmax(v: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty_like(v)
    check(oracle().fmo_softmax(_p(v), v.size, _p(out)), "fmo_softmax")
    return out


def topk(scores: np.ndarray, k: int) -> np.ndarray:
    s = np.ascontiguousarray(scores, np.float32)
    ids = np.empty(max(k, 1), np.uint32)
    check(oracle().fmo_topk(_p(s), s.size, k, _p(ids)), "fmo_topk")
    return ids[:k]


def bucket(ids: np.ndarray, experts: int):
    ids = np.ascontiguousarray(ids, np.uint32)
    tokens, k = ids.shape
    offsets = np.empty(experts + 1, np.uint32)
    tl = np.empty(max(tokens * k, 1), np.uint32)
    rl = np.empty(max(tokens * k, 1), np.uint32)
    check(oracle().fmo_moe_bucket(_p(ids), tokens, k, experts, _p(offsets), _p(tl), _p(rl)), "fmo_moe_bucket")
    return offsets, tl[:tokens * k], rl[:tokens * k]


# ------------------------------------------------------------------- layer --

class HostLayer:
    """A MoE layer held in host memory in raw GGUF block layout."""

    def __init__(self, *, hidden, ffn, experts, top_k, norm_weight, rms_eps, router, gate, up, down,
                 gate_type, up_type=None, down_type=None, router_type=TYPE_F32, router_bias=None,
                 norm_bias=0.0, weights_norm=True, epsilon_additive=False, weights_epsilon=6.103515625e-5,
                 weights_scale=1.0):
        self.hidden, self.ffn, self.experts, self.top_k = hidden, ffn, experts, top_k
        self.norm_weight = None if norm_weight is None else np.ascontiguousarray(norm_weight, np.float32)
        self.rms_eps, self.norm_bias = rms_eps, norm_bias
        self.router_type = router_type
        self.router = np.ascontiguousarray(router)
        self.router_bias = None if router_bias is None else np.ascontiguousarray(router_bias, np.float32)
        self.weights_norm, self.epsilon_additive = weights_norm, epsilon_additive
        self.weights_epsilon, self.weights_scale = weights_epsilon, weights_scale
        self.gate_type = gate_type
        self.up_type = gate_type if up_type is None else up_type
        self.down_type = gate_type if down_type is None else down_type
        self.gate = [np.ascontiguousarray(g) for g in gate]
        self.up = [np.ascontiguousarray(u) for u in up]
        self.down = [np.ascontiguousarray(d) for d in down]
        self._ptrs = [(ctypes.c_void_p * experts)(*[g.ctypes.data for g in arr]) for arr in (self.gate, self.up, self.down)]

    def struct(self) -> Layer:
        return Layer(self.hidden, self.ffn, self.experts, self.top_k, _p(self.norm_weight), self.rms_eps,
                     self.norm_bias, self.router_type, _p(self.router), _p(self.router_bias),
                     int(self.weights_norm), int(self.epsilon_additive), self.weights_epsilon, self.weights_scale,
                     self.gate_type, self.up_type, self.down_type,
                     ctypes.cast(self._ptrs[0], c_void_p), ctypes.cast(self._ptrs[1], c_void_p),
                     ctypes.cast(self._ptrs[2], c_void_p))

    def route(self, x: np.ndarray, isa: int = ISA_AVX2):
        x = np.ascontiguousarray(x, np.float32)
        h = np.empty(self.hidden, np.float32)
        logits = np.empty(self.experts, np.float32)
        probs = np.empty(self.experts, np.float32)
        ids = np.empty(self.top_k, np.uint32)
        w = np.empty(self.top_k, np.float32)
        L = self.struct()
        check(oracle().fmo_route(isa, ctypes.byref(L), _p(x), _p(h), _p(logits), _p(probs), _p(ids), _p(w)),
              "fmo_route")
        return h, logits, probs, ids, w

    def forward(self, x: np.ndarray, isa: int = ISA_AVX2):
        """One token: (out, ids, weights, h, act[top_k x ffn])."""
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(self.hidden, np.float32)
        ids = np.empty(self.top_k, np.uint32)
        w = np.empty(self.top_k, np.float32)
        h = np.empty(self.hidden, np.float32)
        act = np.empty((self.top_k, self.ffn), np.float32)
        L = self.struct()
        check(oracle().fmo_moe_layer(isa, ctypes.byref(L), _p(x), _p(out), _p(ids), _p(w), _p(h), _p(act)),
              "fmo_moe_layer")
        return out, ids, w, h, act

    def experts_for(self, x: np.ndarray, h: np.ndarray, ids, weights, isa: int = ISA_AVX2) -> np.ndarray:
        """The expert half and the residual for a given routing (ids and
        weights in rank order): x + sum_i w_i * down_i(SwiGLU(gate_i h, up_i h))."""
        x = np.ascontiguousarray(x, np.float32)
        h = np.ascontiguousarray(h, np.float32)
        ids = np.ascontiguousarray(ids, np.uint32)
        weights = np.ascontiguousarray(weights, np.float32)
        if ids.size != self.top_k or weights.size != self.top_k:
            raise ValueError("ids and weights must hold top_k entries")
        out = np.empty(self.hidden, np.float32)
        L = self.struct()
        check(oracle().fmo_moe_experts(isa, ctypes.byref(L), _p(x), _p(h), _p(ids), _p(weights), _p(out), None),
              "fmo_moe_experts")
        return out

    def forward_batch(self, x: np.ndarray, isa: int = ISA_AVX2, threads: int = 1):
        """Every row of x as its own token. `threads` > 1 splits the rows over
        that many threads (the C calls release the GIL; each token's result
        does not depend on the split)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.hidden)
        t = x.shape[0]
        out = np.empty_like(x)
        ids = np.empty((t, self.top_k), np.uint32)
        w = np.empty((t, self.top_k), np.float32)
        L = self.struct()

        def run(a: int, b: int) -> int:
            return oracle().fmo_moe_layer_batch(isa, ctypes.byref(L), _p(x[a:]), _p(out[a:]), _p(ids[a:]),
                                                _p(w[a:]), b - a)

        threads = max(1, min(threads, t))
        if threads == 1:
            check(run(0, t), "fmo_moe_layer_batch")
            return out, ids, w
        from concurrent.futures import ThreadPoolExecutor
        cuts = [t * i // threads for i in range(threads + 1)]
        with ThreadPoolExecutor(threads) as pool:
            rcs = list(pool.map(lambda i: run(cuts[i], cuts[i + 1]), range(threads)))
        for rc in rcs:
            check(rc, "fmo_moe_layer_batch")
        return out, ids, w

    def ref_forward_batch(self, x: np.ndarray, isa: int = ISA_AVX2, threads: int = 0):
        """The same layer through the reference's own kernels (libfmref)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.hidden)
        t = x.shape[0]
        out = np.empty_like(x)
        ids = np.empty((t, self.top_k), np.uint32)
        w = np.empty((t, self.top_k), np.float32)
        L = self.struct()
        check(ref().fmr_moe_layer_batch(isa, threads, ctypes.byref(L), _p(x), _p(out), _p(ids), _p(w), t),
              "fmr_moe_layer_batch")
        return out, ids, w


def host_layer(lw) -> HostLayer:
    """HostLayer from freemoe_amd.workloads.LayerWeights (same arrays, no copies)."""
    return HostLayer(hidden=lw.hidden, ffn=lw.ffn, experts=lw.experts, top_k=lw.top_k,
                     norm_weight=lw.norm_weight, rms_eps=lw.rms_eps, router=lw.router_bytes,
                     router_type=lw.router_type, router_bias=lw.router_bias, gate=lw.gate, up=lw.up,
                     down=lw.down, gate_type=lw.gate_type, down_type=lw.down_type,
                     norm_bias=lw.norm_bias, weights_norm=lw.weights_norm,
                     epsilon_additive=lw.epsilon_additive, weights_epsilon=lw.weights_epsilon,
                     weights_scale=lw.weights_scale)
