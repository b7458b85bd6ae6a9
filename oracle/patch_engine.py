"""Writes copies of FreeMoe's include/fm/backend.hpp, src/backend.cpp and
src/engine.cpp with the integration's edits applied, into a build directory
(oracle/_ref/patched by oracle/Makefile). The FreeMoe tree is only read.

TEST INFRASTRUCTURE ONLY: the patched engine is what a FreeMoe maintainer
would compile after making the edits the integration describes; the tests
run it on HipBackend next to the unedited CPU engine.

    python oracle/patch_engine.py <FreeMoe tree> <output directory>

Edits (each located by a short anchor in the original; the script stops if
an anchor is missing or not unique):

  backend.hpp  four virtuals on fm::Backend: matvec_quant (block-type
               matrix times vector), gemm_quant (the batched product),
               moe_layer (the whole routed block, default: not taken) and
               attention (one token's attention, default: not taken).
  backend.cpp  their defaults: FreeMoe's own gemv_quant / gemm_quant with
               the engine's kernel settings and the engine's op records
               ("cpu-quant", "cpu-batched"), so every CPU backend behaves as
               before.
  engine.cpp   matvec_view's block-type branch (engine.cpp:358-366) and the
               batched prefill's product (2008-2022) call those virtuals; the
               routed MoE branch (1602) first offers the layer to
               Backend::moe_layer and, when the backend ran it, records the
               routing, keeps residency's selected / executed accounting and
               takes the layer's output as the new residual stream; the
               per-token attention loop (1367-1420) is first offered to
               Backend::attention (a fourth virtual, default: declined) for
               the full-context multi-head / grouped-query case.
"""
from __future__ import annotations

import sys
from pathlib import Path


def once(text: str, anchor: str, where: str) -> int:
    n = text.count(anchor)
    if n != 1:
        raise SystemExit(f"patch_engine: anchor found {n} times in {where}: {anchor!r}")
    return text.index(anchor)


def line_start(text: str, at: int) -> int:
    return text.rfind("\n", 0, at) + 1


def line_end(text: str, at: int) -> int:
    e = text.find("\n", at)
    return len(text) if e < 0 else e + 1


def replace_call(text: str, call: str, start_anchor: str, end_anchor: str, new: str, where: str) -> str:
    """Replaces the lines from the last `start_anchor` before `call` through
    the first `end_anchor` after it with `new` (at the first line's indent)."""
    c = once(text, call, where)
    s = text.rfind(start_anchor, 0, c)
    e = text.find(end_anchor, c)
    if s < 0 or e < 0 or c - s > 400 or e - c > 800:
        raise SystemExit(f"patch_engine: {call!r} is not where {where} is expected to hold it")
    s = line_start(text, s)
    indent = text[s:text.index(start_anchor, s)]
    return text[:s] + indent + new + "\n" + text[line_end(text, e):]


BACKEND_HPP_DECL = """struct MoeLayerView;  // moe_layer_view.hpp (fmx integration)
struct AttentionView; // moe_layer_view.hpp (fmx integration)

"""

BACKEND_HPP_VIRTUALS = """    // fmx integration: block-type products and the routed MoE block reach
    // the backend. The defaults are FreeMoe's CPU kernels; moe_layer's
    // default declines, and the engine then runs its own per-expert loop.
    virtual void matvec_quant(uint32_t type_id, const void *weights, const float *x, float *y,
                              uint32_t out_dim, uint32_t in_dim, const std::string &op_name);
    virtual void gemm_quant(uint32_t type_id, const void *weights, const float *x, float *y,
                            uint32_t tokens, uint32_t out_dim, uint32_t in_dim,
                            const std::string &op_name);
    virtual bool moe_layer(const MoeLayerView &layer, const float *x, float *out, uint32_t *ids,
                           float *weights) {
        (void)layer, (void)x, (void)out, (void)ids, (void)weights;
        return false;
    }
    virtual bool attention(const AttentionView &view, const float *q, float *out) {
        (void)view, (void)q, (void)out;
        return false;
    }
"""

BACKEND_CPP_DEFAULTS = """
// fmx integration: the defaults of the three virtuals, FreeMoe's CPU path as
// the engine ran it before the edit (engine.cpp:358-366, 2008-2022).
#include "fm/quant.hpp"

namespace fm {

void Backend::matvec_quant(uint32_t type_id, const void *weights, const float *x, float *y,
                           uint32_t out_dim, uint32_t in_dim, const std::string &op_name) {
    KernelConfig kernels;
    kernels.requested = config_.kernel_isa;
    kernels.threads = config_.kernel_threads;
    gemv_quant(kernels, type_id, static_cast<const uint8_t *>(weights), x, y, out_dim, in_dim);
    record_control(op_name, in_dim * static_cast<uint64_t>(out_dim) * quant_geometry(type_id).block_bytes /
                                quant_geometry(type_id).block_size,
                   out_dim * sizeof(float), "cpu-quant");
}

void Backend::gemm_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t tokens,
                         uint32_t out_dim, uint32_t in_dim, const std::string &op_name) {
    KernelConfig kernels;
    kernels.requested = config_.kernel_isa;
    kernels.threads = config_.kernel_threads;
    // qualified: the free kernel, not this member of the same name
    ::fm::gemm_quant(kernels, type_id, static_cast<const uint8_t *>(weights), x, y, tokens, out_dim, in_dim);
    record_control(op_name,
                   static_cast<uint64_t>(out_dim) * in_dim * tokens *
                       (type_id == 0 ? 4 : quant_geometry(type_id).block_bytes / quant_geometry(type_id).block_size),
                   static_cast<uint64_t>(out_dim) * tokens * sizeof(float), "cpu-batched");
}

} // namespace fm
"""

ENGINE_HOOK = """            // fmx integration: offer the whole routed block to the backend when
            // the block is the one its kernels compute (softmax gating, SwiGLU
            // experts on RMSNorm(x), no selection bias, groups, shared expert,
            // projection biases, post-norm or residual scale) and every expert
            // of the layer fits in the residency slots at once.
            if (c.expert_gating == "softmax" && !c.expert_selection_bias && c.expert_groups <= 1 &&
                !c.shared_expert && !c.expert_projection_bias && !c.post_norms &&
                !c.residual_scale_applied && c.activation == "silu" && !c.layer_norm &&
                !c.weightless_norm && !c.parallel_residual && !c.no_branch_norms &&
                !c.ffn_norm_is_post && !c.ffn_norm_ada && !c.layer_is_recurrent(layer) &&
                residency_->slots().size() >= c.expert_count) {
                const uint32_t E = c.expert_count, K = c.expert_top_k;
                const ExpertRecord *first = manifest_.expert(layer, 0);
                if (first && first->extents[0].type_id == first->extents[1].type_id) {
                    MoeLayerView v;
                    v.layer = layer;
                    v.hidden = c.hidden;
                    v.ffn = c.layer_expert_width(layer);
                    v.experts = E;
                    v.top_k = K;
                    v.norm_weight = norm_weights(prefix + "ffn_norm.weight");
                    v.rms_eps = c.rms_eps;
                    v.norm_bias = norm_bias;
                    const TensorView router_view = tensor_view(prefix + "ffn_router.weight");
                    v.router_type = router_view.type_id;
                    v.router = router_view.data;
                    v.router_bias =
                        c.expert_router_bias ? bias_weights(prefix + "ffn_gate_inp.bias") : nullptr;
                    v.weights_norm = c.expert_weights_norm;
                    v.epsilon_additive = c.expert_weights_epsilon_additive;
                    v.weights_epsilon = c.expert_weights_epsilon;
                    v.weights_scale = c.expert_weights_scale;
                    v.gate_type = first->extents[0].type_id;
                    v.up_type = first->extents[1].type_id;
                    v.down_type = first->extents[2].type_id;
                    std::vector<SlotHandle> held;
                    held.reserve(E);
                    for (uint32_t e = 0; e < E; ++e) {
                        held.push_back(residency_->acquire(layer, e, position, false));
                        v.expert_payloads.push_back(held.back().data());
                    }
                    std::vector<uint32_t> fused_ids(K);
                    std::vector<float> fused_w(K), fused_out(c.hidden);
                    if (backend_->moe_layer(v, x.data(), fused_out.data(), fused_ids.data(),
                                            fused_w.data())) {
                        held.clear();
                        residency_->note_selected(layer, fused_ids, position);
                        if (routing) routing->push_back({position, layer, fused_ids});
                        for (uint32_t expert : fused_ids)
                            residency_->issue_prefetch(layer, expert, position + 1);
                        for (uint32_t expert : fused_ids)
                            residency_->with_expert(layer, expert, position, [](const float *) {});
                        residency_->assert_selected_executed();
                        x = std::move(fused_out);
                        continue;
                    }
                }
            }
"""


ENGINE_ATTENTION_HOOK = """        // fmx integration: offer the attention loop below to the backend for
        // the full-context case its kernel computes (no ALiBi, logit soft-cap,
        // sinks or window; values as wide as keys; not MLA). The cache rows
        // stay where the engine wrote them.
        bool attention_on_backend = false;
        if (alibi_slopes.empty() && !(c.attn_logit_softcap > 0.0) && !c.attn_sinks &&
            !c.layer_uses_window(layer) && !c.mla && c.head_v_dim() == c.head_dim) {
            AttentionView av;
            av.layer = layer;
            av.heads = c.heads;
            av.kv_heads = c.kv_heads;
            av.head_dim = c.head_dim;
            av.positions = position + 1;
            av.scale = scale;
            const uint64_t row0 = c.cache_index(layer, 0, c.context);
            av.kv = kv_ + row0;
            av.row_stride = c.cache_index(layer, 1, c.context) - row0;
            av.v_offset = kv_dim;
            attention_on_backend = backend_->attention(av, q.data(), attention.data());
        }
        if (!attention_on_backend)
"""


def patch(tree: Path, out: Path) -> None:
    hpp = (tree / "include/fm/backend.hpp").read_text()
    at = once(hpp, "class Backend {\n", "backend.hpp")
    hpp = hpp[:at] + BACKEND_HPP_DECL + hpp[at:]
    at = once(hpp, "    virtual void inject_fault(BackendFault fault)", "backend.hpp")
    hpp = hpp[:at] + BACKEND_HPP_VIRTUALS + hpp[at:]

    cpp = (tree / "src/backend.cpp").read_text()
    first_ns = once(cpp, "#include \"fm/backend.hpp\"\n", "backend.cpp")
    cut = line_end(cpp, first_ns)
    cpp = cpp[:cut] + "#include \"fm/kernels.hpp\"\n" + cpp[cut:] + BACKEND_CPP_DEFAULTS

    eng = (tree / "src/engine.cpp").read_text()
    at = once(eng, "#include \"fm/engine.hpp\"\n", "engine.cpp")
    cut = line_end(eng, at)
    eng = eng[:cut] + "#include \"moe_layer_view.hpp\"\n" + eng[cut:]
    eng = replace_call(eng, "gemv_quant(kernels, view.type_id", "KernelConfig kernels;", "\"cpu-quant\");",
                       "backend_->matvec_quant(view.type_id, view.data, x.data(), y.data(), out_dim, in_dim, op);",
                       "engine.cpp matvec_view")
    eng = replace_call(eng, "gemm_quant(kernels, view.type_id", "KernelConfig kernels;", "\"cpu-batched\");",
                       "backend_->gemm_quant(view.type_id, view.data, in.data(), out.data(), batch, out_dim, "
                       "in_dim, op + \".batch\");",
                       "engine.cpp prefill_batch")
    router = once(eng, "tensor_view(prefix + \"ffn_router.weight\")", "engine.cpp routed branch")
    decl = eng.rfind("std::vector<float> scores =", 0, router)
    if decl < 0 or router - decl > 200:
        raise SystemExit("patch_engine: the routed branch does not start where expected")
    s = line_start(eng, decl)
    eng = eng[:s] + ENGINE_HOOK + eng[s:]
    att = once(eng, "std::vector<float> attention(attn_out_dim, 0.0f);", "engine.cpp attention")
    loop = eng.find("        for (uint32_t head = 0; head < c.heads; ++head) {", att)
    if loop < 0 or loop - att > 400:
        raise SystemExit("patch_engine: the attention loop does not follow the attention vector")
    eng = eng[:loop] + ENGINE_ATTENTION_HOOK + eng[loop:]

    (out / "include/fm").mkdir(parents=True, exist_ok=True)
    (out / "src").mkdir(parents=True, exist_ok=True)
    for path, text in ((out / "include/fm/backend.hpp", hpp), (out / "src/backend.cpp", cpp),
                       (out / "src/engine.cpp", eng)):
        if not path.exists() or path.read_text() != text:
            path.write_text(text)


if __name__ == "__main__":
    if len(sys.argv) != 3:
        raise SystemExit(__doc__)
    patch(Path(sys.argv[1]), Path(sys.argv[2]))
