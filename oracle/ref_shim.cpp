// ref_shim.cpp — C entry points into FreeMoe's own kernels, compiled from the
// FreeMoe sources into oracle/_ref/libfmref.so by oracle/Makefile.
//
// TEST INFRASTRUCTURE ONLY. Used to pin the oracle (tests compare fmoracle's
// restatement with these bit for bit) and as bench.py's CPU baseline
// (cpu_baseline.kind = "reference"): the MoE layer below runs every matvec
// through the reference's gemv / gemv_quant, including its WorkerPool
// threading, and SwiGLU through the reference's fm::gated_activation; the
// O(E + H) routing glue comes from the oracle. The fmr_engine_* entry points
// run the reference's whole fm::Engine on a checkpoint (its RMSNorm, router,
// softmax, top-k, weights, combine and residual included), for goldens the
// oracle must reproduce.
#include "fm/activation.hpp"
#include "fm/common.hpp"
#include "fm/engine.hpp"
#include "fm/gguf.hpp"
#include "fm/kernels.hpp"
#include "fm/quant.hpp"

#include "fmoracle.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

namespace {

int status_of(const fm::Error &e) {
    switch (e.code) {
    case fm::ErrorCode::INVALID_ARGUMENT: return FMO_ERR_INVALID_ARGUMENT;
    case fm::ErrorCode::UNSUPPORTED_QUANTISATION: return FMO_ERR_UNSUPPORTED_QUANTISATION;
    case fm::ErrorCode::SHAPE_MISMATCH: return FMO_ERR_SHAPE_MISMATCH;
    default: return FMO_ERR_INTERNAL;
    }
}

fm::KernelConfig config_of(int isa, uint32_t threads) {
    fm::KernelConfig c;
    c.requested = isa == FMO_ISA_SCALAR ? fm::KernelIsa::Scalar : fm::KernelIsa::Auto;
    c.threads = threads;
    return c;
}

} // namespace

extern "C" {

float fmr_fp16_to_f32(uint16_t h) { return fm::fp16_to_f32(h); }

int fmr_dequantize_block(uint32_t type_id, const uint8_t *src, float *dst) {
    try {
        fm::dequantize_block(type_id, src, dst);
        return FMO_OK;
    } catch (const fm::Error &e) {
        return status_of(e);
    }
}

// 0 scalar, 1 avx2_fma, 2 avx512: what the reference resolves `isa` to here.
int fmr_resolved_isa(int isa) {
    const fm::KernelIsa r = fm::resolved_isa(config_of(isa, 1));
    return r == fm::KernelIsa::Scalar ? 0 : r == fm::KernelIsa::Avx2Fma ? 1 : 2;
}

uint32_t fmr_resolved_threads(uint32_t threads) {
    return fm::resolved_threads(config_of(FMO_ISA_AVX2, threads));
}

int fmr_gemv(int isa, uint32_t threads, uint32_t type_id, const uint8_t *w, const float *x,
             float *y, uint32_t out_dim, uint32_t in_dim) {
    try {
        fm::gemv_quant(config_of(isa, threads), type_id, w, x, y, out_dim, in_dim);
        return FMO_OK;
    } catch (const fm::Error &e) {
        return status_of(e);
    }
}

int fmr_gemm(int isa, uint32_t threads, uint32_t type_id, const uint8_t *w, const float *x, float *y,
             uint32_t tokens, uint32_t out_dim, uint32_t in_dim) {
    try {
        fm::gemm_quant(config_of(isa, threads), type_id, w, x, y, tokens, out_dim, in_dim);
        return FMO_OK;
    } catch (const fm::Error &e) {
        return status_of(e);
    }
}

// The decode MoE block per token (engine.cpp:1602-1776, 1822) with the
// reference's kernels for the router and all expert projections.
int fmr_moe_layer_batch(int isa, uint32_t threads, const fmo_layer *L, const float *x,
                        float *out, uint32_t *ids, float *weights, uint32_t tokens) {
    const uint32_t H = L->hidden, F = L->ffn, E = L->experts, K = L->top_k;
    const fm::KernelConfig cfg = config_of(isa, threads);
    const fm::ModelConfig activation_cfg; // the default activation: SwiGLU
    std::vector<float> h(H), logits(E), probs(E), gate(F), up(F), act(F), down(H), ffn(H);
    try {
        for (uint32_t t = 0; t < tokens; ++t) {
            const float *xt = x + static_cast<size_t>(t) * H;
            uint32_t *it = ids + static_cast<size_t>(t) * K;
            float *wt = weights + static_cast<size_t>(t) * K;
            int rc = fmo_rmsnorm(xt, L->norm_weight, H, L->rms_eps, L->norm_bias, h.data());
            if (rc) return rc;
            fm::gemv_quant(cfg, L->router_type, L->router, h.data(), logits.data(), E, H);
            if (L->router_bias)
                for (uint32_t e = 0; e < E; ++e) logits[e] += L->router_bias[e];
            rc = fmo_softmax(logits.data(), E, probs.data());
            if (!rc) rc = fmo_topk(probs.data(), E, K, it);
            if (rc) return rc;
            float total = 0.0f;
            for (uint32_t i = 0; i < K; ++i) {
                wt[i] = probs[it[i]];
                total += wt[i];
            }
            if (L->weights_norm) {
                const double den = L->epsilon_additive
                                       ? static_cast<double>(total) + L->weights_epsilon
                                       : std::max(static_cast<double>(total), L->weights_epsilon);
                for (uint32_t i = 0; i < K; ++i) wt[i] = static_cast<float>(wt[i] / den);
            }
            for (uint32_t i = 0; i < K; ++i)
                wt[i] = static_cast<float>(wt[i] * L->weights_scale);
            std::fill(ffn.begin(), ffn.end(), 0.0f);
            for (uint32_t i = 0; i < K; ++i) {
                const uint32_t e = it[i];
                fm::gemv_quant(cfg, L->gate_type, L->gate[e], h.data(), gate.data(), F, H);
                fm::gemv_quant(cfg, L->up_type, L->up[e], h.data(), up.data(), F, H);
                for (uint32_t j = 0; j < F; ++j) act[j] = fm::gated_activation(activation_cfg, gate[j], up[j], 0);
                fm::gemv_quant(cfg, L->down_type, L->down[e], act.data(), down.data(), H, F);
                for (uint32_t j = 0; j < H; ++j) ffn[j] += wt[i] * down[j];
            }
            float *ot = out + static_cast<size_t>(t) * H;
            for (uint32_t j = 0; j < H; ++j) ot[j] = xt[j] + ffn[j];
        }
        return FMO_OK;
    } catch (const fm::Error &e) {
        return status_of(e);
    }
}

// ------------------------------------------------------------ fm::Engine --

struct FmrEngine {
    std::unique_ptr<fm::Engine> engine;
};

// Opens `model_path` with the reference's engine on the scalar CPU backend
// (kernel dispatch `isa`, `threads`; batched prefill off, so every prompt
// token runs forward_token). NULL on failure, with the message in err.
void *fmr_engine_open(const char *model_path, int isa, uint32_t threads, char *err, uint32_t err_cap) {
    try {
        fm::RunConfig rc;
        rc.model_path = model_path;
        rc.backend.kind = fm::BackendKind::ScalarCPU;
        rc.backend.kernel_isa = isa == FMO_ISA_SCALAR ? fm::KernelIsa::Scalar : fm::KernelIsa::Auto;
        rc.backend.kernel_threads = threads;
        rc.backend.batched_prefill = false;
        auto h = std::make_unique<FmrEngine>();
        h->engine = std::make_unique<fm::Engine>(rc);
        h->engine->initialize();
        return h.release();
    } catch (const std::exception &e) {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", e.what());
        return nullptr;
    }
}

void fmr_engine_close(void *handle) { delete static_cast<FmrEngine *>(handle); }

// One prompt (raw bytes) through Engine::run_prompt with `generate` greedy
// tokens. Outputs: the prompt's token ids, the last prompt token's logits,
// the generated ids, and the routing record as rows (position, layer,
// top_k expert ids). Capacities are in elements (routing: rows).
int fmr_engine_prompt(void *handle, const char *prompt, uint32_t prompt_len, uint32_t generate,
                      int32_t *input_ids, uint32_t input_cap, uint32_t *n_input, float *logits,
                      uint32_t vocab_cap, uint32_t *n_vocab, int32_t *generated, uint32_t gen_cap,
                      uint32_t *n_generated, uint32_t *routing, uint32_t routing_cap, uint32_t top_k,
                      uint32_t *n_routing, char *err, uint32_t err_cap) {
    try {
        fm::Engine &e = *static_cast<FmrEngine *>(handle)->engine;
        const fm::PromptResult r = e.run_prompt(std::string(prompt, prompt_len), generate);
        if (r.input_ids.size() > input_cap || r.prefill_logits.size() > vocab_cap ||
            r.generated_ids.size() > gen_cap || r.routing.size() > routing_cap)
            return FMO_ERR_INVALID_ARGUMENT;
        *n_input = static_cast<uint32_t>(r.input_ids.size());
        std::memcpy(input_ids, r.input_ids.data(), r.input_ids.size() * sizeof(int32_t));
        *n_vocab = static_cast<uint32_t>(r.prefill_logits.size());
        std::memcpy(logits, r.prefill_logits.data(), r.prefill_logits.size() * sizeof(float));
        *n_generated = static_cast<uint32_t>(r.generated_ids.size());
        std::memcpy(generated, r.generated_ids.data(), r.generated_ids.size() * sizeof(int32_t));
        *n_routing = static_cast<uint32_t>(r.routing.size());
        for (size_t i = 0; i < r.routing.size(); ++i) {
            const fm::RoutingEvent &ev = r.routing[i];
            if (ev.experts.size() != top_k) return FMO_ERR_SHAPE_MISMATCH;
            uint32_t *row = routing + i * (2 + top_k);
            row[0] = static_cast<uint32_t>(ev.token_index);
            row[1] = ev.layer;
            for (uint32_t k = 0; k < top_k; ++k) row[2 + k] = ev.experts[k];
        }
        return FMO_OK;
    } catch (const fm::Error &ex) {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", ex.what());
        return status_of(ex);
    } catch (const std::exception &ex) {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", ex.what());
        return FMO_ERR_INTERNAL;
    }
}

// The reference's parser and adapter on a checkpoint file (parse_gguf over
// the mapped file, then build_manifest): info = {layers, expert_count, top_k,
// hidden, records, slot_bytes (2 words: low, high), fixed_weight_bytes (low,
// high)}; extents[record][projection] = {offset, bytes, type_id} for up to
// `cap` expert records in manifest order, with the record's (layer, expert)
// in who[record].
int fmr_manifest_probe(const char *path, uint32_t *info, uint64_t *extents, uint32_t *who, uint32_t cap,
                       char *err, uint32_t err_cap) {
    try {
        const fm::GGUFDocument doc = fm::parse_gguf_file(path);
        const fm::ModelManifest m = fm::build_manifest(doc, path);
        info[0] = m.config.layers;
        info[1] = m.config.expert_count;
        info[2] = m.config.expert_top_k;
        info[3] = m.config.hidden;
        info[4] = static_cast<uint32_t>(m.experts.size());
        info[5] = static_cast<uint32_t>(m.slot_bytes);
        info[6] = static_cast<uint32_t>(m.slot_bytes >> 32);
        info[7] = static_cast<uint32_t>(m.fixed_weight_bytes);
        info[8] = static_cast<uint32_t>(m.fixed_weight_bytes >> 32);
        for (size_t i = 0; i < m.experts.size() && i < cap; ++i) {
            who[2 * i] = m.experts[i].layer;
            who[2 * i + 1] = m.experts[i].expert;
            for (int r = 0; r < 3; ++r) {
                uint64_t *x = extents + (i * 3 + r) * 3;
                x[0] = m.experts[i].extents[r].offset;
                x[1] = m.experts[i].extents[r].bytes;
                x[2] = m.experts[i].extents[r].type_id;
            }
        }
        return FMO_OK;
    } catch (const fm::Error &ex) {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", ex.what());
        return status_of(ex);
    } catch (const std::exception &ex) {
        if (err && err_cap) std::snprintf(err, err_cap, "%s", ex.what());
        return FMO_ERR_INTERNAL;
    }
}

} // extern "C"
