// ref_shim.cpp — C entry points into FreeMoe's own kernels, compiled from the
// FreeMoe sources into oracle/_ref/libfmref.so by oracle/Makefile.
//
// TEST INFRASTRUCTURE ONLY. Used to pin the oracle (tests compare fmoracle's
// restatement with these bit for bit) and as bench.py's CPU baseline
// (cpu_baseline.kind = "reference"): the MoE layer below runs every matvec
// through the reference's gemv / gemv_quant, including its WorkerPool
// threading, and only the O(E + F + H) glue comes from the oracle.
#include "fm/common.hpp"
#include "fm/kernels.hpp"
#include "fm/quant.hpp"

#include "fmoracle.h"

#include <cmath>
#include <cstring>
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

// The decode MoE block per token (engine.cpp:1602-1776, 1822) with the
// reference's kernels for the router and all expert projections.
int fmr_moe_layer_batch(int isa, uint32_t threads, const fmo_layer *L, const float *x,
                        float *out, uint32_t *ids, float *weights, uint32_t tokens) {
    const uint32_t H = L->hidden, F = L->ffn, E = L->experts, K = L->top_k;
    const fm::KernelConfig cfg = config_of(isa, threads);
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
                for (uint32_t j = 0; j < F; ++j) {
                    const double g = gate[j];
                    act[j] = static_cast<float>(g / (1.0 + std::exp(-g))) * up[j];
                }
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

} // extern "C"
