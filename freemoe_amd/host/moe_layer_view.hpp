// moe_layer_view.hpp — one routed MoE layer, and one token's attention, as
// FreeMoe's engine holds them, for a backend that runs the whole block
// (engine.cpp:1602-1776) or the attention loop (1360-1420) on the device.
//
// Host pointers as the engine has them: weights inside the backend's buffers
// (the fixed-weight buffer, the expert slots); the norm gains and the logit
// bias may also be ordinary host memory (FreeMoe decodes block-type norm and
// bias vectors into host vectors, engine.cpp:223-266). Header-only and free of
// FreeMoe's headers, so FreeMoe's backend.hpp can name it in a virtual.
#pragma once

#include <cstdint>
#include <vector>

namespace fm {

struct MoeLayerView {
    uint32_t layer = 0;
    uint32_t hidden = 0, ffn = 0, experts = 0, top_k = 0;
    const float *norm_weight = nullptr; // [hidden]
    double rms_eps = 1e-5, norm_bias = 0.0;
    uint32_t router_type = 0;
    const void *router = nullptr;       // [experts x hidden] raw rows
    const float *router_bias = nullptr; // [experts], or nullptr
    bool weights_norm = false, epsilon_additive = false;
    double weights_epsilon = 6.103515625e-5, weights_scale = 1.0;
    // Every expert's slot payload (gate | up | down, raw rows, the layout of
    // residency's slots), all resident: the kernels route on the device.
    std::vector<const void *> expert_payloads;
    uint32_t gate_type = 0, up_type = 0, down_type = 0;
};

// One token's attention in one layer: the engine's KV cache (a host pointer
// inside a backend buffer) with `positions` rows written, position t's row at
// kv + t * row_stride floats (every kv head's key, the values at +
// v_offset), and the query [heads x head_dim] the call passes.
struct AttentionView {
    uint32_t layer = 0;
    uint32_t heads = 0, kv_heads = 0, head_dim = 0;
    uint64_t positions = 0;
    double scale = 1.0;
    const float *kv = nullptr;
    uint64_t row_stride = 0;
    uint32_t v_offset = 0;
};

} // namespace fm
