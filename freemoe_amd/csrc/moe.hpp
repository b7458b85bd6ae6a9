// moe.hpp — argument blocks and launchers shared by the MoE entry points.
#pragma once

#include "fmx_internal.hpp"

namespace fmx {

// Routing arguments (device pointers). An F32 router is raw row-major
// (`router`); a block-type router is packed (`router_packed`, geometry `rg`,
// LDS tile of `rtile` blocks) and its rows run the experts' lane chains.
struct RouteArgs {
    uint32_t hidden, experts, top_k;
    const float *norm_weight;
    double rms_eps, norm_bias;
    uint32_t router_type;
    const float *router;
    const void *router_packed;
    PackedGeometry rg;
    uint32_t rtile;
    const float *router_bias;
    int32_t weights_norm, epsilon_additive;
    double weights_epsilon, weights_scale;
};

// Expert projections of one layer: packed geometry of gate/up ([ffn x hidden])
// and down ([hidden x ffn]) plus the LDS tile sizes (in blocks) of each pass.
struct ExpertArgs {
    uint32_t hidden, ffn, experts, top_k;
    uint32_t type_gu, type_dn;
    const void *const *gate;
    const void *const *up;
    const void *const *down;
    PackedGeometry gu, dn;
    uint32_t gu_tile, dn_tile;
    RouteArgs route; // softmax / top-k / weight options, for routing from logits
};

// Device scratch of one decode step (in the caller's workspace).
struct DecodeScratch {
    float *act; // [top_k x ffn] SwiGLU activations
};

// Router logits of `tokens` rows of x ([tokens x experts]); h (optional)
// receives the normalised rows.
int launch_route_logits(const RouteArgs &a, const float *x, uint32_t tokens, float *h, float *logits,
                        hipStream_t s);
// launch_route_logits, then ids / weights ([tokens x top_k]) from the logits.
// clear_status: zero *status first (by the first routing kernel where that
// is the batched RMSNorm, else by a kernel of its own).
int launch_route(const RouteArgs &a, const float *x, uint32_t tokens, float *h, float *logits,
                 uint32_t *ids, float *weights, uint32_t *status, hipStream_t s, bool clear_status = false);
int prepare_expert_args(const fmx_moe_layer *L, const RouteArgs &route, ExpertArgs *a);
// Routing arguments of a layer (geometry and LDS tile of a block-type router).
int prepare_route_args(const fmx_moe_layer *L, RouteArgs *a);
// Decode experts for one token: gate/up + SwiGLU into act[top_k x ffn], then
// down + combine + residual into out[hidden].
// With `logits` ([experts]), the gate/up kernel computes the token's routing
// from them and stores it into ids / w (top_k each) for the down kernel and
// the caller; without, ids / w hold the routing already.
// `kev`, when given, holds four events: the gate/up kernel's start and end
// and the down kernel's start and end, recorded by the launches themselves
// (hipExtLaunchKernelGGL), so that they bracket each kernel's execution.
// The 16-lane Q4_K down kernel (down_pair.hpp) for layers its fit test admits.
int launch_down_pair_q4k(const ExpertArgs &a, const float *x, const float *act, const uint32_t *ids, const float *w,
                         float *out, uint32_t *status, hipStream_t s, const hipEvent_t *kev);
int launch_experts(const ExpertArgs &a, const float *x, const float *h, const float *logits, uint32_t *ids,
                   float *w, const DecodeScratch &ws, float *out, uint32_t *status, hipStream_t s,
                   const hipEvent_t *kev = nullptr);

} // namespace fmx
