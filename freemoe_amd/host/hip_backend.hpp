// hip_backend.hpp — fm::Backend on MI355X through libfmx (include/fmx.h).
//
// The drop-in for FreeMoe's physical-GPU placeholder (src/backend.cpp:528-571):
// same BackendKind::PhysicalGPU, same `--backend gpu`, same fault and error
// codes. It is compiled inside the FreeMoe tree (it includes FreeMoe's own
// headers) and linked with libfmx.so; backend_factory.cpp wires it into
// Backend::create.
//
// Memory. FreeMoe's engine and residency read DeviceBuffer::data on the host
// (engine.cpp:203, 330, 346, 824-836, 1733-1737; residency.cpp:703-719), so
// `data` is a pinned host mirror and each buffer has an HBM twin. upload()
// copies into the mirror and queues the H2D copy of the twin; the fence is the
// HIP event recorded after it. Kernels read the twins; a host pointer anywhere
// inside a buffer resolves to the same offset in its twin.
//
// Lifetime. The twins, packed copies, fences and stream live in a device
// state object that every buffer's cleanup closure shares, as FreeMoe's VNPU
// backend shares its runtime (backend.cpp:441-446): a buffer released after
// its backend still frees its memory on a live device.
#pragma once

#include "fm/backend.hpp"
#include "moe_layer_view.hpp"

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

namespace fm {

class HipBackend final : public Backend {
public:
    explicit HipBackend(BackendConfig config, TraceWriter *trace = nullptr);
    ~HipBackend() override;

    std::string name() const override { return "hip-gfx950"; }
    DeviceInfo info() const override;
    std::unique_ptr<DeviceBuffer> allocate(uint64_t bytes, AllocationTag tag) override;
    Fence upload(DeviceBuffer &buffer, const void *src, uint64_t bytes) override;
    bool fence_complete(const Fence &fence) const override;
    void wait_fence(const Fence &fence, uint32_t timeout_ms) override;
    void matvec(const float *weights, const float *x, float *y, uint32_t out_dim, uint32_t in_dim,
                const std::string &op_name) override;
    void inject_fault(BackendFault fault) override;
    void clear_faults() override;

    // gemv_quant (include/fm/kernels.hpp:79) for a block-type matrix that lives
    // in one of this backend's buffers: the engine's quantised branch of
    // matvec_view (engine.cpp:358-366) calls this instead of the CPU kernels.
    // Logged under this backend's label with the engine's operation name. A
    // matrix outside this backend's buffers is an INVALID_ARGUMENT: there is
    // no CPU fallback. Where FreeMoe's Backend declares the same virtual (the
    // integration's edit), this overrides it.
    void matvec_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t out_dim,
                      uint32_t in_dim, const std::string &op_name);

    // The whole MoE block for one token on the device (fmx_moe_decode):
    // out[hidden] = x + sum_i w_i down_i(SwiGLU(gate_i h, up_i h)) with
    // h = RMSNorm(x); ids / weights receive the routing in rank order (the
    // RoutingEvent's experts). Logs the reference's operation names
    // (router.L*, router_logit_bias.L* with a bias, router_gating.L*,
    // router_topk.L*, expert_gate/up/down.L*.E*, expert_swiglu.L*,
    // expert_combine.L*) under this backend's label. Meant for a call at the
    // top of the engine's routed branch (engine.cpp:1602), which skips the
    // per-expert loop when the layer ran here; returns true (the layer ran)
    // or throws.
    bool moe_layer(const MoeLayerView &layer, const float *x, float *out, uint32_t *ids, float *weights);

    // One token's attention in one layer on the device (fmx_attention_decode):
    // the engine's full-context loop (engine.cpp:1360-1420) for the cache
    // rows the view describes. The cache is a buffer of this backend whose
    // rows the engine writes on the host: the rows written since the last call
    // go to its HBM twin first (one row when the call continues the previous
    // one, every row otherwise). Returns false for a shape the kernel does not
    // take, so the engine runs its own loop. Where FreeMoe's Backend declares
    // the same virtual (the integration's fourth edit), this overrides it.
    bool attention(const AttentionView &view, const float *q, float *out);

    // gemm_quant (include/fm/kernels.hpp:68) for a matrix (raw rows, any
    // supported type) inside one of this backend's buffers: y[t][o] for
    // tokens t, bit for bit the reference's (fmx_gemm_quant). The batched
    // prefill's projections (engine.cpp:2007-2024) call this.
    void gemm_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t tokens,
                    uint32_t out_dim, uint32_t in_dim, const std::string &op_name);

    // Device address of a host pointer inside one of this backend's buffers
    // (nullptr when it is not in one).
    void *device_address(const void *host) const;

    // The live HipBackend whose buffers hold `host`, or nullptr.
    static HipBackend *owner_of(const void *host);

    struct State;

private:
    void check(int status, const std::string &where) const;
    void ensure_scratch(uint64_t x_bytes, uint64_t y_bytes);

    std::shared_ptr<State> state_;
    BackendFault fault_ = BackendFault::None;
};

} // namespace fm
