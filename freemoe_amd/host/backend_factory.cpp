// backend_factory.cpp — fm::Backend::create with BackendKind::PhysicalGPU
// served by fm::HipBackend.
//
// FreeMoe's factory (src/backend.cpp:579-586) maps PhysicalGPU to its
// placeholder (backend.cpp:528-571). In a FreeMoe tree the integration is a
// one-line change to that switch (`return std::make_unique<HipBackend>(config,
// trace);`). Where FreeMoe's sources are compiled unmodified, this definition
// takes the factory's symbol instead and the original stays reachable under
// the name `fmx_reference_backend_create` (the object's symbol renamed at link
// time), which serves every other backend kind exactly as before.
#include "hip_backend.hpp"

#include <memory>

namespace fm {

// FreeMoe's own factory, renamed in its object file.
std::unique_ptr<Backend> reference_backend_create(const BackendConfig &config, TraceWriter *trace) __asm__(
    "fmx_reference_backend_create");

std::unique_ptr<Backend> Backend::create(const BackendConfig &config, TraceWriter *trace) {
    if (config.kind == BackendKind::PhysicalGPU) return std::make_unique<HipBackend>(config, trace);
    return reference_backend_create(config, trace);
}

} // namespace fm

extern "C" void fmx_engine_gemv_quant(const fm::KernelConfig &config, uint32_t type_id, const uint8_t *weights,
                                      const float *x, float *y, uint32_t out_dim, uint32_t in_dim) {
    if (fm::HipBackend *b = fm::HipBackend::owner_of(weights)) {
        b->matvec_quant(type_id, weights, x, y, out_dim, in_dim, "gemv_quant");
        return;
    }
    fm::gemv_quant(config, type_id, weights, x, y, out_dim, in_dim);
}

extern "C" void fmx_engine_gemm_quant(const fm::KernelConfig &config, uint32_t type_id, const uint8_t *weights,
                                      const float *x, float *y, uint32_t tokens, uint32_t out_dim,
                                      uint32_t in_dim) {
    if (fm::HipBackend *b = fm::HipBackend::owner_of(weights)) {
        b->gemm_quant(type_id, weights, x, y, tokens, out_dim, in_dim, "gemm_quant");
        return;
    }
    fm::gemm_quant(config, type_id, weights, x, y, tokens, out_dim, in_dim);
}
