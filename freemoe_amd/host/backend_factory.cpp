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
//
// The unmodified engine also calls two kernels directly instead of through
// its backend: gemv_quant for block-type projections (engine.cpp:355-366)
// and gemm_quant in the dense batched prefill (engine.cpp:2007-2024). Those
// call sites are renamed to the two hooks below. A matrix inside a
// HipBackend buffer runs on the device. Any other matrix belongs to an engine
// on another backend kind: it runs FreeMoe's CPU kernel only when such a
// backend exists in the process; in a process whose every backend is a
// HipBackend it is an INTERNAL_ERROR, since it would mean a GPU engine's
// projection ran on the host. Fallbacks are counted
// (fmx_engine_hook_fallbacks) for the accounting checks.
#include "hip_backend.hpp"

#include "fm/kernels.hpp"

#include <atomic>
#include <memory>

namespace {

std::atomic<uint64_t> g_other_backends{0}; // backends of another kind created so far
std::atomic<uint64_t> g_fallbacks{0};      // hook calls that ran FreeMoe's CPU kernel

void check_fallback(const char *kernel) {
    if (g_other_backends.load() == 0)
        fm::fail(fm::ErrorCode::INTERNAL_ERROR,
                 std::string(kernel) + ": a matrix outside every HipBackend buffer, with no CPU backend in "
                                       "the process (a GPU engine's projection would have run on the host)");
    g_fallbacks.fetch_add(1);
}

} // namespace

namespace fm {

// FreeMoe's own factory, renamed in its object file.
std::unique_ptr<Backend> reference_backend_create(const BackendConfig &config, TraceWriter *trace) __asm__(
    "fmx_reference_backend_create");

std::unique_ptr<Backend> Backend::create(const BackendConfig &config, TraceWriter *trace) {
    if (config.kind == BackendKind::PhysicalGPU) return std::make_unique<HipBackend>(config, trace);
    g_other_backends.fetch_add(1);
    return reference_backend_create(config, trace);
}

} // namespace fm

extern "C" uint64_t fmx_engine_hook_fallbacks() { return g_fallbacks.load(); }

extern "C" void fmx_engine_gemv_quant(const fm::KernelConfig &config, uint32_t type_id, const uint8_t *weights,
                                      const float *x, float *y, uint32_t out_dim, uint32_t in_dim) {
    if (fm::HipBackend *b = fm::HipBackend::owner_of(weights)) {
        b->matvec_quant(type_id, weights, x, y, out_dim, in_dim, "gemv_quant");
        return;
    }
    check_fallback("gemv_quant");
    fm::gemv_quant(config, type_id, weights, x, y, out_dim, in_dim);
}

extern "C" void fmx_engine_gemm_quant(const fm::KernelConfig &config, uint32_t type_id, const uint8_t *weights,
                                      const float *x, float *y, uint32_t tokens, uint32_t out_dim,
                                      uint32_t in_dim) {
    if (fm::HipBackend *b = fm::HipBackend::owner_of(weights)) {
        b->gemm_quant(type_id, weights, x, y, tokens, out_dim, in_dim, "gemm_quant");
        return;
    }
    check_fallback("gemm_quant");
    fm::gemm_quant(config, type_id, weights, x, y, tokens, out_dim, in_dim);
}
