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
