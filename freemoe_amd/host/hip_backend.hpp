// hip_backend.hpp — fm::Backend on MI355X through libfmx (include/fmx.h).
//
// The drop-in for FreeMoe's physical-GPU placeholder (src/backend.cpp:528-571):
// same BackendKind::PhysicalGPU, same `--backend gpu`, same fault and error
// codes. It is compiled inside the FreeMoe tree (it includes FreeMoe's own
// headers) and linked with libfmx.so; see INTEGRATION.md for the three edits
// that wire it in.
//
// Memory. FreeMoe's engine and residency read DeviceBuffer::data on the host
// (engine.cpp:203, 330, 346, 824-836, 1733-1737; residency.cpp:703-719), so
// `data` is a pinned host mirror and each buffer has an HBM twin. upload()
// copies into the mirror and queues the H2D copy of the twin; the fence is the
// HIP event recorded after it. Kernels read the twins; a host pointer anywhere
// inside a buffer resolves to the same offset in its twin.
#pragma once

#include "fm/backend.hpp"

#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>

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
    void matvec_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t out_dim,
                      uint32_t in_dim, const std::string &op_name);

    // Device address of a host pointer inside one of this backend's buffers
    // (nullptr when it is not in one).
    void *device_address(const void *host) const;

private:
    struct Twin {
        void *device = nullptr;
        uint64_t bytes = 0;
    };
    const Twin *find_twin(const void *host, uint64_t *offset) const;
    void *packed_twin(uint32_t type_id, const void *weights, uint32_t rows, uint32_t cols);
    void ensure_scratch(uint64_t x_bytes, uint64_t y_bytes);
    void check(int status, const std::string &where) const;

    bool have_device_ = false;
    void *stream_ = nullptr;
    mutable std::mutex mutex_;
    std::map<uintptr_t, Twin> twins_;                                           // host mirror start -> twin
    std::map<std::tuple<uintptr_t, uint32_t, uint32_t, uint32_t>, void *> packed_; // packed block matrices
    std::map<uint64_t, void *> fences_;                                         // fence id -> fmx fence
    uint64_t next_fence_ = 1;
    void *x_dev_ = nullptr, *y_dev_ = nullptr;
    uint64_t x_cap_ = 0, y_cap_ = 0;
    BackendFault fault_ = BackendFault::None;
};

} // namespace fm
