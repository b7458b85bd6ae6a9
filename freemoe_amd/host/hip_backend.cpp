// hip_backend.cpp — fm::Backend on MI355X through libfmx (see hip_backend.hpp).
#include "hip_backend.hpp"

#include "fmx.h"

#include <cstring>
#include <vector>

namespace fm {

namespace {

ErrorCode code_of(int status) {
    switch (status) {
    case FMX_ERR_INVALID_ARGUMENT: return ErrorCode::INVALID_ARGUMENT;
    case FMX_ERR_UNSUPPORTED_QUANTISATION: return ErrorCode::UNSUPPORTED_QUANTISATION;
    case FMX_ERR_SHAPE_MISMATCH: return ErrorCode::SHAPE_MISMATCH;
    case FMX_ERR_ALLOCATION_FAILED: return ErrorCode::ALLOCATION_FAILED;
    case FMX_ERR_TRANSFER_FAILED: return ErrorCode::TRANSFER_FAILED;
    case FMX_ERR_FENCE_TIMEOUT: return ErrorCode::FENCE_TIMEOUT;
    case FMX_ERR_DEVICE_LOSS: return ErrorCode::DEVICE_LOSS;
    case FMX_ERR_NO_DEVICE: return ErrorCode::GPU_BACKEND_UNIMPLEMENTED;
    default: return ErrorCode::INTERNAL_ERROR;
    }
}

int fmx_fault_of(BackendFault f) {
    switch (f) {
    case BackendFault::None: return FMX_FAULT_NONE;
    case BackendFault::TransferFailure: return FMX_FAULT_TRANSFER;
    case BackendFault::FenceDeferred: return FMX_FAULT_FENCE_DEFERRED;
    case BackendFault::FenceTimeout: return FMX_FAULT_FENCE_TIMEOUT;
    case BackendFault::DeviceLoss: return FMX_FAULT_DEVICE_LOSS;
    }
    return FMX_FAULT_NONE;
}

} // namespace

HipBackend::HipBackend(BackendConfig config, TraceWriter *trace) : Backend(std::move(config), trace) {
    fmx_device_info info;
    have_device_ = fmx_device_info_get(0, &info) == FMX_OK;
}

HipBackend::~HipBackend() {
    std::lock_guard<std::mutex> lock(mutex_);
    for (auto &f : fences_) fmx_fence_release(f.second);
    for (auto &p : packed_) fmx_free(p.second);
    fmx_free(x_dev_);
    fmx_free(y_dev_);
}

void HipBackend::check(int status, const std::string &where) const {
    if (status != FMX_OK) fail(code_of(status), where + ": " + fmx_status_name(status));
}

DeviceInfo HipBackend::info() const {
    DeviceInfo d;
    d.backend = name();
    fmx_device_info fi;
    if (fmx_device_info_get(0, &fi) != FMX_OK) {
        d.name = "no gfx950 device";
        d.memory_type = "none";
        d.notes = "libfmx found no MI355X (gfx950) device";
        return d;
    }
    d.name = fi.name;
    d.memory_type = "hbm3e";
    d.api_version = "hip";
    d.driver_version = fi.arch;
    d.notes = "expert slots in HBM with pinned host mirrors; kernels for gfx950";
    d.total_memory_bytes = fi.total_memory_bytes;
    d.free_memory_bytes = fi.free_memory_bytes;
    d.dedicated_vram_bytes = fi.total_memory_bytes;
    d.simd_bits = 64 * 32; // one wavefront of 32-bit lanes
    d.threads = fi.compute_units;
    return d;
}

std::unique_ptr<DeviceBuffer> HipBackend::allocate(uint64_t bytes, AllocationTag tag) {
    if (!have_device_) fail(ErrorCode::GPU_BACKEND_UNIMPLEMENTED, "no MI355X (gfx950) device visible");
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    void *host = nullptr, *dev = nullptr;
    check(fmx_host_alloc(bytes, &host), "pinned host mirror");
    const int rc = fmx_alloc(bytes, &dev);
    if (rc != FMX_OK) {
        fmx_host_free(host);
        check(rc, "HBM allocation");
    }
    {
        std::lock_guard<std::mutex> lock(mutex_);
        twins_[reinterpret_cast<uintptr_t>(host)] = Twin{dev, bytes};
    }
    auto buffer = std::make_unique<DeviceBuffer>();
    buffer->data = host;
    buffer->bytes = bytes;
    buffer->tag = tag;
    auto tracker = tracker_;
    buffer->allocation_id = tracker->allocate(tag, bytes);
    // The closure frees this backend's twin too, so buffers must not outlive
    // the backend (the engine and residency release theirs first).
    buffer->cleanup = [this, tracker, id = buffer->allocation_id, host, dev, bytes]() {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            twins_.erase(reinterpret_cast<uintptr_t>(host));
            const uintptr_t lo = reinterpret_cast<uintptr_t>(host);
            for (auto it = packed_.begin(); it != packed_.end();) {
                if (std::get<0>(it->first) >= lo && std::get<0>(it->first) < lo + bytes) {
                    fmx_free(it->second);
                    it = packed_.erase(it);
                } else {
                    ++it;
                }
            }
        }
        tracker->free(id);
        fmx_free(dev);
        fmx_host_free(host);
    };
    return buffer;
}

const HipBackend::Twin *HipBackend::find_twin(const void *host, uint64_t *offset) const {
    const uintptr_t p = reinterpret_cast<uintptr_t>(host);
    auto it = twins_.upper_bound(p);
    if (it == twins_.begin()) return nullptr;
    --it;
    if (p - it->first >= it->second.bytes) return nullptr;
    *offset = p - it->first;
    return &it->second;
}

void *HipBackend::device_address(const void *host) const {
    std::lock_guard<std::mutex> lock(mutex_);
    uint64_t off = 0;
    const Twin *t = find_twin(host, &off);
    return t ? static_cast<uint8_t *>(t->device) + off : nullptr;
}

Fence HipBackend::upload(DeviceBuffer &buffer, const void *src, uint64_t bytes) {
    if (fault_ == BackendFault::TransferFailure) fail(ErrorCode::TRANSFER_FAILED, "injected transfer failure");
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (!buffer.data || bytes > buffer.bytes || (!src && bytes)) fail(ErrorCode::INVALID_ARGUMENT, "bad upload");
    std::lock_guard<std::mutex> lock(mutex_);
    uint64_t off = 0;
    const Twin *t = find_twin(buffer.data, &off);
    if (!t) fail(ErrorCode::INVALID_ARGUMENT, "upload into a buffer this backend did not allocate");
    if (bytes) std::memcpy(buffer.data, src, static_cast<size_t>(bytes));
    // a refilled buffer (an expert slot reused for another expert) drops its packed copies
    const uintptr_t lo = reinterpret_cast<uintptr_t>(buffer.data);
    for (auto it = packed_.begin(); it != packed_.end();) {
        if (std::get<0>(it->first) >= lo && std::get<0>(it->first) < lo + buffer.bytes) {
            fmx_free(it->second);
            it = packed_.erase(it);
        } else {
            ++it;
        }
    }
    void *ev = nullptr;
    check(fmx_upload(static_cast<uint8_t *>(t->device) + off, buffer.data, bytes, stream_, &ev), "upload");
    Fence f;
    f.id = next_fence_++;
    f.ready_at_ms = now_ms();
    f.deferred = fault_ == BackendFault::FenceDeferred;
    fences_[f.id] = ev;
    return f;
}

bool HipBackend::fence_complete(const Fence &fence) const {
    if (fence.deferred && fault_ == BackendFault::FenceDeferred) return false;
    std::lock_guard<std::mutex> lock(mutex_);
    auto it = fences_.find(fence.id);
    if (it == fences_.end()) return true; // already waited on and released
    int done = 0;
    check(fmx_fence_query(it->second, &done), "fence query");
    return done != 0;
}

void HipBackend::wait_fence(const Fence &fence, uint32_t timeout_ms) {
    if (fault_ == BackendFault::FenceTimeout) {
        fault_ = BackendFault::None;
        fmx_clear_faults();
        fail(ErrorCode::FENCE_TIMEOUT, "injected fence timeout");
    }
    void *ev = nullptr;
    {
        std::lock_guard<std::mutex> lock(mutex_);
        auto it = fences_.find(fence.id);
        if (it == fences_.end()) return;
        ev = it->second;
    }
    if (fence.deferred) Backend::wait_fence(fence, timeout_ms); // polls fence_complete until timeout
    check(fmx_fence_wait(ev, timeout_ms), "fence " + std::to_string(fence.id));
    std::lock_guard<std::mutex> lock(mutex_);
    fences_.erase(fence.id);
    fmx_fence_release(ev);
}

void HipBackend::ensure_scratch(uint64_t x_bytes, uint64_t y_bytes) {
    if (x_bytes > x_cap_) {
        fmx_free(x_dev_);
        x_dev_ = nullptr;
        check(fmx_alloc(x_bytes, &x_dev_), "matvec input");
        x_cap_ = x_bytes;
    }
    if (y_bytes > y_cap_) {
        fmx_free(y_dev_);
        y_dev_ = nullptr;
        check(fmx_alloc(y_bytes, &y_dev_), "matvec output");
        y_cap_ = y_bytes;
    }
}

void HipBackend::matvec(const float *weights, const float *x, float *y, uint32_t out_dim, uint32_t in_dim,
                        const std::string &op_name) {
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (!weights || !x || !y || out_dim == 0 || in_dim == 0)
        fail(ErrorCode::INVALID_ARGUMENT, "invalid matvec arguments");
    std::lock_guard<std::mutex> lock(mutex_);
    uint64_t off = 0;
    const Twin *t = find_twin(weights, &off);
    if (!t || off + static_cast<uint64_t>(out_dim) * in_dim * 4 > t->bytes)
        fail(ErrorCode::INVALID_ARGUMENT, "matvec weights are not in a device buffer: " + op_name);
    ensure_scratch(static_cast<uint64_t>(in_dim) * 4, static_cast<uint64_t>(out_dim) * 4);
    check(fmx_upload(x_dev_, x, static_cast<uint64_t>(in_dim) * 4, stream_, nullptr), op_name);
    check(fmx_matvec(FMX_TYPE_F32, static_cast<uint8_t *>(t->device) + off, static_cast<const float *>(x_dev_),
                     static_cast<float *>(y_dev_), out_dim, in_dim, stream_),
          op_name);
    check(fmx_download(y, y_dev_, static_cast<uint64_t>(out_dim) * 4, stream_), op_name);
    record_operation({op_name, name(), (static_cast<uint64_t>(out_dim) * in_dim + in_dim) * sizeof(float),
                      static_cast<uint64_t>(out_dim) * sizeof(float)});
}

void *HipBackend::packed_twin(uint32_t type_id, const void *weights, uint32_t rows, uint32_t cols) {
    const auto key = std::make_tuple(reinterpret_cast<uintptr_t>(weights), type_id, rows, cols);
    auto it = packed_.find(key);
    if (it != packed_.end()) return it->second;
    uint64_t off = 0;
    const Twin *t = find_twin(weights, &off);
    uint32_t bs = 0, bb = 0;
    check(fmx_quant_geometry(type_id, &bs, &bb), "block geometry");
    if (!t || cols % bs || off + static_cast<uint64_t>(rows) * (cols / bs) * bb > t->bytes)
        fail(ErrorCode::INVALID_ARGUMENT, "quantised weights are not in a device buffer");
    const uint64_t n = fmx_packed_bytes(type_id, rows, cols);
    if (n == 0) fail(ErrorCode::SHAPE_MISMATCH, "no packed layout for this shape");
    void *packed = nullptr;
    check(fmx_alloc(n, &packed), "packed weights");
    const int rc = fmx_pack(type_id, static_cast<uint8_t *>(t->device) + off, packed, rows, cols, stream_);
    if (rc != FMX_OK) {
        fmx_free(packed);
        check(rc, "pack");
    }
    packed_[key] = packed;
    return packed;
}

void HipBackend::matvec_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t out_dim,
                              uint32_t in_dim, const std::string &op_name) {
    if (type_id == FMX_TYPE_F32) {
        matvec(static_cast<const float *>(weights), x, y, out_dim, in_dim, op_name);
        return;
    }
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (!weights || !x || !y || out_dim == 0 || in_dim == 0)
        fail(ErrorCode::INVALID_ARGUMENT, "invalid matvec arguments");
    std::lock_guard<std::mutex> lock(mutex_);
    void *packed = packed_twin(type_id, weights, out_dim, in_dim);
    ensure_scratch(static_cast<uint64_t>(in_dim) * 4, static_cast<uint64_t>(out_dim) * 4);
    check(fmx_upload(x_dev_, x, static_cast<uint64_t>(in_dim) * 4, stream_, nullptr), op_name);
    check(fmx_matvec(type_id, packed, static_cast<const float *>(x_dev_), static_cast<float *>(y_dev_), out_dim,
                     in_dim, stream_),
          op_name);
    check(fmx_download(y, y_dev_, static_cast<uint64_t>(out_dim) * 4, stream_), op_name);
    uint32_t bs = 1, bb = 4;
    fmx_quant_geometry(type_id, &bs, &bb);
    record_operation({op_name, name(), static_cast<uint64_t>(out_dim) * (in_dim / bs) * bb + in_dim * 4ull,
                      static_cast<uint64_t>(out_dim) * sizeof(float)});
}

void HipBackend::inject_fault(BackendFault fault) {
    fault_ = fault;
    fmx_inject_fault(fmx_fault_of(fault));
}

void HipBackend::clear_faults() {
    fault_ = BackendFault::None;
    fmx_clear_faults();
}

} // namespace fm
