// hip_backend.cpp — fm::Backend on MI355X through libfmx (see hip_backend.hpp).
#include "hip_backend.hpp"

#include "fm/kernels.hpp"
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

void check_status(int status, const std::string &where) {
    if (status != FMX_OK) fail(code_of(status), where + ": " + fmx_status_name(status));
}

uint64_t raw_bytes(uint32_t type_id, uint32_t rows, uint32_t cols) {
    uint32_t bs = 0, bb = 0;
    if (fmx_quant_geometry(type_id, &bs, &bb) != FMX_OK || cols % bs) return 0;
    return static_cast<uint64_t>(rows) * (cols / bs) * bb;
}

} // namespace

// Device-side state shared by the backend and every buffer it hands out.
struct HipBackend::State {
    struct Twin {
        void *device = nullptr;
        uint64_t bytes = 0;
    };
    std::mutex mutex;
    std::map<uintptr_t, Twin> twins;                                           // host mirror start -> twin
    std::map<std::tuple<uintptr_t, uint32_t, uint32_t, uint32_t>, void *> packed; // packed block matrices
    std::map<uint64_t, void *> fences;                                         // fence id -> fmx fence
    uint64_t next_fence = 1;
    void *stream = nullptr; // the default stream
    bool have_device = false;
    // matvec / MoE scratch
    void *x_dev = nullptr, *y_dev = nullptr;
    uint64_t x_cap = 0, y_cap = 0;
    void *moe_ws = nullptr, *moe_small = nullptr;
    uint64_t moe_ws_cap = 0, moe_small_cap = 0;
    std::map<std::vector<uintptr_t>, void *> slot_tables; // packed expert pointers -> device table
    // KV caches seen by attention(): per layer cache (its row 0's host
    // address), the position count of the last call and a copy of the last
    // row it uploaded
    struct KvSync {
        uint64_t positions = 0;
        std::vector<float> last_row;
    };
    std::map<uintptr_t, KvSync> kv_sync;
    void *attn_status = nullptr;
    // pinned host staging of a call's inputs and outputs (the engine's
    // vectors are pageable): one copy in and one out per call
    void *stage_in = nullptr, *stage_out = nullptr;
    uint64_t stage_in_cap = 0, stage_out_cap = 0;
    // pinned host word receiving a fused call's device error word, read in
    // the same synchronisation as the call's outputs
    void *status_word = nullptr;
    uint64_t status_word_cap = 0;

    uint8_t *pinned(void *&buf, uint64_t &cap, uint64_t bytes) {
        if (bytes > cap) {
            fmx_host_free(buf);
            buf = nullptr;
            cap = 0;
            check_status(fmx_host_alloc(bytes, &buf), "pinned staging");
            cap = bytes;
        }
        return static_cast<uint8_t *>(buf);
    }
    // bytes of src to device dst through the pinned input staging; the copy
    // is queued on the stream (a later download's synchronisation covers it)
    void upload_staged(void *dst, const void *src, uint64_t bytes) {
        uint8_t *h = pinned(stage_in, stage_in_cap, bytes);
        std::memcpy(h, src, static_cast<size_t>(bytes));
        check_status(fmx_upload(dst, h, bytes, stream, nullptr), "staged upload");
    }
    // bytes of device src to dst through the pinned output staging (waits)
    void download_staged(void *dst, const void *src, uint64_t bytes) {
        uint8_t *h = pinned(stage_out, stage_out_cap, bytes);
        check_status(fmx_download(h, src, bytes, stream), "staged download");
        std::memcpy(dst, h, static_cast<size_t>(bytes));
    }

    ~State() {
        for (auto &f : fences) fmx_fence_release(f.second);
        for (auto &p : packed) fmx_free(p.second);
        for (auto &t : slot_tables) fmx_free(t.second);
        fmx_free(x_dev);
        fmx_free(y_dev);
        fmx_free(moe_ws);
        fmx_free(moe_small);
        fmx_free(attn_status);
        fmx_host_free(stage_in);
        fmx_host_free(stage_out);
        fmx_host_free(status_word);
    }

    const Twin *find_twin(const void *host, uint64_t *offset) const {
        const uintptr_t p = reinterpret_cast<uintptr_t>(host);
        auto it = twins.upper_bound(p);
        if (it == twins.begin()) return nullptr;
        --it;
        if (p - it->first >= it->second.bytes) return nullptr;
        *offset = p - it->first;
        return &it->second;
    }

    // Drops the packed copies (and the slot tables that point at them) of
    // matrices inside [lo, lo + bytes): the buffer was refilled or released.
    void drop_packed(uintptr_t lo, uint64_t bytes) {
        bool dropped = false;
        for (auto it = packed.begin(); it != packed.end();) {
            if (std::get<0>(it->first) >= lo && std::get<0>(it->first) < lo + bytes) {
                fmx_free(it->second);
                it = packed.erase(it);
                dropped = true;
            } else {
                ++it;
            }
        }
        if (dropped) {
            for (auto &t : slot_tables) fmx_free(t.second);
            slot_tables.clear();
        }
    }

    // The packed device copy of a [rows x cols] matrix of `type_id` stored in a
    // buffer at host address `weights` (made once, kept until the buffer is
    // refilled or released). F32 copies are 16-byte aligned raw copies.
    void *packed_twin(uint32_t type_id, const void *weights, uint32_t rows, uint32_t cols) {
        const auto key = std::make_tuple(reinterpret_cast<uintptr_t>(weights), type_id, rows, cols);
        auto it = packed.find(key);
        if (it != packed.end()) return it->second;
        uint64_t off = 0;
        const Twin *t = find_twin(weights, &off);
        const uint64_t need = raw_bytes(type_id, rows, cols);
        if (!t || need == 0 || off + need > t->bytes)
            fail(ErrorCode::INVALID_ARGUMENT, "weights are not in a device buffer of this backend");
        const uint64_t n = fmx_packed_bytes(type_id, rows, cols);
        if (n == 0) fail(ErrorCode::SHAPE_MISMATCH, "no packed layout for this shape");
        void *p = nullptr;
        check_status(fmx_alloc(n, &p), "packed weights");
        const int rc = fmx_pack(type_id, static_cast<uint8_t *>(t->device) + off, p, rows, cols, stream);
        if (rc != FMX_OK) {
            fmx_free(p);
            check_status(rc, "pack");
        }
        packed[key] = p;
        return p;
    }
};

namespace {

// Live backends, for owner_of.
std::mutex g_backends_mutex;
std::vector<HipBackend *> g_backends;

} // namespace

HipBackend::HipBackend(BackendConfig config, TraceWriter *trace)
    : Backend(std::move(config), trace), state_(std::make_shared<State>()) {
    // The device kernels reproduce the summation order KernelIsa::Auto
    // resolves to on an AVX2+FMA host (kernels.cpp:147-174, 639-771); the
    // scalar and AVX-512 orders exist only on the CPU backend, so asking for
    // them here is refused rather than answered in another order.
    if (config_.kernel_isa != KernelIsa::Auto && config_.kernel_isa != KernelIsa::Avx2Fma)
        fail(ErrorCode::INVALID_ARGUMENT, std::string("hip-gfx950 computes the avx2_fma order; kernel ISA '") +
                                              kernel_isa_name(config_.kernel_isa) + "' runs on the CPU backend");
    fmx_device_info fi;
    state_->have_device = fmx_device_info_get(0, &fi) == FMX_OK;
    std::lock_guard<std::mutex> lock(g_backends_mutex);
    g_backends.push_back(this);
}

HipBackend::~HipBackend() { // buffers still out hold the state
    std::lock_guard<std::mutex> lock(g_backends_mutex);
    for (auto it = g_backends.begin(); it != g_backends.end(); ++it)
        if (*it == this) {
            g_backends.erase(it);
            break;
        }
}

HipBackend *HipBackend::owner_of(const void *host) {
    std::lock_guard<std::mutex> lock(g_backends_mutex);
    for (HipBackend *b : g_backends) {
        std::lock_guard<std::mutex> state_lock(b->state_->mutex);
        uint64_t off = 0;
        if (b->state_->find_twin(host, &off)) return b;
    }
    return nullptr;
}

void HipBackend::check(int status, const std::string &where) const { check_status(status, where); }

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
    if (!state_->have_device) fail(ErrorCode::GPU_BACKEND_UNIMPLEMENTED, "no MI355X (gfx950) device visible");
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    void *host = nullptr, *dev = nullptr;
    check(fmx_host_alloc(bytes, &host), "pinned host mirror");
    const int rc = fmx_alloc(bytes, &dev);
    if (rc != FMX_OK) {
        fmx_host_free(host);
        check(rc, "HBM allocation");
    }
    {
        std::lock_guard<std::mutex> lock(state_->mutex);
        state_->twins[reinterpret_cast<uintptr_t>(host)] = State::Twin{dev, bytes};
    }
    auto buffer = std::make_unique<DeviceBuffer>();
    buffer->data = host;
    buffer->bytes = bytes;
    buffer->tag = tag;
    auto tracker = tracker_;
    buffer->allocation_id = tracker->allocate(tag, bytes);
    buffer->cleanup = [state = state_, tracker, id = buffer->allocation_id, host, dev, bytes]() {
        {
            std::lock_guard<std::mutex> lock(state->mutex);
            state->twins.erase(reinterpret_cast<uintptr_t>(host));
            state->drop_packed(reinterpret_cast<uintptr_t>(host), bytes);
        }
        tracker->free(id);
        fmx_free(dev);
        fmx_host_free(host);
    };
    return buffer;
}

void *HipBackend::device_address(const void *host) const {
    std::lock_guard<std::mutex> lock(state_->mutex);
    uint64_t off = 0;
    const State::Twin *t = state_->find_twin(host, &off);
    return t ? static_cast<uint8_t *>(t->device) + off : nullptr;
}

Fence HipBackend::upload(DeviceBuffer &buffer, const void *src, uint64_t bytes) {
    if (fault_ == BackendFault::TransferFailure) fail(ErrorCode::TRANSFER_FAILED, "injected transfer failure");
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (!buffer.data || bytes > buffer.bytes || (!src && bytes)) fail(ErrorCode::INVALID_ARGUMENT, "bad upload");
    std::lock_guard<std::mutex> lock(state_->mutex);
    uint64_t off = 0;
    const State::Twin *t = state_->find_twin(buffer.data, &off);
    if (!t) fail(ErrorCode::INVALID_ARGUMENT, "upload into a buffer this backend did not allocate");
    if (bytes) std::memcpy(buffer.data, src, static_cast<size_t>(bytes));
    // a refilled buffer (an expert slot reused for another expert) drops its packed copies
    state_->drop_packed(reinterpret_cast<uintptr_t>(buffer.data), buffer.bytes);
    void *ev = nullptr;
    check(fmx_upload(static_cast<uint8_t *>(t->device) + off, buffer.data, bytes, state_->stream, &ev), "upload");
    Fence f;
    f.id = state_->next_fence++;
    f.ready_at_ms = now_ms();
    f.deferred = fault_ == BackendFault::FenceDeferred;
    state_->fences[f.id] = ev;
    return f;
}

bool HipBackend::fence_complete(const Fence &fence) const {
    if (fence.deferred && fault_ == BackendFault::FenceDeferred) return false;
    std::lock_guard<std::mutex> lock(state_->mutex);
    auto it = state_->fences.find(fence.id);
    if (it == state_->fences.end()) return true; // already waited on and released
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
        std::lock_guard<std::mutex> lock(state_->mutex);
        auto it = state_->fences.find(fence.id);
        if (it == state_->fences.end()) return;
        ev = it->second;
    }
    if (fence.deferred) Backend::wait_fence(fence, timeout_ms); // polls fence_complete until timeout
    check(fmx_fence_wait(ev, timeout_ms), "fence " + std::to_string(fence.id));
    std::lock_guard<std::mutex> lock(state_->mutex);
    state_->fences.erase(fence.id);
    fmx_fence_release(ev);
}

void HipBackend::ensure_scratch(uint64_t x_bytes, uint64_t y_bytes) {
    State &s = *state_;
    if (x_bytes > s.x_cap) {
        fmx_free(s.x_dev);
        s.x_dev = nullptr;
        s.x_cap = 0;
        check(fmx_alloc(x_bytes, &s.x_dev), "matvec input");
        s.x_cap = x_bytes;
    }
    if (y_bytes > s.y_cap) {
        fmx_free(s.y_dev);
        s.y_dev = nullptr;
        s.y_cap = 0;
        check(fmx_alloc(y_bytes, &s.y_dev), "matvec output");
        s.y_cap = y_bytes;
    }
}

void HipBackend::matvec(const float *weights, const float *x, float *y, uint32_t out_dim, uint32_t in_dim,
                        const std::string &op_name) {
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (!weights || !x || !y || out_dim == 0 || in_dim == 0)
        fail(ErrorCode::INVALID_ARGUMENT, "invalid matvec arguments");
    std::lock_guard<std::mutex> lock(state_->mutex);
    State &s = *state_;
    uint64_t off = 0;
    const State::Twin *t = s.find_twin(weights, &off);
    if (!t || off + static_cast<uint64_t>(out_dim) * in_dim * 4 > t->bytes)
        fail(ErrorCode::INVALID_ARGUMENT, "matvec weights are not in a device buffer: " + op_name);
    ensure_scratch(static_cast<uint64_t>(in_dim) * 4, static_cast<uint64_t>(out_dim) * 4);
    s.upload_staged(s.x_dev, x, static_cast<uint64_t>(in_dim) * 4);
    check(fmx_matvec(FMX_TYPE_F32, static_cast<uint8_t *>(t->device) + off, static_cast<const float *>(s.x_dev),
                     static_cast<float *>(s.y_dev), out_dim, in_dim, s.stream),
          op_name);
    s.download_staged(y, s.y_dev, static_cast<uint64_t>(out_dim) * 4);
    record_operation({op_name, name(), (static_cast<uint64_t>(out_dim) * in_dim + in_dim) * sizeof(float),
                      static_cast<uint64_t>(out_dim) * sizeof(float)});
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
    std::lock_guard<std::mutex> lock(state_->mutex);
    State &s = *state_;
    void *packed = s.packed_twin(type_id, weights, out_dim, in_dim);
    ensure_scratch(static_cast<uint64_t>(in_dim) * 4, static_cast<uint64_t>(out_dim) * 4);
    s.upload_staged(s.x_dev, x, static_cast<uint64_t>(in_dim) * 4);
    check(fmx_matvec(type_id, packed, static_cast<const float *>(s.x_dev), static_cast<float *>(s.y_dev), out_dim,
                     in_dim, s.stream),
          op_name);
    s.download_staged(y, s.y_dev, static_cast<uint64_t>(out_dim) * 4);
    record_operation({op_name, name(), raw_bytes(type_id, out_dim, in_dim) + in_dim * 4ull,
                      static_cast<uint64_t>(out_dim) * sizeof(float)});
}

void HipBackend::gemm_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t tokens,
                            uint32_t out_dim, uint32_t in_dim, const std::string &op_name) {
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (tokens == 0 || out_dim == 0 || in_dim == 0) return;
    if (!weights || !x || !y) fail(ErrorCode::INVALID_ARGUMENT, "invalid batched product arguments");
    uint32_t bs = 0, bb = 0;
    if (fmx_quant_geometry(type_id, &bs, &bb) != FMX_OK)
        fail(ErrorCode::UNSUPPORTED_QUANTISATION, "no kernel for tensor type " + std::to_string(type_id));
    if (in_dim % bs) fail(ErrorCode::SHAPE_MISMATCH, "quantised row length is not a whole number of blocks");
    const uint64_t w_bytes = raw_bytes(type_id, out_dim, in_dim);
    std::lock_guard<std::mutex> lock(state_->mutex);
    State &s = *state_;
    uint64_t off = 0;
    const State::Twin *t = s.find_twin(weights, &off);
    if (!t || off + w_bytes > t->bytes)
        fail(ErrorCode::INVALID_ARGUMENT, "batched product weights are not in a device buffer: " + op_name);
    const uint64_t x_bytes = static_cast<uint64_t>(tokens) * in_dim * 4, y_bytes = static_cast<uint64_t>(tokens) * out_dim * 4;
    ensure_scratch(x_bytes, y_bytes);
    s.upload_staged(s.x_dev, x, x_bytes);
    check(fmx_gemm_quant(type_id, static_cast<uint8_t *>(t->device) + off, static_cast<const float *>(s.x_dev),
                         static_cast<float *>(s.y_dev), tokens, out_dim, in_dim, s.stream),
          op_name);
    s.download_staged(y, s.y_dev, y_bytes);
    record_operation({op_name, name(), w_bytes + x_bytes, y_bytes});
}

bool HipBackend::moe_layer(const MoeLayerView &L, const float *x, float *out, uint32_t *ids, float *weights) {
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    const uint32_t H = L.hidden, F = L.ffn, E = L.experts, K = L.top_k;
    if (!x || !out || !ids || !weights || !L.router || H == 0 || F == 0 || E == 0 || K == 0 || K > E ||
        L.expert_payloads.size() != E)
        fail(ErrorCode::INVALID_ARGUMENT, "invalid MoE layer arguments");
    // a layer the fused kernels do not take is declined (false): the engine
    // then runs its own per-expert loop, whose projections still come here
    if (L.up_type != L.gate_type) return false;
    const uint64_t gate_bytes = raw_bytes(L.gate_type, F, H), down_bytes = raw_bytes(L.down_type, H, F);
    const uint64_t router_bytes = raw_bytes(L.router_type, E, H);
    if (gate_bytes == 0 || down_bytes == 0 || router_bytes == 0) return false;
    {
        // the library's own layer checks, on stand-in addresses
        alignas(16) static const uint64_t probe[4] = {};
        fmx_moe_layer d{};
        d.hidden = H;
        d.ffn = F;
        d.experts = E;
        d.top_k = K;
        d.router_type = L.router_type;
        d.router = probe;
        d.gate_type = d.up_type = L.gate_type;
        d.down_type = L.down_type;
        d.gate = d.up = d.down = reinterpret_cast<const void *const *>(probe);
        if (fmx_moe_workspace_bytes(&d, 1) == 0) return false;
    }
    const std::string l = std::to_string(L.layer);

    std::lock_guard<std::mutex> lock(state_->mutex);
    State &s = *state_;
    // the experts' packed slots and the device table of their addresses
    std::vector<uintptr_t> key;
    key.reserve(3 * E);
    for (uint32_t e = 0; e < E; ++e) {
        const uint8_t *base = static_cast<const uint8_t *>(L.expert_payloads[e]);
        key.push_back(reinterpret_cast<uintptr_t>(s.packed_twin(L.gate_type, base, F, H)));
        key.push_back(reinterpret_cast<uintptr_t>(s.packed_twin(L.up_type, base + gate_bytes, F, H)));
        key.push_back(reinterpret_cast<uintptr_t>(s.packed_twin(L.down_type, base + 2 * gate_bytes, H, F)));
    }
    void *table = nullptr;
    auto tit = s.slot_tables.find(key);
    if (tit != s.slot_tables.end()) {
        table = tit->second;
    } else {
        std::vector<uint64_t> host(3 * E);
        for (uint32_t e = 0; e < E; ++e)
            for (uint32_t r = 0; r < 3; ++r) host[r * E + e] = key[3 * e + r];
        check(fmx_alloc(host.size() * 8, &table), "expert slot table");
        const int rc = fmx_upload(table, host.data(), host.size() * 8, s.stream, nullptr);
        if (rc == FMX_OK) check(fmx_stream_sync(s.stream), "expert slot table");
        if (rc != FMX_OK) {
            fmx_free(table);
            check(rc, "expert slot table");
        }
        s.slot_tables[key] = table;
    }
    void *router = s.packed_twin(L.router_type, L.router, E, H);

    // small per-call inputs and outputs: x, the norm gains (when not resident
    // in a buffer), the logit bias, out, ids, weights
    const uint64_t o_x = 0, o_norm = o_x + ((H * 4ull + 255) & ~255ull), o_bias = o_norm + ((H * 4ull + 255) & ~255ull),
                   o_out = o_bias + ((E * 4ull + 255) & ~255ull), o_ids = o_out + ((H * 4ull + 255) & ~255ull),
                   o_w = o_ids + 256, small = o_w + 256;
    if (K > 64) fail(ErrorCode::INVALID_ARGUMENT, "top_k above 64");
    if (small > s.moe_small_cap) {
        fmx_free(s.moe_small);
        s.moe_small = nullptr;
        s.moe_small_cap = 0;
        check(fmx_alloc(small, &s.moe_small), "MoE inputs");
        s.moe_small_cap = small;
    }
    uint8_t *sm = static_cast<uint8_t *>(s.moe_small);
    // x, the norm gains (when not resident in a buffer) and the logit bias go
    // up in one copy of the block [x | norm | bias] as laid out on the device
    uint8_t *hin = s.pinned(s.stage_in, s.stage_in_cap, o_out);
    const float *norm_dev = nullptr;
    uint64_t in_bytes = H * 4ull;
    std::memcpy(hin + o_x, x, H * 4ull);
    if (L.norm_weight) {
        uint64_t off = 0;
        const State::Twin *t = s.find_twin(L.norm_weight, &off);
        const uintptr_t addr = t ? reinterpret_cast<uintptr_t>(t->device) + off : 0;
        if (t && off + H * 4ull <= t->bytes && addr % 16 == 0) {
            norm_dev = reinterpret_cast<const float *>(addr);
        } else {
            std::memcpy(hin + o_norm, L.norm_weight, H * 4ull);
            in_bytes = o_norm + H * 4ull;
            norm_dev = reinterpret_cast<const float *>(sm + o_norm);
        }
    }
    if (L.router_bias) {
        std::memcpy(hin + o_bias, L.router_bias, E * 4ull);
        in_bytes = o_bias + E * 4ull;
    }
    check(fmx_upload(sm + o_x, hin + o_x, in_bytes, s.stream, nullptr), "MoE inputs");

    fmx_moe_layer d;
    std::memset(&d, 0, sizeof(d));
    d.hidden = H;
    d.ffn = F;
    d.experts = E;
    d.top_k = K;
    d.norm_weight = norm_dev;
    d.rms_eps = L.rms_eps;
    d.norm_bias = L.norm_bias;
    d.router_type = L.router_type;
    d.router = router;
    d.router_bias = L.router_bias ? reinterpret_cast<const float *>(sm + o_bias) : nullptr;
    d.weights_norm = L.weights_norm ? 1 : 0;
    d.epsilon_additive = L.epsilon_additive ? 1 : 0;
    d.weights_epsilon = L.weights_epsilon;
    d.weights_scale = L.weights_scale;
    d.gate_type = L.gate_type;
    d.up_type = L.up_type;
    d.down_type = L.down_type;
    const void *const *tab = static_cast<const void *const *>(table);
    d.gate = tab;
    d.up = tab + E;
    d.down = tab + 2 * E;
    const uint64_t ws = fmx_moe_workspace_bytes(&d, 1);
    if (ws == 0) fail(ErrorCode::SHAPE_MISMATCH, "MoE layer shape not supported");
    if (ws > s.moe_ws_cap) {
        fmx_free(s.moe_ws);
        s.moe_ws = nullptr;
        s.moe_ws_cap = 0;
        check(fmx_alloc(ws, &s.moe_ws), "MoE workspace");
        s.moe_ws_cap = ws;
    }
    check(fmx_moe_decode(&d, reinterpret_cast<const float *>(sm + o_x), reinterpret_cast<float *>(sm + o_out), 1,
                         reinterpret_cast<uint32_t *>(sm + o_ids), reinterpret_cast<float *>(sm + o_w), s.moe_ws,
                         s.moe_ws_cap, s.stream),
          "moe layer " + l);
    // the error word comes back with the outputs (one synchronisation)
    uint32_t *word = reinterpret_cast<uint32_t *>(s.pinned(s.status_word, s.status_word_cap, 4));
    check(fmx_moe_status_copy(s.moe_ws, word, s.stream), "router scores of layer " + l);
    {
        // out, ids and weights back in one copy of [out | ids | weights]
        uint8_t *hout = s.pinned(s.stage_out, s.stage_out_cap, small - o_out);
        check(fmx_download(hout, sm + o_out, o_w + K * 4ull - o_out, s.stream), "MoE outputs");
        std::memcpy(out, hout, H * 4ull);
        std::memcpy(ids, hout + (o_ids - o_out), K * 4ull);
        std::memcpy(weights, hout + (o_w - o_out), K * 4ull);
    }
    check(fmx_moe_status_of(*word), "router scores of layer " + l);

    // the reference's operation log for this block (engine.cpp:1603-1776)
    record_operation({"router.L" + l, name(), router_bytes + H * 4ull, E * 4ull});
    if (L.router_bias) record_control("router_logit_bias.L" + l, E * 4ull, 0, name());
    record_control("router_gating.L" + l, E * 4ull, E * 4ull, name());
    record_control("router_topk.L" + l, E * 4ull, K * 4ull, name());
    for (uint32_t i = 0; i < K; ++i) {
        const std::string ex = ".L" + l + ".E" + std::to_string(ids[i]);
        record_operation({"expert_gate" + ex, name(), gate_bytes + H * 4ull, F * 4ull});
        record_operation({"expert_up" + ex, name(), gate_bytes + H * 4ull, F * 4ull});
        record_control("expert_swiglu.L" + l, 2 * F * 4ull, F * 4ull, name());
        record_operation({"expert_down" + ex, name(), down_bytes + F * 4ull, H * 4ull});
    }
    record_control("expert_combine.L" + l, K * H * 4ull, H * 4ull, name());
    return true;
}

bool HipBackend::attention(const AttentionView &A, const float *q, float *out) {
    if (fault_ == BackendFault::DeviceLoss) fail(ErrorCode::DEVICE_LOSS, "injected device loss");
    if (!q || !out || !A.kv || A.positions == 0 || A.heads == 0 || A.head_dim == 0)
        fail(ErrorCode::INVALID_ARGUMENT, "invalid attention arguments");
    const uint64_t P = A.positions, D = A.head_dim, H = A.heads;
    // shapes fmx_attention_decode does not take run the engine's own loop
    if (P > 8192 || D > 256 || D % 4 || A.kv_heads == 0 || H % A.kv_heads || A.row_stride % 4 || A.v_offset % 4 ||
        A.v_offset < A.kv_heads * D || A.v_offset + A.kv_heads * D > A.row_stride)
        return false;
    std::lock_guard<std::mutex> lock(state_->mutex);
    State &s = *state_;
    uint64_t off = 0;
    const State::Twin *t = s.find_twin(A.kv, &off);
    const uint64_t row_bytes = A.row_stride * 4;
    if (!t || off % 16 || off + P * row_bytes > t->bytes) return false;
    float *kv_dev = reinterpret_cast<float *>(static_cast<uint8_t *>(t->device) + off);
    // rows written on the host since the last call: the next row when this
    // call continues the last one (its row P - 2 still as uploaded), every
    // row otherwise (a new sequence, or rows a batched prefill wrote)
    State::KvSync &ks = s.kv_sync[reinterpret_cast<uintptr_t>(A.kv)];
    const float *prev = A.kv + (P >= 2 ? (P - 2) * A.row_stride : 0);
    const bool next_row = P >= 2 && ks.positions + 1 == P && ks.last_row.size() == A.row_stride &&
                          std::memcmp(prev, ks.last_row.data(), row_bytes) == 0;
    const uint64_t from = next_row ? P - 1 : 0;
    check(fmx_upload(kv_dev + from * A.row_stride, A.kv + from * A.row_stride, (P - from) * row_bytes, s.stream,
                     nullptr),
          "attention cache rows");
    ks.positions = P;
    ks.last_row.assign(A.kv + (P - 1) * A.row_stride, A.kv + P * A.row_stride);
    if (!s.attn_status) check(fmx_alloc(256, &s.attn_status), "attention status");
    const uint64_t qo_bytes = H * D * 4;
    ensure_scratch(qo_bytes, qo_bytes);
    s.upload_staged(s.x_dev, q, qo_bytes);
    check(fmx_attention_decode(static_cast<const float *>(s.x_dev), kv_dev, A.row_stride, A.v_offset,
                               static_cast<uint32_t>(H), A.kv_heads, static_cast<uint32_t>(D),
                               static_cast<uint32_t>(P), A.scale, static_cast<float *>(s.y_dev), s.attn_status, 256,
                               s.stream),
          "attention.L" + std::to_string(A.layer));
    uint32_t *word = reinterpret_cast<uint32_t *>(s.pinned(s.status_word, s.status_word_cap, 4));
    check(fmx_moe_status_copy(s.attn_status, word, s.stream), "attention status");
    s.download_staged(out, s.y_dev, qo_bytes);
    check(fmx_moe_status_of(*word), "non-finite attention score in layer " + std::to_string(A.layer));
    record_operation({"attention.L" + std::to_string(A.layer), name(), P * A.kv_heads * D * 8 + qo_bytes, qo_bytes});
    return true;
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
