// capi.cpp — host side of the C ABI: devices, memory, fences, faults, and the
// MoE entry points that validate arguments and sequence the kernels.
#include "bucket.hpp"
#include "fmx_internal.hpp"
#include "moe.hpp"
#include "prefill.hpp"

#include <atomic>
#include <chrono>
#include <cstdio>
#include <mutex>
#include <thread>

namespace fmx {

namespace {

std::atomic<int> g_fault{FMX_FAULT_NONE};

constexpr uint64_t kStatusBytes = 256;

struct Fence {
    hipEvent_t event = nullptr;
    bool deferred = false;
};

// Workspace layout of fmx_moe_route / fmx_moe_decode (all offsets 256-byte
// aligned):
//   [0, 256)     error word (uint32)
//   h            hidden floats (decode: one token)
//   act          top_k x ffn floats (decode)
//   logits       tokens x experts floats (decode: one token; routing without a
//                caller's logits array: every token)
struct DecodeWorkspace {
    uint64_t h = 0, act = 0, logits = 0, total = 0;
};

DecodeWorkspace decode_workspace(const fmx_moe_layer *L, uint32_t tokens) {
    DecodeWorkspace w;
    w.h = kStatusBytes;
    w.act = w.h + align_up(static_cast<uint64_t>(L->hidden) * 4, 256);
    w.logits = w.act + align_up(static_cast<uint64_t>(L->top_k) * L->ffn * 4, 256);
    const uint64_t t = tokens ? tokens : 1;
    w.total = w.logits + align_up(t * L->experts * 4, 256);
    return w;
}

// Prefill workspace (all offsets 256-byte aligned), pairs = tokens * top_k:
//   [0, 256) error word | h [tokens x hidden] f32 | offsets [experts + 1] |
//   token_list, slot_of [pairs] | row tiles [1 + 3 * max_tiles] |
//   tile order [max_tiles] | chunk counts | x [tokens x hidden] bf16 | act [pairs + 192 rows x ffn] bf16 |
//   dn [splits x pairs x hidden] f32 |
//   the decode scratch (act of one token) for shapes the GEMMs do not tile |
//   logits [tokens x experts] f32
struct PrefillWorkspace {
    uint64_t h = 0, offsets = 0, token_list = 0, slot_of = 0, tiles = 0, tile_order = 0,
             chunk_counts = 0, x = 0, act = 0, dn = 0,
             dec_act = 0, logits = 0, total = 0;
    uint32_t pairs = 0, max_tiles = 0;
};

PrefillWorkspace prefill_workspace(const fmx_moe_layer *L, uint32_t tokens) {
    PrefillWorkspace w;
    const uint64_t H = L->hidden, F = L->ffn, E = L->experts;
    w.pairs = tokens * L->top_k;
    w.max_tiles = bucket_max_tiles(tokens, L->top_k, L->experts, kPrefillTileRows);
    const uint64_t P = w.pairs;
    uint64_t o = kStatusBytes;
    auto take = [&o](uint64_t bytes) { const uint64_t at = o; o += align_up(bytes, 256); return at; };
    w.h = take(static_cast<uint64_t>(tokens) * H * 4);
    w.offsets = take((E + 1) * 4);
    w.token_list = take(P * 4);
    w.slot_of = take(P * 4);
    w.tiles = take((1 + 3ull * w.max_tiles) * 4);
    w.tile_order = take(static_cast<uint64_t>(w.max_tiles) * 4);
    w.chunk_counts = take(bucket_chunk_counts_bytes(tokens, L->experts));
    // h in bf16 (the gate/up GEMM's rows, through token_list); the GEMMs read
    // a whole 192-row tile from every tile's first row of act, which carries
    // that many rows of padding
    w.x = take(static_cast<uint64_t>(tokens) * H * 2);
    w.act = take((P + kPrefillTileRows) * F * 2);
    w.dn = take(prefill_down_splits(L->experts, L->ffn) * P * H * 4);
    w.dec_act = take(static_cast<uint64_t>(L->top_k) * F * 4);
    w.logits = take(static_cast<uint64_t>(tokens) * E * 4);
    w.total = o;
    return w;
}

// Zeroes the error word with a kernel, not a memset, so a caller may capture
// the sequence in a HIP graph.
__global__ void clear_word_kernel(uint32_t *word) { *word = 0; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int validate_layer(const fmx_moe_layer *L) {
    if (!L) return FMX_ERR_INVALID_ARGUMENT;
    if (L->hidden == 0 || L->ffn == 0 || L->experts == 0 || L->top_k == 0) return FMX_ERR_INVALID_ARGUMENT;
    if (L->top_k > L->experts) return FMX_ERR_INVALID_ARGUMENT;      // engine.cpp:408
    if (L->top_k > 32 || L->experts > 256) return FMX_ERR_INVALID_ARGUMENT;
    if (L->hidden > 16384 || L->hidden % 4) return FMX_ERR_SHAPE_MISMATCH; // routing stages x as float4
    if (!L->router || !L->gate || !L->up || !L->down) return FMX_ERR_INVALID_ARGUMENT;
    // the routing kernels read x, the router rows and the norm gains as float4
    if (!aligned16(L->router) || (L->norm_weight && !aligned16(L->norm_weight))) return FMX_ERR_INVALID_ARGUMENT;
    if (L->router_type != FMX_TYPE_F32 && L->router_type != FMX_TYPE_Q4_0 && L->router_type != FMX_TYPE_Q8_0 &&
        L->router_type != FMX_TYPE_Q4_K && L->router_type != FMX_TYPE_Q6_K)
        return FMX_ERR_UNSUPPORTED_QUANTISATION;
    if (L->router_type == FMX_TYPE_Q6_K && L->hidden % 256) return FMX_ERR_SHAPE_MISMATCH;
    return FMX_OK;
}

// The decode sequence of fmx_moe_decode for `tokens` rows of x, with the
// one-token workspace at `base` (layout of decode_workspace) and the error
// word at `status`. Arguments are validated by the caller.
int decode_tokens(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                  float *weights, uint8_t *base, uint32_t *status, hipStream_t s) {
    RouteArgs ra;
    if (int rc = prepare_route_args(L, &ra)) return rc;
    ExpertArgs ea;
    if (int rc = prepare_expert_args(L, ra, &ea)) return rc;
    const DecodeWorkspace ws = decode_workspace(L, 1);
    float *h = reinterpret_cast<float *>(base + ws.h);
    float *lg = reinterpret_cast<float *>(base + ws.logits);
    DecodeScratch sc;
    sc.act = reinterpret_cast<float *>(base + ws.act);
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, status);
    FMX_LAUNCH_CHECK();
    const uint64_t H = L->hidden, K = L->top_k;
    for (uint32_t t = 0; t < tokens; ++t) {
        if (int rc = launch_route_logits(ra, x + t * H, 1, h, lg, s)) return rc;
        if (int rc = launch_experts(ea, x + t * H, h, lg, ids + t * K, weights + t * K, sc, out + t * H, status, s))
            return rc;
    }
    return FMX_OK;
}

// The decode workspace of fmx_moe_decode_static: a device array of fixed size
// that every call on one GPU shares. Each GPU holds its own copy at its own
// address; host code uses that address (from hipGetSymbolAddress, looked up
// once per device), never the array's name, which on the host is only a
// stand-in.
static __device__ __align__(256) uint8_t scratch[FMX_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t *g_scratch_ptr[kMaxDevices];

// `scratch` of the current device.
int static_scratch(uint8_t **ptr) {
    int dev = 0;
    FMX_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return FMX_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        FMX_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return FMX_ERR_LAUNCH_FAILED;
        g_scratch_ptr[dev] = static_cast<uint8_t *>(p);
    }
    *ptr = g_scratch_ptr[dev];
    return FMX_OK;
}

} // namespace

int current_fault() { return g_fault.load(); }

void consume_fault(int fault) {
    int expected = fault;
    g_fault.compare_exchange_strong(expected, FMX_FAULT_NONE);
}

int fault_gate() { return g_fault.load() == FMX_FAULT_DEVICE_LOSS ? FMX_ERR_DEVICE_LOSS : FMX_OK; }

int status_of_hip(hipError_t e) {
    switch (e) {
    case hipSuccess: return FMX_OK;
    case hipErrorOutOfMemory: return FMX_ERR_ALLOCATION_FAILED;
    case hipErrorNoDevice:
    case hipErrorInvalidDevice:
    case hipErrorNoBinaryForGpu: return FMX_ERR_NO_DEVICE;
    case hipErrorInvalidValue: return FMX_ERR_INVALID_ARGUMENT;
    default: return FMX_ERR_LAUNCH_FAILED;
    }
}

} // namespace fmx

using namespace fmx;

extern "C" {

int fmx_abi_version(void) { return FMX_ABI_VERSION; }

// Spelled as fm::error_name spells fm::ErrorCode (common.cpp).
const char *fmx_status_name(int status) {
    switch (status) {
    case FMX_OK: return "OK";
    case FMX_ERR_INVALID_ARGUMENT: return "INVALID_ARGUMENT";
    case FMX_ERR_UNSUPPORTED_QUANTISATION: return "UNSUPPORTED_QUANTISATION";
    case FMX_ERR_SHAPE_MISMATCH: return "SHAPE_MISMATCH";
    case FMX_ERR_INTERNAL: return "INTERNAL_ERROR";
    case FMX_ERR_ALLOCATION_FAILED: return "ALLOCATION_FAILED";
    case FMX_ERR_TRANSFER_FAILED: return "TRANSFER_FAILED";
    case FMX_ERR_FENCE_TIMEOUT: return "FENCE_TIMEOUT";
    case FMX_ERR_DEVICE_LOSS: return "DEVICE_LOSS";
    case FMX_ERR_NO_DEVICE: return "GPU_BACKEND_UNIMPLEMENTED";
    case FMX_ERR_LAUNCH_FAILED: return "INTERNAL_ERROR";
    }
    return "UNKNOWN";
}

int fmx_device_info_get(int ordinal, fmx_device_info *info) {
    if (!info) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = fault_gate()) return rc;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= ordinal || ordinal < 0) return FMX_ERR_NO_DEVICE;
    hipDeviceProp_t p;
    FMX_HIP_TRY(hipGetDeviceProperties(&p, ordinal));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0) return FMX_ERR_NO_DEVICE;
    std::memset(info, 0, sizeof(*info));
    std::snprintf(info->name, sizeof(info->name), "%s", p.name);
    std::snprintf(info->arch, sizeof(info->arch), "%s", p.gcnArchName);
    size_t free_b = 0, total_b = 0;
    int prev = 0;
    FMX_HIP_TRY(hipGetDevice(&prev));
    FMX_HIP_TRY(hipSetDevice(ordinal));
    const hipError_t me = hipMemGetInfo(&free_b, &total_b);
    FMX_HIP_TRY(hipSetDevice(prev));
    FMX_HIP_TRY(me);
    info->total_memory_bytes = total_b;
    info->free_memory_bytes = free_b;
    info->compute_units = p.multiProcessorCount;
    info->wavefront_size = p.warpSize;
    info->lds_bytes_per_cu = static_cast<uint32_t>(p.maxSharedMemoryPerMultiProcessor);
    info->clock_khz = p.clockRate;
    info->memory_clock_khz = p.memoryClockRate;
    info->memory_bus_bits = p.memoryBusWidth;
    return FMX_OK;
}

int fmx_alloc(uint64_t bytes, void **device_ptr) {
    if (!device_ptr || bytes == 0) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = fault_gate()) return rc;
    *device_ptr = nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return FMX_ERR_ALLOCATION_FAILED;
    if (hipMemset(p, 0, bytes) != hipSuccess) {
        (void)hipFree(p);
        return FMX_ERR_ALLOCATION_FAILED;
    }
    *device_ptr = p;
    return FMX_OK;
}

int fmx_free(void *device_ptr) {
    if (!device_ptr) return FMX_OK;
    FMX_HIP_TRY(hipFree(device_ptr));
    return FMX_OK;
}

int fmx_host_alloc(uint64_t bytes, void **host_ptr) {
    if (!host_ptr || bytes == 0) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = fault_gate()) return rc;
    *host_ptr = nullptr;
    void *p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) return FMX_ERR_ALLOCATION_FAILED;
    std::memset(p, 0, bytes);
    *host_ptr = p;
    return FMX_OK;
}

int fmx_host_free(void *host_ptr) {
    if (!host_ptr) return FMX_OK;
    FMX_HIP_TRY(hipHostFree(host_ptr));
    return FMX_OK;
}

int fmx_upload(void *device_dst, const void *host_src, uint64_t bytes, void *stream, void **fence) {
    if (fence) *fence = nullptr;
    const int fault = current_fault();
    if (fault == FMX_FAULT_TRANSFER) return FMX_ERR_TRANSFER_FAILED;
    if (fault == FMX_FAULT_DEVICE_LOSS) return FMX_ERR_DEVICE_LOSS;
    if (!device_dst || (!host_src && bytes)) return FMX_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (bytes) FMX_HIP_TRY(hipMemcpyAsync(device_dst, host_src, bytes, hipMemcpyHostToDevice, s));
    if (fence) {
        Fence *f = new Fence();
        f->deferred = fault == FMX_FAULT_FENCE_DEFERRED;
        if (hipEventCreateWithFlags(&f->event, hipEventDisableTiming) != hipSuccess ||
            hipEventRecord(f->event, s) != hipSuccess) {
            if (f->event) (void)hipEventDestroy(f->event);
            delete f;
            return FMX_ERR_TRANSFER_FAILED;
        }
        *fence = f;
    }
    return FMX_OK;
}

int fmx_download(void *host_dst, const void *device_src, uint64_t bytes, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (current_fault() == FMX_FAULT_TRANSFER) return FMX_ERR_TRANSFER_FAILED;
    if (!host_dst || (!device_src && bytes)) return FMX_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (bytes) FMX_HIP_TRY(hipMemcpyAsync(host_dst, device_src, bytes, hipMemcpyDeviceToHost, s));
    FMX_HIP_TRY(hipStreamSynchronize(s));
    return FMX_OK;
}

int fmx_fence_query(void *fence, int *complete) {
    if (!fence || !complete) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = fault_gate()) return rc;
    Fence *f = static_cast<Fence *>(fence);
    if (f->deferred && current_fault() == FMX_FAULT_FENCE_DEFERRED) {
        *complete = 0;
        return FMX_OK;
    }
    const hipError_t e = hipEventQuery(f->event);
    if (e == hipSuccess) *complete = 1;
    else if (e == hipErrorNotReady) *complete = 0;
    else return status_of_hip(e);
    return FMX_OK;
}

// Polls with a 1 ms sleep, as Backend::wait_fence (backend.cpp:128-135).
int fmx_fence_wait(void *fence, uint32_t timeout_ms) {
    if (!fence) return FMX_ERR_INVALID_ARGUMENT;
    if (current_fault() == FMX_FAULT_FENCE_TIMEOUT) {
        consume_fault(FMX_FAULT_FENCE_TIMEOUT); // CpuBackend clears the fault when it fires
        return FMX_ERR_FENCE_TIMEOUT;
    }
    const auto start = std::chrono::steady_clock::now();
    for (;;) {
        int done = 0;
        if (int rc = fmx_fence_query(fence, &done)) return rc;
        if (done) return FMX_OK;
        const auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(
                            std::chrono::steady_clock::now() - start).count();
        if (static_cast<uint64_t>(ms) >= timeout_ms) return FMX_ERR_FENCE_TIMEOUT;
        std::this_thread::sleep_for(std::chrono::milliseconds(1));
    }
}

int fmx_fence_release(void *fence) {
    if (!fence) return FMX_OK;
    Fence *f = static_cast<Fence *>(fence);
    (void)hipEventSynchronize(f->event);
    (void)hipEventDestroy(f->event);
    delete f;
    return FMX_OK;
}

int fmx_stream_sync(void *stream) {
    if (int rc = fault_gate()) return rc;
    FMX_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return FMX_OK;
}

int fmx_inject_fault(int fault) {
    if (fault < FMX_FAULT_NONE || fault > FMX_FAULT_DEVICE_LOSS) return FMX_ERR_INVALID_ARGUMENT;
    g_fault.store(fault);
    return FMX_OK;
}

int fmx_clear_faults(void) {
    g_fault.store(FMX_FAULT_NONE);
    return FMX_OK;
}

// ------------------------------------------------------------------- MoE --

uint64_t fmx_moe_workspace_bytes(const fmx_moe_layer *L, uint32_t tokens) {
    if (validate_layer(L)) return 0;
    return decode_workspace(L, tokens).total;
}

int fmx_moe_route(const fmx_moe_layer *L, const float *x, uint32_t tokens, float *h, float *logits,
                  uint32_t *ids, float *weights, void *workspace, uint64_t workspace_bytes,
                  void *stream) {
    if (int rc = fault_gate()) return rc;
    if (int rc = validate_layer(L)) return rc;
    if (tokens == 0) return FMX_OK;
    if (!x || !ids || !weights || !workspace || workspace_bytes < kStatusBytes) return FMX_ERR_INVALID_ARGUMENT;
    if (!aligned16(x) || (h && !aligned16(h))) return FMX_ERR_INVALID_ARGUMENT;
    const DecodeWorkspace ws = decode_workspace(L, tokens);
    if (!logits && workspace_bytes < ws.total) return FMX_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t *base = static_cast<uint8_t *>(workspace);
    uint32_t *status = reinterpret_cast<uint32_t *>(base);
    float *lg = logits ? logits : reinterpret_cast<float *>(base + ws.logits);
    RouteArgs ra;
    if (int rc = prepare_route_args(L, &ra)) return rc;
    const bool per_token = !h && ra.router_type != FMX_TYPE_F32;
    // a block-type router without a caller's h runs one token at a time
    // through the workspace's h: checked before anything is launched
    if (per_token && workspace_bytes < ws.total) return FMX_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, status);
    FMX_LAUNCH_CHECK();
    if (!per_token) return launch_route(ra, x, tokens, h, lg, ids, weights, status, s);
    float *hw = reinterpret_cast<float *>(base + ws.h);
    const uint64_t H = L->hidden, E = L->experts, K = L->top_k;
    for (uint32_t t = 0; t < tokens; ++t)
        if (int rc = launch_route(ra, x + t * H, 1, hw, lg + t * E, ids + t * K, weights + t * K, status, s))
            return rc;
    return FMX_OK;
}

int fmx_moe_decode(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                   float *weights, void *workspace, uint64_t workspace_bytes, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (int rc = validate_layer(L)) return rc;
    if (tokens == 0) return FMX_OK;
    if (!x || !out || !ids || !weights || !workspace) return FMX_ERR_INVALID_ARGUMENT;
    if (!aligned16(x) || !aligned16(workspace)) return FMX_ERR_INVALID_ARGUMENT;
    if (workspace_bytes < decode_workspace(L, 1).total) return FMX_ERR_INVALID_ARGUMENT;
    uint8_t *base = static_cast<uint8_t *>(workspace);
    return decode_tokens(L, x, out, tokens, ids, weights, base, reinterpret_cast<uint32_t *>(base),
                         static_cast<hipStream_t>(stream));
}

int fmx_moe_decode_static(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                          float *weights, uint32_t *status, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (int rc = validate_layer(L)) return rc;
    if (tokens == 0) return FMX_OK;
    if (!x || !out || !ids || !weights) return FMX_ERR_INVALID_ARGUMENT;
    if (!aligned16(x)) return FMX_ERR_INVALID_ARGUMENT;
    if (decode_workspace(L, 1).total > FMX_STATIC_SCRATCH_BYTES) return FMX_ERR_SHAPE_MISMATCH;
    uint8_t *base = nullptr;
    if (int rc = static_scratch(&base)) return rc;
    return decode_tokens(L, x, out, tokens, ids, weights, base, status ? status : reinterpret_cast<uint32_t *>(base),
                         static_cast<hipStream_t>(stream));
}

int fmx_moe_decode_timed(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                         float *weights, void *workspace, uint64_t workspace_bytes, void *stream,
                         double *kernel_ms) {
    if (int rc = fault_gate()) return rc;
    if (int rc = validate_layer(L)) return rc;
    if (!kernel_ms) return FMX_ERR_INVALID_ARGUMENT;
    kernel_ms[0] = kernel_ms[1] = kernel_ms[2] = 0.0;
    if (tokens == 0) return FMX_OK;
    if (!x || !out || !ids || !weights || !workspace) return FMX_ERR_INVALID_ARGUMENT;
    const DecodeWorkspace ws = decode_workspace(L, 1);
    if (workspace_bytes < ws.total) return FMX_ERR_INVALID_ARGUMENT;
    RouteArgs ra;
    if (int rc = prepare_route_args(L, &ra)) return rc;
    ExpertArgs ea;
    if (int rc = prepare_expert_args(L, ra, &ea)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!aligned16(x) || !aligned16(workspace)) return FMX_ERR_INVALID_ARGUMENT;
    uint8_t *base = static_cast<uint8_t *>(workspace);
    uint32_t *status = reinterpret_cast<uint32_t *>(base);
    float *h = reinterpret_cast<float *>(base + ws.h);
    float *lg = reinterpret_cast<float *>(base + ws.logits);
    DecodeScratch sc;
    sc.act = reinterpret_cast<float *>(base + ws.act);
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, status);
    FMX_LAUNCH_CHECK();
    // events in batches: [token][route start, route end, then the gate/up and
    // the down kernels' start and end, recorded by their launches]
    constexpr uint32_t kBatch = 64;
    hipEvent_t ev[kBatch][6];
    for (auto &row : ev)
        for (auto &e : row) FMX_HIP_TRY(hipEventCreate(&e));
    int rc = FMX_OK;
    const uint64_t H = L->hidden, K = L->top_k;
    for (uint32_t t0 = 0; t0 < tokens && rc == FMX_OK; t0 += kBatch) {
        const uint32_t n = tokens - t0 < kBatch ? tokens - t0 : kBatch;
        for (uint32_t i = 0; i < n && rc == FMX_OK; ++i) {
            const uint64_t t = t0 + i;
            (void)hipEventRecord(ev[i][0], s);
            rc = launch_route_logits(ra, x + t * H, 1, h, lg, s);
            (void)hipEventRecord(ev[i][1], s);
            if (rc == FMX_OK)
                rc = launch_experts(ea, x + t * H, h, lg, ids + t * K, weights + t * K, sc, out + t * H, status,
                                    s, &ev[i][2]);
        }
        if (hipStreamSynchronize(s) != hipSuccess) rc = FMX_ERR_LAUNCH_FAILED;
        for (uint32_t i = 0; i < n && rc == FMX_OK; ++i) {
            float a = 0, b = 0, c = 0;
            if (hipEventElapsedTime(&a, ev[i][0], ev[i][1]) != hipSuccess ||
                hipEventElapsedTime(&b, ev[i][2], ev[i][3]) != hipSuccess ||
                hipEventElapsedTime(&c, ev[i][4], ev[i][5]) != hipSuccess)
                rc = FMX_ERR_LAUNCH_FAILED;
            kernel_ms[0] += a;
            kernel_ms[1] += b;
            kernel_ms[2] += c;
        }
    }
    for (auto &row : ev)
        for (auto &e : row) (void)hipEventDestroy(e);
    return rc;
}

uint64_t fmx_moe_prefill_workspace_bytes(const fmx_moe_layer *L, uint32_t tokens) {
    if (validate_layer(L) || tokens == 0) return 0;
    return prefill_workspace(L, tokens).total;
}

namespace {

// fmx_moe_prefill; kev (optional) as launch_prefill_experts. *tiled: whether
// the grouped GEMMs ran (false: the decode kernels, per token).
int prefill_layer(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                  float *weights, void *workspace, uint64_t workspace_bytes, void *stream, hipEvent_t *kev,
                  bool *tiled) {
    *tiled = false;
    if (int rc = fault_gate()) return rc;
    if (int rc = validate_layer(L)) return rc;
    if (tokens == 0) return FMX_OK;
    if (!x || !out || !ids || !weights || !workspace) return FMX_ERR_INVALID_ARGUMENT;
    if (!aligned16(x) || !aligned16(workspace)) return FMX_ERR_INVALID_ARGUMENT;
    const PrefillWorkspace ws = prefill_workspace(L, tokens);
    if (workspace_bytes < ws.total) return FMX_ERR_INVALID_ARGUMENT;
    RouteArgs ra;
    if (int rc = prepare_route_args(L, &ra)) return rc;
    ExpertArgs ea;
    if (int rc = prepare_expert_args(L, ra, &ea)) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint8_t *base = static_cast<uint8_t *>(workspace);
    uint32_t *status = reinterpret_cast<uint32_t *>(base);
    float *h = reinterpret_cast<float *>(base + ws.h);
    // the routing's first kernel zeroes the error word
    if (int rc = launch_route(ra, x, tokens, h, reinterpret_cast<float *>(base + ws.logits), ids, weights, status,
                              s, true))
        return rc;
    const uint64_t H = L->hidden, K = L->top_k;
    if (!prefill_gemm_supported(ea)) {
        // shapes the grouped GEMMs do not tile (and F32 experts): the decode
        // expert kernels, one token at a time, on the routing just computed
        DecodeScratch sc;
        sc.act = reinterpret_cast<float *>(base + ws.dec_act);
        for (uint32_t t = 0; t < tokens; ++t)
            if (int rc = launch_experts(ea, x + t * H, h + t * H, nullptr, ids + t * K, weights + t * K, sc, out + t * H,
                                        status, s))
                return rc;
        return FMX_OK;
    }
    uint32_t *slot_of = reinterpret_cast<uint32_t *>(base + ws.slot_of);
    PrefillBuffers b;
    b.h = h;
    b.token_list = reinterpret_cast<uint32_t *>(base + ws.token_list);
    b.slot_of = slot_of;
    b.top_k = L->top_k;
    b.tiles = reinterpret_cast<uint32_t *>(base + ws.tiles);
    b.tile_order = reinterpret_cast<uint32_t *>(base + ws.tile_order);
    b.tokens = tokens;
    b.pairs = ws.pairs;
    b.x = reinterpret_cast<__bf16 *>(base + ws.x);
    b.act = reinterpret_cast<__bf16 *>(base + ws.act);
    b.dn = reinterpret_cast<float *>(base + ws.dn);
    b.splits = prefill_down_splits(L->experts, L->ffn);
    if (int rc = launch_bucket_chunked(ids, tokens, L->top_k, L->experts,
                                       reinterpret_cast<uint32_t *>(base + ws.offsets), slot_of,
                                       reinterpret_cast<uint32_t *>(base + ws.token_list), status,
                                       reinterpret_cast<uint32_t *>(base + ws.chunk_counts), s,
                                       reinterpret_cast<uint32_t *>(base + ws.tiles),
                                       reinterpret_cast<uint32_t *>(base + ws.tile_order), kPrefillTileRows))
        return rc;
    if (int rc = launch_prefill_experts(ea, b, ws.max_tiles, s, kev)) return rc;
    *tiled = true;
    return launch_combine(x, b.dn, b.splits, b.pairs, slot_of, weights, L->hidden, L->top_k, tokens, out, s);
}

} // namespace

int fmx_moe_prefill(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                    float *weights, void *workspace, uint64_t workspace_bytes, void *stream) {
    bool tiled;
    return prefill_layer(L, x, out, tokens, ids, weights, workspace, workspace_bytes, stream, nullptr, &tiled);
}

int fmx_moe_prefill_timed(const fmx_moe_layer *L, const float *x, float *out, uint32_t tokens, uint32_t *ids,
                          float *weights, void *workspace, uint64_t workspace_bytes, void *stream,
                          double *kernel_ms) {
    if (!kernel_ms) return FMX_ERR_INVALID_ARGUMENT;
    kernel_ms[0] = kernel_ms[1] = 0.0;
    hipEvent_t kev[4] = {};
    for (auto &e : kev)
        if (hipEventCreate(&e) != hipSuccess) {
            for (auto &f : kev)
                if (f) (void)hipEventDestroy(f);
            return FMX_ERR_LAUNCH_FAILED;
        }
    bool tiled = false;
    int rc = prefill_layer(L, x, out, tokens, ids, weights, workspace, workspace_bytes, stream, kev, &tiled);
    if (rc == FMX_OK && hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess)
        rc = FMX_ERR_LAUNCH_FAILED;
    if (rc == FMX_OK && !tiled) rc = FMX_ERR_SHAPE_MISMATCH;
    if (rc == FMX_OK) {
        float a = 0, b = 0;
        if (hipEventElapsedTime(&a, kev[0], kev[1]) != hipSuccess ||
            hipEventElapsedTime(&b, kev[2], kev[3]) != hipSuccess)
            rc = FMX_ERR_LAUNCH_FAILED;
        kernel_ms[0] = a;
        kernel_ms[1] = b;
    }
    for (auto &e : kev) (void)hipEventDestroy(e);
    return rc;
}

int fmx_attention_decode(const float *q, const float *kv, uint64_t row_stride, uint32_t v_offset,
                         uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t positions,
                         double scale, float *out, void *workspace, uint64_t workspace_bytes, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (!q || !kv || !out || !workspace || workspace_bytes < kStatusBytes) return FMX_ERR_INVALID_ARGUMENT;
    if (!aligned16(q) || !aligned16(kv) || !aligned16(out) || !aligned16(workspace)) return FMX_ERR_INVALID_ARGUMENT;
    if (!(scale == scale)) return FMX_ERR_INVALID_ARGUMENT;
    return attention_decode(q, kv, row_stride, v_offset, heads, kv_heads, head_dim, positions, scale, out,
                            static_cast<uint32_t *>(workspace), static_cast<hipStream_t>(stream));
}

int fmx_moe_status_of(uint32_t word) {
    if (word & STATUS_BAD_EXPERT) return FMX_ERR_INVALID_ARGUMENT;
    if (word & STATUS_NONFINITE_SCORE) return FMX_ERR_INTERNAL;
    return FMX_OK;
}

int fmx_moe_status(void *workspace, void *stream) {
    if (!workspace) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = fault_gate()) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t word = 0;
    FMX_HIP_TRY(hipMemcpyAsync(&word, workspace, 4, hipMemcpyDeviceToHost, s));
    FMX_HIP_TRY(hipStreamSynchronize(s));
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, static_cast<uint32_t *>(workspace));
    FMX_LAUNCH_CHECK();
    return fmx_moe_status_of(word);
}

int fmx_moe_status_copy(void *workspace, uint32_t *host_word, void *stream) {
    if (!workspace || !host_word) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = fault_gate()) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    FMX_HIP_TRY(hipMemcpyAsync(host_word, workspace, 4, hipMemcpyDeviceToHost, s));
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, static_cast<uint32_t *>(workspace));
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

int fmx_moe_bucket(const uint32_t *ids, uint32_t tokens, uint32_t top_k, uint32_t experts,
                   uint32_t *offsets, uint32_t *token_list, uint32_t *rank_list, void *workspace,
                   uint64_t workspace_bytes, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (experts == 0 || experts > kBucketMaxExperts || top_k == 0 || top_k > experts)
        return FMX_ERR_INVALID_ARGUMENT;
    if (!offsets || !workspace || workspace_bytes < kStatusBytes) return FMX_ERR_INVALID_ARGUMENT;
    if (tokens && (!ids || !token_list || !rank_list)) return FMX_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t *status = static_cast<uint32_t *>(workspace);
    hipLaunchKernelGGL(clear_word_kernel, dim3(1), dim3(1), 0, s, status);
    FMX_LAUNCH_CHECK();
    return launch_bucket(ids, tokens, top_k, experts, offsets, token_list, rank_list, nullptr, status, s);
}

} // extern "C"
