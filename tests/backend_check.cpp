// backend_check — fm::HipBackend driven through FreeMoe's own fm::Backend
// interface, against FreeMoe's CPU backend and kernels, in one process.
//
// Built by oracle/Makefile (target _ref/backend_check) from this file,
// freemoe_amd/host/hip_backend.cpp, FreeMoe's sources and libfmx.so. Test
// infrastructure: tests/test_integration.py runs it. Prints one line per
// check and exits non-zero on the first failure.
//
// Without a gfx950 device it checks the placeholder contract FreeMoe's tests
// pin (tests.cpp:558-627): allocate fails with GPU_BACKEND_UNIMPLEMENTED.
#include "hip_backend.hpp"

#include "fm/kernels.hpp"
#include "fm/quant.hpp"

#include <cstdio>
#include <cstring>
#include <vector>

namespace {

int failures = 0;

void report(bool ok, const char *what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
    if (!ok) ++failures;
}

template <class F>
fm::ErrorCode code_of_call(F &&f) {
    try {
        f();
    } catch (const fm::Error &e) {
        return e.code;
    }
    return fm::ErrorCode::OK;
}

uint32_t lcg(uint32_t &s) { return s = s * 1664525u + 1013904223u; }

// A [rows x cols] matrix of raw blocks of `type` with finite scales.
std::vector<uint8_t> quant_matrix(uint32_t type, uint32_t rows, uint32_t cols, uint32_t seed) {
    const fm::QuantGeometry g = fm::quant_geometry(type);
    const uint64_t blocks = static_cast<uint64_t>(rows) * (cols / g.block_size);
    std::vector<uint8_t> w(blocks * g.block_bytes);
    for (auto &b : w) b = static_cast<uint8_t>(lcg(seed) >> 24);
    for (uint64_t i = 0; i < blocks; ++i) {
        uint8_t *blk = w.data() + i * g.block_bytes;
        const uint16_t d = static_cast<uint16_t>(0x2000 + (lcg(seed) >> 22)); // small positive half
        std::memcpy(blk, &d, 2);
        if (type == 12) std::memcpy(blk + 2, &d, 2); // Q4_K dmin
    }
    return w;
}

} // namespace

int main() {
    fm::BackendConfig gcfg;
    gcfg.kind = fm::BackendKind::PhysicalGPU;
    fm::HipBackend gpu(gcfg);
    fm::BackendConfig ccfg;
    ccfg.kind = fm::BackendKind::ScalarCPU;
    auto cpu = fm::Backend::create(ccfg);

    const fm::DeviceInfo info = gpu.info();
    std::printf("device: %s (%s)\n", info.name.c_str(), info.driver_version.c_str());
    if (info.memory_type == "none") {
        report(code_of_call([&] { gpu.allocate(64, fm::AllocationTag::Weights); }) ==
                   fm::ErrorCode::GPU_BACKEND_UNIMPLEMENTED,
               "no device: allocate fails with GPU_BACKEND_UNIMPLEMENTED");
        return failures ? 1 : 0;
    }

    // ---- F32 matvec through buffers, bitwise against the CPU backend (AVX2 order)
    const uint32_t rows = 37, cols = 4103;
    std::vector<float> w(static_cast<size_t>(rows) * cols), x(cols), yc(rows), yg(rows);
    uint32_t s = 7;
    for (auto &v : w) v = static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 26);
    for (auto &v : x) v = static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 23);
    auto gw = gpu.allocate(w.size() * 4, fm::AllocationTag::Weights);
    fm::Fence f = gpu.upload(*gw, w.data(), w.size() * 4);
    gpu.wait_fence(f, 5000);
    report(gpu.fence_complete(f), "fence complete after wait");
    report(std::memcmp(gw->data, w.data(), w.size() * 4) == 0, "host mirror holds the uploaded bytes");
    auto cw = cpu->allocate(w.size() * 4, fm::AllocationTag::Weights);
    cpu->wait_fence(cpu->upload(*cw, w.data(), w.size() * 4), 5000);
    cpu->matvec(cw->f32(), x.data(), yc.data(), rows, cols, "check.f32");
    gpu.matvec(gw->f32(), x.data(), yg.data(), rows, cols, "check.f32");
    report(std::memcmp(yc.data(), yg.data(), rows * 4) == 0, "matvec F32 bit-identical to CpuBackend (Auto)");
    report(!gpu.operations().empty() && gpu.operations().back().backend == "hip-gfx950", "op log names hip-gfx950");

    // a pointer inside a buffer resolves to its twin
    gpu.matvec(gw->f32() + cols, x.data(), yg.data(), rows - 1, cols, "check.f32.offset");
    report(std::memcmp(yc.data() + 1, yg.data(), (rows - 1) * 4) == 0, "matvec on a row offset inside a buffer");

    // ---- block types: matvec_quant vs the reference's gemv_quant (KernelIsa::Auto)
    fm::KernelConfig kc;
    for (uint32_t type : {2u, 8u, 12u}) {
        const uint32_t qr = 23, qc = 2048;
        std::vector<uint8_t> q = quant_matrix(type, qr, qc, 100 + type);
        std::vector<float> xq(qc), yr(qr), yq(qr);
        for (auto &v : xq) v = static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 23);
        auto qb = gpu.allocate(q.size(), fm::AllocationTag::ExpertCache);
        gpu.wait_fence(gpu.upload(*qb, q.data(), q.size()), 5000);
        fm::gemv_quant(kc, type, q.data(), xq.data(), yr.data(), qr, qc);
        gpu.matvec_quant(type, qb->data, xq.data(), yq.data(), qr, qc, "check.quant");
        char what[96];
        std::snprintf(what, sizeof what, "matvec_quant type %u bit-identical to gemv_quant (Auto)", type);
        report(std::memcmp(yr.data(), yq.data(), qr * 4) == 0, what);
        // refill the slot with another matrix: the packed copy must follow
        std::vector<uint8_t> q2 = quant_matrix(type, qr, qc, 200 + type);
        gpu.wait_fence(gpu.upload(*qb, q2.data(), q2.size()), 5000);
        fm::gemv_quant(kc, type, q2.data(), xq.data(), yr.data(), qr, qc);
        gpu.matvec_quant(type, qb->data, xq.data(), yq.data(), qr, qc, "check.quant.refill");
        std::snprintf(what, sizeof what, "matvec_quant type %u follows a slot refill", type);
        report(std::memcmp(yr.data(), yq.data(), qr * 4) == 0, what);
    }

    // ---- faults forced from the host (backend.hpp:118), as the CPU backend raises them
    gpu.inject_fault(fm::BackendFault::TransferFailure);
    report(code_of_call([&] { gpu.upload(*gw, w.data(), 64); }) == fm::ErrorCode::TRANSFER_FAILED,
           "TransferFailure -> TRANSFER_FAILED");
    gpu.clear_faults();
    gpu.inject_fault(fm::BackendFault::FenceTimeout);
    fm::Fence f2 = gpu.upload(*gw, w.data(), 64);
    report(code_of_call([&] { gpu.wait_fence(f2, 5000); }) == fm::ErrorCode::FENCE_TIMEOUT,
           "FenceTimeout -> FENCE_TIMEOUT, once");
    report(code_of_call([&] { gpu.wait_fence(f2, 5000); }) == fm::ErrorCode::OK, "the timeout fault is consumed");
    gpu.inject_fault(fm::BackendFault::DeviceLoss);
    report(code_of_call([&] { gpu.matvec(gw->f32(), x.data(), yg.data(), rows, cols, "x"); }) ==
               fm::ErrorCode::DEVICE_LOSS,
           "DeviceLoss -> DEVICE_LOSS");
    gpu.clear_faults();
    report(code_of_call([&] { gpu.matvec(gw->f32(), x.data(), yg.data(), rows, cols, "x"); }) == fm::ErrorCode::OK,
           "clear_faults restores service");
    report(code_of_call([&] { gpu.matvec(x.data(), x.data(), yg.data(), 1, cols, "x"); }) ==
               fm::ErrorCode::INVALID_ARGUMENT,
           "weights outside any buffer -> INVALID_ARGUMENT");

    // ---- release: tracker back to zero live bytes (tests.cpp:888-893)
    gw.reset();
    report(gpu.tracker()->snapshot().live_bytes == 0, "zero live bytes after release");
    std::printf("%s\n", failures ? "backend_check: FAILED" : "backend_check: all ok");
    return failures ? 1 : 0;
}
