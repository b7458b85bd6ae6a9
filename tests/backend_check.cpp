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

#include "fmoracle.h"

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

    // ---- the fused MoE block (moe_layer) on buffers laid out as the engine and
    // residency hold them, against the oracle's layer (which reproduces
    // FreeMoe's engine bit for bit): output, routing and the operation log
    struct MoeCase {
        uint32_t hidden, ffn, experts, top_k, gate_type, down_type, router_type, norm_offset;
    };
    for (const MoeCase &mc : {MoeCase{512, 256, 8, 2, 12, 8, 8, 4}, MoeCase{256, 512, 6, 2, 2, 2, 0, 16}}) {
        const uint32_t H = mc.hidden, F = mc.ffn, E = mc.experts, K = mc.top_k;
        const fm::QuantGeometry gg = fm::quant_geometry(mc.gate_type), gd = fm::quant_geometry(mc.down_type);
        const uint64_t gate_bytes = static_cast<uint64_t>(F) * (H / gg.block_size) * gg.block_bytes;
        const uint64_t down_bytes = static_cast<uint64_t>(H) * (F / gd.block_size) * gd.block_bytes;
        // fixed weights: [pad][norm gains][router rows], contiguous as engine.cpp:216-224 packs them
        std::vector<float> norm(H);
        for (auto &v : norm) v = 1.0f + static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 29);
        std::vector<uint8_t> router;
        if (mc.router_type == 0) {
            router.resize(static_cast<size_t>(E) * H * 4);
            float *rf = reinterpret_cast<float *>(router.data());
            for (uint64_t i = 0; i < static_cast<uint64_t>(E) * H; ++i)
                rf[i] = static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 27);
        } else {
            router = quant_matrix(mc.router_type, E, H, 300);
        }
        std::vector<uint8_t> fixed(mc.norm_offset + H * 4 + router.size());
        std::memcpy(fixed.data() + mc.norm_offset, norm.data(), H * 4);
        std::memcpy(fixed.data() + mc.norm_offset + H * 4, router.data(), router.size());
        auto fb = gpu.allocate(fixed.size(), fm::AllocationTag::Weights);
        gpu.wait_fence(gpu.upload(*fb, fixed.data(), fixed.size()), 5000);
        // one slot per expert: gate | up | down, raw rows
        std::vector<std::vector<uint8_t>> gate(E), up(E), down(E);
        std::vector<std::unique_ptr<fm::DeviceBuffer>> slots;
        fm::MoeLayerView view;
        for (uint32_t e = 0; e < E; ++e) {
            gate[e] = quant_matrix(mc.gate_type, F, H, 400 + e);
            up[e] = quant_matrix(mc.gate_type, F, H, 500 + e);
            down[e] = quant_matrix(mc.down_type, H, F, 600 + e);
            std::vector<uint8_t> payload(2 * gate_bytes + down_bytes);
            std::memcpy(payload.data(), gate[e].data(), gate_bytes);
            std::memcpy(payload.data() + gate_bytes, up[e].data(), gate_bytes);
            std::memcpy(payload.data() + 2 * gate_bytes, down[e].data(), down_bytes);
            slots.push_back(gpu.allocate(payload.size(), fm::AllocationTag::ExpertCache));
            gpu.wait_fence(gpu.upload(*slots.back(), payload.data(), payload.size()), 5000);
            view.expert_payloads.push_back(slots.back()->data);
        }
        view.layer = 3;
        view.hidden = H;
        view.ffn = F;
        view.experts = E;
        view.top_k = K;
        view.norm_weight = reinterpret_cast<const float *>(static_cast<uint8_t *>(fb->data) + mc.norm_offset);
        view.rms_eps = static_cast<double>(1e-5f);
        view.router_type = mc.router_type;
        view.router = static_cast<uint8_t *>(fb->data) + mc.norm_offset + H * 4;
        view.weights_norm = true;
        view.gate_type = view.up_type = mc.gate_type;
        view.down_type = mc.down_type;
        // the oracle's layer on the same bytes
        std::vector<const uint8_t *> gp(E), upp(E), dp(E);
        for (uint32_t e = 0; e < E; ++e) {
            gp[e] = gate[e].data();
            upp[e] = up[e].data();
            dp[e] = down[e].data();
        }
        fmo_layer ol{};
        ol.hidden = H;
        ol.ffn = F;
        ol.experts = E;
        ol.top_k = K;
        ol.norm_weight = norm.data();
        ol.rms_eps = view.rms_eps;
        ol.router_type = mc.router_type;
        ol.router = router.data();
        ol.weights_norm = 1;
        ol.weights_epsilon = view.weights_epsilon;
        ol.weights_scale = 1.0;
        ol.gate_type = ol.up_type = mc.gate_type;
        ol.down_type = mc.down_type;
        ol.gate = gp.data();
        ol.up = upp.data();
        ol.down = dp.data();
        const size_t ops_before = gpu.operations().size();
        bool same = true;
        std::vector<uint32_t> seen;
        for (int t = 0; t < 6; ++t) {
            std::vector<float> xt(H), og(H), orf(H), wg(K), wr(K);
            std::vector<uint32_t> ig(K), ir(K);
            for (auto &v : xt) v = static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 22);
            if (!gpu.moe_layer(view, xt.data(), og.data(), ig.data(), wg.data())) same = false;
            if (fmo_moe_layer(FMO_ISA_AVX2, &ol, xt.data(), orf.data(), ir.data(), wr.data(), nullptr, nullptr))
                same = false;
            same = same && std::memcmp(og.data(), orf.data(), H * 4) == 0 && ig == ir &&
                   std::memcmp(wg.data(), wr.data(), K * 4) == 0;
            seen.insert(seen.end(), ig.begin(), ig.end());
        }
        char what[160];
        std::snprintf(what, sizeof what,
                      "moe_layer (gate/up type %u, down %u, router %u) bit-identical to the oracle's layer, 6 tokens",
                      mc.gate_type, mc.down_type, mc.router_type);
        report(same, what);
        const auto ops = gpu.operations();
        uint32_t named = 0, on_gpu = 0;
        for (size_t i = ops_before; i < ops.size(); ++i) {
            const std::string &n = ops[i].name;
            named += n == "router.L3" || n == "router_gating.L3" || n == "router_topk.L3" ||
                     n.rfind("expert_gate.L3.E", 0) == 0 || n.rfind("expert_up.L3.E", 0) == 0 ||
                     n.rfind("expert_down.L3.E", 0) == 0 || n == "expert_swiglu.L3" || n == "expert_combine.L3";
            on_gpu += ops[i].backend == "hip-gfx950";
        }
        const size_t expect = 6 * (3 + 4 * K + 1);
        report(ops.size() - ops_before == expect && named == expect && on_gpu == expect,
               "moe_layer logs the reference's op names per token under hip-gfx950");
        std::snprintf(what, sizeof what, "op log names the routed experts: expert_gate.L3.E%u present", seen[0]);
        bool found = false;
        for (size_t i = ops_before; i < ops.size(); ++i)
            found = found || ops[i].name == "expert_gate.L3.E" + std::to_string(seen[0]);
        report(found, what);
        // refill one slot with another expert: the fused path follows it
        const uint32_t ex = seen[0];
        std::vector<uint8_t> g2 = quant_matrix(mc.gate_type, F, H, 700);
        std::vector<uint8_t> payload(2 * gate_bytes + down_bytes);
        std::memcpy(payload.data(), g2.data(), gate_bytes);
        std::memcpy(payload.data() + gate_bytes, up[ex].data(), gate_bytes);
        std::memcpy(payload.data() + 2 * gate_bytes, down[ex].data(), down_bytes);
        gpu.wait_fence(gpu.upload(*slots[ex], payload.data(), payload.size()), 5000);
        gate[ex] = g2;
        gp[ex] = gate[ex].data();
        std::vector<float> xt(H), og(H), orf(H), wg(K), wr(K);
        std::vector<uint32_t> ig(K), ir(K);
        for (auto &v : xt) v = static_cast<float>(static_cast<int32_t>(lcg(s) >> 8) - (1 << 23)) / (1 << 22);
        const bool ran = gpu.moe_layer(view, xt.data(), og.data(), ig.data(), wg.data());
        fmo_moe_layer(FMO_ISA_AVX2, &ol, xt.data(), orf.data(), ir.data(), wr.data(), nullptr, nullptr);
        report(ran && std::memcmp(og.data(), orf.data(), H * 4) == 0 && ig == ir,
               "moe_layer follows an expert slot refill");
    }

    // ---- buffers outlive their backend (the device state stays alive, as the
    // VNPU backend keeps its runtime, backend.cpp:441-446)
    {
        auto late = std::make_unique<fm::HipBackend>(gcfg);
        auto tracker = late->tracker();
        auto buf = late->allocate(1 << 20, fm::AllocationTag::Other);
        late->wait_fence(late->upload(*buf, w.data(), 4096), 5000);
        late.reset();
        buf.reset();
        report(tracker->snapshot().live_bytes == 0, "a buffer released after its backend frees cleanly");
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
