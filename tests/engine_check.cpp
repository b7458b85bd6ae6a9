// engine_check — FreeMoe's unchanged fm::Engine with the physical-GPU backend
// kind served by fm::HipBackend (freemoe_amd/host/backend_factory.cpp), next
// to the same engine on FreeMoe's CPU backend, in one process.
//
// Built by oracle/Makefile (target _ref/engine_check) from this file, the
// adapter, FreeMoe's sources and libfmx.so. Test infrastructure:
// tests/test_gpu_engine.py runs it. Every F32 projection of the engine
// (attention, router, experts, head) goes through Backend::matvec, so on the
// GPU it runs libfmx's F32 row chains; routing, softmax, top-k, attention and
// sampling stay the engine's own code.
//
//   engine_check compare <model.gguf> <reference_root> <prompts> <generate> <cpu|gpu>
//       Engine::compare_reference against FreeMoe's goldens; prints one JSON
//       line (prompts within tolerance, token and routing matches, max abs
//       diff, and how many operations the backend logged and under which
//       backend label).
//   engine_check residency <model.gguf> <reference_root> <prompts> <generate> <slots>
//       compare_reference on the GPU backend with `slots` expert slots (fewer
//       than the model's experts, so ResidencyManager::load_slot refills them:
//       host payload -> upload into the slot's pinned mirror and HBM twin ->
//       fence -> FNV-1a read-back, residency.cpp:617-723); prints the
//       comparison and residency's counters.
//   engine_check twin <model.gguf> <prompts> <prompt_len> <generate> <seed> [<hot GiB> <slots>]
//       seeded random byte prompts through a CPU-backend engine and a
//       GPU-backend engine; prints one JSON line with the largest prompt-logit
//       difference, the number of logits that differ in any bit, and whether
//       routing records and greedy ids are identical.
//   engine_check prompt <model.gguf> <generate> <text>
//       the reference's conformance run (tests.cpp:1424-1468: run_prompt of a
//       fixed text) on a CPU-backend and a GPU-backend engine; one JSON line
//       as for twin. Block-type projections reach the GPU through the renamed
//       gemv_quant / gemm_quant calls (backend_factory.cpp).
//   engine_check record <model.gguf> <prompts> <prompt_len> <generate> <seed> <out> [<hot GiB> <slots>]
//       seeded random byte prompts through a CPU-backend engine only; writes
//       the prompts and the engine's input ids, prompt logits, greedy ids and
//       routing records to <out> (a golden file for replay).
//   engine_check replay <model.gguf> <golden> [<hot GiB> <slots>]
//       the golden file's prompts through a GPU-backend engine only; one JSON
//       line as for twin, with the engine's prefill / decode times.
//
// Every mode's JSON carries the GPU backend's operation accounting: records
// by backend label; "quant_records" (the engine's own "cpu-quant" records,
// one per block-type projection), "batch_records" ("cpu-batched" records of
// batched products); "hooked" (projections the renamed direct calls ran on
// the device); "fallbacks" (renamed calls that ran FreeMoe's CPU kernel, for
// an engine on another backend kind in the same process); "fused_layers"
// (MoE blocks HipBackend::moe_layer ran); "device_attention" (token-layer
// attentions HipBackend::attention ran).
// Built twice: on FreeMoe's unchanged sources (engine_check) and on the
// sources with the integration's edits (engine_check_fused, where the engine
// calls Backend::matvec_quant / gemm_quant / moe_layer / attention itself).
// Exits non-zero on an engine error.
#include "fm/engine.hpp"
#include "fm/residency.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

// backend_factory.cpp: renamed gemv_quant / gemm_quant calls that ran
// FreeMoe's CPU kernel
extern "C" uint64_t fmx_engine_hook_fallbacks();

namespace {

// Hot-memory budget and expert slots for models larger than the defaults
// (64 MiB, as many slots as fit): set by the twin mode's optional arguments.
uint64_t g_hot_bytes = 0;
uint32_t g_slots = 0;

fm::RunConfig config_for(const std::string &model, bool gpu) {
    fm::RunConfig rc;
    rc.model_path = model;
    rc.backend.kind = gpu ? fm::BackendKind::PhysicalGPU : fm::BackendKind::ScalarCPU;
    rc.backend.kernel_isa = fm::KernelIsa::Auto;
    // two kernel threads: FreeMoe's WorkerPool finishes a split into at most
    // two ranges (kernels.cpp:414-459), which large projections would exceed
    rc.backend.kernel_threads = 2;
    if (g_hot_bytes) rc.budget.total_hot_bytes = g_hot_bytes;
    if (g_slots) rc.cache_slots = g_slots;
    return rc;
}

// Operations in the backend's log by the backend label they ran under, and
// the accounting of block-type projections (see the header).
std::string op_labels(fm::Backend &b) {
    std::map<std::string, uint64_t> by, hooked;
    uint64_t quant_records = 0, batch_records = 0, fused_layers = 0, device_attention = 0;
    const std::string dev = b.name();
    for (const auto &op : b.operations()) {
        by[op.backend] += 1;
        if (op.name == "gemv_quant" || op.name == "gemm_quant") hooked[op.name] += 1;
        if (op.backend == "cpu-quant") ++quant_records;
        if (op.backend == "cpu-batched" && op.name.size() > 6 &&
            op.name.compare(op.name.size() - 6, 6, ".batch") == 0)
            ++batch_records;
        if (op.backend == dev && op.name.rfind("expert_combine.L", 0) == 0) ++fused_layers;
        if (op.backend == dev && op.name.rfind("attention.L", 0) == 0) ++device_attention;
    }
    auto obj = [](const std::map<std::string, uint64_t> &m) {
        std::string s = "{";
        for (const auto &kv : m) {
            if (s.size() > 1) s += ",";
            s += "\"" + kv.first + "\":" + std::to_string(kv.second);
        }
        return s + "}";
    };
    std::string s = obj(by);
    s.pop_back();
    return s + (by.empty() ? "" : ",") + "\"hooked\":" + obj(hooked) +
           ",\"quant_records\":" + std::to_string(quant_records) +
           ",\"batch_records\":" + std::to_string(batch_records) +
           ",\"fused_layers\":" + std::to_string(fused_layers) +
           ",\"device_attention\":" + std::to_string(device_attention) +
           ",\"fallbacks\":" + std::to_string(fmx_engine_hook_fallbacks()) + "}";
}

int compare(int argc, char **argv) {
    if (argc < 7) return 2;
    const bool gpu = std::string(argv[6]) == "gpu";
    fm::Engine e(config_for(argv[2], gpu));
    e.initialize();
    const fm::ComparisonResult r =
        e.compare_reference(argv[3], static_cast<uint32_t>(std::atoi(argv[4])), static_cast<uint32_t>(std::atoi(argv[5])));
    std::printf("{\"mode\":\"compare\",\"backend\":\"%s\",\"prompts\":%u,\"within_tolerance\":%u,"
                "\"token_match\":%u,\"routing_match\":%u,\"matching_tokens\":%llu,\"reference_tokens\":%llu,"
                "\"max_abs_diff\":%.9g,\"max_rel_diff\":%.9g,\"ops\":%s}\n",
                e.backend().name().c_str(), r.prompts, r.prompts_within_tolerance, r.prompts_token_match,
                r.prompts_routing_match, static_cast<unsigned long long>(r.matching_tokens),
                static_cast<unsigned long long>(r.reference_tokens), r.max_abs_diff, r.max_rel_diff,
                op_labels(e.backend()).c_str());
    return 0;
}

int residency(int argc, char **argv) {
    if (argc < 7) return 2;
    fm::RunConfig rc = config_for(argv[2], true);
    rc.cache_slots = static_cast<uint32_t>(std::atoi(argv[6]));
    fm::Engine e(rc);
    e.initialize();
    const fm::ComparisonResult r =
        e.compare_reference(argv[3], static_cast<uint32_t>(std::atoi(argv[4])), static_cast<uint32_t>(std::atoi(argv[5])));
    const fm::ResidencyMetrics &m = e.residency()->metrics();
    std::printf("{\"mode\":\"residency\",\"backend\":\"%s\",\"slots\":%u,\"prompts\":%u,\"within_tolerance\":%u,"
                "\"token_match\":%u,\"routing_match\":%u,\"cache_hits\":%llu,\"cache_misses\":%llu,"
                "\"evictions\":%llu,\"checksum_checks\":%llu,\"checksum_failures\":%llu,\"h2d_bytes\":%llu,"
                "\"selected_experts\":%llu,\"experts_executed\":%llu,\"transfer_failures\":%llu,"
                "\"fence_timeouts\":%llu}\n",
                e.backend().name().c_str(), rc.cache_slots, r.prompts, r.prompts_within_tolerance,
                r.prompts_token_match, r.prompts_routing_match, static_cast<unsigned long long>(m.cache_hits),
                static_cast<unsigned long long>(m.cache_misses), static_cast<unsigned long long>(m.evictions),
                static_cast<unsigned long long>(m.checksum_checks),
                static_cast<unsigned long long>(m.checksum_failures), static_cast<unsigned long long>(m.h2d_bytes),
                static_cast<unsigned long long>(m.selected_experts),
                static_cast<unsigned long long>(m.experts_executed),
                static_cast<unsigned long long>(m.transfer_failures),
                static_cast<unsigned long long>(m.fence_timeouts));
    return 0;
}

// CPU-backend and GPU-backend engines over the same prompts (explicit texts,
// or `prompts` seeded random byte strings of length len when texts is empty).
int twin_run(const std::string &model, std::vector<std::string> texts, uint32_t prompts, uint32_t len,
             uint32_t gen, uint64_t seed) {
    fm::Engine cpu(config_for(model, false)), gpu(config_for(model, true));
    cpu.initialize();
    gpu.initialize();
    double max_diff = 0.0;
    uint64_t differing = 0, logits = 0, routing_events = 0, generated = 0;
    bool routing_same = true, ids_same = true;
    if (!texts.empty()) prompts = static_cast<uint32_t>(texts.size());
    for (uint32_t p = 0; p < prompts; ++p) {
        std::string prompt(len, '\0');
        if (!texts.empty()) {
            prompt = texts[p];
        } else {
            for (auto &c : prompt) {
                seed = seed * 6364136223846793005ull + 1442695040888963407ull;
                c = static_cast<char>(seed >> 56);
            }
        }
        const fm::PromptResult a = cpu.run_prompt(prompt, gen);
        const fm::PromptResult b = gpu.run_prompt(prompt, gen);
        if (a.prefill_logits.size() != b.prefill_logits.size()) return 3;
        for (size_t i = 0; i < a.prefill_logits.size(); ++i) {
            uint32_t x, y;
            std::memcpy(&x, &a.prefill_logits[i], 4);
            std::memcpy(&y, &b.prefill_logits[i], 4);
            differing += x != y;
            max_diff = std::max(max_diff, std::fabs(static_cast<double>(a.prefill_logits[i]) - b.prefill_logits[i]));
        }
        logits += a.prefill_logits.size();
        ids_same = ids_same && a.generated_ids == b.generated_ids && a.input_ids == b.input_ids;
        generated += a.generated_ids.size();
        routing_same = routing_same && a.routing.size() == b.routing.size();
        for (size_t i = 0; routing_same && i < a.routing.size(); ++i)
            routing_same = a.routing[i].token_index == b.routing[i].token_index &&
                           a.routing[i].layer == b.routing[i].layer && a.routing[i].experts == b.routing[i].experts;
        routing_events += a.routing.size();
    }
    std::printf("{\"mode\":\"twin\",\"backends\":[\"%s\",\"%s\"],\"prompts\":%u,\"logits\":%llu,"
                "\"differing_logits\":%llu,\"max_abs_diff\":%.9g,\"routing_events\":%llu,\"routing_identical\":%s,"
                "\"generated\":%llu,\"ids_identical\":%s,\"gpu_ops\":%s}\n",
                cpu.backend().name().c_str(), gpu.backend().name().c_str(), prompts,
                static_cast<unsigned long long>(logits), static_cast<unsigned long long>(differing), max_diff,
                static_cast<unsigned long long>(routing_events), routing_same ? "true" : "false",
                static_cast<unsigned long long>(generated), ids_same ? "true" : "false",
                op_labels(gpu.backend()).c_str());
    return 0;
}

int twin(int argc, char **argv) {
    if (argc < 7) return 2;
    if (argc >= 9) {
        g_hot_bytes = std::strtoull(argv[7], nullptr, 10) << 30;
        g_slots = static_cast<uint32_t>(std::atoi(argv[8]));
    }
    return twin_run(argv[2], {}, static_cast<uint32_t>(std::atoi(argv[3])), static_cast<uint32_t>(std::atoi(argv[4])),
                    static_cast<uint32_t>(std::atoi(argv[5])), std::strtoull(argv[6], nullptr, 10));
}

int prompt(int argc, char **argv) {
    if (argc < 5) return 2;
    return twin_run(argv[2], {argv[4]}, 1, 0, static_cast<uint32_t>(std::atoi(argv[3])), 0);
}

std::string seeded_prompt(uint32_t len, uint64_t &seed) {
    std::string prompt(len, '\0');
    for (auto &c : prompt) {
        seed = seed * 6364136223846793005ull + 1442695040888963407ull;
        c = static_cast<char>(seed >> 56);
    }
    return prompt;
}

template <typename T> void put(std::ofstream &f, const T &v) { f.write(reinterpret_cast<const char *>(&v), sizeof(T)); }
template <typename T> void put_vec(std::ofstream &f, const std::vector<T> &v) {
    put(f, static_cast<uint32_t>(v.size()));
    f.write(reinterpret_cast<const char *>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
}
template <typename T> T get(std::ifstream &f) {
    T v{};
    f.read(reinterpret_cast<char *>(&v), sizeof(T));
    if (!f) throw fm::Error(fm::ErrorCode::INVALID_ARGUMENT, "golden file truncated");
    return v;
}
template <typename T> std::vector<T> get_vec(std::ifstream &f) {
    std::vector<T> v(get<uint32_t>(f));
    f.read(reinterpret_cast<char *>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
    if (!f) throw fm::Error(fm::ErrorCode::INVALID_ARGUMENT, "golden file truncated");
    return v;
}

struct Golden {
    std::string prompt;
    uint32_t generate = 0;
    std::vector<int32_t> input_ids, generated;
    std::vector<float> logits;
    std::vector<fm::RoutingEvent> routing;
};

int record(int argc, char **argv) {
    if (argc < 8) return 2;
    if (argc >= 10) {
        g_hot_bytes = std::strtoull(argv[8], nullptr, 10) << 30;
        g_slots = static_cast<uint32_t>(std::atoi(argv[9]));
    }
    const uint32_t prompts = static_cast<uint32_t>(std::atoi(argv[3])), len = static_cast<uint32_t>(std::atoi(argv[4]));
    const uint32_t gen = static_cast<uint32_t>(std::atoi(argv[5]));
    uint64_t seed = std::strtoull(argv[6], nullptr, 10);
    fm::Engine cpu(config_for(argv[2], false));
    cpu.initialize();
    std::ofstream f(argv[7], std::ios::binary);
    f.write("FMXG", 4);
    put(f, prompts);
    for (uint32_t p = 0; p < prompts; ++p) {
        const std::string prompt = seeded_prompt(len, seed);
        const fm::PromptResult r = cpu.run_prompt(prompt, gen);
        put_vec(f, std::vector<char>(prompt.begin(), prompt.end()));
        put(f, gen);
        put_vec(f, r.input_ids);
        put_vec(f, r.prefill_logits);
        put_vec(f, r.generated_ids);
        put(f, static_cast<uint32_t>(r.routing.size()));
        for (const fm::RoutingEvent &ev : r.routing) {
            put(f, static_cast<uint64_t>(ev.token_index));
            put(f, static_cast<uint32_t>(ev.layer));
            put_vec(f, ev.experts);
        }
        std::fprintf(stderr, "record: prompt %u of %u done (%zu input, %zu generated)\n", p + 1, prompts,
                     r.input_ids.size(), r.generated_ids.size());
    }
    if (!f) return 3;
    std::printf("{\"mode\":\"record\",\"backend\":\"%s\",\"prompts\":%u}\n", cpu.backend().name().c_str(), prompts);
    return 0;
}

int replay(int argc, char **argv) {
    if (argc < 4) return 2;
    if (argc >= 6) {
        g_hot_bytes = std::strtoull(argv[4], nullptr, 10) << 30;
        g_slots = static_cast<uint32_t>(std::atoi(argv[5]));
    }
    std::ifstream f(argv[3], std::ios::binary);
    char magic[4] = {};
    f.read(magic, 4);
    if (!f || std::memcmp(magic, "FMXG", 4) != 0) return 3;
    std::vector<Golden> gold(get<uint32_t>(f));
    for (Golden &g : gold) {
        const std::vector<char> pr = get_vec<char>(f);
        g.prompt.assign(pr.begin(), pr.end());
        g.generate = get<uint32_t>(f);
        g.input_ids = get_vec<int32_t>(f);
        g.logits = get_vec<float>(f);
        g.generated = get_vec<int32_t>(f);
        g.routing.resize(get<uint32_t>(f));
        for (fm::RoutingEvent &ev : g.routing) {
            ev.token_index = get<uint64_t>(f);
            ev.layer = get<uint32_t>(f);
            ev.experts = get_vec<uint32_t>(f);
        }
    }
    fm::Engine gpu(config_for(argv[2], true));
    gpu.initialize();
    double max_diff = 0.0, prefill_ms = 0.0, decode_ms = 0.0;
    uint64_t differing = 0, logits = 0, routing_events = 0, generated = 0, prompt_tokens = 0;
    bool routing_same = true, ids_same = true;
    for (size_t p = 0; p < gold.size(); ++p) {
        const Golden &a = gold[p];
        const fm::PromptResult b = gpu.run_prompt(a.prompt, a.generate);
        if (a.logits.size() != b.prefill_logits.size()) return 4;
        for (size_t i = 0; i < a.logits.size(); ++i) {
            uint32_t x, y;
            std::memcpy(&x, &a.logits[i], 4);
            std::memcpy(&y, &b.prefill_logits[i], 4);
            differing += x != y;
            max_diff = std::max(max_diff, std::fabs(static_cast<double>(a.logits[i]) - b.prefill_logits[i]));
        }
        logits += a.logits.size();
        ids_same = ids_same && a.generated == b.generated_ids && a.input_ids == b.input_ids;
        generated += b.generated_ids.size();
        prompt_tokens += b.input_ids.size();
        routing_same = routing_same && a.routing.size() == b.routing.size();
        for (size_t i = 0; routing_same && i < a.routing.size(); ++i)
            routing_same = a.routing[i].token_index == b.routing[i].token_index &&
                           a.routing[i].layer == b.routing[i].layer && a.routing[i].experts == b.routing[i].experts;
        routing_events += a.routing.size();
        prefill_ms += b.prefill_ms;
        decode_ms += b.decode_ms;
        std::fprintf(stderr, "replay: prompt %zu of %zu done (prefill %.1f ms, decode %.1f ms)\n", p + 1,
                     gold.size(), b.prefill_ms, b.decode_ms);
    }
    std::printf("{\"mode\":\"replay\",\"backend\":\"%s\",\"prompts\":%zu,\"logits\":%llu,"
                "\"differing_logits\":%llu,\"max_abs_diff\":%.9g,\"routing_events\":%llu,\"routing_identical\":%s,"
                "\"prompt_tokens\":%llu,\"generated\":%llu,\"ids_identical\":%s,\"prefill_ms\":%.3f,"
                "\"decode_ms\":%.3f,\"gpu_ops\":%s}\n",
                gpu.backend().name().c_str(), gold.size(), static_cast<unsigned long long>(logits),
                static_cast<unsigned long long>(differing), max_diff, static_cast<unsigned long long>(routing_events),
                routing_same ? "true" : "false", static_cast<unsigned long long>(prompt_tokens),
                static_cast<unsigned long long>(generated), ids_same ? "true" : "false", prefill_ms, decode_ms,
                op_labels(gpu.backend()).c_str());
    return 0;
}

} // namespace

int main(int argc, char **argv) {
    try {
        if (argc >= 2 && std::string(argv[1]) == "compare") return compare(argc, argv);
        if (argc >= 2 && std::string(argv[1]) == "twin") return twin(argc, argv);
        if (argc >= 2 && std::string(argv[1]) == "residency") return residency(argc, argv);
        if (argc >= 2 && std::string(argv[1]) == "prompt") return prompt(argc, argv);
        if (argc >= 2 && std::string(argv[1]) == "record") return record(argc, argv);
        if (argc >= 2 && std::string(argv[1]) == "replay") return replay(argc, argv);
    } catch (const fm::Error &e) {
        std::fprintf(stderr, "engine_check: %s: %s\n", fm::error_name(e.code), e.what());
        return 1;
    }
    std::fprintf(stderr, "usage: engine_check compare|twin|residency|prompt|record|replay ...\n");
    return 2;
}
