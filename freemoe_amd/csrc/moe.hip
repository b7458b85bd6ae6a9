// moe.hip — the MoE block of Engine::forward_token on gfx950.
//
//   route_kernel    RMSNorm (engine.cpp:723-740) -> router logits (F32, the
//                   gemv_avx2_row order) -> logit bias (engine.cpp:1611-1616) ->
//                   softmax (engine.cpp:378-393) -> stable top-k
//                   (engine.cpp:395-411) -> weights (engine.cpp:1680-1702).
//                   One workgroup per token: 256 threads per token for batches,
//                   1024 threads with the router rows staged in LDS for decode.
//   gate_up_kernel  gate and up rows of each routed expert, fused with SwiGLU
//                   (engine.cpp:1738-1761; activation.hpp:33, 84).
//   down_kernel     down rows of all routed experts of a token, the combine in
//                   rank order (engine.cpp:1770) and the residual add
//                   (engine.cpp:813-816, 1822).
//
// gfx950 gives a workgroup up to 160 KiB of LDS; the decode kernels stage the
// whole router, the whole of h, and every routed expert's activations at once
// so that no pass waits twice on HBM latency.
//
// RMSNorm's sum of squares is a sequential double sum in the reference. Here it
// is a parallel sum plus a certificate: every normalised value is checked to
// lie farther from a float rounding boundary than the worst-case difference
// between the two sums can move it; only when some value is that close does
// one lane redo the sum in the reference's order. Either way h is the
// reference's h bit for bit.
#include "chains.hpp"
#include "matvec.hpp"
#include "moe.hpp"

#include <mutex>
#include <vector>

namespace fmx {

namespace {

constexpr uint32_t kRouteThreads = 256;      // batched routing: one workgroup per token
constexpr uint32_t kDecodeRouteThreads = 1024;
constexpr uint32_t kMaxHidden = 16384;         // hidden sizes the routing kernels accept
// Dynamic LDS these kernels request at most: a gfx950 workgroup may hold
// 160 KiB, of which 1 KiB is left for the kernels' static LDS.
constexpr size_t kMaxLds = 159 * 1024;
constexpr uint32_t kThreads = 256;

__device__ inline double wave_sum_double(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// The float after f towards +infinity (f finite).
__device__ inline float float_up(float f) {
    if (f == 0.0f) return __uint_as_float(1u);
    const uint32_t b = __float_as_uint(f);
    return __uint_as_float((b >> 31) ? b - 1 : b + 1);
}

// True when float(yd) could change if yd moved by rel_tol of itself: the
// rounding boundaries around f are the midpoints to its neighbours, exact in
// double.
__device__ inline bool rounding_unsafe(double yd, float f, double rel_tol) {
    if (!__builtin_isfinite(f) || __builtin_isnan(yd)) return true;
    if (yd == 0.0) return false;
    const double tol = __builtin_fabs(yd) * rel_tol;
    const double lo = (static_cast<double>(f) + static_cast<double>(-float_up(-f))) * 0.5;
    const double hi = (static_cast<double>(f) + static_cast<double>(float_up(f))) * 0.5;
    return (yd - lo) <= tol || (hi - yd) <= tol;
}

__device__ inline float normalised(float x, const float *w, uint32_t k, double scale,
                                   double norm_bias) {
    const float gain = w ? static_cast<float>(norm_bias + static_cast<double>(w[k])) : 1.0f;
    return static_cast<float>(static_cast<double>(x) * scale * static_cast<double>(gain));
}

// Writes RMSNorm(x) into hs (LDS, H floats); NT threads, x held in registers
// (H <= kMaxHidden). The norm gains are requested with x. Every thread of the
// workgroup calls it; ends with a barrier.
// When some value is too close to a float rounding boundary, the sum is redone
// in the reference's order from a copy of x in `scratch` (LDS, H floats; may be
// nullptr, then x is read again from memory); returns true when `scratch` was
// overwritten.
template <uint32_t NT>
__device__ bool rmsnorm_lds(const RouteArgs &a, const float *__restrict__ x, float *hs, float *scratch) {
    constexpr uint32_t kPer = kMaxHidden / NT;
    __shared__ double wave_part[NT / 64];
    __shared__ double ss_s;
    __shared__ int unsafe_s;
    const uint32_t H = a.hidden, tid = threadIdx.x;
    float xv[kPer];
    double part = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t k = tid + i * NT;
        xv[i] = k < H ? x[k] : 0.0f;
        if (k < H) hs[k] = a.norm_weight ? a.norm_weight[k] : 1.0f;
    }
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) part += static_cast<double>(xv[i]) * static_cast<double>(xv[i]);
    part = wave_sum_double(part);
    if ((tid & 63) == 0) wave_part[tid >> 6] = part;
    if (tid == 0) unsafe_s = 0;
    __syncthreads();
    if (tid == 0) {
        double ss = wave_part[0];
        for (uint32_t w = 1; w < NT / 64; ++w) ss += wave_part[w];
        ss_s = ss;
    }
    __syncthreads();
    // |parallel sum - sequential sum| <= (H + 32) u ss; scale moves by half of
    // that plus a few roundings (see header)
    const double rel_tol = 0.6e-16 * static_cast<double>(H + 32) + 2e-15;
    double scale = 1.0 / sqrt(ss_s / static_cast<double>(H) + a.rms_eps);
    bool unsafe = false;
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t k = tid + i * NT;
        if (k < H) {
            const float gain = a.norm_weight ? static_cast<float>(a.norm_bias + static_cast<double>(hs[k])) : 1.0f;
            const double yd = static_cast<double>(xv[i]) * scale * static_cast<double>(gain);
            const float f = static_cast<float>(yd);
            hs[k] = f;
            unsafe |= rounding_unsafe(yd, f, rel_tol);
        }
    }
    if (unsafe) atomicOr(&unsafe_s, 1);
    __syncthreads();
    if (!unsafe_s) return false;
    if (scratch) {
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t k = tid + i * NT;
            if (k < H) scratch[k] = xv[i];
        }
        __syncthreads();
    }
    if (tid == 0) {
        const float *src = scratch ? scratch : x;
        double ss = 0.0;
#pragma unroll 16
        for (uint32_t k = 0; k < H; ++k) ss += static_cast<double>(src[k]) * static_cast<double>(src[k]);
        ss_s = ss;
    }
    __syncthreads();
    scale = 1.0 / sqrt(ss_s / static_cast<double>(H) + a.rms_eps);
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t k = tid + i * NT;
        if (k < H) hs[k] = normalised(xv[i], a.norm_weight, k, scale, a.norm_bias);
    }
    __syncthreads();
    return scratch != nullptr;
}

// Softmax (float max, double exp and sum, float quotient), stable top-k on
// the probabilities (ties to the lower index) and the routing weights, from
// the E logits in logit_s (LDS). exps (E doubles) and prob_s (E floats) are
// LDS scratch. NT threads; every thread of the workgroup calls it.
template <uint32_t NT>
__device__ void finish_routing(const RouteArgs &a, const float *logit_s, double *exps, float *prob_s,
                               uint32_t *__restrict__ ids, float *__restrict__ weights,
                               uint32_t *__restrict__ status) {
    __shared__ float max_s;
    __shared__ int bad_s;
    __shared__ double sum_s;
    const uint32_t E = a.experts, K = a.top_k, tid = threadIdx.x;
    if (tid == 0) {
        float m = logit_s[0];
        int bad = 0;
        for (uint32_t e = 0; e < E; ++e) {
            if (!__builtin_isfinite(logit_s[e])) bad = 1;
            if (logit_s[e] > m) m = logit_s[e];
        }
        max_s = m;
        bad_s = bad;
    }
    __syncthreads();
    if (bad_s) {
        // The reference raises INTERNAL_ERROR here. Record it and emit a
        // routing that keeps every later kernel in bounds.
        if (tid == 0) atomicOr(status, STATUS_NONFINITE_SCORE);
        for (uint32_t i = tid; i < K; i += NT) {
            ids[i] = i < E ? i : 0;
            weights[i] = 0.0f;
        }
        return;
    }
    for (uint32_t e = tid; e < E; e += NT) exps[e] = exp(static_cast<double>(logit_s[e]) - static_cast<double>(max_s));
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
        for (uint32_t e = 0; e < E; ++e) s += exps[e];
        sum_s = s;
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += NT) prob_s[e] = static_cast<float>(exps[e] / sum_s);
    __syncthreads();
    if (tid == 0) {
        uint32_t chosen[32];
        float wv[32];
        float total = 0.0f;
        for (uint32_t r = 0; r < K; ++r) {
            uint32_t best = E;
            for (uint32_t e = 0; e < E; ++e) {
                bool taken = false;
                for (uint32_t q = 0; q < r; ++q) taken |= chosen[q] == e;
                if (taken) continue;
                if (best == E || prob_s[e] > prob_s[best]) best = e;
            }
            chosen[r] = best;
        }
        for (uint32_t r = 0; r < K; ++r) {
            wv[r] = prob_s[chosen[r]];
            total += wv[r];
        }
        if (a.weights_norm) {
            const double den = a.epsilon_additive ? static_cast<double>(total) + a.weights_epsilon
                                                  : fmax(static_cast<double>(total), a.weights_epsilon);
            for (uint32_t r = 0; r < K; ++r) wv[r] = static_cast<float>(static_cast<double>(wv[r]) / den);
        }
        for (uint32_t r = 0; r < K; ++r) {
            ids[r] = chosen[r];
            weights[r] = static_cast<float>(static_cast<double>(wv[r]) * a.weights_scale);
        }
    }
}

// Routing, one workgroup of NT threads per token. rows_lds = 0: the 16 chain
// lanes of a router row read it from global memory (batched prefill: many
// tokens in flight hide the latency). rows_lds > 0: the router is staged into
// LDS rows_lds rows at a time with every thread's loads in flight together,
// and the chains read LDS (decode: one token, latency exposed).
template <uint32_t NT>
__global__ __launch_bounds__(NT) void route_kernel(RouteArgs a, uint32_t rows_lds, const float *__restrict__ x,
                                                   float *__restrict__ h_out, float *__restrict__ logits_out,
                                                   uint32_t *__restrict__ ids, float *__restrict__ weights,
                                                   uint32_t *__restrict__ status) {
    extern __shared__ __align__(16) double lds_d[];
    const uint32_t H = a.hidden, E = a.experts, K = a.top_k;
    const uint32_t tid = threadIdx.x, t = blockIdx.x;
    double *exps = lds_d;                                   // [E]
    float *hs = reinterpret_cast<float *>(lds_d + E);       // [H]
    float *logit_s = hs + H;                                // [E]
    float *prob_s = logit_s + E;                            // [E]
    float *rows = reinterpret_cast<float *>(reinterpret_cast<char *>(lds_d) +
                                            align_up(E * sizeof(double) + (H + 2 * E) * sizeof(float), 16));
    const uint32_t c = tid & 15, grp = tid >> 4;

    if (rows_lds == 0) {
        rmsnorm_lds<NT>(a, x + static_cast<uint64_t>(t) * H, hs, nullptr);
        for (uint32_t e0 = 0; e0 < E; e0 += NT / 16) {
            const uint32_t e = e0 + grp;
            const uint32_t er = e < E ? e : E - 1;
            const float v = f32_row_chains(a.router + static_cast<uint64_t>(er) * H, hs, H, c);
            if (c == 0 && e < E) logit_s[e] = a.router_bias ? v + a.router_bias[e] : v;
        }
    } else {
        for (uint32_t e0 = 0; e0 < E; e0 += rows_lds) {
            const uint32_t nr = E - e0 < rows_lds ? E - e0 : rows_lds;
            if (e0 > 0) __syncthreads(); // the previous rows' chains are done
            const float4 *src = reinterpret_cast<const float4 *>(a.router + static_cast<uint64_t>(e0) * H);
            float4 *dst = reinterpret_cast<float4 *>(rows);
            const uint32_t n4 = nr * H / 4;
            // stage this pass's router rows; a second time when the exact
            // RMSNorm fallback used the rows' LDS as its copy of x
            for (int again = 0; again < 2; ++again) {
                for (uint32_t i0 = tid; i0 < n4; i0 += 8 * NT) {
                    float4 v[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const uint32_t i = i0 + u * NT;
                        v[u] = src[i < n4 ? i : n4 - 1];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (i0 + u * NT < n4) dst[i0 + u * NT] = v[u];
                }
                if (e0 > 0 || again) {
                    __syncthreads();
                    break;
                }
                // ends with a barrier
                if (!rmsnorm_lds<NT>(a, x + static_cast<uint64_t>(t) * H, hs, rows)) break;
            }
            for (uint32_t r = grp; r < nr; r += NT / 16) {
                const float v = f32_row_chains(rows + static_cast<uint64_t>(r) * H, hs, H, c);
                const uint32_t e = e0 + r;
                if (c == 0) logit_s[e] = a.router_bias ? v + a.router_bias[e] : v;
            }
        }
    }
    __syncthreads();
    if (h_out)
        for (uint32_t k = tid; k < H; k += NT) h_out[static_cast<uint64_t>(t) * H + k] = hs[k];
    if (logits_out)
        for (uint32_t e = tid; e < E; e += NT) logits_out[static_cast<uint64_t>(t) * E + e] = logit_s[e];
    finish_routing<NT>(a, logit_s, exps, prob_s, ids + static_cast<uint64_t>(t) * K,
                       weights + static_cast<uint64_t>(t) * K, status);
}

// ------------------------------------------------------------ experts --

__device__ inline float swiglu(float gate, float up) {
    const double g = static_cast<double>(gate);
    return static_cast<float>(g / (1.0 + exp(-g))) * up;
}

// Gate and up rows j of the expert at rank blockIdx.y, RJ rows per thread:
// the first PF chunks of every row are requested before h is staged.
// Four wavefronts per SIMD (at most 128 VGPRs): the whole grid of a Mixtral
// expert pair is then resident at once.
template <class T, int RJ, int PF>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void gate_up_kernel(ExpertArgs a, const float *__restrict__ h,
                                                           const uint32_t *__restrict__ ids,
                                                           float *__restrict__ act,
                                                           uint32_t *__restrict__ status) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t tid = threadIdx.x, l = tid & 7, slot = tid >> 3;
    const uint32_t rank = blockIdx.y;
    const uint32_t e = ids[rank];
    if (e >= a.experts) {
        if (tid == 0 && blockIdx.x == 0) atomicOr(status, STATUS_BAD_EXPERT);
        return;
    }
    const uint8_t *gate = static_cast<const uint8_t *>(a.gate[e]);
    const uint8_t *up = static_cast<const uint8_t *>(a.up[e]);
    const uint32_t F = a.ffn;
    const uint32_t j0 = (blockIdx.x * (kThreads / 8) + slot) * RJ;
    typename T::Row rw[2 * RJ];
    float t[2 * RJ];
#pragma unroll
    for (int m = 0; m < RJ; ++m) {
        const uint32_t j = j0 + m < F ? j0 + m : F - 1;
        rw[2 * m] = T::row(gate, a.gu.scale_bytes, a.gu.blocks_padded, a.gu.chunks, j, l);
        rw[2 * m + 1] = T::row(up, a.gu.scale_bytes, a.gu.blocks_padded, a.gu.chunks, j, l);
        t[2 * m] = 0.0f;
        t[2 * m + 1] = 0.0f;
    }
    const uint32_t blocks = a.gu.blocks;
    const uint32_t c_end = (blocks + T::kPerChunk - 1) / T::kPerChunk;
    ChunkStream<T, 2 * RJ, PF> cs;
    cs.prime(rw, c_end);
    for (uint32_t tb = 0; tb < blocks; tb += a.gu_tile) {
        const uint32_t nb = blocks - tb < a.gu_tile ? blocks - tb : a.gu_tile;
        __syncthreads();
        T::stage(h, tb, nb, lds, tid, kThreads);
        __syncthreads();
        cs.run(rw, tb / T::kPerChunk, (tb + nb + T::kPerChunk - 1) / T::kPerChunk, c_end, blocks, tb, nb, lds, l,
               t);
    }
#pragma unroll
    for (int m = 0; m < RJ; ++m) {
        const float g = T::finish(t[2 * m]);
        const float u = T::finish(t[2 * m + 1]);
        if (l == 0 && j0 + m < F) act[static_cast<uint64_t>(rank) * F + j0 + m] = swiglu(g, u);
    }
}

// Down rows of every routed expert of one token, then the combine in rank
// order (ffn = 0 + w_0 d_0 + w_1 d_1 ..., engine.cpp:1517, 1770) and the
// residual (engine.cpp:813-816, 1822). Row slot s handles rank s / jpw, row
// s % jpw of this workgroup's jpw rows (jpw = 32 / top_k); every rank's
// activations are staged together, so one workgroup finishes its rows alone.
template <class T, int PF>
__global__ __launch_bounds__(kThreads) void down_kernel(ExpertArgs a, const float *__restrict__ x,
                                                        const float *__restrict__ act,
                                                        const uint32_t *__restrict__ ids,
                                                        const float *__restrict__ w,
                                                        float *__restrict__ out,
                                                        uint32_t *__restrict__ status) {
    extern __shared__ __align__(16) float lds[];
    __shared__ float dres[kThreads / 8];
    const uint32_t tid = threadIdx.x, l = tid & 7, slot = tid >> 3;
    const uint32_t K = a.top_k, H = a.hidden;
    const uint32_t jpw = (kThreads / 8) / K;
    const uint32_t rank = slot / jpw < K ? slot / jpw : K - 1;
    const uint32_t j = blockIdx.x * jpw + slot % jpw;
    const uint32_t jr = j < H ? j : H - 1;
    uint32_t e = ids[rank];
    const bool bad = e >= a.experts;
    if (bad) {
        if (l == 0) atomicOr(status, STATUS_BAD_EXPERT);
        e = 0;
    }
    typename T::Row rw[1];
    rw[0] = T::row(static_cast<const uint8_t *>(a.down[e]), a.dn.scale_bytes, a.dn.blocks_padded, a.dn.chunks,
                   jr, l);
    float t[1] = {0.0f};
    const uint32_t blocks = a.dn.blocks;
    const uint32_t c_end = (blocks + T::kPerChunk - 1) / T::kPerChunk;
    const uint32_t tile_floats = a.dn_tile * T::kLdsFloatsPerBlock;
    ChunkStream<T, 1, PF> cs;
    cs.prime(rw, c_end);
    for (uint32_t tb = 0; tb < blocks; tb += a.dn_tile) {
        const uint32_t nb = blocks - tb < a.dn_tile ? blocks - tb : a.dn_tile;
        __syncthreads();
        for (uint32_t r = 0; r < K; ++r)
            T::stage(act + static_cast<uint64_t>(r) * a.ffn, tb, nb, lds + r * tile_floats, tid, kThreads);
        __syncthreads();
        cs.run(rw, tb / T::kPerChunk, (tb + nb + T::kPerChunk - 1) / T::kPerChunk, c_end, blocks, tb, nb,
               lds + rank * tile_floats, l, t);
    }
    const float v = T::finish(t[0]);
    if (l == 0) dres[slot] = bad ? 0.0f : v;
    __syncthreads();
    if (tid < jpw) {
        const uint32_t jo = blockIdx.x * jpw + tid;
        if (jo < H) {
            float ffn = 0.0f;
            for (uint32_t r = 0; r < K; ++r) ffn = ffn + w[r] * dres[r * jpw + tid];
            out[jo] = x[jo] + ffn;
        }
    }
}

// F32 experts: 16 lanes per row, x read through the cache.
__global__ __launch_bounds__(kThreads) void gate_up_f32_kernel(ExpertArgs a, const float *__restrict__ h,
                                                               const uint32_t *__restrict__ ids,
                                                               float *__restrict__ act,
                                                               uint32_t *__restrict__ status) {
    const uint32_t tid = threadIdx.x, c = tid & 15;
    const uint32_t rank = blockIdx.y;
    const uint32_t e = ids[rank];
    if (e >= a.experts) {
        if (tid == 0 && blockIdx.x == 0) atomicOr(status, STATUS_BAD_EXPERT);
        return;
    }
    const uint32_t F = a.ffn, H = a.hidden;
    const uint32_t j = blockIdx.x * (kThreads / 16) + (tid >> 4);
    const uint32_t jr = j < F ? j : F - 1;
    const float *gate = static_cast<const float *>(a.gate[e]) + static_cast<uint64_t>(jr) * H;
    const float *up = static_cast<const float *>(a.up[e]) + static_cast<uint64_t>(jr) * H;
    const float g = f32_row_chains(gate, h, H, c);
    const float u = f32_row_chains(up, h, H, c);
    if (c == 0 && j < F) act[static_cast<uint64_t>(rank) * F + j] = swiglu(g, u);
}

__global__ __launch_bounds__(kThreads) void down_f32_kernel(ExpertArgs a, const float *__restrict__ x,
                                                            const float *__restrict__ act,
                                                            const uint32_t *__restrict__ ids,
                                                            const float *__restrict__ w,
                                                            float *__restrict__ out,
                                                            uint32_t *__restrict__ status) {
    __shared__ float dres[kThreads / 16];
    const uint32_t tid = threadIdx.x, c = tid & 15, slot = tid >> 4; // 16 slots
    const uint32_t K = a.top_k, H = a.hidden, F = a.ffn;
    const uint32_t jpw = (kThreads / 16) / K;
    const uint32_t rank = slot / jpw < K ? slot / jpw : K - 1;
    const uint32_t jj = slot % jpw;
    const uint32_t j = blockIdx.x * jpw + jj;
    const uint32_t jr = j < H ? j : H - 1;
    uint32_t e = ids[rank];
    const bool bad = e >= a.experts;
    if (bad) {
        if (c == 0) atomicOr(status, STATUS_BAD_EXPERT);
        e = 0;
    }
    const float *row = static_cast<const float *>(a.down[e]) + static_cast<uint64_t>(jr) * F;
    const float v = f32_row_chains(row, act + static_cast<uint64_t>(rank) * F, F, c);
    if (c == 0 && slot < K * jpw) dres[slot] = bad ? 0.0f : v;
    __syncthreads();
    if (tid < jpw) {
        const uint32_t jo = blockIdx.x * jpw + tid;
        if (jo < H) {
            float ffn = 0.0f;
            for (uint32_t r = 0; r < K; ++r) ffn = ffn + w[r] * dres[r * jpw + tid];
            out[jo] = x[jo] + ffn;
        }
    }
}

// ------------------------------------------------------------ launchers --

// Prefetch depth (chunks in flight per row) of each pass.
constexpr int kGateUpPF = 1;
constexpr int kDownPF = 8;

template <class T>
int launch_experts_q(const ExpertArgs &a, const float *x, const float *h, const uint32_t *ids,
                     const float *w, const DecodeScratch &ws, float *out, uint32_t *status, hipStream_t s,
                     hipEvent_t mid) {
    constexpr int RJ = 1;
    const size_t lds_gu = static_cast<size_t>(a.gu_tile) * T::kLdsFloatsPerBlock * sizeof(float);
    const size_t lds_dn = static_cast<size_t>(a.dn_tile) * T::kLdsFloatsPerBlock * sizeof(float) * a.top_k;
    if (lds_gu > kMaxLds || lds_dn > kMaxLds) return FMX_ERR_SHAPE_MISMATCH;
    auto gu = gate_up_kernel<T, RJ, kGateUpPF>;
    auto dn = down_kernel<T, kDownPF>;
    if (int rc = allow_lds(reinterpret_cast<const void *>(gu), lds_gu)) return rc;
    if (int rc = allow_lds(reinterpret_cast<const void *>(dn), lds_dn)) return rc;
    hipLaunchKernelGGL(gu, dim3(div_up(a.ffn, (kThreads / 8) * RJ), a.top_k), dim3(kThreads), lds_gu, s, a, h, ids,
                       ws.act, status);
    FMX_LAUNCH_CHECK();
    if (mid) FMX_HIP_TRY(hipEventRecord(mid, s));
    const uint32_t jpw = (kThreads / 8) / a.top_k;
    hipLaunchKernelGGL(dn, dim3(div_up(a.hidden, jpw)), dim3(kThreads), lds_dn, s, a, x, ws.act, ids, w, out,
                       status);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace

// Raises the dynamic LDS limit of kernel `fn` (64 KiB by default) to `bytes`
// when a launch needs more; the limit only grows, and each kernel's is kept.
int allow_lds(const void *fn, size_t bytes) {
    if (bytes <= 64 * 1024) return FMX_OK;
    static std::mutex mu;
    static std::vector<std::pair<const void *, size_t>> limits;
    std::lock_guard<std::mutex> lock(mu);
    for (auto &f : limits)
        if (f.first == fn) {
            if (f.second >= bytes) return FMX_OK;
            FMX_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
            f.second = bytes;
            return FMX_OK;
        }
    FMX_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
    limits.emplace_back(fn, bytes);
    return FMX_OK;
}

size_t route_lds_bytes(uint32_t hidden, uint32_t experts, uint32_t rows_lds) {
    const size_t base = static_cast<size_t>(experts) * sizeof(double) + (hidden + 2ull * experts) * sizeof(float);
    return align_up(base, 16) + static_cast<size_t>(rows_lds) * hidden * sizeof(float);
}

// Router rows that fit in LDS next to the routing state (0: none fit).
uint32_t route_rows_in_lds(const RouteArgs &a) {
    const size_t base = route_lds_bytes(a.hidden, a.experts, 0);
    if (a.hidden % 4 || base + a.hidden * sizeof(float) > kMaxLds) return 0;
    const uint32_t rows = static_cast<uint32_t>((kMaxLds - base) / (a.hidden * sizeof(float)));
    return rows < a.experts ? rows : a.experts;
}

// One 1024-thread workgroup per token with the router staged in LDS; when
// not even one router row fits, 256 threads per token reading it from memory.
int launch_route(const RouteArgs &a, const float *x, uint32_t tokens, float *h, float *logits,
                 uint32_t *ids, float *weights, uint32_t *status, hipStream_t s) {
    if (a.hidden > kMaxHidden) return FMX_ERR_SHAPE_MISMATCH;
    const uint32_t rows = route_rows_in_lds(a);
    if (rows > 0) {
        const size_t lds = route_lds_bytes(a.hidden, a.experts, rows);
        auto k = route_kernel<kDecodeRouteThreads>;
        if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
        hipLaunchKernelGGL(k, dim3(tokens), dim3(kDecodeRouteThreads), lds, s, a, rows, x, h, logits, ids, weights,
                           status);
        FMX_LAUNCH_CHECK();
        return FMX_OK;
    }
    const size_t lds = route_lds_bytes(a.hidden, a.experts, 0);
    if (lds > kMaxLds) return FMX_ERR_SHAPE_MISMATCH;
    auto k = route_kernel<kRouteThreads>;
    if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
    hipLaunchKernelGGL(k, dim3(tokens), dim3(kRouteThreads), lds, s, a, 0u, x, h, logits, ids, weights, status);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

int launch_route_decode(const RouteArgs &a, const float *x, float *h, uint32_t *ids, float *weights,
                        uint32_t *status, hipStream_t s) {
    return launch_route(a, x, 1, h, nullptr, ids, weights, status, s);
}

int prepare_expert_args(const fmx_moe_layer *L, ExpertArgs *a) {
    ExpertArgs e;
    e.hidden = L->hidden;
    e.ffn = L->ffn;
    e.experts = L->experts;
    e.top_k = L->top_k;
    e.type_gu = L->gate_type;
    e.type_dn = L->down_type;
    e.gate = L->gate;
    e.up = L->up;
    e.down = L->down;
    if (L->up_type != L->gate_type) return FMX_ERR_UNSUPPORTED_QUANTISATION;
    if (int rc = packed_geometry(L->gate_type, L->ffn, L->hidden, &e.gu)) return rc;
    if (int rc = packed_geometry(L->down_type, L->hidden, L->ffn, &e.dn)) return rc;
    // LDS tiles (blocks): gate/up stages one tile of h, down one tile of every
    // rank's activations; a tile is the whole row when it fits, else a whole
    // multiple of the pass's chunk ring (prefetch depth + 1)
    constexpr uint32_t kGuBudget = 32 * 1024;                      // floats
    const uint32_t dn_budget = static_cast<uint32_t>(kMaxLds / 4 - 1024) / L->top_k;
    switch (L->gate_type) {
    case FMX_TYPE_Q4_0: e.gu_tile = tile_blocks_for<Q40>(e.gu.blocks, kGuBudget, kGateUpPF + 1); break;
    case FMX_TYPE_Q8_0: e.gu_tile = tile_blocks_for<Q80>(e.gu.blocks, kGuBudget, kGateUpPF + 1); break;
    case FMX_TYPE_Q4_K: e.gu_tile = tile_blocks_for<Q4K>(e.gu.blocks, kGuBudget, kGateUpPF + 1); break;
    default: e.gu_tile = 0; break;
    }
    switch (L->down_type) {
    case FMX_TYPE_Q4_0: e.dn_tile = tile_blocks_for<Q40>(e.dn.blocks, dn_budget, kDownPF + 1); break;
    case FMX_TYPE_Q8_0: e.dn_tile = tile_blocks_for<Q80>(e.dn.blocks, dn_budget, kDownPF + 1); break;
    case FMX_TYPE_Q4_K: e.dn_tile = tile_blocks_for<Q4K>(e.dn.blocks, dn_budget, kDownPF + 1); break;
    default: e.dn_tile = 0; break;
    }
    *a = e;
    return FMX_OK;
}

int launch_experts(const ExpertArgs &a, const float *x, const float *h, const uint32_t *ids,
                   const float *w, const DecodeScratch &ws, float *out, uint32_t *status, hipStream_t s,
                   hipEvent_t mid) {
    float *act = ws.act;
    if (a.type_gu == FMX_TYPE_F32) {
        if (a.top_k > kThreads / 16 || a.type_dn != FMX_TYPE_F32) return FMX_ERR_UNSUPPORTED_QUANTISATION;
        hipLaunchKernelGGL(gate_up_f32_kernel, dim3(div_up(a.ffn, kThreads / 16), a.top_k), dim3(kThreads), 0, s,
                           a, h, ids, act, status);
        FMX_LAUNCH_CHECK();
        if (mid) FMX_HIP_TRY(hipEventRecord(mid, s));
    }
    if (a.type_gu == FMX_TYPE_F32 && a.type_dn == FMX_TYPE_F32) {
        const uint32_t jpw = (kThreads / 16) / a.top_k;
        hipLaunchKernelGGL(down_f32_kernel, dim3(div_up(a.hidden, jpw)), dim3(kThreads), 0, s, a, x, act, ids,
                           w, out, status);
        FMX_LAUNCH_CHECK();
        return FMX_OK;
    }
    if (a.type_gu != a.type_dn) return FMX_ERR_UNSUPPORTED_QUANTISATION;
    switch (a.type_gu) {
    case FMX_TYPE_Q4_0: return launch_experts_q<Q40>(a, x, h, ids, w, ws, out, status, s, mid);
    case FMX_TYPE_Q8_0: return launch_experts_q<Q80>(a, x, h, ids, w, ws, out, status, s, mid);
    case FMX_TYPE_Q4_K: return launch_experts_q<Q4K>(a, x, h, ids, w, ws, out, status, s, mid);
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

} // namespace fmx
