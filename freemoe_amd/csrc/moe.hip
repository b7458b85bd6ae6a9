// moe.hip — the MoE block of Engine::forward_token on gfx950.
//
// Decode, per token:
//   route_rows_kernel  one workgroup per router row: RMSNorm (engine.cpp:723-740)
//                      of the token, then that row's logit (F32, the
//                      gemv_avx2_row order) and its bias (engine.cpp:1611-1616).
//   gate_up_kernel     softmax (engine.cpp:378-393), stable top-k
//                      (engine.cpp:395-411) and the weights (engine.cpp:1680-1702)
//                      in one wavefront from the logits, then gate and up rows
//                      of each routed expert fused with SwiGLU
//                      (engine.cpp:1738-1761; activation.hpp:33, 84).
//   down_pair_kernel / down_kernel
//                      down rows of all routed experts, the combine in rank order
//                      (engine.cpp:1770) and the residual add (engine.cpp:813-816,
//                      1822).
// Batches (prefill routing): rmsnorm_kernel once per token, router_tile_kernel
// (token x row tiles) or router_quant_kernel, route_finish_kernel.
//
// gfx950 gives a workgroup up to 160 KiB of LDS; the decode kernels stage the
// whole of h and every routed expert's activations at once so that no pass
// waits twice on HBM latency.
//
// RMSNorm's sum of squares is a sequential double sum in the reference. Here it
// is a parallel sum plus a certificate: every normalised value is checked to
// lie farther from a float rounding boundary than the worst-case difference
// between the two sums can move it; only when some value is that close does
// one lane redo the sum in the reference's order. Either way h is the
// reference's h bit for bit.
#include "chains.hpp"
#include "down_pair.hpp"
#include "matvec.hpp"
#include "moe.hpp"

#include <hip/hip_ext.h>

#include <mutex>

namespace fmx {

namespace {

constexpr uint32_t kMaxHidden = 16384; // hidden sizes the routing kernels accept
// Code alignment of the decode kernels: each starts on its own 4 KiB
// boundary, so that where their loops fall in the instruction cache does not
// move with the size of the kernels placed before them.
constexpr int kHotAlign = 4096;
// Dynamic LDS these kernels request at most: a gfx950 workgroup may hold
// 160 KiB, of which 1 KiB is left for the kernels' static LDS.
constexpr size_t kMaxLds = 159 * 1024;
constexpr uint32_t kThreads = 256;
// Rings per pass of the down kernel's steady-state loop: for Q4_0, 7 chunks
// in flight make 8-chunk rings, so a Mixtral down row (56 chunks) is one pass.
template <class T>
constexpr int down_rings() {
    return T::kType == FMX_TYPE_Q4_0 ? 7 : 1;
}

// Wavefront reductions in the butterfly order m = 32, 16, ..., 1 (lane i
// combines its value with lane i ^ m's at each step), by VALU lane moves
// (lane_pair / lane_xor) rather than ds_bpermute shuffles. The operations
// are commutative, so every lane ends with the same bits.
__device__ inline double wave_sum_double(double v) {
    uint64_t a, b;
    lane_pair_u64<32>(__builtin_bit_cast(uint64_t, v), a, b);
    v = __builtin_bit_cast(double, a) + __builtin_bit_cast(double, b);
    lane_pair_u64<16>(__builtin_bit_cast(uint64_t, v), a, b);
    v = __builtin_bit_cast(double, a) + __builtin_bit_cast(double, b);
    v += __builtin_bit_cast(double, lane_xor_u64<8>(__builtin_bit_cast(uint64_t, v)));
    v += __builtin_bit_cast(double, lane_xor_u64<4>(__builtin_bit_cast(uint64_t, v)));
    v += __builtin_bit_cast(double, lane_xor_u64<2>(__builtin_bit_cast(uint64_t, v)));
    v += __builtin_bit_cast(double, lane_xor_u64<1>(__builtin_bit_cast(uint64_t, v)));
    return v;
}

// True when float(yd) could change if yd moved by up to tol_ulps(yd) of its
// own units in the last place. For yd in float's normal range the float
// grid points are the doubles whose low 29 mantissa bits are zero and the
// rounding boundaries (midpoints) those whose low 29 bits are 2^28, so the
// distance to the nearest boundary is |low29 - 2^28| ulps. tol0 = ceil(rel *
// 2^52) bounds rel * |yd| / ulp(yd) = rel * 2^52 * 1.m from above through the
// top 8 mantissa bits. Values outside float's normal range (other than 0),
// infinities and NaN always count as unsafe.
// Branch-free (it runs on every element); tol0 < 2^24.
__device__ inline bool rounding_unsafe(double yd, uint32_t tol0) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(yd));
    const uint32_t hi = static_cast<uint32_t>(b >> 32), lo = static_cast<uint32_t>(b);
    const uint32_t ex = (hi >> 20) & 0x7FFu;
    const bool outside = ex - (1023u - 126u) >= 253u; // ex < 897 or ex >= 1150
    const bool nonzero = ((hi << 1) | lo) != 0u;
    const uint32_t low29 = lo & 0x1FFFFFFFu;
    const uint32_t d = low29 >= (1u << 28) ? low29 - (1u << 28) : (1u << 28) - low29;
    const uint32_t m8 = (hi >> 12) & 0xFFu;
    const bool near = d <= tol0 + (__umul24(tol0, m8 + 1u) >> 8) + 1u;
    return outside ? nonzero : near;
}

__device__ inline float normalised(float x, const float *w, uint32_t k, double scale,
                                   double norm_bias) {
    const float gain = w ? static_cast<float>(norm_bias + static_cast<double>(w[k])) : 1.0f;
    return static_cast<float>(static_cast<double>(x) * scale * static_cast<double>(gain));
}

// ------------------------------------------------------------- routing --

__device__ inline double readlane_double(double v, uint32_t lane) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(b), lane);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane);
    return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
    uint64_t a, b;
    lane_pair_u64<32>(v, a, b);
    v = a > b ? a : b;
    lane_pair_u64<16>(v, a, b);
    v = a > b ? a : b;
    uint64_t o = lane_xor_u64<8>(v);
    v = o > v ? o : v;
    o = lane_xor_u64<4>(v);
    v = o > v ? o : v;
    o = lane_xor_u64<2>(v);
    v = o > v ? o : v;
    o = lane_xor_u64<1>(v);
    return o > v ? o : v;
}

__device__ inline float wave_max_float(float v) {
    uint32_t a, b;
    lane_pair_u32<32>(__builtin_bit_cast(uint32_t, v), a, b);
    v = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    lane_pair_u32<16>(__builtin_bit_cast(uint32_t, v), a, b);
    v = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    v = fmaxf(v, lane_xor<8>(v));
    v = fmaxf(v, lane_xor<4>(v));
    v = fmaxf(v, lane_xor<2>(v));
    return fmaxf(v, lane_xor<1>(v));
}

struct Routing {
    uint32_t id;  // expert of rank (lane) r < top_k
    float weight; // its routing weight
};

// Routing of one token from its E <= 256 router logits, by one wavefront
// (every lane calls it; lane r < top_k receives rank r):
//   softmax (engine.cpp:378-393): float max, double exp(v - max) summed in
//   index order (or, kCertified, a certified wavefront sum where that gives
//   the same quotients), float quotients;
//   stable top-k (engine.cpp:395-411): the highest probability first, ties to
//   the lower index; picked as the wave maximum of (probability bits, ~index),
//   which orders non-negative floats and breaks ties the same way;
//   weights (engine.cpp:1680-1702): float sum of the picked probabilities in
//   rank order, optional division by it (plus or at least epsilon), scale.
// A logit that is not finite (the reference raises INTERNAL_ERROR) sets *bad
// and yields expert r with weight 0, which keeps every later kernel in bounds.
// kSlots: experts per lane, 64 kSlots >= experts.
// The logits lane `lane` takes (expert lane + 64 j), read from `logits`.
template <int kSlots = 4>
__device__ __forceinline__ void route_logits_load(const RouteArgs &a, const float *__restrict__ logits,
                                                  float (&v)[kSlots]) {
    const uint32_t E = a.experts, lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const uint32_t e = lane + 64 * j;
        v[j] = e < E ? logits[e] : 0.0f;
    }
}

// wave_route from logits already loaded by route_logits_load. kCertified:
// the softmax sum as a certified wavefront sum (worth it for many experts).
template <int kSlots = 4, bool kCertified = false>
__device__ Routing wave_route_values(const RouteArgs &a, const float (&v)[kSlots], bool *bad) {
    const uint32_t E = a.experts, K = a.top_k, lane = threadIdx.x & 63;
    bool nonfinite = false;
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const uint32_t e = lane + 64 * j;
        if (e < E) {
            nonfinite |= !__builtin_isfinite(v[j]);
            m = fmaxf(m, v[j]);
        }
    }
    Routing r;
    if (__any(nonfinite)) {
        *bad = true;
        r.id = lane;
        r.weight = 0.0f;
        return r;
    }
    *bad = false;
    m = wave_max_float(m);
    double ex[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j)
        ex[j] = lane + 64 * j < E ? exp(static_cast<double>(v[j]) - static_cast<double>(m)) : 0.0;
    // The reference's sum is sequential in index order (readlane by
    // readlane here). kCertified: a wavefront sum first, with a certificate
    // as for RMSNorm: the two sums of E terms in (0, 1] differ by at most
    // (E + kSlots + 5) 2^-53 of the sum, which moves each quotient by that
    // much plus its own rounding; only when a quotient lies that close to a
    // float rounding boundary is the sum taken in order.
    double sum = 0.0;
    bool in_order = true;
    if constexpr (kCertified) {
        double part = 0.0;
#pragma unroll
        for (int j = 0; j < kSlots; ++j) part += ex[j];
        sum = wave_sum_double(part);
        const double rel_tol = 1.2e-16 * static_cast<double>(E + 2 * kSlots + 10);
        const uint32_t tol0 = static_cast<uint32_t>(ceil(rel_tol * 4503599627370496.0)); // rel_tol * 2^52
        bool unsafe = false;
#pragma unroll
        for (int j = 0; j < kSlots; ++j) unsafe |= (lane + 64 * j < E) & rounding_unsafe(ex[j] / sum, tol0);
        in_order = __any(unsafe);
    }
    if (in_order) {
        sum = 0.0;
#pragma unroll
        for (int j = 0; j < kSlots; ++j) {
            if (64u * j >= E) break;
            const uint32_t n = E - 64 * j < 64 ? E - 64 * j : 64;
            for (uint32_t i = 0; i < n; ++i) sum += readlane_double(ex[j], i);
        }
    }
    uint64_t key[kSlots];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const uint32_t e = lane + 64 * j;
        const float p = static_cast<float>(ex[j] / sum);
        key[j] = e < E ? (static_cast<uint64_t>(__float_as_uint(p)) << 32) | (0xFFFFFFFFu - e) : 0;
    }
    float total = 0.0f;
    r.id = 0;
    r.weight = 0.0f;
    for (uint32_t k = 0; k < K; ++k) {
        uint64_t best = key[0];
#pragma unroll
        for (int j = 1; j < kSlots; ++j) best = key[j] > best ? key[j] : best;
        best = wave_max_u64(best);
#pragma unroll
        for (int j = 0; j < kSlots; ++j)
            if (key[j] == best) key[j] = 0;
        const float p = __uint_as_float(static_cast<uint32_t>(best >> 32));
        total += p;
        if (lane == k) {
            r.id = 0xFFFFFFFFu - static_cast<uint32_t>(best);
            r.weight = p;
        }
    }
    float wv = r.weight;
    if (a.weights_norm) {
        const double den = a.epsilon_additive ? static_cast<double>(total) + a.weights_epsilon
                                              : fmax(static_cast<double>(total), a.weights_epsilon);
        wv = static_cast<float>(static_cast<double>(wv) / den);
    }
    r.weight = static_cast<float>(static_cast<double>(wv) * a.weights_scale);
    return r;
}

template <int kSlots = 4, bool kCertified = false>
__device__ Routing wave_route(const RouteArgs &a, const float *__restrict__ logits, bool *bad) {
    float v[kSlots];
    route_logits_load(a, logits, v);
    return wave_route_values<kSlots, kCertified>(a, v, bad);
}

// ------------------------------------------------- the in-order double sum --
// The reference's sum of squares is s = 0; s = fl(s + a_i) for i ascending
// (a_i = x_i^2, exact in double). ordered_sum reproduces it bit for bit with
// the whole workgroup instead of one lane, by a property of the sequence:
// while s stays in one binade [2^e, 2^(e+1)), every s is a multiple of
// u = 2^(e-52) and fl(s + a) = s + q u with q = a / u rounded to an integer
// (the nearest one; at an exact half the one that makes (s + q u) / u even).
// So inside a binade the running sum is an integer prefix sum of s / u whose
// only dependence on s is the parity of s / u at ties: each term is a map
// (P, p) -> (P + inc[p], out[p]) on (s / u, its parity), maps compose
// associatively, and a workgroup scan gives every prefix at once, in 64-bit
// integer arithmetic on the terms' mantissas. The first term that would
// leave the binade (s + a >= 2^(e+1)) is added by one lane as an ordinary
// double add from the exact prefix before it, and the next scan starts there
// in the new binade. The first kSeqTerms terms (where s changes binade
// often) are added by one lane; a token whose sum leaves its binade more than
// kMaxScans times finishes in one lane too.
constexpr uint32_t kSeqTerms = 256;
constexpr uint32_t kMaxScans = 48;
constexpr uint64_t kTwo53 = 1ull << 53;

// A term's map: s / u grows by inc0 or inc1 (parity 0 or 1 before the term)
// and the parity after it is bit 0 / bit 1 of `out`.
struct SumMap {
    uint64_t inc0, inc1;
    uint32_t out;
};

__device__ inline SumMap sum_map_identity() { return SumMap{0, 0, 2u}; }

// f, then g
__device__ inline SumMap sum_map_then(const SumMap &f, const SumMap &g) {
    const uint32_t f0 = f.out & 1u, f1 = f.out >> 1;
    SumMap r;
    r.inc0 = f.inc0 + (f0 ? g.inc1 : g.inc0);
    r.inc1 = f.inc1 + (f1 ? g.inc1 : g.inc0);
    r.out = ((g.out >> f0) & 1u) | (((g.out >> f1) & 1u) << 1);
    return r;
}

// Term a (a double >= 0) in binade e: its map, n = floor(a / u), and whether
// it leaves the binade by itself (a >= 2^(e+1), infinities and NaN included:
// then its map only has to be large). a / u = m 2^(Ea - e) for a = m 2^(Ea - 52),
// m the 53-bit significand, so n is m shifted right by d = e - Ea and the
// shifted-out bits decide the rounding: above half up, at half a tie.
__device__ inline SumMap sum_term(double a, int e, uint64_t &n, bool &big) {
    const uint64_t b = static_cast<uint64_t>(__double_as_longlong(a));
    const uint32_t be = static_cast<uint32_t>(b >> 52) & 0x7FFu;
    const uint64_t m = (b & ((1ull << 52) - 1)) | (be ? 1ull << 52 : 0);
    const int d = e - (static_cast<int>(be) - 1023);
    big = d < 0;
    const uint32_t sh = d < 0 ? 0u : d > 63 ? 63u : static_cast<uint32_t>(d);
    const uint64_t q = m >> sh, r = m & ((1ull << sh) - 1), half = sh ? 1ull << (sh - 1) : 0;
    const bool wide = d > 63; // a < u / 2 (or a == 0): rounds to nothing
    n = wide ? 0 : q;
    const bool up = !wide && sh != 0 && r > half, tie = !wide && sh != 0 && r == half;
    SumMap f;
    const uint64_t base = n + (up ? 1u : 0u);
    f.inc0 = base + (tie ? (n & 1u) : 0u);
    f.inc1 = base + (tie ? ((n & 1u) ^ 1u) : 0u);
    f.out = tie ? 0u : ((f.inc0 & 1u) ? 1u : 2u);
    if (big) f = SumMap{kTwo53, kTwo53, 2u};
    return f;
}

// The map of lane - D within this lane's row of 16 (row_shr:D, DPP), the
// identity for the row's first D lanes.
template <int D>
__device__ inline uint32_t row_shr_u32(uint32_t v, uint32_t fill) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(fill), static_cast<int>(v), 0x110 + D, 0xF, 0xF, false));
}
template <int D>
__device__ inline uint64_t row_shr_u64(uint64_t v) {
    return (static_cast<uint64_t>(row_shr_u32<D>(static_cast<uint32_t>(v >> 32), 0)) << 32) |
           row_shr_u32<D>(static_cast<uint32_t>(v), 0);
}
template <int D>
__device__ inline SumMap row_shr_map(const SumMap &g) {
    return SumMap{row_shr_u64<D>(g.inc0), row_shr_u64<D>(g.inc1), row_shr_u32<D>(g.out, 2u)};
}
__device__ inline SumMap readlane_map(const SumMap &g, int lane) {
    auto rd64 = [lane](uint64_t v) {
        const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(v), lane);
        const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), lane);
        return (static_cast<uint64_t>(hi) << 32) | lo;
    };
    return SumMap{rd64(g.inc0), rd64(g.inc1), static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(g.out), lane))};
}

// The composition of the maps of the lanes below this one (exclusive scan
// over the wavefront) and of all 64 (*total): a scan inside each row of 16
// lanes by DPP row shifts, then the rows' totals read out and put in front.
__device__ inline SumMap wave_scan_maps(SumMap g, SumMap *total) {
    g = sum_map_then(row_shr_map<1>(g), g);
    g = sum_map_then(row_shr_map<2>(g), g);
    g = sum_map_then(row_shr_map<4>(g), g);
    g = sum_map_then(row_shr_map<8>(g), g);
    const SumMap below_in_row = row_shr_map<1>(g);
    const SumMap r0 = readlane_map(g, 15), r1 = readlane_map(g, 31), r2 = readlane_map(g, 47), r3 = readlane_map(g, 63);
    const SumMap p2 = sum_map_then(r0, r1), p3 = sum_map_then(p2, r2);
    *total = sum_map_then(p3, r3);
    const uint32_t row = (threadIdx.x & 63) >> 4;
    const SumMap rows_before = row == 0 ? sum_map_identity() : row == 1 ? r0 : row == 2 ? p2 : p3;
    return sum_map_then(rows_before, below_in_row);
}

__device__ inline uint32_t wave_min_u32(uint32_t v) {
    v = min(v, lane_xor_u32<1>(v));
    v = min(v, lane_xor_u32<2>(v));
    v = min(v, lane_xor_u32<4>(v));
    v = min(v, lane_xor_u32<8>(v));
    uint32_t a, b;
    lane_pair_u32<16>(v, a, b);
    v = min(a, b);
    lane_pair_u32<32>(v, a, b);
    return min(a, b);
}

struct OrderedSumShared {
    double s;          // the running sum
    uint32_t next;     // the first term not yet in it
    SumMap wave_total[16];
    uint32_t wave_first[16]; // per wavefront: the first term leaving the binade
};

// sum(a_j, j = 0 .. n-1) in index order, bit for bit, by all NT threads (a
// in LDS, n <= 16 NT). Every thread calls it and gets the sum; it ends after
// a barrier. Out of line: inlined, its registers would be allocated around
// the callers' common path too. Each scan covers a window of the next c NT terms (c per thread,
// c about 1.5 next / NT: while the terms are alike, s leaves its binade about
// when the count of terms in it has doubled); a window with no term leaving
// the binade still ends exact, and the next scan starts after it.
template <uint32_t NT>
__device__ __attribute__((noinline)) double ordered_sum(const double *a, uint32_t n, OrderedSumShared &sh) {
    static_assert(NT % 64 == 0 && NT / 64 <= 16, "one to sixteen wavefronts");
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) {
        // the first terms in one lane, 8 LDS reads requested ahead of the
        // adds they feed; then on while the sum is still 0
        constexpr uint32_t kB = 8;
        const uint32_t lead = n < kSeqTerms ? n : kSeqTerms, nb = lead / kB;
        double s = 0.0, buf[2][kB];
        if (nb > 0) {
#pragma unroll
            for (uint32_t q = 0; q < kB; ++q) buf[0][q] = a[q];
        }
        for (uint32_t bi = 0; bi < nb; bi += 2) {
#pragma unroll
            for (uint32_t half = 0; half < 2; ++half) {
                const uint32_t b = bi + half;
                if (b >= nb) break;
                const uint32_t nx = (b + 1 < nb ? b + 1 : b) * kB;
#pragma unroll
                for (uint32_t q = 0; q < kB; ++q) buf[half ^ 1][q] = a[nx + q];
#pragma unroll
                for (uint32_t q = 0; q < kB; ++q) s += buf[half][q];
            }
        }
        uint32_t i = nb * kB;
        while (i < n && (i < lead || s == 0.0)) s += a[i++];
        sh.s = s;
        sh.next = i;
    }
    __syncthreads();
    for (uint32_t scan = 0;; ++scan) {
        const double s = sh.s;
        const uint32_t next = sh.next;
        if (next >= n) break;
        if (!__builtin_isfinite(s) || scan >= kMaxScans) {
            __syncthreads();
            if (tid == 0) {
                double r = s;
                for (uint32_t i = next; i < n; ++i) r += a[i];
                sh.s = r;
            }
            __syncthreads();
            break;
        }
        // s > 0 and normal: its binade e and s / u = its significand
        const uint64_t sb = static_cast<uint64_t>(__double_as_longlong(s));
        const int e = static_cast<int>((sb >> 52) & 0x7FFu) - 1023;
        const uint64_t P0 = (sb & ((1ull << 52) - 1)) | (1ull << 52);
        const uint32_t p0 = static_cast<uint32_t>(P0 & 1u);
        // the window [next, end) and this thread's terms [j0, j1) of it
        const uint32_t c0 = (next + next / 2 + NT - 1) / NT, c = c0 < 1 ? 1 : c0 > 16 ? 16 : c0;
        const uint32_t end = n - next < c * NT ? n : next + c * NT;
        const uint32_t j0 = next + tid * c < end ? next + tid * c : end, j1 = end - j0 < c ? end : j0 + c;
        SumMap g = sum_map_identity();
#pragma unroll 4
        for (uint32_t j = j0; j < j1; ++j) {
            uint64_t nj;
            bool big;
            g = sum_map_then(g, sum_term(a[j], e, nj, big));
        }
        SumMap total;
        const SumMap before = wave_scan_maps(g, &total);
        if (lane == 0) sh.wave_total[wave] = total;
        __syncthreads();
        // this thread's starting (s / u, parity): the earlier wavefronts, then
        // the earlier lanes of this one
        uint64_t P = P0;
        uint32_t p = p0;
        for (uint32_t w = 0; w < wave; ++w) {
            const SumMap &t = sh.wave_total[w];
            P += p ? t.inc1 : t.inc0;
            p = (t.out >> p) & 1u;
        }
        P += p ? before.inc1 : before.inc0;
        p = (before.out >> p) & 1u;
        uint32_t mine = n;
        double s_first = 0.0;
#pragma unroll 4
        for (uint32_t j = j0; j < j1; ++j) {
            const double aj = a[j];
            uint64_t nj;
            bool big;
            const SumMap m = sum_term(aj, e, nj, big);
            if (big || P + nj >= kTwo53) {
                mine = j;
                // the reference's add, from the exact prefix (P < 2^53)
                s_first = ldexp(static_cast<double>(P), e - 52) + aj;
                break;
            }
            P += p ? m.inc1 : m.inc0;
            p = (m.out >> p) & 1u;
        }
        const uint32_t first = wave_min_u32(mine);
        if (lane == 0) sh.wave_first[wave] = first;
        __syncthreads();
        uint32_t f = sh.wave_first[0];
        for (uint32_t w = 1; w < NT / 64; ++w) f = min(f, sh.wave_first[w]);
        if (f == n) {
            // no term of the window leaves the binade: the thread holding the
            // window's last term has its sum (P <= 2^53, exact in double)
            if (j1 == end && j0 < j1) {
                sh.s = ldexp(static_cast<double>(P), e - 52);
                sh.next = end;
            }
        } else if (mine == f) {
            sh.s = s_first;
            sh.next = f + 1;
        }
        __syncthreads();
    }
    return sh.s;
}

// RMSNorm (engine.cpp:723-740) of one token held P float4 per thread
// (element 4 (tid + i NT) + j in xv[i], its gain in gv[i]) into hv[4 i + j].
// The reference's sum of squares is a sequential double sum; here it is a
// parallel sum plus a certificate: every normalised value is checked to lie
// farther from a float rounding boundary than the worst-case difference
// between the two sums can move it; only when one is that close does the
// workgroup redo the sum in the reference's order (ordered_sum) from the
// squares (exact in double) written to `scratch` (LDS, at least 2 hidden
// floats, 16-byte aligned). Either way hv is the reference's h bit for bit.
// Every thread of the workgroup calls it; it ends after a barrier.
template <uint32_t NT, uint32_t P>
__device__ __forceinline__ void token_rmsnorm(const RouteArgs &a, const float4 (&xv)[P], const float4 (&gv)[P],
                                              bool has_gain, float (&hv)[4 * P], float *scratch) {
    __shared__ double wave_part[NT / 64];
    __shared__ int unsafe_s;
    __shared__ OrderedSumShared osum;
    const uint32_t H = a.hidden, tid = threadIdx.x, H4 = H / 4;
    double part = 0.0;
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
        if (tid + i * NT < H4) {
            part += static_cast<double>(xv[i].x) * static_cast<double>(xv[i].x);
            part += static_cast<double>(xv[i].y) * static_cast<double>(xv[i].y);
            part += static_cast<double>(xv[i].z) * static_cast<double>(xv[i].z);
            part += static_cast<double>(xv[i].w) * static_cast<double>(xv[i].w);
        }
    }
    part = wave_sum_double(part);
    if ((tid & 63) == 0) wave_part[tid >> 6] = part;
    if (tid == 0) unsafe_s = 0;
    __syncthreads();
    double ss = wave_part[0];
#pragma unroll
    for (uint32_t w = 1; w < NT / 64; ++w) ss += wave_part[w];
    // |parallel sum - sequential sum| <= (H + 32) u ss; scale moves by half of
    // that plus a few roundings
    const double rel_tol = 0.6e-16 * static_cast<double>(H + 32) + 2e-15;
    const uint32_t tol0 = static_cast<uint32_t>(ceil(rel_tol * 4503599627370496.0)); // rel_tol * 2^52
    bool unsafe = false;
    for (int pass = 0; pass < 2; ++pass) {
        const double scale = 1.0 / sqrt(ss / static_cast<double>(H) + a.rms_eps);
#pragma unroll
        for (uint32_t i = 0; i < P; ++i) {
            const float xs[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
            const float gs[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const float gain = has_gain ? static_cast<float>(a.norm_bias + static_cast<double>(gs[j])) : 1.0f;
                const double yd = static_cast<double>(xs[j]) * scale * static_cast<double>(gain);
                hv[4 * i + j] = static_cast<float>(yd);
                if (pass == 0) unsafe |= (tid + i * NT < H4) & rounding_unsafe(yd, tol0);
            }
        }
        if (pass == 1) break;
        if (__any(unsafe) && (tid & 63) == 0) unsafe_s = 1;
        __syncthreads();
        if (!unsafe_s) break;
        // the squares into LDS, then the sum in the reference's order
        double2 *tl = reinterpret_cast<double2 *>(scratch);
#pragma unroll
        for (uint32_t i = 0; i < P; ++i) {
            const uint32_t q = tid + i * NT;
            if (q < H4) {
                tl[2 * q] = make_double2(static_cast<double>(xv[i].x) * static_cast<double>(xv[i].x),
                                         static_cast<double>(xv[i].y) * static_cast<double>(xv[i].y));
                tl[2 * q + 1] = make_double2(static_cast<double>(xv[i].z) * static_cast<double>(xv[i].z),
                                             static_cast<double>(xv[i].w) * static_cast<double>(xv[i].w));
            }
        }
        __syncthreads();
        ss = ordered_sum<NT>(reinterpret_cast<const double *>(scratch), H, osum);
    }
}

// LDS layout of route_rows_kernel: h and the router row each as 16 chains of
// `cs` floats, element k at (k % 16) * cs + k / 16, so that chain lane c reads
// its elements in order with 16-byte loads. cs = 4 (mod 64) puts the 16
// lanes' 16-byte reads on distinct banks.
__host__ __device__ inline uint32_t route_chain_stride(uint32_t hidden) {
    const uint32_t cs = hidden / 16 + 1;
    return cs + (68u - cs % 64u) % 64u;
}

// One F32 router row's logit in the reference's gemv_avx2_row order from h
// and the row staged in LDS in chain layout (chain c at hs / rs + c * cs, see
// route_chain_stride): lane c of a whole 16-lane group runs chain c (FMA over
// the chain's elements in order), then the 8-element tail, the lane tree and
// the sequential tail; every lane of the group returns the value.
// kB float4 of h and of the row per operand batch, the next batch's reads
// issued before this one's FMAs.
template <uint32_t kB>
__device__ inline float chain_layout_logit(const float *hs, const float *rs, uint32_t cs, uint32_t H, uint32_t c) {
    const uint32_t S = H / 16, n16 = S * 16;
    const float4 *h4 = reinterpret_cast<const float4 *>(hs + c * cs);
    const float4 *w4 = reinterpret_cast<const float4 *>(rs + c * cs);
    float acc = 0.0f;
    // the chain is a dependent FMA sequence: its operands come from LDS in
    // batches of 4 kB steps, the next batch requested before this one's FMAs
    const uint32_t nb = S / 4 / kB;
    float4 hb[2][kB], wb[2][kB];
    if (nb > 0) {
#pragma unroll
        for (uint32_t q = 0; q < kB; ++q) {
            hb[0][q] = h4[q];
            wb[0][q] = w4[q];
        }
    }
    for (uint32_t bi = 0; bi < nb; bi += 2) {
#pragma unroll
        for (uint32_t half = 0; half < 2; ++half) {
            const uint32_t b = bi + half;
            if (b >= nb) break;
            const uint32_t nx = (b + 1 < nb ? b + 1 : b) * kB;
#pragma unroll
            for (uint32_t q = 0; q < kB; ++q) {
                hb[half ^ 1][q] = h4[nx + q];
                wb[half ^ 1][q] = w4[nx + q];
            }
#pragma unroll
            for (uint32_t q = 0; q < kB; ++q) {
                acc = fma_rn(wb[half][q].x, hb[half][q].x, acc);
                acc = fma_rn(wb[half][q].y, hb[half][q].y, acc);
                acc = fma_rn(wb[half][q].z, hb[half][q].z, acc);
                acc = fma_rn(wb[half][q].w, hb[half][q].w, acc);
            }
        }
    }
    for (uint32_t i = nb * kB; i < S / 4; ++i) {
        const float4 hq = h4[i], wq = w4[i];
        acc = fma_rn(wq.x, hq.x, acc);
        acc = fma_rn(wq.y, hq.y, acc);
        acc = fma_rn(wq.z, hq.z, acc);
        acc = fma_rn(wq.w, hq.w, acc);
    }
    for (uint32_t s = S / 4 * 4; s < S; ++s) acc = fma_rn(rs[c * cs + s], hs[c * cs + s], acc);
    const bool tail8 = H - n16 >= 8;
    if (tail8 && c < 8) acc = fma_rn(rs[c * cs + S], hs[c * cs + S], acc);
    const float tt = acc + lane_xor<8>(acc);
    float total = hsum8_lanes(tt);
    for (uint32_t k = tail8 ? n16 + 8 : n16; k < H; ++k)
        total = fma_rn(rs[(k - n16) * cs + S], hs[(k - n16) * cs + S], total);
    return total;
}

// Router logit of row blockIdx.y for token blockIdx.x. Every workgroup of the
// token computes the token's RMSNorm (engine.cpp:723-740) from x held in
// registers (4 float4 per thread: hidden <= 16 NT), the first one writes it to
// h_out; then lanes 0-15 run the row's 16 FMA chains of the reference's
// gemv_avx2_row order (8 lanes x 2 accumulators, lane tree, sequential tail)
// and lane 0 adds the logit bias (engine.cpp:1611-1616).
//
// RMSNorm's sum of squares is a sequential double sum in the reference. Here
// it is a parallel sum plus a certificate: every normalised value is checked
// to lie farther from a float rounding boundary than the worst-case
// difference between the two sums can move it; only when one is that close
// does one lane redo the sum in the reference's order. Either way h is the
// reference's h bit for bit.
template <uint32_t NT>
__global__ __launch_bounds__(NT) __attribute__((aligned(kHotAlign))) void route_rows_kernel(RouteArgs a, const float *__restrict__ x,
                                                        float *__restrict__ h_out, float *__restrict__ logits) {
    constexpr uint32_t P = 4;
    extern __shared__ __align__(16) float lds[];
    const uint32_t H = a.hidden, E = a.experts, tid = threadIdx.x;
    const uint32_t t = blockIdx.x, row = blockIdx.y;
    const uint32_t H4 = H / 4, cs = route_chain_stride(H);
    float *hs = lds;
    float *rs = lds + 16 * cs;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + static_cast<uint64_t>(t) * H);
    const float4 *r4 = reinterpret_cast<const float4 *>(a.router + static_cast<uint64_t>(row) * H);
    // unconditional loads (gains from x when there are none, unused): a load
    // under a branch makes the compiler wait for it before the branch
    const bool has_gain = a.norm_weight != nullptr;
    const float4 *g4 = has_gain ? reinterpret_cast<const float4 *>(a.norm_weight) : x4;
    float4 xv[P], gv[P], rv[P];
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
        const uint32_t q = tid + i * NT;
        const uint32_t qc = q < H4 ? q : H4 - 1;
        xv[i] = x4[qc];
        rv[i] = r4[qc];
        gv[i] = g4[qc];
    }
    float hv[4 * P];
    token_rmsnorm<NT, P>(a, xv, gv, has_gain, hv, lds); // hs and rs: see route_lds_bytes
    // h and the router row into the chain layout
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
        const uint32_t q = tid + i * NT;
        if (q < H4) {
            const uint32_t s = q >> 2, c0 = (q & 3) * 4;
            const float rr[4] = {rv[i].x, rv[i].y, rv[i].z, rv[i].w};
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                hs[(c0 + j) * cs + s] = hv[4 * i + j];
                rs[(c0 + j) * cs + s] = rr[j];
            }
            if (row == 0 && h_out)
                reinterpret_cast<float4 *>(h_out + static_cast<uint64_t>(t) * H)[q] =
                    make_float4(hv[4 * i], hv[4 * i + 1], hv[4 * i + 2], hv[4 * i + 3]);
        }
    }
    __syncthreads();
    if (tid < 16) {
        const float total = chain_layout_logit<8>(hs, rs, cs, H, tid);
        if (tid == 0) logits[static_cast<uint64_t>(t) * E + row] = a.router_bias ? total + a.router_bias[row] : total;
    }
}

// RMSNorm of token blockIdx.x into h (batched routing). NT threads, P float4
// per thread (hidden <= 4 P NT; P = 2 up to hidden 2048 keeps the registers
// of the unused half free); LDS: 2 hidden floats (the squares, for the
// in-order sum when the certificate fails).
template <uint32_t NT, uint32_t P = 4>
__global__ __launch_bounds__(NT) void rmsnorm_kernel(RouteArgs a, const float *__restrict__ x,
                                                     float *__restrict__ h, uint32_t *__restrict__ clear) {
    // the call's error word, zeroed by the first kernel of the call (no later
    // kernel of the call runs before this one ends, and this one sets no bit)
    if (clear && blockIdx.x == 0 && threadIdx.x == 0) *clear = 0;
    extern __shared__ __align__(16) float lds[];
    const uint32_t H = a.hidden, H4 = H / 4, tid = threadIdx.x, t = blockIdx.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + static_cast<uint64_t>(t) * H);
    const bool has_gain = a.norm_weight != nullptr;
    const float4 *g4 = has_gain ? reinterpret_cast<const float4 *>(a.norm_weight) : x4; // unconditional loads
    float4 xv[P], gv[P];
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
        const uint32_t q = tid + i * NT;
        const uint32_t qc = q < H4 ? q : H4 - 1;
        xv[i] = x4[qc];
        gv[i] = g4[qc];
    }
    float hv[4 * P];
    token_rmsnorm<NT, P>(a, xv, gv, has_gain, hv, lds);
    float4 *h4 = reinterpret_cast<float4 *>(h + static_cast<uint64_t>(t) * H);
#pragma unroll
    for (uint32_t i = 0; i < P; ++i) {
        const uint32_t q = tid + i * NT;
        if (q < H4) h4[q] = make_float4(hv[4 * i], hv[4 * i + 1], hv[4 * i + 2], hv[4 * i + 3]);
    }
}

// Router logits of a tile of TT = GT PT tokens x TR = (16 / GT) PR router
// rows per workgroup (batched routing): every (token, row) pair runs the 16
// FMA chains of the reference's gemv_avx2_row order (chain c takes elements
// 16 s + c, s = 0, 1, ...), lane c of a 16-lane group owning chain c of a
// PT x PR block of pairs (PT PR independent chains per lane). h and the
// router rows pass through LDS 256 elements (16 steps of every chain) at a
// time, the next tile requested during this one's FMAs and, within a tile,
// the next four steps' operands read from LDS during this four's; then the
// lane tree, the sequential tail and the logit bias, as in f32_row_chains.
// Few experts take small tiles (2 tokens x 8 or 16 rows) so that the grid
// still covers the device; many take 16 x 32 (4 x 8 pairs per lane). grid:
// (ceil(tokens / TT), ceil(experts / TR)).
constexpr uint32_t kRtSteps = 16;              // steps of every chain per LDS tile (16 kRtSteps elements)
constexpr uint32_t kRtF4 = 4 * kRtSteps;       // float4 per token or row per tile
constexpr uint32_t kRtPad = kRtSteps + 4;      // floats per (token or row, chain) in LDS
constexpr uint32_t kRtRow = 16 * kRtPad;       // floats per token or row
template <uint32_t PT, uint32_t PR, uint32_t GT>
__global__ __launch_bounds__(256) void router_tile_kernel(RouteArgs a, const float *__restrict__ h,
                                                          uint32_t tokens, float *__restrict__ logits,
                                                          uint32_t *__restrict__ ids, float *__restrict__ weights,
                                                          uint32_t *__restrict__ status) {
    constexpr uint32_t GR = 16 / GT, TT = GT * PT, TR = GR * PR;
    __shared__ __align__(16) float hl[TT * kRtRow];
    __shared__ __align__(16) float wl[TR * kRtRow];
    __shared__ float lg[TT][TR];
    const uint32_t H = a.hidden, E = a.experts, tid = threadIdx.x;
    const uint32_t c = tid & 15, g = tid >> 4;
    const uint32_t tg = (g % GT) * PT, rg = (g / GT) * PR;
    const uint32_t t0 = blockIdx.x * TT, r0 = blockIdx.y * TR;
    const uint32_t S = H / 16, n16 = S * 16, ntiles = (S + kRtSteps - 1) / kRtSteps;
    // staging: the tile's TT + TR rows of kRtF4 float4 each, item q = tid +
    // 256 i -> row q / kRtF4, float4 q % kRtF4 of the row's 16 kRtSteps elements
    constexpr uint32_t kItems = (TT + TR) * kRtF4, kPer = (kItems + 255) / 256;
    const float *src[kPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t q = tid + 256 * i, row = q / kRtF4 < TT + TR ? q / kRtF4 : 0;
        src[i] = row < TT ? h + static_cast<uint64_t>(t0 + row < tokens ? t0 + row : tokens - 1) * H
                          : a.router + static_cast<uint64_t>(r0 + row - TT < E ? r0 + row - TT : E - 1) * H;
    }
    float4 sv[kPer];
    auto load_tile = [&](uint32_t k) {
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t q = tid + 256 * i;
            if (kItems % 256 != 0 && q >= kItems) break;
            const uint32_t e = 16 * kRtSteps * k + 4 * (q % kRtF4);
            const uint32_t ec = e + 4 <= n16 ? e : 0; // past the chains' elements: unused
            sv[i] = *reinterpret_cast<const float4 *>(src[i] + ec);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t q = tid + 256 * i;
            if (kItems % 256 != 0 && q >= kItems) break;
            const uint32_t row = q / kRtF4, f = q % kRtF4, s0 = f >> 2, c0 = 4 * (f & 3);
            float *dst = (row < TT ? hl + row * kRtRow : wl + (row - TT) * kRtRow) + c0 * kRtPad + s0;
            dst[0] = sv[i].x;
            dst[kRtPad] = sv[i].y;
            dst[2 * kRtPad] = sv[i].z;
            dst[3 * kRtPad] = sv[i].w;
        }
    };
    float acc[PT][PR];
#pragma unroll
    for (uint32_t i = 0; i < PT; ++i)
#pragma unroll
        for (uint32_t j = 0; j < PR; ++j) acc[i][j] = 0.0f;
    if (ntiles > 0) load_tile(0);
    for (uint32_t k = 0; k < ntiles; ++k) {
        store_tile();
        __syncthreads();
        if (k + 1 < ntiles) load_tile(k + 1);
        const uint32_t steps = S - kRtSteps * k < kRtSteps ? S - kRtSteps * k : kRtSteps;
        // operands of steps s4 .. s4 + 3 from LDS, and their FMAs (ns of them)
        auto read_ops = [&](float4 (&hq)[PT], float4 (&wq)[PR], uint32_t s4) {
#pragma unroll
            for (uint32_t i = 0; i < PT; ++i) hq[i] = *reinterpret_cast<const float4 *>(&hl[(tg + i) * kRtRow + c * kRtPad + s4]);
#pragma unroll
            for (uint32_t j = 0; j < PR; ++j) wq[j] = *reinterpret_cast<const float4 *>(&wl[(rg + j) * kRtRow + c * kRtPad + s4]);
        };
        auto fmas = [&](const float4 (&hq)[PT], const float4 (&wq)[PR], uint32_t ns) {
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) {
                if (u >= ns) break;
#pragma unroll
                for (uint32_t i = 0; i < PT; ++i) {
                    const float hu = u == 0 ? hq[i].x : u == 1 ? hq[i].y : u == 2 ? hq[i].z : hq[i].w;
#pragma unroll
                    for (uint32_t j = 0; j < PR; ++j) {
                        const float wu = u == 0 ? wq[j].x : u == 1 ? wq[j].y : u == 2 ? wq[j].z : wq[j].w;
                        acc[i][j] = fma_rn(wu, hu, acc[i][j]);
                    }
                }
            }
        };
        if (steps == kRtSteps) {
            // a whole tile: the next four steps' operands requested before
            // this four's FMAs
            float4 hq[2][PT], wq[2][PR];
            read_ops(hq[0], wq[0], 0);
#pragma unroll
            for (uint32_t s4 = 0; s4 < kRtSteps; s4 += 4) {
                const uint32_t b = (s4 / 4) & 1;
                if (s4 + 4 < kRtSteps) read_ops(hq[b ^ 1], wq[b ^ 1], s4 + 4);
                fmas(hq[b], wq[b], 4);
            }
        } else {
            for (uint32_t s4 = 0; s4 < steps; s4 += 4) {
                float4 hq[PT], wq[PR];
                read_ops(hq, wq, s4);
                fmas(hq, wq, steps - s4 < 4 ? steps - s4 : 4);
            }
        }
        __syncthreads();
    }
    const bool tail8 = H - n16 >= 8;
#pragma unroll
    for (uint32_t i = 0; i < PT; ++i) {
        const uint32_t t = t0 + tg + i;
        const float *hr = h + static_cast<uint64_t>(t < tokens ? t : tokens - 1) * H;
#pragma unroll
        for (uint32_t j = 0; j < PR; ++j) {
            const uint32_t r = r0 + rg + j;
            const float *wr = a.router + static_cast<uint64_t>(r < E ? r : E - 1) * H;
            float v = acc[i][j];
            if (tail8 && c < 8) v = fma_rn(wr[n16 + c], hr[n16 + c], v);
            const float tt = v + lane_xor<8>(v);
            float total = hsum8_lanes(tt);
            for (uint32_t kk = tail8 ? n16 + 8 : n16; kk < H; ++kk) total = fma_rn(wr[kk], hr[kk], total);
            const float logit = a.router_bias ? total + a.router_bias[r < E ? r : E - 1] : total;
            if (c == 0 && t < tokens && r < E) logits[static_cast<uint64_t>(t) * E + r] = logit;
            if (c == 0) lg[tg + i][rg + j] = logit;
        }
    }
    // with ids (the host passes them when one row tile holds every expert):
    // each token's routing from its logits in LDS, one wavefront per token,
    // as route_finish_kernel does it
    if (!ids) return;
    __syncthreads();
    for (uint32_t w = tid >> 6; w < TT; w += 4) {
        const uint32_t t = t0 + w;
        if (t >= tokens) break;
        bool bad;
        const Routing rt = wave_route(a, lg[w], &bad);
        const uint32_t lane = tid & 63;
        if (lane < a.top_k) {
            ids[static_cast<uint64_t>(t) * a.top_k + lane] = rt.id;
            weights[static_cast<uint64_t>(t) * a.top_k + lane] = rt.weight;
        }
        if (bad && lane == 0) atomicOr(status, STATUS_NONFINITE_SCORE);
    }
}

// ids / weights of token blockIdx.x from its logits; one wavefront.
__global__ __launch_bounds__(64) void route_finish_kernel(RouteArgs a, const float *__restrict__ logits,
                                                          uint32_t *__restrict__ ids,
                                                          float *__restrict__ weights,
                                                          uint32_t *__restrict__ status) {
    const uint32_t t = blockIdx.x, lane = threadIdx.x;
    bool bad;
    const Routing r = wave_route<4, true>(a, logits + static_cast<uint64_t>(t) * a.experts, &bad);
    if (lane < a.top_k) {
        ids[static_cast<uint64_t>(t) * a.top_k + lane] = r.id;
        weights[static_cast<uint64_t>(t) * a.top_k + lane] = r.weight;
    }
    if (bad && lane == 0) atomicOr(status, STATUS_NONFINITE_SCORE);
}

// Router logits of a block-type router (the reference's quantised branch,
// engine.cpp:358-366 -> gemv_quant, kernels.cpp:846-878): every row runs the
// lane chains of the experts' rows, so a logit is the reference's bit for
// bit; then the logit bias (engine.cpp:1611-1616). 32 router rows per
// workgroup, token blockIdx.x's h staged in LDS tiles of a.rtile blocks.
// grid: (tokens, ceil(experts / 32)).
template <class T>
__global__ __launch_bounds__(kThreads) void router_quant_kernel(RouteArgs a, const float *__restrict__ h,
                                                                float *__restrict__ logits) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t tid = threadIdx.x, l = tid & 7, slot = tid >> 3;
    const uint32_t t = blockIdx.x, r = blockIdx.y * (kThreads / 8) + slot, E = a.experts;
    const PackedGeometry &g = a.rg;
    typename T::Row rw[1] = {T::row(static_cast<const uint8_t *>(a.router_packed), g.scale_bytes, g.blocks_padded,
                                    g.chunks, r < E ? r : E - 1, l)};
    float acc[1] = {0.0f};
    const float *x = h + static_cast<uint64_t>(t) * a.hidden;
    for (uint32_t tb = 0; tb < g.blocks; tb += a.rtile) {
        const uint32_t nb = g.blocks - tb < a.rtile ? g.blocks - tb : a.rtile;
        __syncthreads();
        T::stage(x, tb, nb, lds, tid, kThreads);
        __syncthreads();
        run_chunks_pf<T, 1, 2>(rw, tb / T::kPerChunk, (tb + nb + T::kPerChunk - 1) / T::kPerChunk, g.blocks, tb, nb,
                               lds, l, acc);
    }
    const float v = T::finish(acc[0]);
    if (l == 0 && r < E) logits[static_cast<uint64_t>(t) * E + r] = a.router_bias ? v + a.router_bias[r] : v;
}

// Router logits of a Q6_K router (raw 210-byte blocks, as FreeMoe stores
// them): one 16-lane group per router row runs the Q6_K row dot of fmx_matvec
// (the reference's gemv_quant order, bit for bit), then the logit bias
// (engine.cpp:1611-1616). grid: (tokens, ceil(experts / 16)).
__global__ __launch_bounds__(kThreads) void router_q6k_kernel(RouteArgs a, const float *__restrict__ h,
                                                              float *__restrict__ logits) {
    const uint32_t tid = threadIdx.x, c = tid & 15;
    const uint32_t t = blockIdx.x, r = blockIdx.y * (kThreads / 16) + (tid >> 4), E = a.experts;
    const float v = RowDot16<FMX_TYPE_Q6_K>::dot(a.router_packed, r < E ? r : E - 1,
                                                 h + static_cast<uint64_t>(t) * a.hidden, a.hidden, c);
    if (c == 0 && r < E) logits[static_cast<uint64_t>(t) * E + r] = a.router_bias ? v + a.router_bias[r] : v;
}

// The expert of rank `rank` for an expert kernel: from the routing computed
// in this wavefront when `logits` is given (the first workgroup also stores
// ids, weights and the error flag for the kernels after it), else from ids.
// The expert of rank `rank` from logits already loaded (route_logits_load);
// the first block also stores the token's routing (ids_out / w_out) and flags
// a non-finite logit.
__device__ inline uint32_t expert_of_rank_values(const RouteArgs &ra, const float (&lv)[4], uint32_t rank,
                                                 bool first_block, uint32_t *__restrict__ ids_out,
                                                 float *__restrict__ w_out, uint32_t *__restrict__ status) {
    bool bad;
    const Routing r = wave_route_values(ra, lv, &bad);
    const uint32_t lane = threadIdx.x & 63;
    if (first_block && threadIdx.x < 64) {
        if (lane < ra.top_k) {
            ids_out[lane] = r.id;
            w_out[lane] = r.weight;
        }
        if (bad && lane == 0) atomicOr(status, STATUS_NONFINITE_SCORE);
    }
    return __builtin_amdgcn_readlane(static_cast<int>(r.id), rank);
}

__device__ inline uint32_t expert_of_rank(const RouteArgs &ra, const float *__restrict__ logits,
                                          const uint32_t *__restrict__ ids, uint32_t rank, bool first_block,
                                          uint32_t *__restrict__ ids_out, float *__restrict__ w_out,
                                          uint32_t *__restrict__ status) {
    if (!logits) return ids[rank];
    bool bad;
    const Routing r = wave_route(ra, logits, &bad);
    const uint32_t lane = threadIdx.x & 63;
    if (first_block && threadIdx.x < 64) {
        if (lane < ra.top_k) {
            ids_out[lane] = r.id;
            w_out[lane] = r.weight;
        }
        if (bad && lane == 0) atomicOr(status, STATUS_NONFINITE_SCORE);
    }
    return __builtin_amdgcn_readlane(static_cast<int>(r.id), rank);
}

// ------------------------------------------------------------ experts --

__device__ inline float swiglu(float gate, float up) {
    const double g = static_cast<double>(gate);
    return static_cast<float>(g / (1.0 + exp(-g))) * up;
}

// Gate and up rows j of the expert at rank blockIdx.y, RJ rows per thread:
// the first PF chunks of every row are requested before h is staged.
// Four wavefronts per SIMD (at most 128 VGPRs): the whole grid of a Mixtral
// expert pair is then resident at once. A wavefront's eight 8-lane groups
// take seven rows (the eighth group repeats the seventh's row, whose loads
// the wavefront's coalescing merges, and stores nothing): the 28672 rows of a
// Mixtral pair are then 4096 wavefronts, four on every SIMD, where eight rows
// per wavefront left half the SIMDs four and half three.
template <class T, int RJ, int PF>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4 / RJ), aligned(kHotAlign))) void gate_up_kernel(
    ExpertArgs a, const float *__restrict__ h, const float *__restrict__ logits, uint32_t *__restrict__ ids,
    float *__restrict__ w, float *__restrict__ act, uint32_t *__restrict__ status) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t tid = threadIdx.x, l = tid & 7, g8 = (tid >> 3) & 7;
    const uint32_t slot = (tid >> 6) * 7 + (g8 < 7 ? g8 : 6);
    const uint32_t rank = blockIdx.y;
    const uint32_t blocks = a.gu.blocks;
    // the logits are requested first, then h's first tile, so that the
    // routing waits only for the logits (loads complete in issue order) and
    // h arrives while it runs; without logits (routing given) ids[rank]
    float lv[4];
    route_logits_load(a.route, logits ? logits : h, lv);
    const uint32_t given = logits ? 0u : ids[rank];
    __builtin_amdgcn_sched_barrier(0);
    XBatch<4> hb;
    load_batch<T>(hb, h, 0, (blocks < a.gu_tile ? blocks : a.gu_tile) * T::kBlock, tid, kThreads);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t e = logits ? expert_of_rank_values(a.route, lv, rank, blockIdx.x == 0 && rank == 0, ids, w, status)
                              : given;
    if (e >= a.experts) {
        if (tid == 0 && blockIdx.x == 0) atomicOr(status, STATUS_BAD_EXPERT);
        return;
    }
    const uint8_t *gate = static_cast<const uint8_t *>(a.gate[e]);
    const uint8_t *up = static_cast<const uint8_t *>(a.up[e]);
    const uint32_t F = a.ffn;
    const uint32_t j0 = (blockIdx.x * (kThreads / 64 * 7) + slot) * RJ;
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
    const uint32_t c_end = (blocks + T::kPerChunk - 1) / T::kPerChunk;
    ChunkStream<T, 2 * RJ, PF> cs;
    cs.prime(rw, c_end);
    for (uint32_t tb = 0; tb < blocks; tb += a.gu_tile) {
        const uint32_t nb = blocks - tb < a.gu_tile ? blocks - tb : a.gu_tile;
        __syncthreads();
        if (tb == 0) T::template stage<4, true>(h, tb, nb, lds, tid, kThreads, hb);
        else T::stage(h, tb, nb, lds, tid, kThreads);
        __syncthreads();
        cs.run(tb / T::kPerChunk, (tb + nb + T::kPerChunk - 1) / T::kPerChunk, c_end, blocks, tb, nb, lds, l, t);
    }
#pragma unroll
    for (int m = 0; m < RJ; ++m) {
        const float g = T::finish(t[2 * m]);
        const float u = T::finish(t[2 * m + 1]);
        if (l == 0 && g8 < 7 && j0 + m < F) act[static_cast<uint64_t>(rank) * F + j0 + m] = swiglu(g, u);
    }
}

// Down rows of every routed expert of one token, then the combine in rank
// order (ffn = 0 + w_0 d_0 + w_1 d_1 ..., engine.cpp:1517, 1770) and the
// residual (engine.cpp:813-816, 1822). Row slot s handles rank s / jpw, row
// s % jpw of this workgroup's jpw rows (jpw = 32 / top_k); every rank's
// activations are staged together, so one workgroup finishes its rows alone.
// The activations fill the LDS, so one workgroup (one wavefront per SIMD)
// runs per CU: the wavefront may use every register, which holds a deep
// prefetch ring.
template <class T, int PF>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1), aligned(kHotAlign))) void down_kernel(ExpertArgs a, const float *__restrict__ x,
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
    ChunkStream<T, 1, PF, down_rings<T>(), T::kType == FMX_TYPE_Q4_0> cs;
    for (uint32_t tb = 0; tb < blocks; tb += a.dn_tile) {
        const uint32_t nb = blocks - tb < a.dn_tile ? blocks - tb : a.dn_tile;
        __syncthreads();
        const uint32_t tile_elems = nb * T::kBlock;
        if (K == 2 && tile_elems <= 16 * 4 * kThreads) {
            // both ranks' activations requested together: one memory latency;
            // the first weight chunks after them, so that staging (which
            // waits for its loads in the order they were issued) does not
            // wait for the weights as well
            XBatch<16> b0, b1;
            load_batch<T>(b0, act, tb * T::kBlock, tile_elems, tid, kThreads);
            load_batch<T>(b1, act + a.ffn, tb * T::kBlock, tile_elems, tid, kThreads);
            if (tb == 0) cs.prime(rw, c_end);
            T::template stage<16, true>(act, tb, nb, lds, tid, kThreads, b0);
            T::template stage<16, true>(act + a.ffn, tb, nb, lds + tile_floats, tid, kThreads, b1);
        } else {
            if (tb == 0) cs.prime(rw, c_end);
            for (uint32_t r = 0; r < K; ++r)
                T::template stage<16>(act + static_cast<uint64_t>(r) * a.ffn, tb, nb, lds + r * tile_floats, tid,
                                      kThreads);
        }
        __syncthreads();
        const uint32_t c0 = tb / T::kPerChunk, c1 = (tb + nb + T::kPerChunk - 1) / T::kPerChunk;
        cs.run(c0, c1, c_end, blocks, tb, nb, lds + rank * tile_floats, l, t);
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

// F32 and Q6_K experts: 16 lanes per row (RowDot16: F32 in gemv_avx2_row's
// order, Q6_K in row_dot_fused_scalar's), h staged in LDS first (every row
// of the workgroup reads all of it; the groups of a wavefront read the same
// elements at once). LDS: hidden floats.
template <uint32_t kT>
__global__ __launch_bounds__(kThreads) void gate_up_rows16_kernel(ExpertArgs a, const float *__restrict__ h,
                                                                  const float *__restrict__ logits,
                                                                  uint32_t *__restrict__ ids, float *__restrict__ w,
                                                                  float *__restrict__ act,
                                                                  uint32_t *__restrict__ status) {
    extern __shared__ __align__(16) float hl16[];
    const uint32_t tid = threadIdx.x, c = tid & 15;
    const uint32_t rank = blockIdx.y;
    const uint32_t e = expert_of_rank(a.route, logits, ids, rank, blockIdx.x == 0 && rank == 0, ids, w, status);
    if (e >= a.experts) {
        if (tid == 0 && blockIdx.x == 0) atomicOr(status, STATUS_BAD_EXPERT);
        return;
    }
    const uint32_t F = a.ffn, H = a.hidden;
    const float4 *h4 = reinterpret_cast<const float4 *>(h);
    for (uint32_t q = tid; q < H / 4; q += kThreads) reinterpret_cast<float4 *>(hl16)[q] = h4[q];
    __syncthreads();
    const uint32_t j = blockIdx.x * (kThreads / 16) + (tid >> 4);
    const uint32_t jr = j < F ? j : F - 1;
    const float g = RowDot16<kT>::dot(a.gate[e], jr, hl16, H, c);
    const float u = RowDot16<kT>::dot(a.up[e], jr, hl16, H, c);
    if (c == 0 && j < F) act[static_cast<uint64_t>(rank) * F + j] = swiglu(g, u);
}

// F32 and Q6_K down rows on 16 lanes each (RowDot16), then the combine in
// rank order and the residual, as down_kernel; 16 slots, 16 / top_k rows of
// every rank per workgroup.
template <uint32_t kT>
__global__ __launch_bounds__(kThreads) void down_rows16_kernel(ExpertArgs a, const float *__restrict__ x,
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
    const float v = RowDot16<kT>::dot(a.down[e], jr, act + static_cast<uint64_t>(rank) * F, F, c);
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

// Q6_K down rows with G 16-lane groups per row: group g takes blocks g,
// g + G, ... (each block's dot is independent), the block dots meet in LDS
// and one lane per row adds them in block order from 0 (as q6_k_row_chains
// does), then the combine in rank order and the residual. 16 / G slots,
// 16 / G / top_k rows of every rank per workgroup. LDS: 16 / G slots x
// blocks floats.
template <uint32_t G>
__global__ __launch_bounds__(kThreads) void down_q6_k_split_kernel(ExpertArgs a, const float *__restrict__ x,
                                                                   const float *__restrict__ act,
                                                                   const uint32_t *__restrict__ ids,
                                                                   const float *__restrict__ w,
                                                                   float *__restrict__ out,
                                                                   uint32_t *__restrict__ status) {
    extern __shared__ float dots[];
    constexpr uint32_t kSlots = kThreads / 16 / G;
    __shared__ float dres[kSlots];
    const uint32_t tid = threadIdx.x, c = tid & 15, grp = tid >> 4;
    const uint32_t slot = grp / G, part = grp % G;
    const uint32_t K = a.top_k, H = a.hidden, F = a.ffn, blocks = F / 256;
    const uint32_t jpw = kSlots / K;
    const uint32_t rank = slot / jpw < K ? slot / jpw : K - 1;
    const uint32_t j = blockIdx.x * jpw + slot % jpw;
    const uint32_t jr = j < H ? j : H - 1;
    uint32_t e = ids[rank];
    const bool bad = e >= a.experts;
    if (bad) {
        if (c == 0 && part == 0) atomicOr(status, STATUS_BAD_EXPERT);
        e = 0;
    }
    q6_k_block_dots(static_cast<const uint8_t *>(a.down[e]) + static_cast<uint64_t>(jr) * blocks * 210,
                    act + static_cast<uint64_t>(rank) * F, blocks, part, G, c, dots + slot * blocks);
    __syncthreads();
    if (tid < K * jpw) {
        // slot tid: rank tid / jpw
        const float *d = dots + tid * blocks;
        float v = 0.0f;
        for (uint32_t b = 0; b < blocks; ++b) v = v + d[b];
        dres[tid] = ids[tid / jpw] >= a.experts ? 0.0f : v;
    }
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
constexpr int kDownPF = 7;
constexpr int kRJ = 1;

// Dynamic LDS of the chain kernels (gate/up: one tile of h; down: one tile
// of every rank's activations); 0 for the 16-lane kernels.
size_t gate_up_lds(const ExpertArgs &a) {
    switch (a.type_gu) {
    case FMX_TYPE_Q4_0: return static_cast<size_t>(a.gu_tile) * Q40::kLdsFloatsPerBlock * sizeof(float);
    case FMX_TYPE_Q8_0: return static_cast<size_t>(a.gu_tile) * Q80::kLdsFloatsPerBlock * sizeof(float);
    case FMX_TYPE_Q4_K: return static_cast<size_t>(a.gu_tile) * Q4K::kLdsFloatsPerBlock * sizeof(float);
    }
    return 0;
}
size_t down_lds(const ExpertArgs &a) {
    switch (a.type_dn) {
    case FMX_TYPE_Q4_0: return static_cast<size_t>(a.dn_tile) * Q40::kLdsFloatsPerBlock * sizeof(float) * a.top_k;
    case FMX_TYPE_Q8_0: return static_cast<size_t>(a.dn_tile) * Q80::kLdsFloatsPerBlock * sizeof(float) * a.top_k;
    case FMX_TYPE_Q4_K: return static_cast<size_t>(a.dn_tile) * Q4K::kLdsFloatsPerBlock * sizeof(float) * a.top_k;
    }
    return 0;
}

// Launches `k` on (grid, kThreads, lds), recording kev[0] / kev[1] at its
// start and end when kev is given.
template <class K, class... Args>
int launch_timed(K k, dim3 grid, size_t lds, hipStream_t s, const hipEvent_t *kev, Args... args) {
    if (kev)
        hipExtLaunchKernelGGL(k, grid, dim3(kThreads), lds, s, kev[0], kev[1], 0, args...);
    else
        hipLaunchKernelGGL(k, grid, dim3(kThreads), lds, s, args...);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

// Gate/up rows of every routed expert in block type TG (the lane chains).
template <class TG>
int launch_gate_up_q(const ExpertArgs &a, const float *h, const float *logits, uint32_t *ids, float *w, float *act,
                     uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    auto gu = gate_up_kernel<TG, kRJ, kGateUpPF>;
    const size_t lds = gate_up_lds(a);
    if (int rc = allow_lds(reinterpret_cast<const void *>(gu), lds)) return rc;
    return launch_timed(gu, dim3(div_up(a.ffn, (kThreads / 64 * 7) * kRJ), a.top_k), lds, s, kev, a, h, logits, ids, w,
                        act, status);
}

// Down rows of every routed expert in block type TD, combine and residual.
template <class TD>
int launch_down_q(const ExpertArgs &a, const float *x, const float *act, const uint32_t *ids, const float *w,
                  float *out, uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    auto dn = down_kernel<TD, kDownPF>;
    const size_t lds = down_lds(a);
    if (int rc = allow_lds(reinterpret_cast<const void *>(dn), lds)) return rc;
    const uint32_t jpw = (kThreads / 8) / a.top_k;
    return launch_timed(dn, dim3(div_up(a.hidden, jpw)), lds, s, kev, a, x, act, ids, w, out, status);
}

int launch_gate_up(const ExpertArgs &a, const float *h, const float *logits, uint32_t *ids, float *w, float *act,
                   uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    const dim3 grid16(div_up(a.ffn, kThreads / 16), a.top_k);
    switch (a.type_gu) {
    case FMX_TYPE_F32:
        return launch_timed(gate_up_rows16_kernel<FMX_TYPE_F32>, grid16, a.hidden * sizeof(float), s, kev, a, h, logits,
                            ids, w, act, status);
    case FMX_TYPE_Q6_K:
        return launch_timed(gate_up_rows16_kernel<FMX_TYPE_Q6_K>, grid16, a.hidden * sizeof(float), s, kev, a, h, logits,
                            ids, w, act, status);
    case FMX_TYPE_Q4_0: return launch_gate_up_q<Q40>(a, h, logits, ids, w, act, status, s, kev);
    case FMX_TYPE_Q8_0: return launch_gate_up_q<Q80>(a, h, logits, ids, w, act, status, s, kev);
    case FMX_TYPE_Q4_K: return launch_gate_up_q<Q4K>(a, h, logits, ids, w, act, status, s, kev);
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

// down_q6_k_split_kernel<G>: 16 / G row slots over the ranks per workgroup.
template <uint32_t G>
int launch_down_q6_k_split(const ExpertArgs &a, const float *x, const float *act, const uint32_t *ids,
                           const float *w, float *out, uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    constexpr uint32_t kSlots = kThreads / 16 / G;
    const size_t lds = static_cast<size_t>(kSlots) * (a.ffn / 256) * sizeof(float);
    if (int rc = allow_lds(reinterpret_cast<const void *>(down_q6_k_split_kernel<G>), lds)) return rc;
    return launch_timed(down_q6_k_split_kernel<G>, dim3(div_up(a.hidden, kSlots / a.top_k)), lds, s, kev, a, x, act,
                        ids, w, out, status);
}

int launch_down(const ExpertArgs &a, const float *x, const float *act, const uint32_t *ids, const float *w,
                float *out, uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    // the 16-lane kernel's rows per workgroup: its 16 slots over the ranks
    // (launch_experts admits it only for top_k <= 16)
    auto grid16 = [&a]() { return dim3(div_up(a.hidden, (kThreads / 16) / a.top_k)); };
    switch (a.type_dn) {
    case FMX_TYPE_F32:
        return launch_timed(down_rows16_kernel<FMX_TYPE_F32>, grid16(), 0, s, kev, a, x, act, ids, w, out, status);
    case FMX_TYPE_Q6_K:
        // Q6_K rows of many blocks split over four (or two) lane groups
        // each, while every rank keeps a row slot
        if (a.top_k <= kThreads / 64 && a.ffn / 256 >= 8)
            return launch_down_q6_k_split<4>(a, x, act, ids, w, out, status, s, kev);
        if (a.top_k <= kThreads / 32 && a.ffn / 256 >= 8)
            return launch_down_q6_k_split<2>(a, x, act, ids, w, out, status, s, kev);
        return launch_timed(down_rows16_kernel<FMX_TYPE_Q6_K>, grid16(), 0, s, kev, a, x, act, ids, w, out,
                            status);
    case FMX_TYPE_Q4_0:
        if (pair_down_fits<PairQ40>(a)) return launch_down_pair<PairQ40>(a, x, act, ids, w, out, status, s, kev);
        return launch_down_q<Q40>(a, x, act, ids, w, out, status, s, kev);
    case FMX_TYPE_Q8_0: return launch_down_q<Q80>(a, x, act, ids, w, out, status, s, kev);
    case FMX_TYPE_Q4_K:
        if (pair_down_fits<PairQ4K>(a)) return launch_down_pair_q4k(a, x, act, ids, w, out, status, s, kev);
        return launch_down_q<Q4K>(a, x, act, ids, w, out, status, s, kev);
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

} // namespace

// Raises the dynamic LDS limit of kernel `fn` (64 KiB by default) to `bytes`
// when a launch needs more; the limit only grows, and each kernel's is kept.
// The table is a fixed array (no allocation on a compute call); a kernel past
// its capacity has its attribute set on every such launch instead.
int allow_lds(const void *fn, size_t bytes) {
    if (bytes <= 64 * 1024) return FMX_OK;
    constexpr int kKernels = 256;
    static std::mutex mu;
    static const void *fns[kKernels];
    static size_t limits[kKernels];
    static int used = 0;
    std::lock_guard<std::mutex> lock(mu);
    int i = 0;
    while (i < used && fns[i] != fn) ++i;
    if (i < used && limits[i] >= bytes) return FMX_OK;
    FMX_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
    if (i == used && used < kKernels) ++used;
    if (i < used) {
        fns[i] = fn;
        limits[i] = bytes;
    }
    return FMX_OK;
}

// route_rows_kernel's LDS: h and the router row in chain layout (32 cs >= 2
// hidden floats, which first hold the squares of an in-order sum of squares).
size_t route_lds_bytes(uint32_t hidden) { return 2ull * 16 * route_chain_stride(hidden) * sizeof(float); }

// RMSNorm of `tokens` rows of x into h: one workgroup per token.
int launch_rmsnorm(const RouteArgs &a, const float *x, uint32_t tokens, float *h, hipStream_t s,
                   uint32_t *clear = nullptr) {
    const size_t lds = 2ull * a.hidden * sizeof(float);
    if (a.hidden <= 8 * 256) {
        auto k = rmsnorm_kernel<256, 2>;
        if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
        hipLaunchKernelGGL(k, dim3(tokens), dim3(256), lds, s, a, x, h, clear);
    } else if (a.hidden <= 16 * 256) {
        auto k = rmsnorm_kernel<256>;
        if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
        hipLaunchKernelGGL(k, dim3(tokens), dim3(256), lds, s, a, x, h, clear);
    } else {
        auto k = rmsnorm_kernel<1024>;
        if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
        hipLaunchKernelGGL(k, dim3(tokens), dim3(1024), lds, s, a, x, h, clear);
    }
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

template <class T>
int launch_router_quant_t(const RouteArgs &a, const float *h, uint32_t tokens, float *logits, hipStream_t s) {
    const size_t lds = static_cast<size_t>(a.rtile) * T::kLdsFloatsPerBlock * sizeof(float);
    auto k = router_quant_kernel<T>;
    if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
    hipLaunchKernelGGL(k, dim3(tokens, div_up(a.experts, kThreads / 8)), dim3(kThreads), lds, s, a, h, logits);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

// Logits of a block-type router from h ([tokens x hidden]).
int launch_router_quant(const RouteArgs &a, const float *h, uint32_t tokens, float *logits, hipStream_t s) {
    switch (a.router_type) {
    case FMX_TYPE_Q4_0: return launch_router_quant_t<Q40>(a, h, tokens, logits, s);
    case FMX_TYPE_Q8_0: return launch_router_quant_t<Q80>(a, h, tokens, logits, s);
    case FMX_TYPE_Q4_K: return launch_router_quant_t<Q4K>(a, h, tokens, logits, s);
    case FMX_TYPE_Q6_K:
        hipLaunchKernelGGL(router_q6k_kernel, dim3(tokens, div_up(a.experts, kThreads / 16)), dim3(kThreads), 0, s, a,
                           h, logits);
        FMX_LAUNCH_CHECK();
        return FMX_OK;
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

// One workgroup per (token, router row): 256 threads up to hidden 4096, 1024
// beyond (each thread holds 16 elements of the token). A block-type router
// takes RMSNorm into h (which it then needs) and the router rows after it.
int launch_route_logits(const RouteArgs &a, const float *x, uint32_t tokens, float *h, float *logits,
                        hipStream_t s) {
    if (a.hidden > kMaxHidden || a.hidden % 4 || a.experts == 0) return FMX_ERR_SHAPE_MISMATCH;
    if (a.router_type != FMX_TYPE_F32) {
        if (!h) return FMX_ERR_INVALID_ARGUMENT;
        if (int rc = launch_rmsnorm(a, x, tokens, h, s)) return rc;
        return launch_router_quant(a, h, tokens, logits, s);
    }
    const size_t lds = route_lds_bytes(a.hidden);
    if (lds > kMaxLds) return FMX_ERR_SHAPE_MISMATCH;
    const dim3 grid(tokens, a.experts);
    if (a.hidden <= 16 * 256) {
        auto k = route_rows_kernel<256>;
        if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
        hipLaunchKernelGGL(k, grid, dim3(256), lds, s, a, x, h, logits);
    } else {
        auto k = route_rows_kernel<1024>;
        if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
        hipLaunchKernelGGL(k, grid, dim3(1024), lds, s, a, x, h, logits);
    }
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

// Batched routing: RMSNorm once per token into h, then the router logits in
// token x row tiles shaped by the expert count (a workgroup per router row and
// token would redo each token's RMSNorm once per expert).
// With ids (and weights, status), an F32 router of at most 32 experts (one
// row tile) also routes each token in the same launch; *routed tells whether
// it did.
int launch_route_batched(const RouteArgs &a, const float *x, uint32_t tokens, float *h, float *logits,
                         hipStream_t s, uint32_t *ids = nullptr, float *weights = nullptr,
                         uint32_t *status = nullptr, bool *routed = nullptr, uint32_t *clear = nullptr) {
    if (routed) *routed = false;
    if (a.hidden > kMaxHidden || a.hidden % 4 || a.experts == 0) return FMX_ERR_SHAPE_MISMATCH;
    if (int rc = launch_rmsnorm(a, x, tokens, h, s, clear)) return rc;
    if (a.router_type != FMX_TYPE_F32) return launch_router_quant(a, h, tokens, logits, s);
    const bool fuse = ids && weights && status && routed && a.experts <= 32;
    uint32_t *fi = fuse ? ids : nullptr;
    if (a.experts <= 8)
        hipLaunchKernelGGL((router_tile_kernel<1, 1, 2>), dim3(div_up(tokens, 2), div_up(a.experts, 8)), dim3(256), 0,
                           s, a, h, tokens, logits, fi, weights, status);
    else if (a.experts <= 16)
        hipLaunchKernelGGL((router_tile_kernel<1, 2, 2>), dim3(div_up(tokens, 2), div_up(a.experts, 16)), dim3(256), 0,
                           s, a, h, tokens, logits, fi, weights, status);
    else
        hipLaunchKernelGGL((router_tile_kernel<4, 8, 4>), dim3(div_up(tokens, 16), div_up(a.experts, 32)), dim3(256),
                           0, s, a, h, tokens, logits, fi, weights, status);
    FMX_LAUNCH_CHECK();
    if (fuse) *routed = true;
    return FMX_OK;
}

__global__ void route_clear_kernel(uint32_t *word) { *word = 0; }

int launch_route(const RouteArgs &a, const float *x, uint32_t tokens, float *h, float *logits,
                 uint32_t *ids, float *weights, uint32_t *status, hipStream_t s, bool clear_status) {
    bool routed = false;
    const bool batched = h && tokens > 1;
    if (clear_status && !batched) {
        hipLaunchKernelGGL(route_clear_kernel, dim3(1), dim3(1), 0, s, status);
        FMX_LAUNCH_CHECK();
    }
    if (int rc = batched ? launch_route_batched(a, x, tokens, h, logits, s, ids, weights, status, &routed,
                                                clear_status ? status : nullptr)
                         : launch_route_logits(a, x, tokens, h, logits, s))
        return rc;
    if (routed) return FMX_OK;
    hipLaunchKernelGGL(route_finish_kernel, dim3(tokens), dim3(64), 0, s, a, logits, ids, weights, status);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

int prepare_route_args(const fmx_moe_layer *L, RouteArgs *out) {
    RouteArgs a;
    a.hidden = L->hidden;
    a.experts = L->experts;
    a.top_k = L->top_k;
    a.norm_weight = L->norm_weight;
    a.rms_eps = L->rms_eps;
    a.norm_bias = L->norm_bias;
    a.router_type = L->router_type;
    a.router = nullptr;
    a.router_packed = nullptr;
    a.rtile = 0;
    switch (L->router_type) {
    case FMX_TYPE_F32: a.router = static_cast<const float *>(L->router); break;
    case FMX_TYPE_Q4_0:
    case FMX_TYPE_Q8_0:
    case FMX_TYPE_Q4_K: {
        if (int rc = packed_geometry(L->router_type, L->experts, L->hidden, &a.rg)) return rc;
        a.router_packed = L->router;
        constexpr uint32_t kBudget = 8 * 1024; // floats of h per LDS tile
        a.rtile = L->router_type == FMX_TYPE_Q4_0   ? tile_blocks_for<Q40>(a.rg.blocks, kBudget)
                  : L->router_type == FMX_TYPE_Q8_0 ? tile_blocks_for<Q80>(a.rg.blocks, kBudget)
                                                    : tile_blocks_for<Q4K>(a.rg.blocks, kBudget);
        break;
    }
    case FMX_TYPE_Q6_K:
        // raw rows (the packed layout of Q6_K is the raw one)
        if (L->hidden % 256) return FMX_ERR_SHAPE_MISMATCH;
        a.router_packed = L->router;
        break;
    default: return FMX_ERR_UNSUPPORTED_QUANTISATION;
    }
    a.router_bias = L->router_bias;
    a.weights_norm = L->weights_norm;
    a.epsilon_additive = L->epsilon_additive;
    a.weights_epsilon = L->weights_epsilon;
    a.weights_scale = L->weights_scale;
    *out = a;
    return FMX_OK;
}

int prepare_expert_args(const fmx_moe_layer *L, const RouteArgs &route, ExpertArgs *a) {
    ExpertArgs e;
    e.route = route;
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

int launch_experts(const ExpertArgs &a, const float *x, const float *h, const float *logits, uint32_t *ids,
                   float *w, const DecodeScratch &ws, float *out, uint32_t *status, hipStream_t s,
                   const hipEvent_t *kev) {
    auto known = [](uint32_t t) {
        return t == FMX_TYPE_F32 || t == FMX_TYPE_Q4_0 || t == FMX_TYPE_Q8_0 || t == FMX_TYPE_Q4_K ||
               t == FMX_TYPE_Q6_K;
    };
    if (!known(a.type_gu) || !known(a.type_dn)) return FMX_ERR_UNSUPPORTED_QUANTISATION;
    // the 16-lane down kernel gives each rank at least one of its 16 row slots
    const bool dn16 = a.type_dn == FMX_TYPE_F32 || a.type_dn == FMX_TYPE_Q6_K;
    if (dn16 && a.top_k > kThreads / 16) return FMX_ERR_UNSUPPORTED_QUANTISATION;
    // both kernels' LDS checked before either launches
    if (gate_up_lds(a) > kMaxLds || down_lds(a) > kMaxLds) return FMX_ERR_SHAPE_MISMATCH;
    if (int rc = launch_gate_up(a, h, logits, ids, w, ws.act, status, s, kev)) return rc;
    return launch_down(a, x, ws.act, ids, w, out, status, s, kev ? kev + 2 : nullptr);
}

} // namespace fmx
