// bucket.hip — per-expert token lists from a routing table, on the GPU.
//
// The reference has no bucketing: it walks each token's routed experts in rank
// order (engine.cpp:1711-1772). A batched path needs, per expert, the tokens
// that chose it; this pass inverts the routing record (engine.cpp:1707) into
// CSR form: offsets[E+1], and for expert e the entries offsets[e]..offsets[e+1]-1
// of token_list / rank_list hold the tokens, ascending, and the rank at which
// they chose e. `slot_of[t*K + r]` receives the entry index of (t, r).
//
// Deterministic by construction: counts are order-independent integer adds,
// and the position of (t, r) inside expert e's list is the number of earlier
// tokens that chose e, taken from a per-expert bitmask of the tokens of the
// current 1024-token chunk (popcounts of the lower bits), never from atomic
// slot grabs.
#include "fmx_internal.hpp"
#include "bucket.hpp"

namespace fmx {

namespace {

constexpr uint32_t kBucketThreads = 1024;
constexpr uint32_t kWords = kBucketThreads / 32; // bitmask words per expert

__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(
    const uint32_t *__restrict__ ids, uint32_t tokens, uint32_t K, uint32_t E,
    uint32_t *__restrict__ offsets, uint32_t *__restrict__ token_list,
    uint32_t *__restrict__ rank_list, uint32_t *__restrict__ slot_of, uint32_t *__restrict__ status,
    uint32_t *__restrict__ tiles, uint32_t tile_rows) {
    extern __shared__ __align__(16) uint32_t sm[];
    uint32_t *count = sm;                  // [E]
    uint32_t *base = count + E;            // [E]
    uint32_t *mask = base + E;             // [E][kWords]
    __shared__ uint32_t bad;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) bad = 0;
    for (uint32_t e = tid; e < E; e += kBucketThreads) count[e] = 0;
    __syncthreads();
    const uint64_t n = static_cast<uint64_t>(tokens) * K;
    for (uint64_t i = tid; i < n; i += kBucketThreads) {
        const uint32_t e = ids[i];
        if (e < E) atomicAdd(&count[e], 1u);
        else atomicOr(&bad, 1u);
    }
    __syncthreads();
    if (bad) {
        if (tid == 0) {
            atomicOr(status, STATUS_BAD_EXPERT);
            if (tiles) tiles[0] = 0; // nothing downstream runs on these lists
        }
        return;
    }
    // exclusive prefix sum over experts (E <= kBucketThreads), one lane;
    // with `tiles`, also the list of row tiles (expert, first row, rows) of
    // at most tile_rows rows each, experts ascending: tiles[0] = count, then
    // 3 words per tile
    if (tid == 0) {
        uint32_t run = 0, nt = 0;
        for (uint32_t e = 0; e < E; ++e) {
            base[e] = run;
            offsets[e] = run;
            if (tiles)
                for (uint32_t r = 0; r < count[e]; r += tile_rows, ++nt) {
                    tiles[1 + 3 * nt] = e;
                    tiles[2 + 3 * nt] = run + r;
                    tiles[3 + 3 * nt] = count[e] - r < tile_rows ? count[e] - r : tile_rows;
                }
            run += count[e];
        }
        offsets[E] = run;
        if (tiles) tiles[0] = nt;
    }
    __syncthreads();
    for (uint32_t t0 = 0; t0 < tokens; t0 += kBucketThreads) {
        for (uint32_t i = tid; i < E * kWords; i += kBucketThreads) mask[i] = 0;
        __syncthreads();
        const uint32_t t = t0 + tid;
        const bool live = t < tokens;
        if (live)
            for (uint32_t r = 0; r < K; ++r) {
                const uint32_t e = ids[static_cast<uint64_t>(t) * K + r];
                atomicOr(&mask[e * kWords + (tid >> 5)], 1u << (tid & 31));
            }
        __syncthreads();
        if (live)
            for (uint32_t r = 0; r < K; ++r) {
                const uint32_t e = ids[static_cast<uint64_t>(t) * K + r];
                const uint32_t w = tid >> 5;
                uint32_t before = 0;
                for (uint32_t q = 0; q < w; ++q) before += __builtin_popcount(mask[e * kWords + q]);
                const uint32_t below = mask[e * kWords + w] & ((1u << (tid & 31)) - 1u);
                const uint32_t pos = base[e] + before + __builtin_popcount(below);
                token_list[pos] = t;
                rank_list[pos] = r;
                if (slot_of) slot_of[static_cast<uint64_t>(t) * K + r] = pos;
            }
        __syncthreads();
        for (uint32_t i = tid; i < E; i += kBucketThreads) {
            uint32_t chosen = 0;
            for (uint32_t q = 0; q < kWords; ++q) chosen += __builtin_popcount(mask[i * kWords + q]);
            base[i] += chosen;
        }
        __syncthreads();
    }
}

} // namespace

size_t bucket_lds_bytes(uint32_t experts) {
    return (2ull * experts + static_cast<uint64_t>(experts) * kWords) * sizeof(uint32_t);
}

int launch_bucket(const uint32_t *ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t *offsets,
                  uint32_t *token_list, uint32_t *rank_list, uint32_t *slot_of, uint32_t *status,
                  hipStream_t s, uint32_t *tiles, uint32_t tile_rows) {
    if (tiles && tile_rows == 0) return FMX_ERR_INVALID_ARGUMENT;
    hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(kBucketThreads), bucket_lds_bytes(E), s, ids, tokens, K,
                       E, offsets, token_list, rank_list, slot_of, status, tiles, tile_rows);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace fmx
