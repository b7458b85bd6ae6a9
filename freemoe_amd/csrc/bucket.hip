// bucket.hip — per-expert token lists from a routing table, on the GPU.
//
// The reference has no bucketing: it walks each token's routed experts in rank
// order (engine.cpp:1711-1772). A batched path needs, per expert, the tokens
// that chose it; this pass inverts the routing record (engine.cpp:1707) into
// CSR form: offsets[E+1], and for expert e the entries offsets[e]..offsets[e+1]-1
// of token_list / rank_list hold the tokens, ascending, and the rank at which
// they chose e. `slot_of[t*K + r]` receives the entry index of (t, r); when it
// is given, a second, many-workgroup pass writes the two lists from it.
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
// Ids are read into registers in batches (their loads overlap; one workgroup
// is latency-bound): kCountBatch per thread when counting, and a token's
// first kIdRegs ids once per chunk.
constexpr uint32_t kCountBatch = 8;
constexpr uint32_t kIdRegs = 16;

__global__ __launch_bounds__(kBucketThreads) void bucket_kernel(
    const uint32_t *__restrict__ ids, uint32_t tokens, uint32_t K, uint32_t E,
    uint32_t *__restrict__ offsets, uint32_t *__restrict__ token_list,
    uint32_t *__restrict__ rank_list, uint32_t *__restrict__ slot_of, uint32_t *__restrict__ status,
    uint32_t *__restrict__ tiles, uint32_t tile_rows) {
    extern __shared__ __align__(16) uint32_t sm[];
    uint32_t *count = sm;                  // [E]
    uint32_t *base = count + E;            // [E]
    uint32_t *mask = base + E;             // [E][kWords]
    uint32_t *below = mask + E * kWords;   // [E][kWords]: chosen tokens in the expert's earlier words
    __shared__ uint32_t bad;
    const uint32_t tid = threadIdx.x;
    if (tid == 0) bad = 0;
    for (uint32_t e = tid; e < E; e += kBucketThreads) count[e] = 0;
    __syncthreads();
    const uint64_t n = static_cast<uint64_t>(tokens) * K;
    for (uint64_t i0 = tid; i0 < n; i0 += kCountBatch * kBucketThreads) {
        uint32_t eb[kCountBatch];
#pragma unroll
        for (uint32_t j = 0; j < kCountBatch; ++j) {
            const uint64_t i = i0 + j * kBucketThreads;
            eb[j] = i < n ? ids[i] : 0;
        }
#pragma unroll
        for (uint32_t j = 0; j < kCountBatch; ++j) {
            if (i0 + j * kBucketThreads >= n) break;
            if (eb[j] < E) atomicAdd(&count[eb[j]], 1u);
            else atomicOr(&bad, 1u);
        }
    }
    __syncthreads();
    if (bad) {
        if (tid == 0) {
            atomicOr(status, STATUS_BAD_EXPERT);
            if (tiles) tiles[0] = 0; // nothing downstream runs on these lists
        }
        // every position out of range: the gather and the combine skip them
        if (slot_of)
            for (uint64_t i = tid; i < n; i += kBucketThreads) slot_of[i] = 0xFFFFFFFFu;
        return;
    }
    // exclusive prefix sums over experts (E <= kBucketMaxExperts), one
    // wavefront, kPerLane consecutive experts per lane: entry offsets and,
    // with `tiles`, the list of row tiles (expert, first row, rows) of at most
    // tile_rows rows each, experts ascending: tiles[0] = count, then 3 words
    // per tile
    if (tid < 64) {
        constexpr uint32_t kPerLane = kBucketMaxExperts / 64;
        uint32_t rows = 0, nts = 0;
#pragma unroll
        for (uint32_t j = 0; j < kPerLane; ++j) {
            const uint32_t e = tid * kPerLane + j;
            const uint32_t c = e < E ? count[e] : 0;
            rows += c;
            if (tiles) nts += (c + tile_rows - 1) / tile_rows;
        }
        uint32_t rincl = rows, tincl = nts;
#pragma unroll
        for (uint32_t d = 1; d < 64; d <<= 1) {
            const uint32_t rv = __shfl_up(rincl, d), tv = __shfl_up(tincl, d);
            if (tid >= d) {
                rincl += rv;
                tincl += tv;
            }
        }
        uint32_t run = rincl - rows, nt = tincl - nts;
        for (uint32_t j = 0; j < kPerLane; ++j) {
            const uint32_t e = tid * kPerLane + j;
            if (e >= E) break;
            const uint32_t c = count[e];
            base[e] = run;
            offsets[e] = run;
            if (tiles)
                for (uint32_t r = 0; r < c; r += tile_rows, ++nt) {
                    tiles[1 + 3 * nt] = e;
                    tiles[2 + 3 * nt] = run + r;
                    tiles[3 + 3 * nt] = c - r < tile_rows ? c - r : tile_rows;
                }
            run += c;
        }
        if (tid == 63) {
            offsets[E] = rincl;
            if (tiles) tiles[0] = tincl;
        }
    }
    __syncthreads();
    for (uint32_t t0 = 0; t0 < tokens; t0 += kBucketThreads) {
        for (uint32_t i = tid; i < E * kWords; i += kBucketThreads) mask[i] = 0;
        __syncthreads();
        const uint32_t t = t0 + tid;
        const bool live = t < tokens;
        const uint32_t *tid_ids = ids + static_cast<uint64_t>(live ? t : 0) * K;
        uint32_t ev[kIdRegs];
#pragma unroll
        for (uint32_t r = 0; r < kIdRegs; ++r) ev[r] = live && r < K ? tid_ids[r] : 0;
        if (live) {
#pragma unroll
            for (uint32_t r = 0; r < kIdRegs; ++r)
                if (r < K) atomicOr(&mask[ev[r] * kWords + (tid >> 5)], 1u << (tid & 31));
            for (uint32_t r = kIdRegs; r < K; ++r) atomicOr(&mask[tid_ids[r] * kWords + (tid >> 5)], 1u << (tid & 31));
        }
        __syncthreads();
        // per expert, the exclusive prefix of its words' popcounts: one
        // 32-lane half-wavefront per expert at a time (kWords = 32)
        for (uint32_t i = tid; i < E * kWords; i += kBucketThreads) {
            const uint32_t c = __builtin_popcount(mask[i]), q = i & (kWords - 1);
            uint32_t incl = c;
#pragma unroll
            for (uint32_t d = 1; d < kWords; d <<= 1) {
                const uint32_t v = __shfl_up(incl, d, kWords);
                if (q >= d) incl += v;
            }
            below[i] = incl - c;
        }
        __syncthreads();
        if (live) {
            const uint32_t w = tid >> 5, lowbits = (1u << (tid & 31)) - 1u;
            // with slot_of, invert_slots_kernel writes the lists from it:
            // their scattered stores would all pass through this one CU
            auto place = [&](uint32_t r, uint32_t e) {
                const uint32_t pos = base[e] + below[e * kWords + w] + __builtin_popcount(mask[e * kWords + w] & lowbits);
                if (slot_of) {
                    slot_of[static_cast<uint64_t>(t) * K + r] = pos;
                } else {
                    token_list[pos] = t;
                    rank_list[pos] = r;
                }
            };
#pragma unroll
            for (uint32_t r = 0; r < kIdRegs; ++r)
                if (r < K) place(r, ev[r]);
            for (uint32_t r = kIdRegs; r < K; ++r) place(r, tid_ids[r]);
        }
        __syncthreads();
        for (uint32_t i = tid; i < E; i += kBucketThreads) {
            const uint32_t chosen = below[i * kWords + kWords - 1] + __builtin_popcount(mask[i * kWords + kWords - 1]);
            base[i] += chosen;
            count[i] -= chosen;
        }
        __syncthreads();
    }
    // a token that lists one expert twice sets one mask bit for two counts:
    // its expert's count is then not used up, and the lists hold a gap
    for (uint32_t e = tid; e < E; e += kBucketThreads)
        if (count[e] != 0) atomicOr(status, STATUS_BAD_EXPERT);
}

// token_list / rank_list from slot_of: entry slot_of[i] = (i / K, i % K).
// Positions outside [0, n) (a table the bucketing rejected) are skipped.
__global__ __launch_bounds__(256) void invert_slots_kernel(const uint32_t *__restrict__ slot_of, uint32_t n,
                                                           uint32_t K, uint32_t *__restrict__ token_list,
                                                           uint32_t *__restrict__ rank_list) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const uint32_t pos = slot_of[i];
    if (pos >= n) return;
    token_list[pos] = i / K;
    rank_list[pos] = i % K;
}

// ------------------------------------------------- many-workgroup bucketing --
// The same lists (and slot_of, tiles, offsets) over many workgroups, for the
// prefill: the tokens in chunks of kChunkTokens, one workgroup per chunk in
// two passes. Pass 1 writes each chunk's per-expert counts (integer adds in
// LDS) and a bad-id word; pass 2 gives each chunk the expert offsets (an
// exclusive scan of the totals) plus the counts of the chunks before it, and
// places the chunk's pairs by the popcounts of per-expert token bitmasks, as
// the single-workgroup pass does per 1024-token chunk. Deterministic: no
// position comes from an atomic slot grab.
constexpr uint32_t kChunkTokens = 256;
constexpr uint32_t kChunkWords = kChunkTokens / 32; // bitmask words per expert

// counts[c][E + 1]: chunk c's per-expert counts, then 1 when one of its ids is
// >= E. grid: chunks.
__global__ __launch_bounds__(kChunkTokens) void bucket_count_kernel(const uint32_t *__restrict__ ids,
                                                                   uint32_t tokens, uint32_t K, uint32_t E,
                                                                   uint32_t *__restrict__ counts) {
    __shared__ uint32_t cnt[kBucketMaxExperts];
    __shared__ uint32_t bad;
    const uint32_t tid = threadIdx.x, c = blockIdx.x;
    if (tid == 0) bad = 0;
    for (uint32_t e = tid; e < E; e += kChunkTokens) cnt[e] = 0;
    __syncthreads();
    const uint32_t t0 = c * kChunkTokens, t1 = tokens - t0 < kChunkTokens ? tokens : t0 + kChunkTokens;
    const uint64_t i1 = static_cast<uint64_t>(t1) * K;
    for (uint64_t i = static_cast<uint64_t>(t0) * K + tid; i < i1; i += kChunkTokens) {
        const uint32_t e = ids[i];
        if (e < E) atomicAdd(&cnt[e], 1u);
        else atomicOr(&bad, 1u);
    }
    __syncthreads();
    uint32_t *out = counts + static_cast<uint64_t>(c) * (E + 1);
    for (uint32_t e = tid; e < E; e += kChunkTokens) out[e] = cnt[e];
    if (tid == 0) out[E] = bad;
}

// Pass 2. grid: chunks; chunk 0 also writes offsets[E + 1] and the tiles.
__global__ __launch_bounds__(kChunkTokens) void bucket_place_kernel(
    const uint32_t *__restrict__ ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t chunks,
    const uint32_t *__restrict__ counts, uint32_t *__restrict__ offsets, uint32_t *__restrict__ slot_of,
    uint32_t *__restrict__ token_list, uint32_t *__restrict__ status, uint32_t *__restrict__ tiles,
    uint32_t *__restrict__ order, uint32_t tile_rows) {
    __shared__ uint32_t total[kBucketMaxExperts], base[kBucketMaxExperts], own[kBucketMaxExperts];
    __shared__ uint32_t mask[kBucketMaxExperts * kChunkWords], below[kBucketMaxExperts * kChunkWords];
    __shared__ uint32_t bad;
    const uint32_t tid = threadIdx.x, c = blockIdx.x;
    const uint32_t t0 = c * kChunkTokens;
    if (tid == 0) bad = 0;
    for (uint32_t i = tid; i < E * kChunkWords; i += kChunkTokens) mask[i] = 0;
    __syncthreads();
    // per expert: the total over chunks and the count of the chunks before c
    // (the chunks' counts requested 8 at a time, so their latencies overlap)
    for (uint32_t e = tid; e < E; e += kChunkTokens) {
        uint32_t tot = 0, pre = 0;
        for (uint32_t q0 = 0; q0 < chunks; q0 += 8) {
            uint32_t v[8];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j)
                v[j] = q0 + j < chunks ? counts[static_cast<uint64_t>(q0 + j) * (E + 1) + e] : 0u;
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
                pre += q0 + j < c ? v[j] : 0u;
                tot += v[j];
            }
        }
        total[e] = tot;
        base[e] = pre;
        own[e] = counts[static_cast<uint64_t>(c) * (E + 1) + e];
    }
    for (uint32_t q = tid; q < chunks; q += kChunkTokens)
        if (counts[static_cast<uint64_t>(q) * (E + 1) + E]) atomicOr(&bad, 1u);
    __syncthreads();
    if (bad) {
        if (c == 0 && tid == 0) {
            atomicOr(status, STATUS_BAD_EXPERT);
            if (tiles) tiles[0] = 0; // nothing downstream runs on these lists
        }
        // every position out of range: the gather and the combine skip them
        const uint64_t i1 = static_cast<uint64_t>(tokens - t0 < kChunkTokens ? tokens : t0 + kChunkTokens) * K;
        for (uint64_t i = static_cast<uint64_t>(t0) * K + tid; i < i1; i += kChunkTokens) slot_of[i] = 0xFFFFFFFFu;
        return;
    }
    // exclusive scan of the totals over experts by one wavefront (as the
    // single-workgroup pass); chunk 0 writes the offsets and the tiles in
    // expert order, and with `order` the same tiles largest first (order[i]:
    // the i-th tile to run), so that a GEMM's last rounds of workgroups hold
    // the short ones: every expert's full tiles (expert order), then the
    // partial tiles by row blocks, most first (expert order within a class).
    // The partial tiles' counts per class (9 bits each, at most 256 experts)
    // are scanned packed in one 64-bit word.
    if (tid < 64) {
        constexpr uint32_t kPerLane = kBucketMaxExperts / 64;
        const uint32_t nb = tile_rows / 32; // row-block classes of a partial tile (<= 7)
        auto cls = [tile_rows](uint32_t v) { return (v % tile_rows + 31) / 32; }; // 0: no partial tile
        uint32_t rows = 0, nts = 0, full = 0;
        uint64_t part = 0;
#pragma unroll
        for (uint32_t j = 0; j < kPerLane; ++j) {
            const uint32_t e = tid * kPerLane + j;
            const uint32_t v = e < E ? total[e] : 0;
            rows += v;
            if (tiles) {
                nts += (v + tile_rows - 1) / tile_rows;
                full += v / tile_rows;
                if (cls(v)) part += 1ull << (9 * (cls(v) - 1));
            }
        }
        uint32_t rincl = rows, tincl = nts, fincl = full;
        uint64_t pincl = part;
#pragma unroll
        for (uint32_t d = 1; d < 64; d <<= 1) {
            const uint32_t rv = __shfl_up(rincl, d), tv = __shfl_up(tincl, d), fv = __shfl_up(fincl, d);
            const uint64_t pv = __shfl_up(pincl, d);
            if (tid >= d) {
                rincl += rv;
                tincl += tv;
                fincl += fv;
                pincl += pv;
            }
        }
        uint32_t run = rincl - rows, nt = tincl - nts, nf = fincl - full;
        // where this lane's next partial tile of each class goes in `order`
        uint32_t np[7] = {};
        if (order) {
            const uint32_t ftotal = __shfl(fincl, 63);
            const uint64_t ptotal = __shfl(pincl, 63), pexcl = pincl - part;
            uint32_t at = ftotal;
            for (uint32_t k = nb; k >= 1; --k) {
                np[k - 1] = at + static_cast<uint32_t>((pexcl >> (9 * (k - 1))) & 511u);
                at += static_cast<uint32_t>((ptotal >> (9 * (k - 1))) & 511u);
            }
        }
        for (uint32_t j = 0; j < kPerLane; ++j) {
            const uint32_t e = tid * kPerLane + j;
            if (e >= E) break;
            const uint32_t v = total[e];
            base[e] += run;
            if (c == 0) {
                offsets[e] = run;
                if (tiles)
                    for (uint32_t r = 0; r < v; r += tile_rows, ++nt) {
                        const uint32_t n = v - r < tile_rows ? v - r : tile_rows;
                        tiles[1 + 3 * nt] = e;
                        tiles[2 + 3 * nt] = run + r;
                        tiles[3 + 3 * nt] = n;
                        if (order) order[n == tile_rows ? nf++ : np[cls(v) - 1]++] = nt;
                    }
            }
            run += v;
        }
        if (tid == 63 && c == 0) {
            offsets[E] = rincl;
            if (tiles) tiles[0] = tincl;
        }
    }
    // the chunk's tokens into per-expert bitmasks
    const uint32_t t = t0 + tid;
    const bool live = t < tokens;
    const uint32_t *tid_ids = ids + static_cast<uint64_t>(live ? t : 0) * K;
    uint32_t ev[kIdRegs];
#pragma unroll
    for (uint32_t r = 0; r < kIdRegs; ++r) ev[r] = live && r < K ? tid_ids[r] : 0;
    if (live) {
#pragma unroll
        for (uint32_t r = 0; r < kIdRegs; ++r)
            if (r < K) atomicOr(&mask[ev[r] * kChunkWords + (tid >> 5)], 1u << (tid & 31));
        for (uint32_t r = kIdRegs; r < K; ++r)
            atomicOr(&mask[tid_ids[r] * kChunkWords + (tid >> 5)], 1u << (tid & 31));
    }
    __syncthreads();
    // per expert, the exclusive prefix of its words' popcounts (8-lane groups)
    for (uint32_t i = tid; i < E * kChunkWords; i += kChunkTokens) {
        const uint32_t pc = __builtin_popcount(mask[i]), q = i & (kChunkWords - 1);
        uint32_t incl = pc;
#pragma unroll
        for (uint32_t d = 1; d < kChunkWords; d <<= 1) {
            const uint32_t v = __shfl_up(incl, d, kChunkWords);
            if (q >= d) incl += v;
        }
        below[i] = incl - pc;
        // a token that lists one expert twice sets one bit for two counts
        if (q == kChunkWords - 1 && incl != own[i / kChunkWords]) atomicOr(status, STATUS_BAD_EXPERT);
    }
    __syncthreads();
    if (live) {
        const uint32_t w = tid >> 5, lowbits = (1u << (tid & 31)) - 1u;
        auto place = [&](uint32_t r, uint32_t e) {
            const uint32_t pos =
                base[e] + below[e * kChunkWords + w] + __builtin_popcount(mask[e * kChunkWords + w] & lowbits);
            slot_of[static_cast<uint64_t>(t) * K + r] = pos;
            if (token_list) token_list[pos] = t;
        };
#pragma unroll
        for (uint32_t r = 0; r < kIdRegs; ++r)
            if (r < K) place(r, ev[r]);
        for (uint32_t r = kIdRegs; r < K; ++r) place(r, tid_ids[r]);
    }
}

} // namespace

uint64_t bucket_chunk_counts_bytes(uint32_t tokens, uint32_t experts) {
    return static_cast<uint64_t>(div_up(tokens, kChunkTokens)) * (experts + 1) * sizeof(uint32_t);
}

int launch_bucket_chunked(const uint32_t *ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t *offsets,
                          uint32_t *slot_of, uint32_t *token_list, uint32_t *status, uint32_t *counts, hipStream_t s,
                          uint32_t *tiles, uint32_t *order, uint32_t tile_rows) {
    // order (with tiles): tile_rows a multiple of 32, at most 7 row blocks
    // (the classes of the partial tiles' packed counts)
    if (!slot_of || !counts || E == 0 || E > kBucketMaxExperts || (tiles && tile_rows == 0) || (order && !tiles) ||
        (order && (tile_rows % 32 || tile_rows > 224)))
        return FMX_ERR_INVALID_ARGUMENT;
    if (tokens == 0) return FMX_OK;
    const uint32_t chunks = div_up(tokens, kChunkTokens);
    hipLaunchKernelGGL(bucket_count_kernel, dim3(chunks), dim3(kChunkTokens), 0, s, ids, tokens, K, E, counts);
    FMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(bucket_place_kernel, dim3(chunks), dim3(kChunkTokens), 0, s, ids, tokens, K, E, chunks, counts,
                       offsets, slot_of, token_list, status, tiles, order, tile_rows);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

size_t bucket_lds_bytes(uint32_t experts) {
    return (2ull * experts + 2ull * experts * kWords) * sizeof(uint32_t);
}

int launch_bucket(const uint32_t *ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t *offsets,
                  uint32_t *token_list, uint32_t *rank_list, uint32_t *slot_of, uint32_t *status,
                  hipStream_t s, uint32_t *tiles, uint32_t tile_rows) {
    if (tiles && tile_rows == 0) return FMX_ERR_INVALID_ARGUMENT;
    if (int rc = allow_lds(reinterpret_cast<const void *>(bucket_kernel), bucket_lds_bytes(E))) return rc;
    hipLaunchKernelGGL(bucket_kernel, dim3(1), dim3(kBucketThreads), bucket_lds_bytes(E), s, ids, tokens, K,
                       E, offsets, token_list, rank_list, slot_of, status, tiles, tile_rows);
    FMX_LAUNCH_CHECK();
    const uint64_t n = static_cast<uint64_t>(tokens) * K;
    if (slot_of && n > 0) {
        hipLaunchKernelGGL(invert_slots_kernel, dim3(static_cast<uint32_t>((n + 255) / 256)), dim3(256), 0, s, slot_of,
                           static_cast<uint32_t>(n), K, token_list, rank_list);
        FMX_LAUNCH_CHECK();
    }
    return FMX_OK;
}

} // namespace fmx
