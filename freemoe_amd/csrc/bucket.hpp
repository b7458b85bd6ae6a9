// bucket.hpp — deterministic per-expert token lists (see bucket.hip).
#pragma once

#include "fmx_internal.hpp"

namespace fmx {

// Experts supported by the single-workgroup bucketing pass (LDS bound).
constexpr uint32_t kBucketMaxExperts = 256;

size_t bucket_lds_bytes(uint32_t experts);
// tiles (optional): [1 + 3 * max_tiles] words, max_tiles = E + tokens*K / tile_rows;
// receives the row tiles of at most tile_rows rows of every non-empty expert.
int launch_bucket(const uint32_t *ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t *offsets,
                  uint32_t *token_list, uint32_t *rank_list, uint32_t *slot_of, uint32_t *status,
                  hipStream_t s, uint32_t *tiles = nullptr, uint32_t tile_rows = 0);

// The prefill's bucketing over many workgroups: slot_of (required),
// offsets, token_list (optional) and tiles as launch_bucket, without
// rank_list; order (optional, with tiles; bucket_max_tiles entries): the
// tiles' indices largest first. counts: the chunk counts' device scratch,
// bucket_chunk_counts_bytes(tokens, E) bytes.
uint64_t bucket_chunk_counts_bytes(uint32_t tokens, uint32_t experts);
int launch_bucket_chunked(const uint32_t *ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t *offsets,
                          uint32_t *slot_of, uint32_t *token_list, uint32_t *status, uint32_t *counts, hipStream_t s,
                          uint32_t *tiles, uint32_t *order, uint32_t tile_rows);

inline uint32_t bucket_max_tiles(uint32_t tokens, uint32_t K, uint32_t E, uint32_t tile_rows) {
    return E + static_cast<uint32_t>((static_cast<uint64_t>(tokens) * K) / tile_rows);
}

} // namespace fmx
