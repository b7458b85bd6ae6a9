// bucket.hpp — deterministic per-expert token lists (see bucket.hip).
#pragma once

#include "fmx_internal.hpp"

namespace fmx {

// Experts supported by the single-workgroup bucketing pass (LDS bound).
constexpr uint32_t kBucketMaxExperts = 256;

size_t bucket_lds_bytes(uint32_t experts);
int launch_bucket(const uint32_t *ids, uint32_t tokens, uint32_t K, uint32_t E, uint32_t *offsets,
                  uint32_t *token_list, uint32_t *rank_list, uint32_t *slot_of, uint32_t *status,
                  hipStream_t s);

} // namespace fmx
