// prefill.hpp — the batched (prefill) MoE path: grouped GEMMs on bf16 MFMA.
#pragma once

#include "moe.hpp"

namespace fmx {

// Device buffers of one prefill call (in the caller's workspace).
struct PrefillBuffers {
    const float *h;              // [tokens x hidden] RMSNorm output
    const uint32_t *token_list;  // [pairs] token of each bucketed (token, expert) pair
    const uint32_t *slot_of;     // [tokens x top_k] pair row of each (token, rank)
    uint32_t top_k;
    const uint32_t *tiles;       // row tiles of the bucketing (count, then expert / first row / rows)
    const uint32_t *tile_order;  // the tiles' indices largest first (the gate/up GEMM's dispatch order)
    uint32_t tokens;
    uint32_t pairs;              // tokens * top_k
    __bf16 *x;                   // [tokens x hidden] h in bf16, in the gate/up packed K order
    __bf16 *act;                 // [pairs x ffn] SwiGLU output in the down packed K order
    float *dn;                   // [splits x pairs x hidden] down projections (partial over K splits)
    uint32_t splits;             // K splits of the down projection (prefill_down_splits)
};

// Token-expert pairs per row tile of the grouped GEMMs (6 blocks of 32).
constexpr uint32_t kPrefillTileRows = 192;

// The grouped GEMMs need block-type experts with hidden and ffn multiples of
// the K step (128), of the types' chunk sizes and of the N tiles (hidden % 256,
// ffn % 128).
bool prefill_gemm_supported(const ExpertArgs &a);
// K splits of the down projection (its partial products are summed by the
// combine).
uint32_t prefill_down_splits(uint32_t experts, uint32_t ffn);
// h to bf16 -> gate/up GEMM (rows through token_list) + SwiGLU -> down GEMM,
// over `max_tiles` row tiles.
// kev (optional): events the gate/up launch records at its start and end
// (kev[0], kev[1]) and the down launch likewise (kev[2], kev[3]).
int launch_prefill_experts(const ExpertArgs &a, const PrefillBuffers &b, uint32_t max_tiles, hipStream_t s,
                           hipEvent_t *kev = nullptr);
// out[t] = x[t] + sum over ranks (rank order) of w * (sum over splits of
// dn[split][slot_of[t, r]]).
int launch_combine(const float *x, const float *dn, uint32_t splits, uint32_t pairs, const uint32_t *slot_of,
                   const float *w, uint32_t hidden, uint32_t K, uint32_t tokens, float *out, hipStream_t s);

} // namespace fmx
