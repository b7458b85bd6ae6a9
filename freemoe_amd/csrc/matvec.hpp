// matvec.hpp — the F32 row dot of gemv_avx2_row (kernels.cpp:147-167) on 16 lanes.
#pragma once

#include "fmx_internal.hpp"

namespace fmx {

// 16 consecutive lanes (c = lane & 15, groups aligned to 16 within the
// wavefront) compute one F32 row dot: chain c accumulates k = c mod 16 with
// FMA, chains 0..7 take the 8-element tail, lanes c and c+8 add (acc0 + acc1),
// the 8-lane tree sum follows, then an FMA tail over the last n mod 8 elements.
// Every lane of the group returns the row's value. `x` may point to LDS.
__device__ inline float f32_row_chains(const float *__restrict__ row, const float *x, uint32_t n,
                                       uint32_t c) {
    float acc = 0.0f;
    const uint32_t n16 = n / 16 * 16;
#pragma unroll 8
    for (uint32_t k = 0; k < n16; k += 16) acc = fma_rn(row[k + c], x[k + c], acc);
    const bool tail8 = n - n16 >= 8;
    if (tail8 && c < 8) acc = fma_rn(row[n16 + c], x[n16 + c], acc);
    const float t = acc + lane_xor(acc, 8);
    float total = hsum8_lanes(t);
    for (uint32_t k = tail8 ? n16 + 8 : n16; k < n; ++k) total = fma_rn(row[k], x[k], total);
    return total;
}

} // namespace fmx
