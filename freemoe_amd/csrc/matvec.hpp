// matvec.hpp — 16-lane row dots: F32 in gemv_avx2_row's order
// (kernels.cpp:147-167), Q6_K in row_dot_fused_scalar's (kernels.cpp:574-590).
#pragma once

#include <utility>

#include "fmx_internal.hpp"

namespace fmx {

// 16 consecutive lanes (c = lane & 15, groups aligned to 16 within the
// wavefront) compute one F32 row dot: chain c accumulates k = c mod 16 with
// FMA, chains 0..7 take the 8-element tail, lanes c and c+8 add (acc0 + acc1),
// the 8-lane tree sum follows, then an FMA tail over the last n mod 8 elements.
// Every lane of the group returns the row's value. `x` may point to LDS.
// kNT: the row's batches read with non-temporal loads. The matrix-vector
// product uses them: from a cold cache [4096 x 4096] 27.9 -> 20.3 µs and
// [14336 x 4096] 80.5 -> 53.3 µs, the 8-layer decoder's 256 tokens through
// the engine 797 -> 775 ms; only a matrix that fits the memory-side cache
// and is read again at once loses ([14336 x 4096] back to back 43.9 -> 51.1
// µs). The decode's F32 expert rows keep plain loads (5% faster there).
template <bool kNT = false>
__device__ inline float f32_row_chains(const float *__restrict__ row, const float *x, uint32_t n,
                                       uint32_t c) {
    auto ld = [](const float *p) {
        if constexpr (kNT) return ldf_nt(p);
        else return *p;
    };
    float acc = 0.0f;
    const uint32_t n16 = n / 16 * 16;
    // the chain is a dependent FMA sequence: the row's elements are requested
    // kB steps at a time, the next batch before this one's FMAs
    constexpr uint32_t kB = 16;
    const uint32_t nb = n16 / (16 * kB);
    float wb[2][kB];
    if (nb > 0) {
#pragma unroll
        for (uint32_t u = 0; u < kB; ++u) wb[0][u] = ld(row + 16 * u + c);
    }
    for (uint32_t bi = 0; bi < nb; bi += 2) {
#pragma unroll
        for (uint32_t half = 0; half < 2; ++half) {
            const uint32_t b = bi + half;
            if (b >= nb) break;
            const uint32_t k0 = 16 * kB * b, kn = 16 * kB * (b + 1 < nb ? b + 1 : b);
#pragma unroll
            for (uint32_t u = 0; u < kB; ++u) wb[half ^ 1][u] = ld(row + kn + 16 * u + c);
#pragma unroll
            for (uint32_t u = 0; u < kB; ++u) acc = fma_rn(wb[half][u], x[k0 + 16 * u + c], acc);
        }
    }
#pragma unroll 8
    for (uint32_t k = 16 * kB * nb; k < n16; k += 16) acc = fma_rn(row[k + c], x[k + c], acc);
    const bool tail8 = n - n16 >= 8;
    if (tail8 && c < 8) acc = fma_rn(row[n16 + c], x[n16 + c], acc);
    const float t = acc + lane_xor<8>(acc);
    float total = hsum8_lanes(t);
    for (uint32_t k = tail8 ? n16 + 8 : n16; k < n; ++k) total = fma_rn(row[k], x[k], total);
    return total;
}

// Element e (< 256) of a raw Q6_K block (quant.cpp:347-371): half n = e / 128;
// in the half, l = e % 32 and quarter qt = (e % 128) / 32 take the low (qt < 2)
// or high nibble of ql[64 n + l + 32 (qt % 2)], the bit pair qt of
// qh[32 n + l], sub-block scale sc[8 n + l / 16 + 2 qt]; (d * sc) * (q - 32).
__device__ inline float q6_k_value(const uint8_t *blk, uint32_t e) {
    const uint32_t n = e >> 7, r = e & 127, l = r & 31, qt = r >> 5;
    const uint32_t ql = blk[64 * n + l + 32 * (qt & 1)];
    const uint32_t qh = blk[128 + 32 * n + l];
    const int q = static_cast<int>((qt >= 2 ? ql >> 4 : ql & 0x0Fu) | (((qh >> (2 * qt)) & 3u) << 4)) - 32;
    const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
    const float sc = static_cast<float>(static_cast<int8_t>(blk[192 + 8 * n + l / 16 + 2 * qt]));
    return d * sc * static_cast<float>(q);
}

// One lane's share of a raw Q6_K block for chain c: element e = 16 m + c
// (m < 16) lies in half n = m / 8, at l = 16 (m % 2) + c of the half, quarter
// qt = (m % 8) / 2; its quant byte is ql[64 n + 16 (m % 2 + 2 (qt % 2)) + c],
// its bit pairs qh[128 + 32 n + 16 (m % 2) + c], its scale sc[8 n + m % 2 +
// 2 qt] = sc[m]: element 16 m + c lies in sub-block m for every c. The lane
// loads those 8 + 4 bytes, scale byte c (its sub-block's scale d sc[c] is
// formed once per block and handed to the other lanes of its 16-lane group
// by DPP row broadcasts) and d, and its 16 inputs x[16 m + c], all requested
// together. The lanes of a group must be the 16 lanes of one DPP row.
struct Q6Lane {
    uint32_t ql[2][4], qh[2][2];
    uint32_t scb; // scale byte c
    uint32_t d;
    float xv[16];
    __device__ __forceinline__ void load(const uint8_t *__restrict__ blk, const float *xb, uint32_t c) {
#pragma unroll
        for (uint32_t n = 0; n < 2; ++n) {
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) ql[n][k] = blk[64 * n + 16 * k + c];
#pragma unroll
            for (uint32_t a = 0; a < 2; ++a) qh[n][a] = blk[128 + 32 * n + 16 * a + c];
        }
        scb = blk[192 + c];
        d = *reinterpret_cast<const uint16_t *>(blk + 208);
#pragma unroll
        for (uint32_t m = 0; m < 16; ++m) xv[m] = xb[16 * m + c];
    }
    // q - 32 of element 16 m + c.
    template <uint32_t m>
    __device__ __forceinline__ int q_of() const {
        constexpr uint32_t n = m >> 3, a = m & 1, qt = (m & 7) >> 1;
        const uint32_t qlb = ql[n][a + 2 * (qt & 1)];
        return static_cast<int>((qt >= 2 ? qlb >> 4 : qlb & 0x0Fu) | (((qh[n][a] >> (2 * qt)) & 3u) << 4)) - 32;
    }
    template <uint32_t... M>
    __device__ __forceinline__ float chain_over(float dsc, std::integer_sequence<uint32_t, M...>) const {
        float acc = 0.0f;
        ((acc = fma_rn(row_bcast<M>(dsc) * static_cast<float>(q_of<M>()), xv[M], acc)), ...);
        return acc;
    }
    // Chain c of dot_avx2 over the block's decoded values (d * sc) * (q - 32)
    // in element order: d * sc[m] (exact) from lane m of the row, handed over
    // as the multiply's DPP operand.
    __device__ __forceinline__ float chain() const {
        const float dsc = half_bits_to_float(d) * static_cast<float>(static_cast<int8_t>(scb & 0xFFu));
        return chain_over(dsc, std::make_integer_sequence<uint32_t, 16>());
    }
};

// One Q6_K row dot on 16 consecutive lanes (c = lane & 15): for each block,
// lane c runs chain c of dot_avx2 over the block's 256 decoded values
// (elements 16 m + c), the chains meet as in f32_row_chains, and the block's
// dot is added to the row total in block order. The next block's bytes and
// inputs are requested before this block's chain runs. Every lane returns the
// row's value.
__device__ inline float q6_k_row_chains(const uint8_t *__restrict__ row, const float *x, uint32_t blocks,
                                        uint32_t c) {
    float total = 0.0f;
    Q6Lane q[2];
    if (blocks > 0) q[0].load(row, x, c);
    for (uint32_t b = 0; b < blocks; b += 2) {
#pragma unroll
        for (uint32_t u = 0; u < 2; ++u) {
            if (b + u >= blocks) break;
            if (b + u + 1 < blocks)
                q[u ^ 1].load(row + static_cast<uint64_t>(b + u + 1) * 210, x + static_cast<uint64_t>(b + u + 1) * 256,
                              c);
            const float acc = q[u].chain();
            // t is the same in lanes i and i + 8, so hsum8_first's rotation
            // reads a lane holding the xor-4 partner's value in every lane
            const float t = acc + lane_xor<8>(acc);
            total = total + hsum8_first(t);
        }
    }
    return total;
}

// Floats per Q6_K block of inputs staged in LDS: the 16 floats between
// blocks put 16-lane groups of one wavefront that work on different blocks
// on different banks.
constexpr uint32_t kQ6XStride = 272;

// Dots of blocks b0, b0 + stride, ... (< blocks) of one Q6_K row on 16
// consecutive lanes, each as in q6_k_row_chains (chain c over elements
// 16 m + c, the lanes' chains joined), the next block's share requested
// before a block's chain runs; lane 0 writes block b's dot to out[b]. Block
// b's 256 inputs start at x + b * xstride (256 in memory; more where x is
// staged in LDS with padding between blocks).
__device__ __forceinline__ void q6_k_block_dots(const uint8_t *__restrict__ row, const float *x, uint32_t blocks,
                                                uint32_t b0, uint32_t stride, uint32_t c, float *out,
                                                uint32_t xstride = 256) {
    Q6Lane q[2];
    if (b0 < blocks) q[0].load(row + static_cast<uint64_t>(b0) * 210, x + static_cast<uint64_t>(b0) * xstride, c);
    for (uint32_t b = b0; b < blocks; b += 2 * stride) {
#pragma unroll
        for (uint32_t u = 0; u < 2; ++u) {
            const uint32_t bu = b + u * stride;
            if (bu >= blocks) break;
            const uint32_t nb = bu + stride;
            if (nb < blocks)
                q[u ^ 1].load(row + static_cast<uint64_t>(nb) * 210, x + static_cast<uint64_t>(nb) * xstride, c);
            const float acc = q[u].chain();
            const float t = acc + lane_xor<8>(acc);
            const float dot = hsum8_first(t); // exact in every lane, as above
            if (c == 0) out[bu] = dot;
        }
    }
}

// Row dots on 16 lanes by type, for kernels that take F32 or Q6_K rows: the
// value of row r of matrix m ([rows x n], raw rows) against x.
template <uint32_t kType>
struct RowDot16 {
    __device__ static float dot(const void *m, uint32_t r, const float *x, uint32_t n, uint32_t c) {
        if constexpr (kType == FMX_TYPE_Q6_K)
            return q6_k_row_chains(static_cast<const uint8_t *>(m) + static_cast<uint64_t>(r) * (n / 256) * 210, x,
                                   n / 256, c);
        else
            return f32_row_chains(static_cast<const float *>(m) + static_cast<uint64_t>(r) * n, x, n, c);
    }
};

} // namespace fmx
