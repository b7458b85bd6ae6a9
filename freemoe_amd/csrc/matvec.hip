// matvec.hip — y = W x for one matrix (Backend::matvec / gemv_quant).
//
// Block-type rows use the lane chains of chains.hpp (Q4_0, Q8_0, Q4_K: the
// reference's dedicated AVX2 row dots); Q6_K rows, which the reference runs
// through row_dot_fused_scalar (kernels.cpp:574-590: each block decoded,
// dotted by dot_avx2, the block's dot added to the row total), use that order
// on 16 lanes per row; F32 rows use the
// reference's gemv_avx2_row order (kernels.cpp:147-167): per row 16 chains
// (chain c takes k = c mod 16; chains 0..7 are acc0, 8..15 acc1), an 8-element
// tail into acc0, lane-wise acc0 + acc1, the 8-lane tree sum, then a scalar
// FMA tail over the last in_dim mod 8 elements.
#include "chains.hpp"
#include "matvec.hpp"

namespace fmx {

namespace {

constexpr uint32_t kThreads = 256;              // 4 wavefronts
constexpr uint32_t kLdsBudgetFloats = 8 * 1024; // 32 KiB of x per tile
constexpr size_t kMatvecMaxLds = 128 * 1024;     // the Q6_K split kernel's x and dots

template <class T, int NR>
__global__ __launch_bounds__(kThreads) void matvec_kernel(
    const uint8_t *__restrict__ packed, const float *__restrict__ x, float *__restrict__ y,
    uint32_t rows, uint32_t blocks, uint32_t blocks_padded, uint32_t chunks, uint64_t scale_bytes,
    uint32_t tile_blocks) {
    extern __shared__ __align__(16) float lds[];
    const uint32_t tid = threadIdx.x;
    const uint32_t l = tid & 7;
    const uint32_t slot = tid >> 3; // 0..31
    const uint32_t r0 = (blockIdx.x * (kThreads / 8) + slot) * NR;
    typename T::Row rw[NR];
    float t[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const uint32_t r = r0 + i < rows ? r0 + i : rows - 1; // clamp: loads stay in bounds
        rw[i] = T::row(packed, scale_bytes, blocks_padded, chunks, r, l);
        t[i] = 0.0f;
    }
    for (uint32_t tb = 0; tb < blocks; tb += tile_blocks) {
        const uint32_t nb = blocks - tb < tile_blocks ? blocks - tb : tile_blocks;
        __syncthreads();
        T::stage(x, tb, nb, lds, tid, kThreads);
        __syncthreads();
        const uint32_t c0 = tb / T::kPerChunk;
        const uint32_t c1 = (tb + nb + T::kPerChunk - 1) / T::kPerChunk;
        run_chunks_pf<T, NR, 2>(rw, c0, c1, blocks, tb, nb, lds, l, t);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const float v = T::finish(t[i]);
        if (l == 0 && r0 + i < rows) y[r0 + i] = v;
    }
}

// F32: 16 lanes per row (4 row slots per wavefront, 16 per workgroup).
// kXs: x staged in LDS first (n floats), so each input is read from memory
// once per workgroup instead of once per row; the groups of a wavefront read
// the same elements at once.
template <bool kXs>
__global__ __launch_bounds__(kThreads) void matvec_f32_kernel(const float *__restrict__ w,
                                                              const float *__restrict__ x,
                                                              float *__restrict__ y,
                                                              uint32_t rows, uint32_t n) {
    extern __shared__ __align__(16) float xs_f32[];
    const uint32_t tid = threadIdx.x;
    const uint32_t c = tid & 15;
    const float *xr = x;
    if constexpr (kXs) {
        if ((reinterpret_cast<uintptr_t>(x) & 15u) == 0 && n % 4 == 0) {
            const float4 *x4 = reinterpret_cast<const float4 *>(x);
            for (uint32_t q = tid; q < n / 4; q += kThreads) reinterpret_cast<float4 *>(xs_f32)[q] = x4[q];
        } else {
            for (uint32_t q = tid; q < n; q += kThreads) xs_f32[q] = x[q];
        }
        __syncthreads();
        xr = xs_f32;
    }
    const uint32_t r = blockIdx.x * (kThreads / 16) + (tid >> 4);
    const uint32_t rr = r < rows ? r : rows - 1;
    const float *row = w + static_cast<uint64_t>(rr) * n;
    const float total = f32_row_chains<true>(row, xr, n, c);
    if (c == 0 && r < rows) y[r] = total;
}

// Q6_K: 16 lanes per row over raw blocks (q6_k_row_chains).
__global__ __launch_bounds__(kThreads) void matvec_q6_k_kernel(const uint8_t *__restrict__ w,
                                                               const float *__restrict__ x,
                                                               float *__restrict__ y, uint32_t rows,
                                                               uint32_t blocks) {
    const uint32_t tid = threadIdx.x, c = tid & 15;
    const uint32_t r = blockIdx.x * (kThreads / 16) + (tid >> 4);
    const uint32_t rr = r < rows ? r : rows - 1;
    const float total = q6_k_row_chains(w + static_cast<uint64_t>(rr) * blocks * 210, x, blocks, c);
    if (c == 0 && r < rows) y[r] = total;
}

// Q6_K with few rows: G lane groups per row, group g taking blocks
// g, g + G, ... (each block's dot is independent); the block dots meet in LDS
// and one lane adds them in block order from 0, as q6_k_row_chains does.
// kXs: x staged in LDS first (block b at xs + b * kQ6XStride), so each input
// is read from memory once per workgroup instead of once per row (worth its
// LDS at 8 rows per workgroup).
// LDS: (16 / G) rows x blocks dots, then x.
__host__ __device__ inline uint32_t q6_split_dots_floats(uint32_t rows, uint32_t blocks) {
    return (rows * blocks + 3u) & ~3u;
}
template <uint32_t G, bool kXs>
__global__ __launch_bounds__(kThreads) void matvec_q6_k_split_kernel(const uint8_t *__restrict__ w,
                                                                     const float *__restrict__ x,
                                                                     float *__restrict__ y, uint32_t rows,
                                                                     uint32_t blocks) {
    extern __shared__ __align__(16) float q6_lds[];
    constexpr uint32_t kRows = kThreads / 16 / G;
    float *dots = q6_lds;
    const uint32_t tid = threadIdx.x, c = tid & 15, grp = tid >> 4;
    const float *xr = x;
    uint32_t xstride = 256;
    if constexpr (kXs) {
        float *xs = q6_lds + q6_split_dots_floats(kRows, blocks);
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (uint32_t q = tid; q < blocks * 64; q += kThreads)
            reinterpret_cast<float4 *>(xs + (q >> 6) * kQ6XStride)[q & 63] = x4[q];
        __syncthreads();
        xr = xs;
        xstride = kQ6XStride;
    }
    const uint32_t lr = grp / G, part = grp % G;
    const uint32_t r = blockIdx.x * kRows + lr;
    const uint32_t rr = r < rows ? r : rows - 1;
    q6_k_block_dots(w + static_cast<uint64_t>(rr) * blocks * 210, xr, blocks, part, G, c, dots + lr * blocks,
                    xstride);
    __syncthreads();
    if (tid < kRows && blockIdx.x * kRows + tid < rows) {
        const float *d = dots + tid * blocks;
        float total = 0.0f;
        for (uint32_t b = 0; b < blocks; ++b) total = total + d[b];
        y[blockIdx.x * kRows + tid] = total;
    }
}

template <class T, int NR>
int launch_matvec(const PackedGeometry &g, const void *packed, const float *x, float *y,
                  hipStream_t s) {
    const uint32_t tb = tile_blocks_for<T>(g.blocks, kLdsBudgetFloats);
    const size_t lds = static_cast<size_t>(tb) * T::kLdsFloatsPerBlock * sizeof(float);
    const uint32_t rows_per_wg = (kThreads / 8) * NR;
    hipLaunchKernelGGL((matvec_kernel<T, NR>), dim3(div_up(g.rows, rows_per_wg)), dim3(kThreads),
                       lds, s, static_cast<const uint8_t *>(packed), x, y, g.rows, g.blocks,
                       g.blocks_padded, g.chunks, g.scale_bytes, tb);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace

} // namespace fmx

using namespace fmx;

extern "C" int fmx_matvec(uint32_t type_id, const void *packed, const float *x, float *y,
                          uint32_t out_dim, uint32_t in_dim, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (out_dim == 0 || in_dim == 0) return FMX_OK;
    PackedGeometry g;
    if (int rc = packed_geometry(type_id, out_dim, in_dim, &g)) return rc;
    if (!packed || !x || !y) return FMX_ERR_INVALID_ARGUMENT;
    // block-type kernels stage x with 16-byte loads
    if (type_id != FMX_TYPE_F32 && (reinterpret_cast<uintptr_t>(x) & 15u)) return FMX_ERR_INVALID_ARGUMENT;
    // Q6_K blocks: scales and d are read as 2-byte words
    if (type_id == FMX_TYPE_Q6_K && (reinterpret_cast<uintptr_t>(packed) & 1u)) return FMX_ERR_INVALID_ARGUMENT;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (type_id) {
    case FMX_TYPE_F32:
        if (in_dim <= 16384)
            hipLaunchKernelGGL(matvec_f32_kernel<true>, dim3(div_up(out_dim, kThreads / 16)), dim3(kThreads),
                               static_cast<size_t>(in_dim) * sizeof(float), s, static_cast<const float *>(packed), x, y,
                               out_dim, in_dim);
        else
            hipLaunchKernelGGL(matvec_f32_kernel<false>, dim3(div_up(out_dim, kThreads / 16)), dim3(kThreads), 0, s,
                               static_cast<const float *>(packed), x, y, out_dim, in_dim);
        FMX_LAUNCH_CHECK();
        return FMX_OK;
    case FMX_TYPE_Q4_0: return launch_matvec<Q40, 2>(g, packed, x, y, s);
    case FMX_TYPE_Q8_0: return launch_matvec<Q80, 2>(g, packed, x, y, s);
    case FMX_TYPE_Q4_K: return launch_matvec<Q4K, 1>(g, packed, x, y, s);
    case FMX_TYPE_Q6_K: {
        // one lane group per row leaves the device short of wavefronts below
        // 32768 rows: split each row's blocks over 4 (fewer than 8192 rows)
        // or 2 groups
        const bool four = out_dim < 8192;
        const uint32_t rows_per_wg = four ? kThreads / 64 : kThreads / 32;
        const size_t dots = q6_split_dots_floats(rows_per_wg, g.blocks) * sizeof(float);
        const size_t with_x = dots + static_cast<size_t>(g.blocks) * kQ6XStride * sizeof(float);
        if (out_dim < 32768 && g.blocks >= 8 && dots <= 64 * 1024) {
            auto k = four ? matvec_q6_k_split_kernel<4, false>
                          : with_x <= kMatvecMaxLds ? matvec_q6_k_split_kernel<2, true>
                                                    : matvec_q6_k_split_kernel<2, false>;
            const size_t lds = !four && with_x <= kMatvecMaxLds ? with_x : dots;
            if (int rc = allow_lds(reinterpret_cast<const void *>(k), lds)) return rc;
            hipLaunchKernelGGL(k, dim3(div_up(out_dim, rows_per_wg)), dim3(kThreads), lds, s,
                               static_cast<const uint8_t *>(packed), x, y, out_dim, g.blocks);
            FMX_LAUNCH_CHECK();
            return FMX_OK;
        }
        hipLaunchKernelGGL(matvec_q6_k_kernel, dim3(div_up(out_dim, kThreads / 16)), dim3(kThreads), 0, s,
                           static_cast<const uint8_t *>(packed), x, y, out_dim, g.blocks);
        FMX_LAUNCH_CHECK();
        return FMX_OK;
    }
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}
