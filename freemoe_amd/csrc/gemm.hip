// gemm.hip — the batched product gemm_quant (kernels.cpp:289-345) on gfx950.
//
// y[t][o] = dot(dequantize_row(W row o), x_t) for every token t: the row is
// dequantised exactly (dequantize_row, quant.cpp:163-318) and each dot is the
// reference's dot_avx2 (kernels.cpp:206-223): two 8-lane FMA chains (k mod 16
// < 8 and >= 8), their sum, the 8-lane tree, then an FMA tail. Every output is
// the reference's bit for bit.
//
// Tiles. A workgroup (16 lane groups of 16) owns 32 weight rows x 32 tokens.
// Lane c of a group runs chain k = c (mod 16) for 8 rows x 8 tokens at once,
// so each LDS value it reads feeds several chains; the K loop stages 256
// columns at a time: the 32 rows dequantised from their raw blocks, the 32
// tokens' inputs (requested a stage ahead). Chains persist in registers
// across the stages, so the K order of every chain is the reference's. The
// group's rows are gr, gr + 4, ..., gr + 28 (gr = group % 4) and LDS rows are
// 272 floats apart, so the four groups of a wavefront read 16 distinct banks
// each; they share tokens (group / 4), which the LDS broadcasts. Every
// token's inputs are read once per 32 rows, the largest traffic of the
// kernel.
#include "fmx_internal.hpp"

namespace fmx {

namespace {

constexpr uint32_t kGmThreads = 256;
constexpr uint32_t kGmRows = 32;     // weight rows per workgroup
constexpr uint32_t kGmTokens = 32;   // tokens per workgroup
constexpr uint32_t kGmK = 256;       // columns per stage (a multiple of every block size)
constexpr uint32_t kGmWStride = 272; // LDS floats between weight rows
constexpr uint32_t kGmMR = 8, kGmMT = 8;

// Elements 16 s .. 16 s + 15 of one raw block (dequantize_block): the same
// expressions as the library's block dequantiser, so the values are exact.
__device__ inline void dequant_segment(uint32_t type_id, const uint8_t *blk, uint32_t s, float *o) {
    switch (type_id) {
    case FMX_TYPE_Q4_0: {
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        // s = 0: low nibbles of bytes 0..15 (elements 0..15); s = 1: high
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t b = blk[2 + j];
            o[j] = d * static_cast<float>(static_cast<int>(s ? b >> 4 : b & 0x0Fu) - 8);
        }
        break;
    }
    case FMX_TYPE_Q8_0: {
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
#pragma unroll
        for (int j = 0; j < 16; ++j) o[j] = d * static_cast<float>(static_cast<int8_t>(blk[2 + 16 * s + j]));
        break;
    }
    case FMX_TYPE_Q4_K: {
        // 64-element group g = s / 4: elements 64 g + 0..31 are the low
        // nibbles of qs[32 g + 0..31] (sub-block 2 g), 64 g + 32..63 the high
        // nibbles (sub-block 2 g + 1); segment s covers 16 of them
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
        const uint32_t g = s >> 2, hi = (s >> 1) & 1, part = s & 1;
        uint32_t sc, m;
        k4_scale_min(static_cast<int>(2 * g + hi), blk + 4, sc, m);
        const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(m);
        const uint8_t *qs = blk + 16 + 32 * g + 16 * part;
#pragma unroll
        for (int j = 0; j < 16; ++j) o[j] = d1 * static_cast<float>(hi ? qs[j] >> 4 : qs[j] & 0x0Fu) - m1;
        break;
    }
    case FMX_TYPE_Q6_K: {
        // segment s: half n = s / 8, quarter qt = (s / 2) % 4 of the half,
        // l = 16 (s % 2) + j; sub-block scale 8 n + s % 2 + 2 qt
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const uint32_t n = s >> 3, qt = (s >> 1) & 3, l0 = 16 * (s & 1);
        const float sc = static_cast<float>(static_cast<int8_t>(blk[192 + 8 * n + (s & 1) + 2 * qt]));
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t l = l0 + j;
            const uint32_t ql = blk[64 * n + l + 32 * (qt & 1)], qh = blk[128 + 32 * n + l];
            const int q = static_cast<int>((qt >= 2 ? ql >> 4 : ql & 0x0Fu) | (((qh >> (2 * qt)) & 3u) << 4)) - 32;
            o[j] = d * sc * static_cast<float>(q);
        }
        break;
    }
    default:
        break;
    }
}

// grid: (ceil(out_dim / 32), ceil(tokens / 32)).
__global__ __launch_bounds__(kGmThreads) void gemm_quant_kernel(uint32_t type_id, const uint8_t *__restrict__ w,
                                                                const float *__restrict__ x, float *__restrict__ y,
                                                                uint32_t tokens, uint32_t out_dim, uint32_t in_dim,
                                                                uint32_t block_size, uint32_t block_bytes) {
    __shared__ float wl[kGmRows * kGmWStride];
    __shared__ float xl[kGmTokens * kGmK];
    const uint32_t tid = threadIdx.x, c = tid & 15, grp = tid >> 4;
    const uint32_t gr = grp & 3, gt = grp >> 2;
    const uint32_t o0 = blockIdx.x * kGmRows, t0 = blockIdx.y * kGmTokens;
    const uint64_t row_bytes = static_cast<uint64_t>(in_dim / block_size) * block_bytes;
    const uint32_t n16 = in_dim / 16 * 16;
    float acc[kGmMR][kGmMT];
#pragma unroll
    for (uint32_t i = 0; i < kGmMR; ++i)
#pragma unroll
        for (uint32_t j = 0; j < kGmMT; ++j) acc[i][j] = 0.0f;
    // thread tid's column of the 32 tokens' inputs for the stage at k0 (all
    // 32 loads requested before any is used)
    static_assert(kGmThreads == kGmK, "one staged input column per thread");
    float xs[kGmTokens];
    auto load_x = [&](uint32_t k0) {
        const uint32_t k = k0 + tid < in_dim ? k0 + tid : in_dim - 1;
#pragma unroll
        for (uint32_t p = 0; p < kGmTokens; ++p) {
            const uint32_t t = t0 + p < tokens ? t0 + p : tokens - 1;
            xs[p] = x[static_cast<uint64_t>(t) * in_dim + k];
        }
    };
    load_x(0);
    for (uint32_t k0 = 0; k0 < in_dim; k0 += kGmK) {
        const uint32_t nk = in_dim - k0 < kGmK ? in_dim - k0 : kGmK;
        __syncthreads();
        // weights: thread -> (rows tid / 16 and tid / 16 + 16, 16-column
        // segment tid % 16)
#pragma unroll
        for (uint32_t half = 0; half < kGmRows / 16; ++half) {
            const uint32_t r = (tid >> 4) + 16 * half, seg = tid & 15, col = 16 * seg;
            const uint32_t o = o0 + r < out_dim ? o0 + r : out_dim - 1;
            float v[16];
            if (col < nk) {
                const uint8_t *row = w + static_cast<uint64_t>(o) * row_bytes;
                if (type_id == FMX_TYPE_F32) {
                    const uint32_t n = nk - col < 16 ? nk - col : 16;
                    for (uint32_t j = 0; j < 16; ++j) {
                        float f = 0.0f;
                        if (j < n) memcpy(&f, row + 4ull * (k0 + col + j), 4);
                        v[j] = f;
                    }
                } else {
                    const uint32_t e = k0 + col; // first element; blocks hold 32 or 256
                    const uint8_t *blk = row + static_cast<uint64_t>(e / block_size) * block_bytes;
                    dequant_segment(type_id, blk, (e % block_size) / 16, v);
                }
#pragma unroll
                for (uint32_t j = 0; j < 16; ++j) wl[r * kGmWStride + col + j] = v[j];
            }
        }
        // inputs: column tid of the 32 tokens, requested one stage ahead
        if (tid < nk) {
#pragma unroll
            for (uint32_t p = 0; p < kGmTokens; ++p) xl[p * kGmK + tid] = xs[p];
        }
        __syncthreads();
        if (k0 + kGmK < in_dim) load_x(k0 + kGmK);
        // the chains: k = k0 + 16 m + c over whole 16-groups below n16
        const uint32_t m_end = (n16 > k0 ? (n16 - k0 < nk ? n16 - k0 : nk) : 0) / 16;
        for (uint32_t m = 0; m < m_end; ++m) {
            const uint32_t k = 16 * m + c;
            float wv[kGmMR], xv[kGmMT];
#pragma unroll
            for (uint32_t i = 0; i < kGmMR; ++i) wv[i] = wl[(gr + 4 * i) * kGmWStride + k];
#pragma unroll
            for (uint32_t j = 0; j < kGmMT; ++j) xv[j] = xl[(gt * kGmMT + j) * kGmK + k];
#pragma unroll
            for (uint32_t i = 0; i < kGmMR; ++i)
#pragma unroll
                for (uint32_t j = 0; j < kGmMT; ++j) acc[i][j] = fma_rn(wv[i], xv[j], acc[i][j]);
        }
        if (k0 + nk == in_dim && in_dim - n16 >= 8 && c < 8) {
            // dot_avx2's 8-wide step after the 16-wide loop (chain 0 only)
            const uint32_t k = n16 - k0 + c;
#pragma unroll
            for (uint32_t i = 0; i < kGmMR; ++i)
#pragma unroll
                for (uint32_t j = 0; j < kGmMT; ++j)
                    acc[i][j] = fma_rn(wl[(gr + 4 * i) * kGmWStride + k], xl[(gt * kGmMT + j) * kGmK + k], acc[i][j]);
        }
        if (k0 + nk == in_dim) {
            // acc0 + acc1, the 8-lane tree, the scalar tail; then the stores
            const uint32_t kt = in_dim - n16 >= 8 ? n16 + 8 : n16;
#pragma unroll
            for (uint32_t i = 0; i < kGmMR; ++i) {
#pragma unroll
                for (uint32_t j = 0; j < kGmMT; ++j) {
                    const float s = acc[i][j] + lane_xor<8>(acc[i][j]);
                    float total = hsum8_lanes(s);
                    for (uint32_t k = kt; k < in_dim; ++k)
                        total = fma_rn(wl[(gr + 4 * i) * kGmWStride + k - k0], xl[(gt * kGmMT + j) * kGmK + k - k0],
                                       total);
                    acc[i][j] = total;
                }
            }
        }
    }
    if (c != 0) return;
#pragma unroll
    for (uint32_t i = 0; i < kGmMR; ++i) {
        const uint32_t o = o0 + gr + 4 * i;
#pragma unroll
        for (uint32_t j = 0; j < kGmMT; ++j) {
            const uint32_t t = t0 + gt * kGmMT + j;
            if (o < out_dim && t < tokens) y[static_cast<uint64_t>(t) * out_dim + o] = acc[i][j];
        }
    }
}

} // namespace
} // namespace fmx

using namespace fmx;

extern "C" int fmx_gemm_quant(uint32_t type_id, const void *weights, const float *x, float *y, uint32_t tokens,
                              uint32_t out_dim, uint32_t in_dim, void *stream) {
    if (int rc = fault_gate()) return rc;
    if (tokens == 0 || out_dim == 0 || in_dim == 0) return FMX_OK;
    if (!weights || !x || !y) return FMX_ERR_INVALID_ARGUMENT;
    uint32_t bs = 0, bb = 0;
    if (int rc = raw_geometry(type_id, &bs, &bb)) return rc;
    if (in_dim % bs) return FMX_ERR_SHAPE_MISMATCH;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(gemm_quant_kernel, dim3(div_up(out_dim, kGmRows), div_up(tokens, kGmTokens)),
                       dim3(kGmThreads), 0, s, type_id, static_cast<const uint8_t *>(weights), x, y, tokens,
                       out_dim, in_dim, bs, bb);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}
