// attention.hip — one token's decode attention over its cached positions
// (FreeMoe's engine.cpp:1360-1420, the full-context MHA / GQA case) on
// gfx950, for fm::HipBackend::attention.
//
// Per query head h (kv head h / (heads / kv_heads)), over cached positions
// t = 0 .. P-1:
//   s_t   = float(dot(q_h, k_t) * scale), the dot a double sum over the head
//           dimension in index order (a float times a float is exact in
//           double, so every rounding is the engine's);
//   p     = the engine's softmax of s (engine.cpp:378-393): the float
//           maximum m, e_t = exp(double(s_t) - m), their double sum in
//           position order, p_t = float(e_t / sum);
//   out_j = float(sum_t double(p_t) v_t[j]) in position order.
// Only exp is the device's own (the engine calls the host libm's); both are
// within an ulp, so a result can differ in its last bit where a value sits
// on a rounding boundary. A non-finite score (the engine raises
// INTERNAL_ERROR) sets bit 0 of the status word.
//
// One workgroup per query head: the head's scores and exponentials stay in
// LDS (positions <= kMaxPositions), one lane adds the exponentials in order,
// and head_dim lanes run the value sums.
#include "fmx_internal.hpp"

namespace fmx {

namespace {

constexpr uint32_t kAttnThreads = 256;
constexpr uint32_t kMaxHeadDim = 256;
constexpr uint32_t kMaxPositions = 8192;

__device__ inline float block_max(float v, float *red) {
    for (uint32_t m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
    for (uint32_t i = 1; i < kAttnThreads / 64; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

// grid: heads; LDS: positions floats (scores, then probabilities) and
// positions doubles (exponentials).
__global__ __launch_bounds__(kAttnThreads) void attention_decode_kernel(
    const float *__restrict__ q, const float *__restrict__ kv, uint64_t row_stride, uint32_t v_offset,
    uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t positions, double scale,
    float *__restrict__ out, uint32_t *__restrict__ status) {
    extern __shared__ __align__(16) char lds[];
    __shared__ __align__(16) float qs[kMaxHeadDim];
    __shared__ float red[kAttnThreads / 64];
    __shared__ double sum_s;
    __shared__ int bad_s;
    float *sc = reinterpret_cast<float *>(lds);
    double *ex = reinterpret_cast<double *>(lds + ((positions * 4 + 15) & ~15u));
    const uint32_t tid = threadIdx.x, head = blockIdx.x;
    const uint32_t kvh = head / (heads / kv_heads);
    const uint32_t D = head_dim, D4 = D / 4;
    for (uint32_t j = tid; j < D; j += kAttnThreads) qs[j] = q[static_cast<uint64_t>(head) * D + j];
    if (tid == 0) bad_s = 0;
    __syncthreads();
    // scores: one position per thread, its key read as float4s
    bool bad = false;
    for (uint32_t t = tid; t < positions; t += kAttnThreads) {
        const float4 *k4 = reinterpret_cast<const float4 *>(kv + t * row_stride + static_cast<uint64_t>(kvh) * D);
        double dot = 0.0;
        for (uint32_t j4 = 0; j4 < D4; ++j4) {
            const float4 k = k4[j4];
            dot += static_cast<double>(qs[4 * j4]) * static_cast<double>(k.x);
            dot += static_cast<double>(qs[4 * j4 + 1]) * static_cast<double>(k.y);
            dot += static_cast<double>(qs[4 * j4 + 2]) * static_cast<double>(k.z);
            dot += static_cast<double>(qs[4 * j4 + 3]) * static_cast<double>(k.w);
        }
        const float s = static_cast<float>(dot * scale);
        bad |= !__builtin_isfinite(s);
        sc[t] = s;
    }
    if (__any(bad) && (tid & 63) == 0) bad_s = 1;
    __syncthreads();
    if (bad_s) {
        if (tid == 0) atomicOr(status, STATUS_NONFINITE_SCORE);
        for (uint32_t j = tid; j < D; j += kAttnThreads) out[static_cast<uint64_t>(head) * D + j] = 0.0f;
        return;
    }
    float m = -__builtin_inff();
    for (uint32_t t = tid; t < positions; t += kAttnThreads) m = fmaxf(m, sc[t]);
    m = block_max(m, red);
    const double md = static_cast<double>(m);
    for (uint32_t t = tid; t < positions; t += kAttnThreads) ex[t] = exp(static_cast<double>(sc[t]) - md);
    __syncthreads();
    if (tid == 0) {
        double s = 0.0;
        for (uint32_t t = 0; t < positions; ++t) s += ex[t];
        sum_s = s;
    }
    __syncthreads();
    const double sum = sum_s;
    for (uint32_t t = tid; t < positions; t += kAttnThreads) sc[t] = static_cast<float>(ex[t] / sum);
    __syncthreads();
    // values: one output element per thread, positions in order
    for (uint32_t j = tid; j < D; j += kAttnThreads) {
        const float *v = kv + v_offset + static_cast<uint64_t>(kvh) * D + j;
        double acc = 0.0;
        for (uint32_t t = 0; t < positions; ++t)
            acc += static_cast<double>(sc[t]) * static_cast<double>(v[t * row_stride]);
        out[static_cast<uint64_t>(head) * D + j] = static_cast<float>(acc);
    }
}

__global__ void attention_clear_kernel(uint32_t *status) { *status = 0; }

} // namespace

size_t attention_lds_bytes(uint32_t positions) {
    return ((static_cast<size_t>(positions) * 4 + 15) & ~static_cast<size_t>(15)) + static_cast<size_t>(positions) * 8;
}

int attention_decode(const float *q, const float *kv, uint64_t row_stride, uint32_t v_offset, uint32_t heads,
                     uint32_t kv_heads, uint32_t head_dim, uint32_t positions, double scale, float *out,
                     uint32_t *status, hipStream_t s) {
    if (heads == 0 || kv_heads == 0 || heads % kv_heads || head_dim == 0 || head_dim > kMaxHeadDim ||
        head_dim % 4 || positions == 0 || positions > kMaxPositions || row_stride % 4 || v_offset % 4)
        return FMX_ERR_SHAPE_MISMATCH;
    if (v_offset + static_cast<uint64_t>(kv_heads) * head_dim > row_stride ||
        static_cast<uint64_t>(kv_heads) * head_dim > v_offset)
        return FMX_ERR_SHAPE_MISMATCH;
    const size_t lds = attention_lds_bytes(positions);
    if (int rc = allow_lds(reinterpret_cast<const void *>(attention_decode_kernel), lds)) return rc;
    hipLaunchKernelGGL(attention_clear_kernel, dim3(1), dim3(1), 0, s, status);
    FMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(attention_decode_kernel, dim3(heads), dim3(kAttnThreads), lds, s, q, kv, row_stride, v_offset,
                       heads, kv_heads, head_dim, positions, scale, out, status);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace fmx
