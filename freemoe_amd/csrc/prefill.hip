// prefill.hip — the MoE block over a batch of tokens at once (prefill).
//
// The reference has no batched MoE path: it runs Engine::forward_token per
// prompt token (engine.cpp:1870, 2395-2399). Here the batch is
//   route (bit-identical to the per-token routing, moe.hip)
//   -> bucket (per-expert token lists and row tiles, bucket.hip)
//   -> gather: h rows of each (token, expert) pair into an expert-contiguous
//      bf16 matrix X [pairs x hidden]
//   -> gate/up grouped GEMM on bf16 MFMA, weights dequantised from their
//      packed blocks into LDS, SwiGLU in the epilogue -> act [pairs x ffn] bf16
//   -> down grouped GEMM -> D [pairs x hidden] f32
//   -> combine per token in rank order plus the residual.
//
// K order. The packed expert slots (quant.hip) keep each lane's 16-byte slice
// of a chunk together, so a chunk's elements are stored permuted. A GEMM
// contracts over K in any order, so instead of re-permuting the weights the
// activations are written in the same permuted order ("packed positions"):
// one packed slot serves both decode and prefill, and every weight byte is
// read from HBM in 16-byte runs straight into the dequantiser.
//
// Tiles. A workgroup (8 wavefronts) owns one row tile of one expert (up to 256
// token-expert pairs, 32 per wavefront) and 128 weight rows (gate/up: 64 gate
// rows and the same 64 up rows, so SwiGLU pairs meet in one lane). It walks K
// in steps of 128 packed positions: the weight slices of step s+1 are in
// flight while step s is dequantised into one of two LDS buffers and fed to
// v_mfma_f32_32x32x16_bf16 with the activations read straight from memory.
#include "bucket.hpp"
#include "fmx_internal.hpp"
#include "moe.hpp"
#include "prefill.hpp"

namespace fmx {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kGemmThreads = 512;            // 8 wavefronts
constexpr uint32_t kTileN = 128;                  // weight rows per workgroup
constexpr uint32_t kStepK = 128;                  // packed K positions per step
constexpr uint32_t kWStride = kStepK + 8;         // bf16 per LDS weight row (16-byte pad)
constexpr uint32_t kWBufElems = kTileN * kWStride;

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const __bf16 x = static_cast<__bf16>(a), y = static_cast<__bf16>(b);
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, x)) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, y)) << 16);
}

// ------------------------------------------------------------ block types --
// kChunkK: elements per packed chunk. kSlices: 16-byte lane slices a step of
// kStepK positions covers. elem(p) / pos(e): element held at packed position p
// of a chunk, and its inverse. Slice: a slice's raw bytes plus its scales;
// dequant() writes the slice's values, in position order, as bf16 pairs.

struct GQ80 {
    static constexpr uint32_t kType = FMX_TYPE_Q8_0;
    static constexpr uint32_t kChunkK = 128;
    static constexpr uint32_t kSlices = 8;                 // a step is a whole chunk
    static constexpr uint32_t kValsPerSlice = 16;
    // position p = 16 l + 4 j + k holds element 32 j + 8 k + l
    __host__ __device__ static uint32_t elem(uint32_t p) { return 32 * ((p & 15) >> 2) + 8 * (p & 3) + (p >> 4); }
    __host__ __device__ static uint32_t pos(uint32_t e) { return 16 * (e & 7) + 4 * (e >> 5) + ((e & 31) >> 3); }
    struct Slice {
        uint4 q;
        uint2 d; // the chunk's four block scales
    };
    // Slice s (0..7) of chunk c of row r.
    __device__ static Slice load(const uint8_t *packed, const PackedGeometry &g, uint32_t r, uint32_t c,
                                 uint32_t s) {
        Slice v;
        v.q = ld16(packed + g.scale_bytes + ((static_cast<uint64_t>(r) * g.chunks + c) * 8 + s) * 16);
        v.d = ld8(packed + static_cast<uint64_t>(r) * g.blocks_padded * 2 + static_cast<uint64_t>(c) * 8);
        return v;
    }
    __device__ static void dequant(const Slice &v, uint32_t *out) {
        const uint32_t w[4] = {v.q.x, v.q.y, v.q.z, v.q.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float d = half_bits_to_float(j & 2 ? ((j & 1) ? v.d.y >> 16 : v.d.y & 0xFFFFu)
                                                     : ((j & 1) ? v.d.x >> 16 : v.d.x & 0xFFFFu));
            const float q0 = static_cast<float>(static_cast<int32_t>(w[j] << 24) >> 24);
            const float q1 = static_cast<float>(static_cast<int32_t>(w[j] << 16) >> 24);
            const float q2 = static_cast<float>(static_cast<int32_t>(w[j] << 8) >> 24);
            const float q3 = static_cast<float>(static_cast<int32_t>(w[j]) >> 24);
            out[2 * j] = pack_bf16x2(d * q0, d * q1);
            out[2 * j + 1] = pack_bf16x2(d * q2, d * q3);
        }
    }
};

struct GQ40 {
    static constexpr uint32_t kType = FMX_TYPE_Q4_0;
    static constexpr uint32_t kChunkK = 256;
    static constexpr uint32_t kSlices = 4;                 // a step is half a chunk
    static constexpr uint32_t kValsPerSlice = 32;
    // position p = 32 l + 4 j + 2 which + nib holds element 32 j + 16 nib + 8 which + l
    __host__ __device__ static uint32_t elem(uint32_t p) {
        const uint32_t l = p >> 5, q = p & 31, nib = q & 1, which = (q >> 1) & 1, j = q >> 2;
        return 32 * j + 16 * nib + 8 * which + l;
    }
    __host__ __device__ static uint32_t pos(uint32_t e) {
        const uint32_t j = e >> 5, r = e & 31, nib = r >> 4, which = (r >> 3) & 1, l = r & 7;
        return 32 * l + 4 * j + 2 * which + nib;
    }
    struct Slice {
        uint4 q;
        uint4 d; // the chunk's eight block scales
    };
    __device__ static Slice load(const uint8_t *packed, const PackedGeometry &g, uint32_t r, uint32_t c,
                                 uint32_t s) {
        Slice v;
        v.q = ld16(packed + g.scale_bytes + ((static_cast<uint64_t>(r) * g.chunks + c) * 8 + s) * 16);
        v.d = ld16(packed + static_cast<uint64_t>(r) * g.blocks_padded * 2 + static_cast<uint64_t>(c) * 16);
        return v;
    }
    __device__ static void dequant(const Slice &v, uint32_t *out) {
        const uint32_t w[4] = {v.q.x, v.q.y, v.q.z, v.q.w};
        const uint32_t dw[4] = {v.d.x, v.d.y, v.d.z, v.d.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // dword i holds bytes b = 4i..4i+3: blocks 2i (bytes 4i, 4i+1) and 2i+1
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float d = half_bits_to_float(h ? dw[i] >> 16 : dw[i] & 0xFFFFu);
#pragma unroll
                for (int bb = 0; bb < 2; ++bb) {
                    const uint32_t byte = (w[i] >> (8 * (2 * h + bb))) & 0xFFu;
                    const float lo = d * static_cast<float>(static_cast<int32_t>(byte & 15u) - 8);
                    const float hi = d * static_cast<float>(static_cast<int32_t>(byte >> 4) - 8);
                    out[4 * i + 2 * h + bb] = pack_bf16x2(lo, hi);
                }
            }
        }
    }
};

struct GQ4K {
    static constexpr uint32_t kType = FMX_TYPE_Q4_K;
    static constexpr uint32_t kChunkK = 256;
    static constexpr uint32_t kSlices = 4;
    static constexpr uint32_t kValsPerSlice = 32;
    // position p = 32 l + 8 g + 2 k + nib holds element 64 g + 32 nib + 8 k + l
    __host__ __device__ static uint32_t elem(uint32_t p) {
        const uint32_t l = p >> 5, q = p & 31, nib = q & 1, k = (q >> 1) & 3, g = q >> 3;
        return 64 * g + 32 * nib + 8 * k + l;
    }
    __host__ __device__ static uint32_t pos(uint32_t e) {
        const uint32_t g = e >> 6, r = e & 63, nib = r >> 5, k = (r >> 3) & 3, l = r & 7;
        return 32 * l + 8 * g + 2 * k + nib;
    }
    struct Slice {
        uint4 q;
        uint4 h; // the super-block header: d, dmin, 12 bytes of 6-bit scales and mins
    };
    __device__ static Slice load(const uint8_t *packed, const PackedGeometry &g, uint32_t r, uint32_t c,
                                 uint32_t s) {
        Slice v;
        v.q = ld16(packed + g.scale_bytes + ((static_cast<uint64_t>(r) * g.chunks + c) * 8 + s) * 16);
        v.h = ld16(packed + (static_cast<uint64_t>(r) * g.chunks + c) * 16);
        return v;
    }
    __device__ static void dequant(const Slice &v, uint32_t *out) {
        uint8_t hdr[16];
        memcpy(hdr, &v.h, 16);
        const float d = half_bits_to_float(hdr[0] | (hdr[1] << 8));
        const float dmin = half_bits_to_float(hdr[2] | (hdr[3] << 8));
        const uint32_t w[4] = {v.q.x, v.q.y, v.q.z, v.q.w};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            uint32_t sc1, m1, sc2, m2;
            k4_scale_min(2 * g, hdr + 4, sc1, m1);
            k4_scale_min(2 * g + 1, hdr + 4, sc2, m2);
            // dequantize_block's values: (d * sc) * q - dmin * m (quant.cpp:297-318)
            const float d1 = d * static_cast<float>(sc1), mm1 = dmin * static_cast<float>(m1);
            const float d2 = d * static_cast<float>(sc2), mm2 = dmin * static_cast<float>(m2);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t byte = (w[g] >> (8 * k)) & 0xFFu;
                out[4 * g + k] = pack_bf16x2(d1 * static_cast<float>(byte & 15u) - mm1,
                                             d2 * static_cast<float>(byte >> 4) - mm2);
            }
        }
    }
};

// Weight rows of a tile: the LDS row lr (0..127) reads matrix `w0` row
// base0 + lr for lr < split, else matrix `w1` row base1 + lr - split.
struct TileRows {
    const uint8_t *w0, *w1;
    uint32_t base0, base1, split;
};

// One K step of the weight tile: thread t loads slices of LDS row t / 4.
template <class T>
struct WeightStep {
    static constexpr uint32_t kPerThread = T::kSlices * kTileN / kGemmThreads; // 2 (Q8_0) or 1 (Q4)
    typename T::Slice s[kPerThread];

    __device__ void load(const TileRows &tr, const PackedGeometry &g, uint32_t step, uint32_t tid) {
        const uint32_t lr = tid >> 2;
        const uint8_t *w = lr < tr.split ? tr.w0 : tr.w1;
        const uint32_t r = lr < tr.split ? tr.base0 + lr : tr.base1 + lr - tr.split;
        const uint32_t c = step * kStepK / T::kChunkK;
        const uint32_t s0 = (step * kStepK % T::kChunkK) / (T::kChunkK / 8); // first slice of the step
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) s[i] = T::load(w, g, r, c, s0 + (tid & 3) * kPerThread + i);
    }

    // Dequantised values into LDS row tid / 4 at the step's positions of the slices.
    __device__ void store(__bf16 *wbuf, uint32_t tid) const {
        const uint32_t lr = tid >> 2;
#pragma unroll
        for (uint32_t i = 0; i < kPerThread; ++i) {
            uint32_t v[T::kValsPerSlice / 2];
            T::dequant(s[i], v);
            const uint32_t p0 = ((tid & 3) * kPerThread + i) * T::kValsPerSlice;
            uint4 *dst = reinterpret_cast<uint4 *>(wbuf + lr * kWStride + p0);
#pragma unroll
            for (uint32_t q = 0; q < T::kValsPerSlice / 8; ++q)
                dst[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        }
    }
};

// Activation fragments of one K step for this lane: row `xrow`, positions
// k0 + 16 kk + 8 (lane / 32) .. +8, kk = 0..7.
struct XStep {
    bf16x8 f[kStepK / 16];
    __device__ void load(const __bf16 *x, uint64_t ld, uint32_t xrow, uint32_t k0, uint32_t lane) {
        const __bf16 *base = x + static_cast<uint64_t>(xrow) * ld + k0 + 8 * (lane >> 5);
#pragma unroll
        for (uint32_t kk = 0; kk < kStepK / 16; ++kk) {
            const uint4 v = ld16(base + 16 * kk);
            f[kk] = __builtin_bit_cast(bf16x8, v);
        }
    }
};

// The shared main loop: acc[nb] (32 x 32 blocks nb = 0..3 over the tile's 128
// weight rows) += X[rows of this wavefront] . W^T over `steps` K steps.
template <class T>
__device__ void gemm_tile(const TileRows &tr, const PackedGeometry &g, const __bf16 *x, uint64_t ldx,
                          uint32_t xrow, bool active, uint32_t steps, __bf16 *wlds, f32x16 (&acc)[4]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    WeightStep<T> ws;
    XStep xs[2];
    ws.load(tr, g, 0, tid);
    if (active) xs[0].load(x, ldx, xrow, 0, lane);
    for (uint32_t st = 0; st < steps; ++st) {
        __bf16 *wbuf = wlds + (st & 1) * kWBufElems;
        ws.store(wbuf, tid);
        if (st + 1 < steps) ws.load(tr, g, st + 1, tid);
        __syncthreads();
        if (active) {
            XStep &cur = xs[st & 1];
            if (st + 1 < steps) xs[(st + 1) & 1].load(x, ldx, xrow, (st + 1) * kStepK, lane);
#pragma unroll
            for (uint32_t kk = 0; kk < kStepK / 16; ++kk) {
#pragma unroll
                for (uint32_t nb = 0; nb < 4; ++nb) {
                    const uint4 bv = *reinterpret_cast<const uint4 *>(
                        wbuf + (32 * nb + (lane & 31)) * kWStride + 16 * kk + 8 * (lane >> 5));
                    acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.f[kk], __builtin_bit_cast(bf16x8, bv),
                                                                     acc[nb], 0, 0, 0);
                }
            }
        }
    }
}

// Row tile `mt` of the bucketed pairs: (expert, first row, rows); false when
// mt is past the tiles the bucketing produced (or a tile is malformed).
__device__ inline bool row_tile(const uint32_t *tiles, uint32_t mt, uint32_t experts, uint32_t pairs, uint32_t &e,
                                uint32_t &row0, uint32_t &rows) {
    if (mt >= tiles[0]) return false;
    e = tiles[1 + 3 * mt];
    row0 = tiles[2 + 3 * mt];
    rows = tiles[3 + 3 * mt];
    return e < experts && rows > 0 && rows <= 32 * (kGemmThreads / 64) && row0 <= pairs && rows <= pairs - row0;
}

// ------------------------------------------------------------------ kernels --

// X[s][p] = bf16(h[token_list[s]][element at packed position p]), 8 positions
// per thread. grid: (ceil(hidden / 8 / 256), pairs).
template <class T>
__global__ __launch_bounds__(256) void gather_kernel(const float *__restrict__ h, uint32_t hidden, uint32_t tokens,
                                                     const uint32_t *__restrict__ token_list,
                                                     __bf16 *__restrict__ x) {
    const uint32_t s = blockIdx.y;
    const uint32_t p0 = (blockIdx.x * 256 + threadIdx.x) * 8;
    if (p0 >= hidden) return;
    const uint32_t tok = token_list[s];
    const float *src = h + static_cast<uint64_t>(tok < tokens ? tok : tokens - 1) * hidden;
    const uint32_t cbase = p0 / T::kChunkK * T::kChunkK, pc = p0 % T::kChunkK;
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        v[i] = pack_bf16x2(src[cbase + T::elem(pc + 2 * i)], src[cbase + T::elem(pc + 2 * i + 1)]);
    *reinterpret_cast<uint4 *>(x + static_cast<uint64_t>(s) * hidden + p0) = make_uint4(v[0], v[1], v[2], v[3]);
}

// Gate and up of 64 ffn rows (tile nt) for one row tile, SwiGLU, and the
// activations written as bf16 in the down projection's packed K order.
// grid: (ffn / 64, max row tiles).
template <class T, class TD>
__global__ __launch_bounds__(kGemmThreads) void gate_up_gemm_kernel(ExpertArgs a, const uint32_t *__restrict__ tiles,
                                                                     uint32_t pairs, const __bf16 *__restrict__ x,
                                                                     __bf16 *__restrict__ act) {
    extern __shared__ __align__(16) __bf16 wlds[];
    uint32_t e, row0, rows;
    if (!row_tile(tiles, blockIdx.y, a.experts, pairs, e, row0, rows)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n0 = blockIdx.x * 64;
    TileRows tr{static_cast<const uint8_t *>(a.gate[e]), static_cast<const uint8_t *>(a.up[e]), n0, n0, 64};
    const uint32_t m_local = 32 * wave + (lane & 31);
    const bool active = 32 * wave < rows;
    const uint32_t xrow = row0 + (m_local < rows ? m_local : rows - 1);
    f32x16 acc[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;
    gemm_tile<T>(tr, a.gu, x, a.hidden, xrow, active, a.hidden / kStepK, wlds, acc);
    if (!active) return;
    const uint32_t F = a.ffn;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t m = 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= rows) continue;
        __bf16 *dst = act + static_cast<uint64_t>(row0 + m) * F;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const uint32_t n = n0 + 32 * nb + (lane & 31);
            const float gv = acc[nb][r], uv = acc[nb + 2][r];
            const float sv = gv / (1.0f + expf(-gv)) * uv;
            dst[n / TD::kChunkK * TD::kChunkK + TD::pos(n % TD::kChunkK)] = static_cast<__bf16>(sv);
        }
    }
}

// Down rows [128 nt, +128) for one row tile into D [pairs x hidden] f32.
// grid: (hidden / 128, max row tiles).
template <class T>
__global__ __launch_bounds__(kGemmThreads) void down_gemm_kernel(ExpertArgs a, const uint32_t *__restrict__ tiles,
                                                                  uint32_t pairs, const __bf16 *__restrict__ act,
                                                                  float *__restrict__ dn) {
    extern __shared__ __align__(16) __bf16 wlds[];
    uint32_t e, row0, rows;
    if (!row_tile(tiles, blockIdx.y, a.experts, pairs, e, row0, rows)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n0 = blockIdx.x * kTileN;
    const uint8_t *w = static_cast<const uint8_t *>(a.down[e]);
    TileRows tr{w, w, n0, n0, kTileN};
    const uint32_t m_local = 32 * wave + (lane & 31);
    const bool active = 32 * wave < rows;
    const uint32_t xrow = row0 + (m_local < rows ? m_local : rows - 1);
    f32x16 acc[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;
    gemm_tile<T>(tr, a.dn, act, a.ffn, xrow, active, a.ffn / kStepK, wlds, acc);
    if (!active) return;
    const uint32_t H = a.hidden;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t m = 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= rows) continue;
        float *dst = dn + static_cast<uint64_t>(row0 + m) * H + n0 + (lane & 31);
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) dst[32 * nb] = acc[nb][r];
    }
}

// out[t] = x[t] + ((0 + w_0 D_0) + w_1 D_1 ...) in rank order (engine.cpp:1517,
// 1770, 813-816). grid: (ceil(hidden / 256), tokens).
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ x, const float *__restrict__ dn,
                                                      const uint32_t *__restrict__ slot_of,
                                                      const float *__restrict__ w, uint32_t hidden, uint32_t K,
                                                      float *__restrict__ out) {
    const uint32_t t = blockIdx.y, j = blockIdx.x * 256 + threadIdx.x;
    if (j >= hidden) return;
    float ffn = 0.0f;
    for (uint32_t r = 0; r < K; ++r) {
        const uint64_t i = static_cast<uint64_t>(t) * K + r;
        ffn = ffn + w[i] * dn[static_cast<uint64_t>(slot_of[i]) * hidden + j];
    }
    out[static_cast<uint64_t>(t) * hidden + j] = x[static_cast<uint64_t>(t) * hidden + j] + ffn;
}

// ---------------------------------------------------------------- launchers --

template <class T>
int launch_gather(const float *h, uint32_t hidden, uint32_t tokens, const uint32_t *token_list, uint32_t pairs,
                  __bf16 *x, hipStream_t s) {
    hipLaunchKernelGGL(gather_kernel<T>, dim3(div_up(hidden / 8, 256), pairs), dim3(256), 0, s, h, hidden, tokens,
                       token_list, x);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

template <class T, class TD>
int launch_gemms(const ExpertArgs &a, const PrefillBuffers &b, uint32_t max_tiles, hipStream_t s) {
    const size_t lds = 2ull * kWBufElems * sizeof(__bf16);
    auto gu = gate_up_gemm_kernel<T, TD>;
    auto dn = down_gemm_kernel<TD>;
    if (int rc = allow_lds(reinterpret_cast<const void *>(gu), lds)) return rc;
    if (int rc = allow_lds(reinterpret_cast<const void *>(dn), lds)) return rc;
    if (b.pairs == 0) return FMX_OK;
    if (int rc = launch_gather<T>(b.h, a.hidden, b.tokens, b.token_list, b.pairs, b.x, s)) return rc;
    hipLaunchKernelGGL(gu, dim3(a.ffn / 64, max_tiles), dim3(kGemmThreads), lds, s, a, b.tiles, b.pairs, b.x,
                       b.act);
    FMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dn, dim3(a.hidden / kTileN, max_tiles), dim3(kGemmThreads), lds, s, a, b.tiles, b.pairs,
                       b.act, b.dn);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

uint32_t chunk_k_of(uint32_t type) {
    switch (type) {
    case FMX_TYPE_Q8_0: return GQ80::kChunkK;
    case FMX_TYPE_Q4_0: return GQ40::kChunkK;
    case FMX_TYPE_Q4_K: return GQ4K::kChunkK;
    }
    return 0;
}

} // namespace

bool prefill_gemm_supported(const ExpertArgs &a) {
    const uint32_t ck_gu = chunk_k_of(a.type_gu), ck_dn = chunk_k_of(a.type_dn);
    if (ck_gu == 0 || ck_dn == 0) return false;
    return a.hidden % ck_gu == 0 && a.hidden % kTileN == 0 && a.ffn % ck_dn == 0 && a.ffn % 64 == 0 &&
           a.hidden % kStepK == 0 && a.ffn % kStepK == 0;
}

int launch_prefill_experts(const ExpertArgs &a, const PrefillBuffers &b, uint32_t max_tiles, hipStream_t s) {
    if (!prefill_gemm_supported(a)) return FMX_ERR_SHAPE_MISMATCH;
    switch (a.type_gu) {
    case FMX_TYPE_Q8_0:
        switch (a.type_dn) {
        case FMX_TYPE_Q8_0: return launch_gemms<GQ80, GQ80>(a, b, max_tiles, s);
        case FMX_TYPE_Q4_0: return launch_gemms<GQ80, GQ40>(a, b, max_tiles, s);
        case FMX_TYPE_Q4_K: return launch_gemms<GQ80, GQ4K>(a, b, max_tiles, s);
        }
        break;
    case FMX_TYPE_Q4_0:
        switch (a.type_dn) {
        case FMX_TYPE_Q8_0: return launch_gemms<GQ40, GQ80>(a, b, max_tiles, s);
        case FMX_TYPE_Q4_0: return launch_gemms<GQ40, GQ40>(a, b, max_tiles, s);
        case FMX_TYPE_Q4_K: return launch_gemms<GQ40, GQ4K>(a, b, max_tiles, s);
        }
        break;
    case FMX_TYPE_Q4_K:
        switch (a.type_dn) {
        case FMX_TYPE_Q8_0: return launch_gemms<GQ4K, GQ80>(a, b, max_tiles, s);
        case FMX_TYPE_Q4_0: return launch_gemms<GQ4K, GQ40>(a, b, max_tiles, s);
        case FMX_TYPE_Q4_K: return launch_gemms<GQ4K, GQ4K>(a, b, max_tiles, s);
        }
        break;
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

int launch_combine(const float *x, const float *dn, const uint32_t *slot_of, const float *w, uint32_t hidden,
                   uint32_t K, uint32_t tokens, float *out, hipStream_t s) {
    hipLaunchKernelGGL(combine_kernel, dim3(div_up(hidden, 256), tokens), dim3(256), 0, s, x, dn, slot_of, w, hidden,
                       K, out);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace fmx
