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
// Tiles. A workgroup (8 wavefronts) owns one row tile of one expert (up to 128
// token-expert pairs) and 128 weight rows (gate/up: 64 gate rows and the same
// 64 up rows, arranged so SwiGLU pairs meet in one lane); wavefront w computes
// rows 32 (w / 2) .. +32 against weight rows 64 (w % 2) .. +64. It walks K in
// steps of 128 packed positions with three steps of weight slices and
// activation rows in flight: each step is dequantised (weights) and copied
// (activations) into one of two LDS buffer pairs and fed from LDS to
// v_mfma_f32_32x32x16_bf16.
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
constexpr uint32_t kWBufElems = kTileN * kStepK;  // one LDS weight tile (bf16)

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
            const float q0 = static_cast<float>(static_cast<int8_t>(w[j]));
            const float q1 = static_cast<float>(static_cast<int8_t>(w[j] >> 8));
            const float q2 = static_cast<float>(static_cast<int8_t>(w[j] >> 16));
            const float q3 = static_cast<float>(static_cast<int8_t>(w[j] >> 24));
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

// Weight rows of a tile. Gated (gate/up): LDS row block b = lr / 32 holds
// gate rows (b even) or up rows (b odd) n0 + 32 (b / 2) + lr % 32, so each
// wavefront's two 32-row blocks are the gate and up rows of the same ffn
// rows. Plain (down): LDS row lr is matrix row n0 + lr.
struct TileRows {
    const uint8_t *gate_or_w, *up;
    uint32_t n0;
    bool gated;
    __device__ void at(uint32_t lr, const uint8_t *&w, uint32_t &r) const {
        if (gated) {
            const uint32_t b = lr >> 5;
            w = (b & 1) ? up : gate_or_w;
            r = n0 + 32 * (b >> 1) + (lr & 31);
        } else {
            w = gate_or_w;
            r = n0 + lr;
        }
    }
};

// LDS tiles (weights and activations): 128 rows x 128 bf16 (256 bytes), the
// 16-byte granule g of row r stored at granule g ^ (r & 15), so the 16 rows an
// MFMA operand read or a store touches at once fall in 16 distinct bank groups.
__device__ __forceinline__ uint32_t tile_offset(uint32_t row, uint32_t granule) {
    return row * kStepK + ((granule ^ (row & 15)) << 3);
}

// One K step of the weight tile: thread t loads slices of LDS row t / 4.
template <class T>
struct WeightStep {
    static constexpr uint32_t kPerThread = T::kSlices * kTileN / kGemmThreads; // 2 (Q8_0) or 1 (Q4)
    typename T::Slice s[kPerThread];

    // w / r: the matrix and row of this thread's LDS row (tid / 4).
    __device__ void load(const uint8_t *w, uint32_t r, const PackedGeometry &g, uint32_t step, uint32_t tid) {
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
            const uint32_t g0 = ((tid & 3) * kPerThread + i) * (T::kValsPerSlice / 8);
#pragma unroll
            for (uint32_t q = 0; q < T::kValsPerSlice / 8; ++q)
                *reinterpret_cast<uint4 *>(wbuf + tile_offset(lr, g0 + q)) =
                    make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        }
    }
};

// One K step of the activation tile: thread t copies 64 bytes (positions
// 32 (t % 4) .. +32) of tile row t / 4, i.e. matrix row `xrow`.
struct XStep {
    uint4 v[4];
    __device__ void load(const __bf16 *x, uint64_t ld, uint32_t xrow, uint32_t step, uint32_t tid) {
        const __bf16 *src = x + static_cast<uint64_t>(xrow) * ld + step * kStepK + 32 * (tid & 3);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = ld16(src + 8 * q);
    }
    __device__ void store(__bf16 *xbuf, uint32_t tid) const {
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) *reinterpret_cast<uint4 *>(xbuf + tile_offset(tid >> 2, 4 * (tid & 3) + q)) = v[q];
    }
};

// K steps whose loads are in flight ahead of the step being consumed. The
// loads of a step are issued together and consumed together, in issue order,
// so a wait for one step never waits on a later one. Every step issues its
// loads unconditionally (past the last step they re-read the last step, which
// the caches still hold), so the compiler's wait counts stay exact.
constexpr uint32_t kLead = 4;

// The shared main loop over `steps` K steps. Per step: wait for that step's
// weight slices and activation rows, dequantise / copy them into one of two
// LDS buffer pairs, request step + kLead, barrier, then wavefront w multiplies
// tile rows 32 (w / 2) .. +32 against weight row blocks 2 (w % 2), +1:
// acc[j] += X . W^T, operands read from LDS.
template <class T>
__device__ void gemm_tile(const TileRows &tr, const PackedGeometry &g, const __bf16 *x, uint64_t ldx,
                          uint32_t xrow, bool active, uint32_t steps, __bf16 *lds, f32x16 (&acc)[2]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63, mb = tid >> 7, nb0 = 2 * ((tid >> 6) & 1);
    const uint8_t *wrow;
    uint32_t rrow;
    tr.at(tid >> 2, wrow, rrow);
    WeightStep<T> ws[kLead];
    XStep xs[kLead];
    const uint32_t last = steps - 1;
#pragma unroll
    for (uint32_t p = 0; p < kLead; ++p) {
        ws[p].load(wrow, rrow, g, p < last ? p : last, tid);
        xs[p].load(x, ldx, xrow, p < last ? p : last, tid);
    }
    for (uint32_t st0 = 0; st0 < steps; st0 += kLead) {
#pragma unroll
        for (uint32_t u = 0; u < kLead; ++u) {
            const uint32_t st = st0 + u;
            if (st >= steps) break;
            __bf16 *wbuf = lds + (st & 1) * 2 * kWBufElems;
            __bf16 *xbuf = wbuf + kWBufElems;
            ws[u].store(wbuf, tid);
            xs[u].store(xbuf, tid);
            const uint32_t nxt = st + kLead < last ? st + kLead : last;
            ws[u].load(wrow, rrow, g, nxt, tid);
            xs[u].load(x, ldx, xrow, nxt, tid);
            __syncthreads();
            if (active) {
                const uint32_t arow = 32 * mb + (lane & 31);
#pragma unroll
                for (uint32_t kk = 0; kk < kStepK / 16; ++kk) {
                    const uint32_t gr = 2 * kk + (lane >> 5);
                    const bf16x8 av = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(xbuf + tile_offset(arow, gr)));
#pragma unroll
                    for (uint32_t j = 0; j < 2; ++j) {
                        const uint32_t brow = 32 * (nb0 + j) + (lane & 31);
                        const uint4 bv = *reinterpret_cast<const uint4 *>(wbuf + tile_offset(brow, gr));
                        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8, bv), acc[j], 0,
                                                                        0, 0);
                    }
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
    return e < experts && rows > 0 && rows <= kPrefillTileRows && row0 <= pairs && rows <= pairs - row0;
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

// Gate and up of 64 ffn rows for one row tile, SwiGLU, and the activations
// written as bf16 in the down projection's packed K order.
// grid: (max row tiles, ffn / 64): row tiles of one ffn slice run together,
// so tiles of one expert share the slice's weights through the caches.
template <class T, class TD>
__global__ __launch_bounds__(kGemmThreads) void gate_up_gemm_kernel(ExpertArgs a, const uint32_t *__restrict__ tiles,
                                                                     uint32_t pairs, const __bf16 *__restrict__ x,
                                                                     __bf16 *__restrict__ act) {
    extern __shared__ __align__(16) __bf16 tiles_lds[];
    uint32_t e, row0, rows;
    if (!row_tile(tiles, blockIdx.x, a.experts, pairs, e, row0, rows)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n0 = blockIdx.y * 64;
    const TileRows tr{static_cast<const uint8_t *>(a.gate[e]), static_cast<const uint8_t *>(a.up[e]), n0, true};
    const uint32_t mb = wave >> 1;
    const bool active = 32 * mb < rows;
    const uint32_t xr = tid >> 2; // the tile row this thread copies
    const uint32_t xrow = row0 + (xr < rows ? xr : rows - 1);
    f32x16 acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    gemm_tile<T>(tr, a.gu, x, a.hidden, xrow, active, a.hidden / kStepK, tiles_lds, acc);
    if (!active) return;
    const uint32_t F = a.ffn;
    // acc[0] = gate, acc[1] = up of ffn row n0 + 32 (wave % 2) + lane % 32
    const uint32_t n = n0 + 32 * (wave & 1) + (lane & 31);
    const uint32_t col = n / TD::kChunkK * TD::kChunkK + TD::pos(n % TD::kChunkK);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t m = 32 * mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= rows) continue;
        const float gv = acc[0][r], uv = acc[1][r];
        act[static_cast<uint64_t>(row0 + m) * F + col] = static_cast<__bf16>(gv / (1.0f + expf(-gv)) * uv);
    }
}

// Down rows [128 nt, +128) for one row tile into D [pairs x hidden] f32.
// grid: (max row tiles, hidden / 128).
template <class T>
__global__ __launch_bounds__(kGemmThreads) void down_gemm_kernel(ExpertArgs a, const uint32_t *__restrict__ tiles,
                                                                  uint32_t pairs, const __bf16 *__restrict__ act,
                                                                  float *__restrict__ dn) {
    extern __shared__ __align__(16) __bf16 tiles_lds[];
    uint32_t e, row0, rows;
    if (!row_tile(tiles, blockIdx.x, a.experts, pairs, e, row0, rows)) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t n0 = blockIdx.y * kTileN;
    const TileRows tr{static_cast<const uint8_t *>(a.down[e]), nullptr, n0, false};
    const uint32_t mb = wave >> 1;
    const bool active = 32 * mb < rows;
    const uint32_t xr = tid >> 2; // the tile row this thread copies
    const uint32_t xrow = row0 + (xr < rows ? xr : rows - 1);
    f32x16 acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
    gemm_tile<T>(tr, a.dn, act, a.ffn, xrow, active, a.ffn / kStepK, tiles_lds, acc);
    if (!active) return;
    const uint32_t H = a.hidden;
    const uint32_t nb0 = 2 * (wave & 1);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const uint32_t m = 32 * mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m >= rows) continue;
        float *dst = dn + static_cast<uint64_t>(row0 + m) * H + n0 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 2; ++j) dst[32 * (nb0 + j)] = acc[j][r];
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
    const size_t lds = 4ull * kWBufElems * sizeof(__bf16); // two (weights, activations) tile pairs
    auto gu = gate_up_gemm_kernel<T, TD>;
    auto dn = down_gemm_kernel<TD>;
    if (int rc = allow_lds(reinterpret_cast<const void *>(gu), lds)) return rc;
    if (int rc = allow_lds(reinterpret_cast<const void *>(dn), lds)) return rc;
    if (b.pairs == 0) return FMX_OK;
    if (int rc = launch_gather<T>(b.h, a.hidden, b.tokens, b.token_list, b.pairs, b.x, s)) return rc;
    hipLaunchKernelGGL(gu, dim3(max_tiles, a.ffn / 64), dim3(kGemmThreads), lds, s, a, b.tiles, b.pairs, b.x,
                       b.act);
    FMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dn, dim3(max_tiles, a.hidden / kTileN), dim3(kGemmThreads), lds, s, a, b.tiles, b.pairs,
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
