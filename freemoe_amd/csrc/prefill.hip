// prefill.hip — the MoE block over a batch of tokens at once (prefill).
//
// The reference has no batched MoE path: it runs Engine::forward_token per
// prompt token (engine.cpp:1870, 2395-2399). Here the batch is
//   route (bit-identical to the per-token routing, moe.hip)
//   -> bucket (per-expert token lists and row tiles, bucket.hip)
//   -> h into bf16 rows in the packed K order, one per token
//   -> gate/up grouped GEMM on bf16 MFMA over each expert's pairs (their
//      tokens' rows read through the bucketing's token list), weights
//      dequantised from their packed blocks in registers, SwiGLU in the
//      epilogue -> act [pairs x ffn] bf16
//   -> down grouped GEMM (K split in two for few experts) -> D f32 partials
//   -> combine per token in rank order plus the residual.
//
// K order. The packed expert slots (quant.hip) keep each lane's 16-byte slice
// of a chunk together, so a chunk's elements are stored permuted. A GEMM
// contracts over K in any order, so instead of re-permuting the weights the
// activations are written in the same permuted order ("packed positions"):
// one packed slot serves both decode and prefill, and every weight byte is
// read from HBM in 16-byte runs straight into the dequantiser.
//
// Tiles: see "the GEMMs" below.
#include "bucket.hpp"
#include "fmx_internal.hpp"
#include "moe.hpp"
#include "prefill.hpp"

#include <hip/hip_ext.h>

namespace fmx {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));


typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// (bf16(a), bf16(b)) rounded to nearest even, a in the low half: one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// float((int8_t)(byte B of w)) in one instruction: v_cvt_f32_i32 reading the
// byte through its sign-extending operand select (SDWA). Written out because
// the compiler otherwise shifts, sign-extends and converts (three
// instructions per byte).
template <int B>
__device__ __forceinline__ float i8_to_f32(uint32_t w) {
    float r;
    if constexpr (B == 0)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (B == 1)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}

// ------------------------------------------------------------ block types --
// kChunkK: elements per packed chunk (eight 16-byte lane slices). elem(p) /
// pos(e): element held at packed position p of a chunk, and its inverse.
// WStep: a lane's packed bytes (and scales) for one GEMM K step; decode()
// turns its scales into floats once per step (Dec), and dequant_kk() turns 8
// consecutive positions of it into the bf16 B operand of one MFMA.

struct GQ80 {
    static constexpr uint32_t kChunkK = 128;
    // position p = 16 l + 4 j + k holds element 32 j + 8 k + l
    __host__ __device__ static uint32_t elem(uint32_t p) { return 32 * ((p & 15) >> 2) + 8 * (p & 3) + (p >> 4); }
    __host__ __device__ static uint32_t pos(uint32_t e) { return 16 * (e & 7) + 4 * (e >> 5) + ((e & 31) >> 3); }
    // A lane's half of a K step (128 positions = one chunk): slices 4 h ..
    // 4 h + 3 (positions 64 h .. +64 of the step) and the chunk's four block
    // scales.
    struct WStep {
        uint4 q[4];
        uint2 d;
    };
    __device__ static void load_step(WStep &w, const uint8_t *packed, const PackedGeometry &g, uint32_t r,
                                     uint32_t step, uint32_t h) {
        const uint8_t *q = packed + g.scale_bytes + (static_cast<uint64_t>(r) * g.chunks + step) * 128 + h * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.q[i] = ld16(q + 16 * i);
        w.d = ld8(packed + static_cast<uint64_t>(r) * g.blocks_padded * 2 + static_cast<uint64_t>(step) * 8);
    }
    // The step's block scales as floats (once per step, not per K slice).
    struct Dec {
        float d[4];
    };
    __device__ static void decode(const WStep &w, Dec &c) {
        c.d[0] = half_bits_to_float(w.d.x & 0xFFFFu);
        c.d[1] = half_bits_to_float(w.d.x >> 16);
        c.d[2] = half_bits_to_float(w.d.y & 0xFFFFu);
        c.d[3] = half_bits_to_float(w.d.y >> 16);
    }
    // Positions 64 h + 8 kk .. +8 of the step: bytes 8 (kk % 2) .. +8 of the
    // lane's slice kk / 2, i.e. blocks 2 (kk % 2) and 2 (kk % 2) + 1. Each
    // int8 is converted straight from its byte of the dword (i8_to_f32).
    __device__ static bf16x8 dequant_kk(const WStep &w, const Dec &c, int kk) {
        const uint4 q = w.q[kk >> 1];
        const uint32_t lo = (kk & 1) ? q.z : q.x, hi = (kk & 1) ? q.w : q.y;
        const float d0 = c.d[2 * (kk & 1)], d1 = c.d[2 * (kk & 1) + 1];
        uint32_t v[4];
        v[0] = pack_bf16x2(d0 * i8_to_f32<0>(lo), d0 * i8_to_f32<1>(lo));
        v[1] = pack_bf16x2(d0 * i8_to_f32<2>(lo), d0 * i8_to_f32<3>(lo));
        v[2] = pack_bf16x2(d1 * i8_to_f32<0>(hi), d1 * i8_to_f32<1>(hi));
        v[3] = pack_bf16x2(d1 * i8_to_f32<2>(hi), d1 * i8_to_f32<3>(hi));
        return __builtin_bit_cast(bf16x8, make_uint4(v[0], v[1], v[2], v[3]));
    }
};

struct GQ40 {
    static constexpr uint32_t kChunkK = 256;
    // position p = 32 l + 4 j + 2 which + nib holds element 32 j + 16 nib + 8 which + l
    __host__ __device__ static uint32_t elem(uint32_t p) {
        const uint32_t l = p >> 5, q = p & 31, nib = q & 1, which = (q >> 1) & 1, j = q >> 2;
        return 32 * j + 16 * nib + 8 * which + l;
    }
    __host__ __device__ static uint32_t pos(uint32_t e) {
        const uint32_t j = e >> 5, r = e & 31, nib = r >> 4, which = (r >> 3) & 1, l = r & 7;
        return 32 * l + 4 * j + 2 * which + nib;
    }
    // A lane's half of a K step (128 positions = half a chunk): slices
    // 4 (step % 2) + 2 h and the next (positions 64 h .. +64 of the step), and
    // the chunk's eight block scales.
    struct WStep {
        uint4 q[2];
        uint4 d;
    };
    __device__ static void load_step(WStep &w, const uint8_t *packed, const PackedGeometry &g, uint32_t r,
                                     uint32_t step, uint32_t h) {
        const uint32_t c = step >> 1, s0 = 4 * (step & 1) + 2 * h;
        const uint8_t *q = packed + g.scale_bytes + ((static_cast<uint64_t>(r) * g.chunks + c) * 8 + s0) * 16;
        w.q[0] = ld16(q);
        w.q[1] = ld16(q + 16);
        w.d = ld16(packed + static_cast<uint64_t>(r) * g.blocks_padded * 2 + static_cast<uint64_t>(c) * 16);
    }
    // The chunk's block scales as 2^9 d and -8 d, once per step.
    struct Dec {
        float d9[8], nd[8];
    };
    __device__ static void decode(const WStep &w, Dec &c) {
        const uint32_t dw[4] = {w.d.x, w.d.y, w.d.z, w.d.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float d = half_bits_to_float((j & 1) ? dw[j >> 1] >> 16 : dw[j >> 1] & 0xFFFFu);
            c.d9[j] = d * 0x1p9f;
            c.nd[j] = -8.0f * d;
        }
    }
    // Positions 64 h + 8 kk .. +8 of the step: dword kk % 4 of the lane's slice
    // kk / 4; its bytes are blocks 2 (kk % 4) (bytes 0, 1) and 2 (kk % 4) + 1
    // (bytes 2, 3), low nibble first. The nibbles, one per byte, become floats
    // two at a time read as fp8 (q 2^-9, exact), and d (q - 8) =
    // fma(2^9 d, q 2^-9, -8 d) exactly (the product is d q, exact in f32; d
    // comes from an f16, so 2^9 d is exact too).
    __device__ static bf16x8 dequant_kk(const WStep &w, const Dec &c, int kk) {
        const uint4 q = w.q[kk >> 2];
        const int i = kk & 3;
        const uint32_t qw = i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
        const uint32_t lo = qw & 0x0F0F0F0Fu, hi = (qw >> 4) & 0x0F0F0F0Fu;
        const float2 l01 = fp8_pair<false>(lo), l23 = fp8_pair<true>(lo);
        const float2 h01 = fp8_pair<false>(hi), h23 = fp8_pair<true>(hi);
        const float lq[4] = {l01.x, l01.y, l23.x, l23.y}, hq[4] = {h01.x, h01.y, h23.x, h23.y};
        uint32_t v[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float d = c.d9[2 * i + (b >> 1)], nd = c.nd[2 * i + (b >> 1)];
            v[b] = pack_bf16x2(__builtin_fmaf(d, lq[b], nd), __builtin_fmaf(d, hq[b], nd));
        }
        return __builtin_bit_cast(bf16x8, make_uint4(v[0], v[1], v[2], v[3]));
    }
};

struct GQ4K {
    static constexpr uint32_t kChunkK = 256;
    // position p = 32 l + 8 g + 2 k + nib holds element 64 g + 32 nib + 8 k + l
    __host__ __device__ static uint32_t elem(uint32_t p) {
        const uint32_t l = p >> 5, q = p & 31, nib = q & 1, k = (q >> 1) & 3, g = q >> 3;
        return 64 * g + 32 * nib + 8 * k + l;
    }
    __host__ __device__ static uint32_t pos(uint32_t e) {
        const uint32_t g = e >> 6, r = e & 63, nib = r >> 5, k = (r >> 3) & 3, l = r & 7;
        return 32 * l + 8 * g + 2 * k + nib;
    }
    // A lane's half of a K step: as Q4_0, with the super-block header.
    struct WStep {
        uint4 q[2];
        uint4 hd;
    };
    __device__ static void load_step(WStep &w, const uint8_t *packed, const PackedGeometry &g, uint32_t r,
                                     uint32_t step, uint32_t h) {
        const uint32_t c = step >> 1, s0 = 4 * (step & 1) + 2 * h;
        const uint8_t *q = packed + g.scale_bytes + ((static_cast<uint64_t>(r) * g.chunks + c) * 8 + s0) * 16;
        w.q[0] = ld16(q);
        w.q[1] = ld16(q + 16);
        w.hd = ld16(packed + (static_cast<uint64_t>(r) * g.chunks + c) * 16);
    }
    // The super-block's sub-block scales 2^9 d sc_j and negated mins
    // -dmin m_j (j < 8) as floats, once per step; the products are exact in
    // f32 (an f16 times a 6-bit integer, times a power of two).
    struct Dec {
        float d[8], nm[8];
    };
    __device__ static void decode(const WStep &w, Dec &c) {
        uint8_t hdr[16];
        memcpy(hdr, &w.hd, 16);
        const float d = half_bits_to_float(hdr[0] | (hdr[1] << 8));
        const float dmin = half_bits_to_float(hdr[2] | (hdr[3] << 8));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, m;
            k4_scale_min(j, hdr + 4, sc, m);
            c.d[j] = d * static_cast<float>(sc) * 0x1p9f;
            c.nm[j] = -(dmin * static_cast<float>(m));
        }
    }
    // Positions 64 h + 8 kk .. +8 of the step: dword g = kk % 4 of the lane's
    // slice kk / 4, group g: low nibbles sub-block 2 g, high 2 g + 1. The
    // nibbles become floats two at a time read as fp8 (q 2^-9, exact), and
    // d sc q - dmin m = fma(2^9 d sc, q 2^-9, -dmin m) exactly (d sc q is exact).
    __device__ static bf16x8 dequant_kk(const WStep &w, const Dec &c, int kk) {
        const uint4 q = w.q[kk >> 2];
        const int gi = kk & 3;
        const uint32_t qw = gi == 0 ? q.x : gi == 1 ? q.y : gi == 2 ? q.z : q.w;
        const uint32_t lo = qw & 0x0F0F0F0Fu, hi = (qw >> 4) & 0x0F0F0F0Fu;
        const float d1 = c.d[2 * gi], m1 = c.nm[2 * gi], d2 = c.d[2 * gi + 1], m2 = c.nm[2 * gi + 1];
        const float2 l01 = fp8_pair<false>(lo), l23 = fp8_pair<true>(lo);
        const float2 h01 = fp8_pair<false>(hi), h23 = fp8_pair<true>(hi);
        const float lq[4] = {l01.x, l01.y, l23.x, l23.y}, hq[4] = {h01.x, h01.y, h23.x, h23.y};
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            v[k] = pack_bf16x2(__builtin_fmaf(d1, lq[k], m1), __builtin_fmaf(d2, hq[k], m2));
        return __builtin_bit_cast(bf16x8, make_uint4(v[0], v[1], v[2], v[3]));
    }
};

// Q6_K raw blocks (256 elements in 210 bytes: ql[128], qh[64], sc[16], d).
// Positions are elements (the identity order): K step s is half n = s % 2 of
// block s / 2, elements 128 n + 0..127; lanes 0-31 take 128 n + 0..63 (ql
// low nibbles, quarters 0 and 1), lanes 32-63 128 n + 64..127 (high
// nibbles, quarters 2 and 3). Blocks are only 2-byte aligned, so the quant
// bytes come in with unaligned 16-byte loads (each inside its block).
typedef unsigned int fmx_u32x4_u1 __attribute__((ext_vector_type(4), aligned(1)));
__device__ __forceinline__ uint4 ld16u(const uint8_t *p) {
    const fmx_u32x4_u1 v = *(const __attribute__((address_space(1))) fmx_u32x4_u1 *)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

struct GQ6K {
    static constexpr uint32_t kChunkK = 256;
    __host__ __device__ static uint32_t elem(uint32_t p) { return p; }
    __host__ __device__ static uint32_t pos(uint32_t e) { return e; }
    // The lane's half of a K step: the half block's 64 ql bytes and 32 qh
    // bytes (both lane halves read them: low or high nibbles, other bit
    // pairs), its four sub-block scales and d.
    struct WStep {
        uint4 ql[4], qh[2];
        uint32_t sc, d;
    };
    __device__ static void load_step(WStep &w, const uint8_t *packed, const PackedGeometry &g, uint32_t r,
                                     uint32_t step, uint32_t h) {
        const uint32_t n = step & 1;
        const uint8_t *blk = packed + (static_cast<uint64_t>(r) * g.blocks + (step >> 1)) * 210;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.ql[i] = ld16u(blk + 64 * n + 16 * i);
#pragma unroll
        for (int i = 0; i < 2; ++i) w.qh[i] = ld16u(blk + 128 + 32 * n + 16 * i);
        // scales 8 n + 4 h .. +3 (quarters 2 h and 2 h + 1 of the half, two
        // 16-element sub-blocks each)
        const uint16_t *s16 = reinterpret_cast<const uint16_t *>(blk + 192 + 8 * n + 4 * h);
        w.sc = s16[0] | (static_cast<uint32_t>(s16[1]) << 16);
        w.d = *reinterpret_cast<const uint16_t *>(blk + 208);
    }
    // d sc (exact: 11 x 8 bits) and -32 d sc per sub-block, once per step.
    struct Dec {
        float dsc[4], nd[4];
    };
    __device__ static void decode(const WStep &w, Dec &c) {
        const float d = half_bits_to_float(w.d);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c.dsc[i] = d * static_cast<float>(static_cast<int8_t>((w.sc >> (8 * i)) & 0xFFu));
            c.nd[i] = -32.0f * c.dsc[i];
        }
    }
    // Positions 64 h + 8 kk .. +8 of the step: ql bytes 8 kk .. +8 of the
    // half, qh bytes 8 (kk % 4) .. +8 at bit pair 2 h + kk / 4, scale
    // (kk % 4) / 2 + 2 (kk / 4) of the lane's four. (d sc) (q - 32) =
    // fma(d sc, q, -32 d sc) exactly: the product has at most 24 bits.
    __device__ static bf16x8 dequant_kk(const WStep &w, const Dec &c, int kk) {
        const uint32_t h = (threadIdx.x & 63) >> 5;
        const uint4 q = w.ql[kk >> 1];
        const uint4 b = w.qh[(kk & 3) >> 1];
        const uint32_t q0 = (kk & 1) ? q.z : q.x, q1 = (kk & 1) ? q.w : q.y;
        const uint32_t b0 = ((kk & 3) & 1) ? b.z : b.x, b1 = ((kk & 3) & 1) ? b.w : b.y;
        const uint32_t sh = 4 * h + 2 * (kk >> 2);
        const uint32_t v0 = ((h ? q0 >> 4 : q0) & 0x0F0F0F0Fu) | (((b0 >> sh) & 0x03030303u) << 4);
        const uint32_t v1 = ((h ? q1 >> 4 : q1) & 0x0F0F0F0Fu) | (((b1 >> sh) & 0x03030303u) << 4);
        const int si = ((kk & 3) >> 1) + 2 * (kk >> 2);
        const float ds = c.dsc[si], nd = c.nd[si];
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t vv = i ? v1 : v0;
            v[2 * i] = pack_bf16x2(__builtin_fmaf(ds, static_cast<float>(vv & 0xFFu), nd),
                                   __builtin_fmaf(ds, static_cast<float>((vv >> 8) & 0xFFu), nd));
            v[2 * i + 1] = pack_bf16x2(__builtin_fmaf(ds, static_cast<float>((vv >> 16) & 0xFFu), nd),
                                       __builtin_fmaf(ds, static_cast<float>(vv >> 24), nd));
        }
        return __builtin_bit_cast(bf16x8, make_uint4(v[0], v[1], v[2], v[3]));
    }
};

// ------------------------------------------------------------ the GEMMs --
//
// One workgroup (8 wavefronts, two per SIMD, so one wavefront's dequantising
// overlaps the other's MFMAs) multiplies a row tile of one expert (up to 192
// token-expert pairs = 6 blocks of 32) by 128 (gate/up) or 256 (down) weight
// columns; wavefront w owns one 32-column block (gate/up: wavefronts 0-3 the
// gate rows, 4-7 the up rows of the same 128 ffn rows; down: 32 rows each).
//
// Weights never touch LDS: each lane loads its own row's packed bytes for
// a K step (128 packed positions; lanes 0-31 take positions 0-63, lanes 32-63
// positions 64-127) from HBM into registers, two steps ahead, and dequantises
// 8 positions (one MFMA K slice) at a time as the B operand. Each weight byte
// is read once per row tile, and a row tile holds all of an expert's pairs up
// to 192. Activations: the tile's rows for the next step are loaded during
// this one straight into the other of two LDS buffers (direct-to-LDS loads),
// where all eight wavefronts read their A operands.
//
// v_mfma_f32_32x32x16_bf16: A lane l = tile row 32 mb + l % 32, B lane l =
// column l % 32, both at positions 64 (l / 32) + 8 kk .. +8 of the step (a GEMM
// may contract over K in any order, as long as A and B agree); C element r of
// lane l = row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.

constexpr uint32_t kGThreads = 512;                           // 8 wavefronts, two per SIMD
constexpr uint32_t kGStepK = 128;                             // packed positions per K step
constexpr uint32_t kGRowBytes = kGStepK * 2;                  // 256 bytes of a tile row
constexpr uint32_t kGBufBytes = kPrefillTileRows * kGRowBytes; // one LDS activation buffer

// LDS activation tile: 192 rows x 128 bf16 (256 bytes = the 64 banks, sixteen
// 16-byte granules); granule g of row r sits at granule g ^ (r % 16). A pass
// of 16 lanes of an A-operand read (16 consecutive rows, one granule) or of a
// store (one row, 16 granules) then touches 16 distinct bank groups.
__device__ __forceinline__ uint32_t xswz(uint32_t row) { return row & 15u; }

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

typedef const __attribute__((address_space(1))) void *fmx_gptr;
typedef __attribute__((address_space(3))) void *fmx_lptr;

// 16 bytes per lane from global `src` to LDS `dst_base` + 16 lane (dst_base
// wave-uniform): global_load_lds_dwordx4.
__device__ __forceinline__ void load_lds16(const void *src, char *dst_base) {
    __builtin_amdgcn_global_load_lds((fmx_gptr)src, (fmx_lptr)dst_base, 16, 0, 0);
}

// The workgroup barrier of a K step, after wait_vm_lgkm0 has waited for this
// wavefront's LDS reads and for its loads (the direct-to-LDS ones among
// them): s_barrier itself, the empty asm statements keeping the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (expcnt not waited for), n < 64.
template <uint32_t N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N < 64, "vmcnt has six bits");
    __builtin_amdgcn_s_waitcnt((N & 15u) | ((N >> 4) << 14) | (7u << 4));
}

// One GEMM of a workgroup: weight steps in a ring of three register slots
// and the accumulators of NMB row blocks (the kernels instantiate one per
// possible block count, so no MFMA sits under a branch). The activations go
// from global memory straight into LDS (global_load_lds_dwordx4: no
// registers, no LDS store instructions): a wavefront's load fills 1 KiB of
// LDS, 16 bytes per lane in lane order, so thread t (wavefront w, lane l)
// fills slot l % 16 of tile row sr = 4 w + l / 16 (+ 32 i for row block i)
// and loads the granule the swizzle puts there, granule (l % 16) ^ (sr % 16).
// Every staging row has a readable source (gate/up: the token of the pair,
// or of the last pair for rows past them; down: the workspace pads act by a
// tile), and rows past the tile (up to 32 NMB) only feed output rows that
// are never written.
//
// Requests: step st requests the activations of step st + 1 (into the LDS
// buffer that step st - 1 read) and the weights of step st + 2, and at its
// end waits for all of its requests (vmcnt(0)): the activations must be in
// LDS before the barrier, and the weights have had the step's MFMAs to
// arrive (waiting only for the activations, with the weights left in flight
// across the barrier, measured the same). No direct-to-LDS load is in flight
// when the K loop ends, so the epilogue may reuse the LDS.
template <class T, uint32_t NMB>
struct GemmWave {
    static constexpr uint32_t kPass = 6; // steps per pass: the ring (3) and the buffers (2) both turn
    typename T::WStep w[3];
    f32x16 acc[NMB];

    // xrow[i]: this thread's granule of staging row sr + 32 i at K position 0
    // (see run).
    const __bf16 *xrow[NMB];

    // This thread's granules of step k0's activations into LDS buffer `dst`
    // (the wavefront's 1 KiB of row block 0 of the buffer: wave-uniform).
    __device__ __forceinline__ void load_x(char *dst, uint32_t k0) {
#pragma unroll
        for (uint32_t i = 0; i < NMB; ++i) load_lds16(xrow[i] + k0, dst + i * 32 * kGRowBytes);
    }

    // The MFMAs of one K step from ring slot `slot`; a_kk[kk]: byte address of
    // the lane's A operand of slice kk in row block 0 of the step's buffer.
    // Software-pipelined over the 8 K slices: the A operands (LDS) and the B
    // operands (dequantised weights) of slice kk + 1 are prepared while the
    // MFMAs of slice kk run, so the VALU work overlaps the matrix unit.
    __device__ __forceinline__ void multiply(int slot, const char *const (&a_kk)[8]) {
        bf16x8 av[2][NMB], bv[2];
        typename T::Dec dc;
        T::decode(w[slot], dc);
#pragma unroll
        for (uint32_t mb = 0; mb < NMB; ++mb)
            av[0][mb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(a_kk[0] + mb * 32 * kGRowBytes));
        bv[0] = T::dequant_kk(w[slot], dc, 0);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const int c = kk & 1, n = c ^ 1;
            if (kk + 1 < 8) {
#pragma unroll
                for (uint32_t mb = 0; mb < NMB; ++mb)
                    av[n][mb] = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const uint4 *>(a_kk[kk + 1] + mb * 32 * kGRowBytes));
                bv[n] = T::dequant_kk(w[slot], dc, kk + 1);
            }
#pragma unroll
            for (uint32_t mb = 0; mb < NMB; ++mb)
                acc[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[c][mb], bv[c], acc[mb], 0, 0, 0);
        }
    }

    // One step: request the activations of step `nx` into the other LDS
    // buffer and the weights of step `nw` into `slot_next`, multiply step
    // (ring slot `slot`, LDS buffer `buf`), wait for the activations, barrier.
    __device__ __forceinline__ void step(int slot, int slot_next, uint32_t buf, uint32_t nw, uint32_t nx,
                                         const uint8_t *m0, uint32_t r0, const PackedGeometry &g, char *lds,
                                         uint32_t wbase, uint32_t aoff0, uint32_t h) {
        load_x(lds + (buf ^ 1) * kGBufBytes + wbase, nx * kGStepK);
        T::load_step(w[slot_next], m0, g, r0, nw, h);
        __builtin_amdgcn_sched_barrier(0);
        const char *a_kk[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) a_kk[kk] = lds + buf * kGBufBytes + (aoff0 ^ (kk << 4));
        multiply(slot, a_kk);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_lgkm0<0>();
        lds_barrier();
    }

    // K steps [s0, s0 + steps) against weight row (m0, r0). Staging row r of
    // the tile (r < 32 NMB) is the activation row row_of(r) (a pointer to
    // its K position 0).
    template <class RowOf>
    __device__ __forceinline__ void run(const uint8_t *m0, uint32_t r0, const PackedGeometry &g, RowOf row_of,
                                        uint32_t s0, uint32_t steps, char *lds) {
        const uint32_t tid = threadIdx.x, lane = tid & 63, h = lane >> 5;
        const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t last = s0 + steps - 1;
        auto clampk = [last](uint32_t k) { return k < last ? k : last; };
        // A operand of slice kk: row lane % 32 of the block, granule 8 h + kk
        const uint32_t ar = lane & 31;
        const uint32_t aoff0 = ar * kGRowBytes + (((8 * h) ^ xswz(ar)) << 4);
        // staging: row sr = 4 w + l / 16 (= tid / 16), slot l % 16
        const uint32_t sr = tid >> 4;
#pragma unroll
        for (uint32_t i = 0; i < NMB; ++i) xrow[i] = row_of(sr + 32 * i) + 8 * ((lane & 15) ^ xswz(sr));
        const uint32_t wbase = 1024 * wave;
#pragma unroll
        for (uint32_t mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mb][i] = 0.0f;
        // prologue: activations of s0 into LDS buffer 0, weights of s0 and
        // s0 + 1
        load_x(lds + wbase, s0 * kGStepK);
#pragma unroll
        for (int p = 0; p < 2; ++p) T::load_step(w[p], m0, g, r0, clampk(s0 + p), h);
        wait_vm_lgkm0<0>();
        __syncthreads();
        uint32_t s = 0;
        // steady state: kPass steps per pass
        for (; s + kPass <= steps; s += kPass) {
#pragma unroll
            for (uint32_t u = 0; u < kPass; ++u) {
                const uint32_t st = s0 + s + u;
                step(u % 3, (u + 2) % 3, u & 1, clampk(st + 2), clampk(st + 1), m0, r0, g, lds, wbase, aoff0, h);
            }
        }
        // the remaining steps (fewer than kPass)
#pragma unroll
        for (uint32_t u = 0; u < kPass; ++u) {
            if (s + u >= steps) break;
            const uint32_t st = s0 + s + u;
            step(u % 3, (u + 2) % 3, u & 1, clampk(st + 2), clampk(st + 1), m0, r0, g, lds, wbase, aoff0, h);
        }
    }
};

// ------------------------------------------------------------------ kernels --

// hb[t][p] = bf16(h[t][element at packed position p]): one workgroup per
// (2048-element segment, token), the h segment staged in LDS by 16-byte
// loads, 8 positions (one 16-byte store) per thread. The gate/up GEMM reads
// each pair's row of hb through token_list. grid: (ceil(hidden / 2048),
// tokens).
constexpr uint32_t kPackSeg = 2048;
template <class T>
__global__ __launch_bounds__(256) void pack_h_kernel(const float *__restrict__ h, uint32_t hidden,
                                                     __bf16 *__restrict__ hb) {
    __shared__ __align__(16) float seg[kPackSeg];
    const uint32_t t = blockIdx.y, e0 = blockIdx.x * kPackSeg, tid = threadIdx.x;
    const uint32_t n = hidden - e0 < kPackSeg ? hidden - e0 : kPackSeg;
    const float4 *src = reinterpret_cast<const float4 *>(h + static_cast<uint64_t>(t) * hidden + e0);
    for (uint32_t q = tid; q < n / 4; q += 256) reinterpret_cast<float4 *>(seg)[q] = src[q];
    __syncthreads();
    const uint32_t p = tid * 8;
    if (p >= n) return;
    const uint32_t cb = p / T::kChunkK * T::kChunkK, pc = p % T::kChunkK;
    uint32_t v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(seg[cb + T::elem(pc + 2 * i)], seg[cb + T::elem(pc + 2 * i + 1)]);
    *reinterpret_cast<uint4 *>(hb + static_cast<uint64_t>(t) * hidden + e0 + p) = make_uint4(v[0], v[1], v[2], v[3]);
}

// Column of activation element f (an ffn index) in the down projection's
// packed K order (the down matrices' block type decides it; the activations
// are written straight into that order).
__device__ __forceinline__ uint32_t down_k_position(uint32_t down_type, uint32_t f) {
    switch (down_type) {
    case FMX_TYPE_Q8_0: return f / GQ80::kChunkK * GQ80::kChunkK + GQ80::pos(f % GQ80::kChunkK);
    case FMX_TYPE_Q4_0: return f / GQ40::kChunkK * GQ40::kChunkK + GQ40::pos(f % GQ40::kChunkK);
    case FMX_TYPE_Q4_K: return f / GQ4K::kChunkK * GQ4K::kChunkK + GQ4K::pos(f % GQ4K::kChunkK);
    default: return f; // Q6_K: the identity order
    }
}

// Gate and up of 128 ffn rows (32 per wavefront) for one row tile of NMB row
// blocks, SwiGLU, and the activations written as bf16 in the down
// projection's packed K order.
// Wavefronts 0-3 take the gate rows, 4-7 the up rows of the same 128 ffn
// rows; after the K loop the gate wavefronts hand their results through LDS
// (the activation buffers, free by then) to the up wavefronts of the same
// columns, which apply SwiGLU.
template <class T, uint32_t NMB>
__device__ __forceinline__ void gate_up_tile(const ExpertArgs &a, uint32_t e, uint32_t row0, uint32_t rows,
                                             uint32_t pairs, uint32_t tokens, const __bf16 *__restrict__ hb,
                                             const uint32_t *__restrict__ token_list, __bf16 *__restrict__ act,
                                             char *lds) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t f = blockIdx.x * 128 + 32 * (wave & 3) + (lane & 31);
    const bool is_up = wave >= 4;
    GemmWave<T, NMB> gw;
    const uint32_t H = a.hidden;
    // rows past the pairs read the last pair's token; a token index out of
    // range (a list the bucketing reported as broken) reads token 0
    auto row_of = [=](uint32_t r) {
        const uint32_t pr = row0 + r < pairs ? row0 + r : pairs - 1, t = token_list[pr];
        return hb + static_cast<uint64_t>(t < tokens ? t : 0u) * H;
    };
    gw.run(static_cast<const uint8_t *>(is_up ? a.up[e] : a.gate[e]), f, a.gu, row_of, 0, H / kGStepK, lds);
    // the K loop ended with a barrier after every wavefront's last LDS read
    float *xc = reinterpret_cast<float *>(lds) + (wave & 3) * NMB * 16 * 64 + lane;
    if (!is_up) {
#pragma unroll
        for (uint32_t mb = 0; mb < NMB; ++mb)
#pragma unroll
            for (int r = 0; r < 16; ++r) xc[(mb * 16 + r) * 64] = gw.acc[mb][r];
    }
    __syncthreads();
    if (!is_up) return;
    const uint32_t F = a.ffn;
    const uint32_t col = down_k_position(a.type_dn, f);
#pragma unroll
    for (uint32_t mb = 0; mb < NMB; ++mb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t m = 32 * mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= rows) continue;
            const float gv = xc[(mb * 16 + r) * 64], uv = gw.acc[mb][r];
            act[static_cast<uint64_t>(row0 + m) * F + col] = static_cast<__bf16>(gv / (1.0f + expf(-gv)) * uv);
        }
    }
}

// grid: (ffn / 128, max row tiles): tile order[blockIdx.y] (largest first);
// the row tiles past the bucketing's count (their workgroups return at once)
// come last in dispatch order.
template <class T>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gate_up_gemm_kernel(
    ExpertArgs a, const uint32_t *__restrict__ tiles, const uint32_t *__restrict__ order, uint32_t pairs,
    uint32_t tokens, const __bf16 *__restrict__ hb, const uint32_t *__restrict__ token_list, __bf16 *__restrict__ act) {
    extern __shared__ __align__(16) char xlds[];
    uint32_t e, row0, rows;
    if (blockIdx.y >= tiles[0] || !row_tile(tiles, order[blockIdx.y], a.experts, pairs, e, row0, rows)) return;
    switch ((rows + 31) / 32) {
    case 1: gate_up_tile<T, 1>(a, e, row0, rows, pairs, tokens, hb, token_list, act, xlds); break;
    case 2: gate_up_tile<T, 2>(a, e, row0, rows, pairs, tokens, hb, token_list, act, xlds); break;
    case 3: gate_up_tile<T, 3>(a, e, row0, rows, pairs, tokens, hb, token_list, act, xlds); break;
    case 4: gate_up_tile<T, 4>(a, e, row0, rows, pairs, tokens, hb, token_list, act, xlds); break;
    case 5: gate_up_tile<T, 5>(a, e, row0, rows, pairs, tokens, hb, token_list, act, xlds); break;
    default: gate_up_tile<T, 6>(a, e, row0, rows, pairs, tokens, hb, token_list, act, xlds); break;
    }
}

// Down rows [256 blockIdx.x, +256) (32 per wavefront) for one row tile of NMB
// row blocks, over K steps [blockIdx.y * steps, +steps), into D[blockIdx.y]
// [pairs x hidden] f32.
template <class T, uint32_t NMB>
__device__ __forceinline__ void down_tile(const ExpertArgs &a, uint32_t e, uint32_t row0, uint32_t rows, uint32_t pairs,
                          const __bf16 *__restrict__ act, uint32_t steps, float *__restrict__ dn, char *lds) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = blockIdx.x * 256 + 32 * wave + (lane & 31);
    const uint8_t *wd = static_cast<const uint8_t *>(a.down[e]);
    GemmWave<T, NMB> gw;
    const uint32_t F = a.ffn;
    auto row_of = [=](uint32_t r) { return act + static_cast<uint64_t>(row0 + r) * F; };
    gw.run(wd, n, a.dn, row_of, blockIdx.y * steps, steps, lds);
    const uint32_t H = a.hidden;
    float *dst = dn + static_cast<uint64_t>(blockIdx.y) * pairs * H;
#pragma unroll
    for (uint32_t mb = 0; mb < NMB; ++mb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t m = 32 * mb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= rows) continue;
            dst[static_cast<uint64_t>(row0 + m) * H + n] = gw.acc[mb][r];
        }
    }
}

// grid: (hidden / 256, K splits, max row tiles).
template <class T>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void down_gemm_kernel(
    ExpertArgs a, const uint32_t *__restrict__ tiles, uint32_t pairs, const __bf16 *__restrict__ act,
    uint32_t steps, float *__restrict__ dn) {
    extern __shared__ __align__(16) char xlds[];
    uint32_t e, row0, rows;
    if (!row_tile(tiles, blockIdx.z, a.experts, pairs, e, row0, rows)) return;
    switch ((rows + 31) / 32) {
    case 1: down_tile<T, 1>(a, e, row0, rows, pairs, act, steps, dn, xlds); break;
    case 2: down_tile<T, 2>(a, e, row0, rows, pairs, act, steps, dn, xlds); break;
    case 3: down_tile<T, 3>(a, e, row0, rows, pairs, act, steps, dn, xlds); break;
    case 4: down_tile<T, 4>(a, e, row0, rows, pairs, act, steps, dn, xlds); break;
    case 5: down_tile<T, 5>(a, e, row0, rows, pairs, act, steps, dn, xlds); break;
    default: down_tile<T, 6>(a, e, row0, rows, pairs, act, steps, dn, xlds); break;
    }
}

// out[t] = x[t] + ((0 + w_0 D_0) + w_1 D_1 ...) in rank order (engine.cpp:1517,
// 1770, 813-816), each D the sum of the K splits' partial products in split
// order. V consecutive elements per thread (hidden % V == 0, x and out
// V-float aligned). A rank whose position is at or past `pairs` (a routing
// table the bucketing rejected, which reported it) adds nothing. grid:
// (ceil(hidden / (256 V)), tokens).
template <uint32_t V>
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ x, const float *__restrict__ dn,
                                                      uint32_t splits, uint64_t split_stride,
                                                      const uint32_t *__restrict__ slot_of, uint32_t pairs,
                                                      const float *__restrict__ w, uint32_t hidden, uint32_t K,
                                                      float *__restrict__ out) {
    typedef float fv __attribute__((ext_vector_type(V)));
    const uint32_t t = blockIdx.y, j = (blockIdx.x * 256 + threadIdx.x) * V;
    if (j >= hidden) return;
    fv ffn = 0.0f;
    for (uint32_t r = 0; r < K; ++r) {
        const uint64_t i = static_cast<uint64_t>(t) * K + r;
        const uint32_t pos = slot_of[i];
        if (pos >= pairs) continue;
        const float *d = dn + static_cast<uint64_t>(pos) * hidden + j;
        fv v = *reinterpret_cast<const fv *>(d);
        for (uint32_t sp = 1; sp < splits; ++sp) v += *reinterpret_cast<const fv *>(d + sp * split_stride);
        ffn = ffn + w[i] * v;
    }
    const uint64_t o = static_cast<uint64_t>(t) * hidden + j;
    *reinterpret_cast<fv *>(out + o) = *reinterpret_cast<const fv *>(x + o) + ffn;
}

// ---------------------------------------------------------------- launchers --

template <class T>
int launch_pack_h(const float *h, uint32_t hidden, uint32_t tokens, __bf16 *hb, hipStream_t s) {
    if (tokens == 0) return FMX_OK;
    hipLaunchKernelGGL(pack_h_kernel<T>, dim3(div_up(hidden, kPackSeg), tokens), dim3(256), 0, s, h, hidden, hb);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

template <class T, class TD>
int launch_gemms(const ExpertArgs &a, const PrefillBuffers &b, uint32_t max_tiles, hipStream_t s, hipEvent_t *kev) {
    const size_t lds = 2ull * kGBufBytes; // two activation buffers
    auto gu = gate_up_gemm_kernel<T>;
    auto dn = down_gemm_kernel<TD>;
    if (int rc = allow_lds(reinterpret_cast<const void *>(gu), lds)) return rc;
    if (int rc = allow_lds(reinterpret_cast<const void *>(dn), lds)) return rc;
    if (b.pairs == 0) return FMX_OK;
    if (int rc = launch_pack_h<T>(b.h, a.hidden, b.tokens, b.x, s)) return rc;
    const dim3 gu_grid(a.ffn / 128, max_tiles), dn_grid(a.hidden / 256, b.splits, max_tiles);
    const uint32_t steps = a.ffn / kGStepK / b.splits;
    if (kev) {
        // the launches record kev[0..1] / kev[2..3] at kernel start and end
        hipExtLaunchKernelGGL(gu, gu_grid, dim3(kGThreads), lds, s, kev[0], kev[1], 0, a, b.tiles, b.tile_order,
                              b.pairs, b.tokens, b.x, b.token_list, b.act);
        FMX_LAUNCH_CHECK();
        hipExtLaunchKernelGGL(dn, dn_grid, dim3(kGThreads), lds, s, kev[2], kev[3], 0, a, b.tiles, b.pairs, b.act,
                              steps, b.dn);
        FMX_LAUNCH_CHECK();
        return FMX_OK;
    }
    hipLaunchKernelGGL(gu, gu_grid, dim3(kGThreads), lds, s, a, b.tiles, b.tile_order, b.pairs, b.tokens, b.x,
                       b.token_list, b.act);
    FMX_LAUNCH_CHECK();
    hipLaunchKernelGGL(dn, dn_grid, dim3(kGThreads), lds, s, a, b.tiles, b.pairs, b.act, steps, b.dn);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

template <class T>
int launch_for_down(const ExpertArgs &a, const PrefillBuffers &b, uint32_t max_tiles, hipStream_t s,
                    hipEvent_t *kev) {
    switch (a.type_dn) {
    case FMX_TYPE_Q8_0: return launch_gemms<T, GQ80>(a, b, max_tiles, s, kev);
    case FMX_TYPE_Q4_0: return launch_gemms<T, GQ40>(a, b, max_tiles, s, kev);
    case FMX_TYPE_Q4_K: return launch_gemms<T, GQ4K>(a, b, max_tiles, s, kev);
    case FMX_TYPE_Q6_K: return launch_gemms<T, GQ6K>(a, b, max_tiles, s, kev);
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

uint32_t chunk_k_of(uint32_t type) {
    switch (type) {
    case FMX_TYPE_Q8_0: return GQ80::kChunkK;
    case FMX_TYPE_Q4_0: return GQ40::kChunkK;
    case FMX_TYPE_Q4_K: return GQ4K::kChunkK;
    case FMX_TYPE_Q6_K: return GQ6K::kChunkK;
    }
    return 0;
}

} // namespace

bool prefill_gemm_supported(const ExpertArgs &a) {
    const uint32_t ck_gu = chunk_k_of(a.type_gu), ck_dn = chunk_k_of(a.type_dn);
    if (ck_gu == 0 || ck_dn == 0) return false;
    return a.hidden % ck_gu == 0 && a.hidden % 256 == 0 && a.ffn % ck_dn == 0 && a.ffn % 128 == 0 &&
           a.hidden % kGStepK == 0 && a.ffn % kGStepK == 0;
}

int launch_prefill_experts(const ExpertArgs &a, const PrefillBuffers &b, uint32_t max_tiles, hipStream_t s,
                           hipEvent_t *kev) {
    if (!prefill_gemm_supported(a)) return FMX_ERR_SHAPE_MISMATCH;
    switch (a.type_gu) {
    case FMX_TYPE_Q8_0: return launch_for_down<GQ80>(a, b, max_tiles, s, kev);
    case FMX_TYPE_Q4_0: return launch_for_down<GQ40>(a, b, max_tiles, s, kev);
    case FMX_TYPE_Q4_K: return launch_for_down<GQ4K>(a, b, max_tiles, s, kev);
    case FMX_TYPE_Q6_K: return launch_for_down<GQ6K>(a, b, max_tiles, s, kev);
    }
    return FMX_ERR_UNSUPPORTED_QUANTISATION;
}

uint32_t prefill_down_splits(uint32_t experts, uint32_t ffn) {
    // few experts give few row tiles: split the down projection's K so that
    // the grid still covers the device
    return experts <= 16 && ffn % (2 * kGStepK) == 0 ? 2 : 1;
}

int launch_combine(const float *x, const float *dn, uint32_t splits, uint32_t pairs, const uint32_t *slot_of,
                   const float *w, uint32_t hidden, uint32_t K, uint32_t tokens, float *out, hipStream_t s) {
    const uint64_t stride = static_cast<uint64_t>(pairs) * hidden;
    if (hidden % 4 == 0 && (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 == 0)
        hipLaunchKernelGGL(combine_kernel<4>, dim3(div_up(hidden, 1024), tokens), dim3(256), 0, s, x, dn, splits,
                           stride, slot_of, pairs, w, hidden, K, out);
    else
        hipLaunchKernelGGL(combine_kernel<1>, dim3(div_up(hidden, 256), tokens), dim3(256), 0, s, x, dn, splits,
                           stride, slot_of, pairs, w, hidden, K, out);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace fmx
