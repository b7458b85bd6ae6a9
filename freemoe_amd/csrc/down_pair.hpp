// down_pair.hpp — the down projection of one decode token on 16 lanes per
// row (Q4_0 and Q4_K down matrices); included by moe.hip (Q4_0) and
// down_pair_q4k.hip (Q4_K), each instantiating its own block type.
#pragma once

#include "chains.hpp"
#include "moe.hpp"

#include <hip/hip_ext.h>

namespace fmx {

namespace {

// Prefetch depth (chunks in flight per row) and the dynamic LDS a launch may
// request (a gfx950 workgroup holds 160 KiB, 1 KiB left for static LDS).
constexpr int kPairPF = 7;
constexpr size_t kPairMaxLds = 159 * 1024;

// Down rows as down_kernel, on twice the lanes: 16 per row slot, 512 threads,
// two wavefronts per SIMD (Q4_0 and Q4_K down matrices). A row's sum is a
// sequence of independent per-block values folded into a chain in block
// order: Q4_0's lane chains t_l = fma(c_b, d_b, t_l) with c_b = (lo + hi) -
// 8 sum x, Q4_K's running total t = t + (part_lo + part_hi) per 32-element
// group pair. Lane l < 8 of a slot computes the values of the first half of
// each chunk from its half of lane l's 16-byte slice, lane l + 8 those of
// the second half from the other, a DPP rotation of the 16-lane row by 8
// hands the second half's values to lane l, and lane l folds them all in the
// reference's order, so the row's result is down_kernel's bit for bit. Every
// rank's activations fill the LDS as one tile (the host checks that they
// fit).
constexpr uint32_t kPairThreads = 512;

// Lane (i + 8) mod 16's value within each row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ float row_swap8(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
}

struct PairChunk {
    uint2 q; // dwords 2 hf, 2 hf + 1 of the lane's slice
    uint4 s; // the chunk's block scales (Q4_0) or super-block header (Q4_K)
};

// Q4_0: a chunk is 8 blocks; lane half hf takes blocks 4 hf .. 4 hf + 3.
struct PairQ40 {
    using T = Q40;
    static constexpr int kNV = 4;
    // this lane's quads and sums of the tile (block stride 8, chunk stride 64)
    struct X {
        const float4 *xs4;
        const float *s8;
    };
    __device__ static X x_of(const float *tile, uint32_t nb_tile, uint32_t l) {
        return X{reinterpret_cast<const float4 *>(tile) + l, tile + nb_tile * 32 + l};
    }
    // The lane's LDS operands of one chunk: blocks 4 hf + q, q < 4.
    struct XC {
        float4 xv[4];
        float s8[4];
    };
    __device__ static void read_x(const X &xt, uint32_t ch, uint32_t /*l*/, uint32_t hf, XC &o) {
        const float4 *xs4 = xt.xs4 + ch * 64;
        const float *s8 = xt.s8 + ch * 64;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            o.xv[q] = xs4[(4 * hf + q) * 8];
            o.s8[q] = s8[(4 * hf + q) * 8];
        }
    }
    // c of blocks 4 hf + q, q < 4, of the chunk whose operands `xc` holds.
    __device__ static void values(const PairChunk &k, const XC &xc, uint32_t /*hf*/, float (&c)[kNV]) {
#pragma unroll
        for (uint32_t jj = 0; jj < 2; ++jj) {
            const uint32_t qw = jj ? k.q.y : k.q.x;
            const uint32_t lo4 = qw & 0x0F0F0F0Fu, hi4 = (qw >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const uint32_t q = 2 * jj + h;
                const float4 xv = xc.xv[q];
                const float2 lq = h ? nibble_pair<true>(lo4) : nibble_pair<false>(lo4);
                const float2 hq = h ? nibble_pair<true>(hi4) : nibble_pair<false>(hi4);
                const float lo = fma_rn(lq.x, xv.x, lq.y * xv.y);
                const float hi = fma_rn(hq.x, xv.z, hq.y * xv.w);
                c[q] = (lo + hi) - xc.s8[q];
            }
        }
    }
    // t = fma(c_b, d_b, t) for blocks 0-7: own values, then the partner's.
    __device__ static float chain(const PairChunk &k, const float (&c)[kNV], float t) {
        float r[kNV];
#pragma unroll
        for (int q = 0; q < kNV; ++q) r[q] = row_swap8(c[q]);
        const uint32_t sw[4] = {k.s.x, k.s.y, k.s.z, k.s.w};
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const float cb = b < 4 ? c[b] : r[b - 4];
            const float d = half_bits_to_float((b & 1) ? (sw[b >> 1] >> 16) : (sw[b >> 1] & 0xFFFFu));
            t = fma_rn(cb, d, t);
        }
        return t;
    }
    __device__ static float finish(float t) { return hsum8_lanes(t); }
};

// Q4_K: a chunk is one super-block of four 64-element group pairs; lane half
// hf takes groups 2 hf and 2 hf + 1, each reduced over its 8 lanes by the
// reference's lane tree (as Q4K::step).
struct PairQ4K {
    using T = Q4K;
    static constexpr int kNV = 2;
    struct X {
        const float4 *xs;
        const float *sums;
    };
    __device__ static X x_of(const float *tile, uint32_t nb_tile, uint32_t) {
        return X{reinterpret_cast<const float4 *>(tile), tile + nb_tile * 256};
    }
    // 6-bit scale / min of sub-block j = 4 hf + i (k4_scale_min, quant.cpp:63-71)
    // with i a compile-time constant and hf per lane: both forms from the
    // header's dwords 1-3, then a select.
    template <uint32_t i>
    __device__ static void scale_min(const uint4 &h, uint32_t hf, uint32_t &sc, uint32_t &m) {
        const uint32_t b1 = (h.y >> (8 * i)) & 0xFFu, b2 = (h.z >> (8 * i)) & 0xFFu, b3 = (h.w >> (8 * i)) & 0xFFu;
        sc = hf ? ((b3 & 0x0Fu) | ((b1 >> 6) << 4)) : (b1 & 63u);
        m = hf ? ((b3 >> 4) | ((b2 >> 6) << 4)) : (b2 & 63u);
    }
    // The lane's LDS operands of one super-block: groups 2 hf and 2 hf + 1.
    struct XC {
        float4 xl[2], xh[2];
        float sum_lo[2], sum_hi[2];
    };
    __device__ static void read_x(const X &xt, uint32_t ch, uint32_t l, uint32_t hf, XC &o) {
#pragma unroll
        for (uint32_t gg = 0; gg < 2; ++gg) {
            const uint32_t g = 2 * hf + gg;
            const uint32_t e = (ch * 4 + g) * 8 + l;
            o.xl[gg] = xt.xs[2 * e];
            o.xh[gg] = xt.xs[2 * e + 1];
            o.sum_lo[gg] = xt.sums[(ch * 4 + g) * 2];
            o.sum_hi[gg] = xt.sums[(ch * 4 + g) * 2 + 1];
        }
    }
    __device__ static void values(const PairChunk &k, const XC &xc, uint32_t hf, float (&c)[kNV]) {
        const float d = half_bits_to_float(k.s.x & 0xFFFFu);
        const float dmin = half_bits_to_float(k.s.x >> 16);
#pragma unroll
        for (uint32_t gg = 0; gg < 2; ++gg) {
            const float4 xl = xc.xl[gg], xh = xc.xh[gg];
            const float sum_lo = xc.sum_lo[gg], sum_hi = xc.sum_hi[gg];
            const uint32_t w = gg ? k.q.y : k.q.x;
            const uint32_t lo4 = w & 0x0F0F0F0Fu, hi4 = (w >> 4) & 0x0F0F0F0Fu;
            const float2 l01 = nibble_pair<false>(lo4), l23 = nibble_pair<true>(lo4);
            const float2 h01 = nibble_pair<false>(hi4), h23 = nibble_pair<true>(hi4);
            float alo = fma_rn(l01.x, xl.x, 0.0f);
            alo = fma_rn(l01.y, xl.y, alo);
            alo = fma_rn(l23.x, xl.z, alo);
            alo = fma_rn(l23.y, xl.w, alo);
            float ahi = fma_rn(h01.x, xh.x, 0.0f);
            ahi = fma_rn(h01.y, xh.y, ahi);
            ahi = fma_rn(h23.x, xh.z, ahi);
            ahi = fma_rn(h23.y, xh.w, ahi);
            const float hlo = hsum8_first(alo), hhi = hsum8_first(ahi);
            // sub-blocks 2 g and 2 g + 1 = 4 hf + 2 gg and 4 hf + 2 gg + 1
            uint32_t sc1, m1, sc2, m2;
            if (gg == 0) {
                scale_min<0>(k.s, hf, sc1, m1);
                scale_min<1>(k.s, hf, sc2, m2);
            } else {
                scale_min<2>(k.s, hf, sc1, m1);
                scale_min<3>(k.s, hf, sc2, m2);
            }
            const float dsc1 = d * static_cast<float>(sc1), dm1 = dmin * static_cast<float>(m1);
            const float dsc2 = d * static_cast<float>(sc2), dm2 = dmin * static_cast<float>(m2);
            const float part_lo = fma_rn(dsc1, hlo, -(dm1 * sum_lo));
            const float part_hi = fma_rn(dsc2, hhi, -(dm2 * sum_hi));
            c[gg] = part_lo + part_hi;
        }
    }
    // t = t + value for groups 0-3: own values, then the partner's.
    __device__ static float chain(const PairChunk &, const float (&c)[kNV], float t) {
        const float r0 = row_swap8(c[0]), r1 = row_swap8(c[1]);
        t = t + c[0];
        t = t + c[1];
        t = t + r0;
        return t + r1;
    }
    __device__ static float finish(float t) { return t; }
};

// The row's chunks in rings of PF + 1 register slots, chunk c + PF requested
// while chunk c is computed, and chunk c + 1's LDS operands read during chunk
// c's arithmetic (two operand sets, alternating with the slot's parity). The
// last one or two rings run with each request under a (wavefront-uniform)
// test, so nothing past the row's end is read.
template <class P, int PF>
__device__ __forceinline__ float pair_stream(const uint8_t *qp, const uint8_t *sp, uint32_t c_end, const float *tile,
                                             uint32_t nb_tile, uint32_t l, uint32_t hf, PairChunk (&buf)[PF + 1]) {
    constexpr uint32_t kSlots = PF + 1;
    static_assert(kSlots % 2 == 0, "the operand sets alternate with the parity of the ring slot");
    const typename P::X xt = P::x_of(tile, nb_tile, l);
    typename P::XC xc[2];
    P::read_x(xt, 0, l, hf, xc[0]);
    float t = 0.0f;
    uint32_t c = 0;
    for (; c + 2 * kSlots <= c_end; c += kSlots) {
#pragma unroll
        for (uint32_t p = 0; p < kSlots; ++p) {
            PairChunk &nx = buf[(p + PF) % kSlots];
            nx.q = ld8nt(qp + (p + PF) * 128);
            nx.s = ld16(sp + (p + PF) * 16);
            __builtin_amdgcn_sched_barrier(0);
            P::read_x(xt, c + p + 1, l, hf, xc[(p + 1) & 1]); // c + p + 1 < c_end in this loop
            float cv[P::kNV];
            P::values(buf[p], xc[p & 1], hf, cv);
            t = P::chain(buf[p], cv, t);
        }
        qp += kSlots * 128;
        sp += kSlots * 16;
    }
    // the last chunks (fewer than two rings), in slot order
#pragma unroll
    for (uint32_t p = 0; p < 2 * kSlots; ++p) {
        if (c + p >= c_end) break;
        if (c + p + PF < c_end) {
            PairChunk &nx = buf[(p + PF) % kSlots];
            nx.q = ld8nt(qp + (p + PF) * 128);
            nx.s = ld16(sp + (p + PF) * 16);
        }
        if (c + p + 1 < c_end) P::read_x(xt, c + p + 1, l, hf, xc[(p + 1) & 1]);
        float cv[P::kNV];
        P::values(buf[p % kSlots], xc[p & 1], hf, cv);
        t = P::chain(buf[p % kSlots], cv, t);
    }
    return t;
}

template <class P, int PF>
__global__ __launch_bounds__(kPairThreads) __attribute__((amdgpu_waves_per_eu(2, 2), aligned(4096))) void down_pair_kernel(
    ExpertArgs a, const float *__restrict__ x, const float *__restrict__ act, const uint32_t *__restrict__ ids,
    const float *__restrict__ w, float *__restrict__ out, uint32_t *__restrict__ status) {
    using T = typename P::T;
    extern __shared__ __align__(16) float lds[];
    __shared__ float dres[kPairThreads / 16];
    const uint32_t tid = threadIdx.x, l = tid & 7, hf = (tid >> 3) & 1, slot = tid >> 4;
    const uint32_t K = a.top_k, H = a.hidden;
    const uint32_t jpw = (kPairThreads / 16) / K;
    const uint32_t rank = slot / jpw < K ? slot / jpw : K - 1;
    const uint32_t j = blockIdx.x * jpw + slot % jpw;
    const uint32_t jr = j < H ? j : H - 1;
    uint32_t e = ids[rank];
    const bool bad = e >= a.experts;
    if (bad) {
        if ((tid & 15) == 0) atomicOr(status, STATUS_BAD_EXPERT);
        e = 0;
    }
    // quants of lane l's slice (its half) and the chunk's scales / header
    const typename T::Row rw = T::row(static_cast<const uint8_t *>(a.down[e]), a.dn.scale_bytes, a.dn.blocks_padded,
                                      a.dn.chunks, jr, l);
    const uint8_t *qp = rw.quants + 8 * hf;
    const uint8_t *sp;
    if constexpr (T::kType == FMX_TYPE_Q4_0) sp = rw.scales;
    else sp = rw.header;
    const uint32_t blocks = a.dn.blocks, c_end = blocks / T::kPerChunk;
    const uint32_t tile_floats = blocks * T::kLdsFloatsPerBlock;
    const uint32_t n = blocks * T::kBlock;
    // every rank's activations requested first (staging waits for its loads
    // in issue order), then the first weight chunks, then the staging
    constexpr int kB = 8;
    XBatch<kB> b0, b1;
    load_batch<T>(b0, act, 0, n, tid, kPairThreads);
    if (K > 1) load_batch<T>(b1, act + a.ffn, 0, n, tid, kPairThreads);
    PairChunk buf[PF + 1];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
        const uint32_t c = static_cast<uint32_t>(p) < c_end ? p : c_end - 1;
        buf[p].q = ld8nt(qp + c * 128);
        buf[p].s = ld16(sp + c * 16);
    }
    T::template stage<kB, true>(act, 0, blocks, lds, tid, kPairThreads, b0);
    if (K > 1) T::template stage<kB, true>(act + a.ffn, 0, blocks, lds + tile_floats, tid, kPairThreads, b1);
    for (uint32_t r = 2; r < K; ++r)
        T::template stage<kB>(act + static_cast<uint64_t>(r) * a.ffn, 0, blocks, lds + r * tile_floats, tid,
                              kPairThreads);
    __syncthreads();
    const float t = pair_stream<P, PF>(qp, sp, c_end, lds + rank * tile_floats, blocks, l, hf, buf);
    const float v = P::finish(t);
    if ((tid & 15) == 0) dres[slot] = bad ? 0.0f : v;
    __syncthreads();
    if (tid < jpw) {
        const uint32_t jo = blockIdx.x * jpw + tid;
        if (jo < H) {
            float ffn = 0.0f;
            for (uint32_t r = 0; r < K; ++r) ffn = ffn + w[r] * dres[r * jpw + tid];
            out[jo] = x[jo] + ffn;
        }
    }
}

// The 16-lane down kernel (block type P::T) serves a layer when every rank's
// activations fit the LDS as one tile and the rows are whole chunks.
template <class P>
bool pair_down_fits(const ExpertArgs &a) {
    using T = typename P::T;
    return a.type_dn == T::kType && a.top_k <= kPairThreads / 16 && a.dn.blocks % T::kPerChunk == 0 &&
           static_cast<size_t>(a.dn.blocks) * T::kLdsFloatsPerBlock * sizeof(float) * a.top_k <= kPairMaxLds;
}

template <class P>
int launch_down_pair(const ExpertArgs &a, const float *x, const float *act, const uint32_t *ids, const float *w,
                     float *out, uint32_t *status, hipStream_t s, const hipEvent_t *kev) {
    auto dn = down_pair_kernel<P, kPairPF>;
    const size_t lds = static_cast<size_t>(a.dn.blocks) * P::T::kLdsFloatsPerBlock * sizeof(float) * a.top_k;
    if (int rc = allow_lds(reinterpret_cast<const void *>(dn), lds)) return rc;
    const dim3 grid(div_up(a.hidden, (kPairThreads / 16) / a.top_k));
    if (kev)
        hipExtLaunchKernelGGL(dn, grid, dim3(kPairThreads), lds, s, kev[0], kev[1], 0, a, x, act, ids, w, out, status);
    else
        hipLaunchKernelGGL(dn, grid, dim3(kPairThreads), lds, s, a, x, act, ids, w, out, status);
    FMX_LAUNCH_CHECK();
    return FMX_OK;
}

} // namespace

} // namespace fmx
