// chains.hpp — the reference's per-lane FMA chains as wavefront building blocks.
//
// The reference's AVX2 row dots (kernels.cpp:639-653, 673-694, 720-771) keep
// eight float lanes per row and fold blocks into them in order. Here eight
// consecutive lanes of a wavefront are those eight lanes: lane l (= lane & 7)
// owns chain l of its row and walks the row's blocks in order, so every
// rounding happens in the same sequence as on the CPU. A wavefront holds 8 rows
// ("row slots"); a thread may carry NR rows that share the same x values.
//
// x is staged per K-tile in LDS in the order the lanes consume it, so a lane's
// four x values of a block are one 16-byte LDS read and lanes of different row
// slots read the same address (broadcast).
#pragma once

#include "fmx_internal.hpp"

namespace fmx {

// ------------------------------------------------------------- staging --
// Staging copies a tile of x into LDS as "quads": quad s holds the four x
// values that one lane of one block consumes, elements q, q + 8, q + 16 and
// q + 24 of the tile for q = T::quad_base(s), and goes to LDS as one 16-byte
// write at float4 s. A thread gathers its quads with four 4-byte loads each
// (the lanes of a wavefront still read whole 32-byte runs), so that
// consecutive lanes write consecutive 16-byte slots: spreading a float4 of
// consecutive elements over four slots instead put every lane of a wavefront
// on the same 8 LDS banks.
// One batch of a staging pass: N quads per thread, in flight together. A
// kernel may load the first batch ahead, to request x before it knows what
// else it needs.
template <int N>
struct XBatch {
    float4 v[N];
};

// Quads s0 + u * nthreads (u < N) of the tile of n elements at x + e0.
template <class T, int N>
__device__ __forceinline__ void load_batch(XBatch<N> &b, const float *__restrict__ x, uint32_t e0, uint32_t n,
                                           uint32_t s0, uint32_t nthreads) {
    const float *src = x + e0;
    const uint32_t nq = n / 4;
#pragma unroll
    for (int u = 0; u < N; ++u) {
        const uint32_t s = s0 + u * nthreads;
        const uint32_t q = T::quad_base(s < nq ? s : nq - 1);
        b.v[u] = make_float4(src[q], src[q + 8], src[q + 16], src[q + 24]);
    }
}

// Every quad of the tile of n elements (n a multiple of 32) at x + e0, in
// batches of N per thread, handed to put(s, quad). kPre: `pre` holds the
// first batch, loaded by load_batch<T>(pre, x, e0, n, tid, nthreads).
template <class T, int N, bool kPre, class Put>
__device__ __forceinline__ void gather_quads(const float *__restrict__ x, uint32_t e0, uint32_t n, uint32_t tid,
                                             uint32_t nthreads, const XBatch<N> &pre, Put put) {
    const uint32_t nq = n / 4;
    for (uint32_t s0 = tid; s0 < nq; s0 += N * nthreads) {
        XBatch<N> b;
        if (kPre && s0 == tid) b = pre;
        else load_batch<T>(b, x, e0, n, s0, nthreads);
#pragma unroll
        for (int u = 0; u < N; ++u) {
            const uint32_t s = s0 + u * nthreads;
            if (s < nq) put(s, b.v[u]);
        }
    }
}

// ---------------------------------------------------------------- Q4_0 --
// Block = 32 elements; chunk = 8 blocks (one 16-byte lane load per row).
// LDS per block: 8 lanes x float4 x-values, then 8 floats of 8*sum(x).
struct Q40 {
    static constexpr uint32_t kType = FMX_TYPE_Q4_0;
    static constexpr uint32_t kBlock = 32;
    static constexpr uint32_t kPerChunk = 8;
    static constexpr uint32_t kLdsFloatsPerBlock = 40;

    // Stage blocks [b0, b0 + nb) of x into lds (xs: nb*32 floats, s8: nb*8):
    // Quad s = 8 b + l: block b, lane l.
    __device__ static uint32_t quad_base(uint32_t s) { return (s >> 3) * 32 + (s & 7); }

    // xs[b][l] = (x[l], x[8+l], x[16+l], x[24+l]) of block b, then per (b, l)
    // 8 * ((x[l] + x[8+l]) + (x[16+l] + x[24+l])) (the scaling is exact). The
    // caller's barrier after stage() publishes the tile.
    template <int N = 8, bool kPre = false>
    __device__ static void stage(const float *__restrict__ x, uint32_t b0, uint32_t nb, float *lds, uint32_t tid,
                                 uint32_t nthreads, const XBatch<N> &pre = XBatch<N>()) {
        float4 *xs = reinterpret_cast<float4 *>(lds);
        float *s8 = lds + nb * 32;
        gather_quads<Q40, N, kPre>(x, b0 * 32, nb * 32, tid, nthreads, pre, [&](uint32_t q, float4 v) {
            xs[q] = v;
            s8[q] = 8.0f * ((v.x + v.y) + (v.z + v.w));
        });
    }

    // Row base pointers for this lane: scales of the row, and the lane's
    // 16-byte slot of chunk 0 of the row.
    struct Row {
        const uint8_t *scales;
        const uint8_t *quants;
    };
    __device__ static Row row(const uint8_t *packed, uint64_t scale_bytes, uint32_t blocks_padded,
                              uint32_t chunks, uint32_t r, uint32_t l) {
        Row w;
        w.scales = packed + static_cast<uint64_t>(r) * blocks_padded * 2;
        w.quants = packed + scale_bytes + (static_cast<uint64_t>(r) * chunks * 8 + l) * 16;
        return w;
    }

    struct Chunk {
        uint4 q, s;
    };
    __device__ static Chunk load(const Row &w, uint32_t c) {
        Chunk k;
        k.q = ld16nt(w.quants + static_cast<uint64_t>(c) * 128);
        k.s = ld16(w.scales + static_cast<uint64_t>(c) * 16);
        return k;
    }
    // The row's pointers moved n chunks on.
    __device__ static void advance(Row &w, uint32_t n) {
        w.quants += static_cast<uint64_t>(n) * 128;
        w.scales += static_cast<uint64_t>(n) * 16;
    }

    // The x values of half a chunk (4 blocks) from LDS: per block the lane's
    // float4 and its 8 * sum.
    struct XHalf {
        float4 xv[4];
        float sx8[4];
    };
    // read_half for a full chunk whose first block sits `kb` blocks past the
    // blocks xs0 / s80 point at (xs0 = tile's float4s + 8 b + l, s80 = tile's
    // sums + 8 b + l for a base block b): with kb a compile-time constant the
    // reads carry it as an instruction offset.
    __device__ static void read_half_at(XHalf &xh, const float4 *xs0, const float *s80, uint32_t kb,
                                        uint32_t half) {
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t j = kb + 4 * half + q;
            xh.xv[q] = xs0[j * 8];
            xh.sx8[q] = s80[j * 8];
        }
    }
    // Blocks 4 * half .. 4 * half + 3 of the chunk whose first block sits at
    // tile block tb0 (blocks past nblk read block 0 instead).
    __device__ static void read_half(XHalf &xh, const float *lds, uint32_t nb_tile, uint32_t tb0, uint32_t half,
                                     uint32_t l, uint32_t nblk = kPerChunk) {
        const float4 *xs = reinterpret_cast<const float4 *>(lds) + tb0 * 8 + l;
        const float *s8 = lds + nb_tile * 32 + tb0 * 8 + l;
#pragma unroll
        for (uint32_t q = 0; q < 4; ++q) {
            const uint32_t j = 4 * half + q;
            const uint32_t jr = j < nblk ? j : 0;
            xh.xv[q] = xs[jr * 8];
            xh.sx8[q] = s8[jr * 8];
        }
    }

    // The arithmetic of blocks 4 * half + q, q < nq, of chunk `k`.
    template <int NR, bool FULL>
    __device__ static void compute_half(const Chunk (&k)[NR], const XHalf &xh, uint32_t half, uint32_t nq,
                                        float (&t)[NR]) {
#pragma unroll
        for (uint32_t jj = 2 * half; jj < 2 * half + 2; ++jj) {
            // dword jj holds blocks 2jj and 2jj+1: bytes (A, B, A', B')
            uint32_t lo4[NR], hi4[NR], sw[NR];
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const uint32_t qw = jj == 0 ? k[i].q.x : jj == 1 ? k[i].q.y : jj == 2 ? k[i].q.z : k[i].q.w;
                sw[i] = jj == 0 ? k[i].s.x : jj == 1 ? k[i].s.y : jj == 2 ? k[i].s.z : k[i].s.w;
                lo4[i] = qw & 0x0F0F0F0Fu;
                hi4[i] = (qw >> 4) & 0x0F0F0F0Fu;
            }
#pragma unroll
            for (uint32_t h = 0; h < 2; ++h) {
                const uint32_t q = 2 * jj + h - 4 * half;
                if (!FULL && q >= nq) break;
#pragma unroll
                for (int i = 0; i < NR; ++i) {
                    // (A.lo, B.lo) and (A.hi, B.hi) of block 2jj + h, exact
                    const float2 lq = h ? nibble_pair<true>(lo4[i]) : nibble_pair<false>(lo4[i]);
                    const float2 hq = h ? nibble_pair<true>(hi4[i]) : nibble_pair<false>(hi4[i]);
                    const float qa = lq.x, qb = lq.y, qc = hq.x, qd = hq.y;
                    // lo = fma(q[l], x[l], q[8+l]*x[8+l]); hi likewise for 16+l, 24+l
                    const float lo = fma_rn(qa, xh.xv[q].x, qb * xh.xv[q].y);
                    const float hi = fma_rn(qc, xh.xv[q].z, qd * xh.xv[q].w);
                    const float c = (lo + hi) - xh.sx8[q];
                    const float d = half_bits_to_float(h ? (sw[i] >> 16) : (sw[i] & 0xFFFFu));
                    t[i] = fma_rn(c, d, t[i]);
                }
            }
        }
    }

    // Blocks j < nblk of chunk `k` (block index within the LDS tile: tb0 + j),
    // in two halves of four blocks whose LDS reads are issued before their
    // arithmetic. FULL: all kPerChunk blocks are present.
    template <int NR, bool FULL = false>
    __device__ static void step(const Chunk (&k)[NR], const float *lds, uint32_t nb_tile,
                                uint32_t tb0, uint32_t nblk, uint32_t l, float (&t)[NR]) {
#pragma unroll
        for (uint32_t half = 0; half < 2; ++half) {
            if (!FULL && 4 * half >= nblk) break;
            XHalf xh;
            read_half(xh, lds, nb_tile, tb0, half, l, FULL ? kPerChunk : nblk);
            const uint32_t nq = FULL ? 4 : (nblk - 4 * half < 4 ? nblk - 4 * half : 4);
            compute_half<NR, FULL>(k, xh, half, nq, t);
        }
    }

    // Half-chunk LDS pipelining (ChunkStream with kPipelined): the next half's
    // reads are in flight during this half's arithmetic.
    static constexpr bool kHalves = true;

    // The row's value from the lane chains (all 8 lanes end with it).
    __device__ static float finish(float t) { return hsum8_lanes(t); }
};

// ---------------------------------------------------------------- Q8_0 --
// Block = 32; chunk = 4 blocks. LDS per block: 8 lanes x float4.
struct Q80 {
    static constexpr uint32_t kType = FMX_TYPE_Q8_0;
    static constexpr uint32_t kBlock = 32;
    static constexpr uint32_t kPerChunk = 4;
    static constexpr uint32_t kLdsFloatsPerBlock = 32;

    __device__ static uint32_t quad_base(uint32_t s) { return (s >> 3) * 32 + (s & 7); }

    // xs[b][l] = (x[l], x[8+l], x[16+l], x[24+l]) of block b.
    template <int N = 8, bool kPre = false>
    __device__ static void stage(const float *__restrict__ x, uint32_t b0, uint32_t nb, float *lds, uint32_t tid,
                                 uint32_t nthreads, const XBatch<N> &pre = XBatch<N>()) {
        float4 *xs = reinterpret_cast<float4 *>(lds);
        gather_quads<Q80, N, kPre>(x, b0 * 32, nb * 32, tid, nthreads, pre,
                                   [&](uint32_t q, float4 v) { xs[q] = v; });
    }

    struct Row {
        const uint8_t *scales;
        const uint8_t *quants;
    };
    __device__ static Row row(const uint8_t *packed, uint64_t scale_bytes, uint32_t blocks_padded,
                              uint32_t chunks, uint32_t r, uint32_t l) {
        Row w;
        w.scales = packed + static_cast<uint64_t>(r) * blocks_padded * 2;
        w.quants = packed + scale_bytes + (static_cast<uint64_t>(r) * chunks * 8 + l) * 16;
        return w;
    }

    struct Chunk {
        uint4 q;
        uint2 s;
    };
    __device__ static Chunk load(const Row &w, uint32_t c) {
        Chunk k;
        k.q = ld16nt(w.quants + static_cast<uint64_t>(c) * 128);
        k.s = ld8(w.scales + static_cast<uint64_t>(c) * 8);
        return k;
    }
    __device__ static void advance(Row &w, uint32_t n) {
        w.quants += static_cast<uint64_t>(n) * 128;
        w.scales += static_cast<uint64_t>(n) * 8;
    }

    __device__ static float sbyte(uint32_t w, int k) {
        return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * k)) >> 24);
    }

    template <int NR, bool FULL = false>
    __device__ static void step(const Chunk (&k)[NR], const float *lds, uint32_t /*nb_tile*/,
                                uint32_t tb0, uint32_t nblk, uint32_t l, float (&t)[NR]) {
        const float4 *xs = reinterpret_cast<const float4 *>(lds) + tb0 * 8 + l;
        float4 xv[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) xv[j] = xs[(FULL || j < nblk ? j : 0) * 8];
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            if (!FULL && j >= nblk) break;
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const uint32_t w = j == 0 ? k[i].q.x : j == 1 ? k[i].q.y : j == 2 ? k[i].q.z : k[i].q.w;
                const uint32_t sw = j < 2 ? k[i].s.x : k[i].s.y;
                // acc over elements l, 8+l, 16+l, 24+l from zero, then t += acc*d (both FMA)
                float acc = fma_rn(sbyte(w, 0), xv[j].x, 0.0f);
                acc = fma_rn(sbyte(w, 1), xv[j].y, acc);
                acc = fma_rn(sbyte(w, 2), xv[j].z, acc);
                acc = fma_rn(sbyte(w, 3), xv[j].w, acc);
                const float d = half_bits_to_float((j & 1) ? (sw >> 16) : (sw & 0xFFFFu));
                t[i] = fma_rn(acc, d, t[i]);
            }
        }
    }

    __device__ static float finish(float t) { return hsum8_lanes(t); }
};

// ---------------------------------------------------------------- Q4_K --
// Super-block = 256 elements = one chunk. LDS per super-block: [4 groups]
// [8 lanes][8 floats: x[64g+8k+l], k<4, then x[64g+32+8k+l]] followed, after
// the tile, by 8 floats of per-group sums (lo, hi) in the reference's order.
struct Q4K {
    static constexpr uint32_t kType = FMX_TYPE_Q4_K;
    static constexpr uint32_t kBlock = 256;
    static constexpr uint32_t kPerChunk = 1;
    static constexpr uint32_t kLdsFloatsPerBlock = 264;

    // Quad s = ((4 * super-block + group) * 8 + l) * 2 + half.
    __device__ static uint32_t quad_base(uint32_t s) { return (s >> 4) * 64 + (s & 1) * 32 + ((s >> 1) & 7); }

    // Per super-block and group g: slots (g, l, half) hold x[64g + 32 half + 8k + l],
    // k = 0..3; then per (super-block, g) the low and high 32-element sums in
    // the reference's order (per-lane sums of four, then the 8-lane tree). The
    // caller's barrier after stage() publishes the sums.
    template <int N = 8, bool kPre = false>
    __device__ static void stage(const float *__restrict__ x, uint32_t b0, uint32_t nb, float *lds, uint32_t tid,
                                 uint32_t nthreads, const XBatch<N> &pre = XBatch<N>()) {
        float4 *xw = reinterpret_cast<float4 *>(lds);
        gather_quads<Q4K, N, kPre>(x, b0 * 256, nb * 256, tid, nthreads, pre,
                                   [&](uint32_t q, float4 v) { xw[q] = v; });
        __syncthreads();
        const float4 *xs = reinterpret_cast<const float4 *>(lds);
        float *sums = lds + nb * 256;
        for (uint32_t e = tid; e < nb * 8; e += nthreads) {
            // e = (super-block, group) * 2 + half
            const uint32_t sg = e >> 1, half = e & 1;
            float v[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const float4 q = xs[(sg * 8 + l) * 2 + half];
                v[l] = (q.x + q.y) + (q.z + q.w);
            }
            sums[e] = ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
        }
    }

    struct Row {
        const uint8_t *header;
        const uint8_t *quants;
    };
    __device__ static Row row(const uint8_t *packed, uint64_t scale_bytes, uint32_t /*bp*/,
                              uint32_t chunks, uint32_t r, uint32_t l) {
        Row w;
        w.header = packed + static_cast<uint64_t>(r) * chunks * 16;
        w.quants = packed + scale_bytes + (static_cast<uint64_t>(r) * chunks * 8 + l) * 16;
        return w;
    }

    struct Chunk {
        uint4 q, h;
    };
    __device__ static Chunk load(const Row &w, uint32_t c) {
        Chunk k;
        k.q = ld16nt(w.quants + static_cast<uint64_t>(c) * 128);
        k.h = ld16(w.header + static_cast<uint64_t>(c) * 16);
        return k;
    }
    __device__ static void advance(Row &w, uint32_t n) {
        w.quants += static_cast<uint64_t>(n) * 128;
        w.header += static_cast<uint64_t>(n) * 16;
    }

    template <int NR, bool FULL = false>
    __device__ static void step(const Chunk (&k)[NR], const float *lds, uint32_t nb_tile,
                                uint32_t tb0, uint32_t nblk, uint32_t l, float (&t)[NR]) {
        if (!FULL && nblk == 0) return;
        const float4 *xs = reinterpret_cast<const float4 *>(lds);
        const float *sums = lds + nb_tile * 256;
#pragma unroll
        for (uint32_t g = 0; g < 4; ++g) {
            const uint32_t e = (tb0 * 4 + g) * 8 + l;
            const float4 xl = xs[2 * e], xh = xs[2 * e + 1];
            const float sum_lo = sums[(tb0 * 4 + g) * 2], sum_hi = sums[(tb0 * 4 + g) * 2 + 1];
#pragma unroll
            for (int i = 0; i < NR; ++i) {
                const uint32_t w = g == 0 ? k[i].q.x : g == 1 ? k[i].q.y : g == 2 ? k[i].q.z : k[i].q.w;
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
                uint8_t hdr[16];
                memcpy(hdr, &k[i].h, 16);
                const float d = half_bits_to_float(hdr[0] | (hdr[1] << 8));
                const float dmin = half_bits_to_float(hdr[2] | (hdr[3] << 8));
                uint32_t sc1, m1, sc2, m2;
                k4_scale_min(2 * g, hdr + 4, sc1, m1);
                k4_scale_min(2 * g + 1, hdr + 4, sc2, m2);
                const float dsc1 = d * static_cast<float>(sc1), dm1 = dmin * static_cast<float>(m1);
                const float dsc2 = d * static_cast<float>(sc2), dm2 = dmin * static_cast<float>(m2);
                // part = fma(d*sc, hsum(acc), -((dmin*m) * sum_x)); total += lo + hi
                const float part_lo = fma_rn(dsc1, hlo, -(dm1 * sum_lo));
                const float part_hi = fma_rn(dsc2, hhi, -(dm2 * sum_hi));
                t[i] = t[i] + (part_lo + part_hi);
            }
        }
    }

    // The running total is the row's value in lanes 0-3 of the row's group
    // (its lane trees are hsum8_first's); callers read lane 0.
    __device__ static float finish(float t) { return t; }
};

// ------------------------------------------------ chunked row processing --

// Processes chunks [c0, c1) of NR rows against the LDS tile that starts at
// block `tile_b0` (tile holds nb_tile blocks). PF chunks per row are kept in
// flight in registers: chunk c + PF is requested before chunk c is consumed.
template <class T, int NR, int PF>
__device__ __forceinline__ void run_chunks_pf(const typename T::Row (&rows)[NR], uint32_t c0,
                                              uint32_t c1, uint32_t blocks, uint32_t tile_b0,
                                              uint32_t nb_tile, const float *lds, uint32_t l,
                                              float (&t)[NR]) {
    typename T::Chunk buf[PF][NR];
#pragma unroll
    for (int p = 0; p < PF; ++p)
        if (c0 + p < c1) {
#pragma unroll
            for (int i = 0; i < NR; ++i) buf[p][i] = T::load(rows[i], c0 + p);
        }
    for (uint32_t c = c0; c < c1; c += PF) {
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const uint32_t cc = c + p;
            if (cc >= c1) break;
            typename T::Chunk cur[NR];
#pragma unroll
            for (int i = 0; i < NR; ++i) cur[i] = buf[p][i];
            if (cc + PF < c1) {
#pragma unroll
                for (int i = 0; i < NR; ++i) buf[p][i] = T::load(rows[i], cc + PF);
            }
            const uint32_t b = cc * T::kPerChunk;
            const uint32_t nblk = blocks - b < T::kPerChunk ? blocks - b : T::kPerChunk;
            T::template step<NR>(cur, lds, nb_tile, b - tile_b0, nblk, l, t);
        }
    }
}

// A row stream with PF chunks per row in flight across LDS tiles: prime()
// requests chunks 0..PF-1 (before the first tile is staged, so the weight
// loads overlap the staging); run() consumes chunks [c0, c1) of the current
// tile and keeps requesting chunk c + PF, so the loads of the next tile are
// already in flight when its staging starts.
// The chunks live in a ring of kSlots = PF + 1 register slots: the load for
// chunk c + PF goes into the slot chunk c - 1 just left, before chunk c is
// consumed, with every slot index a compile-time constant. Every load is
// issued unconditionally (past the row's last chunk the steady state reads on
// into the next row or the layout's tail and the last partial ring re-reads
// the last chunk): a load under a branch makes the compiler's wait counts
// conservative, and it then waits for every load in flight before each chunk,
// which removes the prefetch. Every tile must start at a multiple of kSlots
// chunks.
// In the steady state every load is addressed from row pointers that move
// one ring on per pass, with the chunk's distance from them a compile-time
// constant (an instruction offset): no address is computed per load, and the
// prefetch reads up to PF chunks past a row's last chunk, which the packed
// layout's tail keeps inside the matrix's allocation. (Address temporaries
// computed per load made the compiler reuse registers of loads still in
// flight, and wait for all of them at the top of every pass.) U rings per pass
// (U * kSlots chunks) make the loop-head wait rare where it remains.
// kPipe (types with XHalf / read_half / compute_half): in the steady state
// the LDS reads of the next half chunk are in flight during the arithmetic of
// the current one, for kernels with too few wavefronts per SIMD to hide LDS
// latency by switching.
template <class T, int NR, bool FULL>
__device__ __forceinline__ void chain_step(const typename T::Chunk (&k)[NR], const float *lds, uint32_t nb_tile,
                                           uint32_t tb0, uint32_t nblk, uint32_t l, float (&t)[NR]) {
    T::template step<NR, FULL>(k, lds, nb_tile, tb0, nblk, l, t);
}

template <class T, int NR, int PF, int U = 1, bool kPipe = false>
struct ChunkStream {
    static constexpr int kSlots = PF + 1;
    typename T::Chunk buf[kSlots][NR];
    // the rows' pointers at the stream's position (the first chunk run() has
    // not consumed yet)
    typename T::Row at[NR];

    // One full chunk from `cur`, with `xa` holding its first half's x values
    // on entry and the next chunk's on return; first requests the chunk `rel`
    // chunks past the stream position into `dst`. The chunk's and the next
    // chunk's first blocks sit kb and kn blocks past the blocks xs0 / s80
    // point at (read_half_at).
    template <class XH>
    __device__ __forceinline__ void pipe_step(const typename T::Chunk (&cur)[NR], typename T::Chunk (&dst)[NR],
                                              uint32_t rel, const float4 *xs0, const float *s80, uint32_t kb,
                                              uint32_t kn, float (&t)[NR], XH &xa, XH &xb) {
#pragma unroll
        for (int i = 0; i < NR; ++i) dst[i] = T::load(at[i], rel);
        __builtin_amdgcn_sched_barrier(0);
        T::read_half_at(xb, xs0, s80, kb, 1);
        __builtin_amdgcn_sched_barrier(0);
        T::template compute_half<NR, true>(cur, xa, 0, 4, t);
        T::read_half_at(xa, xs0, s80, kn, 0);
        __builtin_amdgcn_sched_barrier(0);
        T::template compute_half<NR, true>(cur, xb, 1, 4, t);
    }

    __device__ __forceinline__ void advance(uint32_t n) {
#pragma unroll
        for (int i = 0; i < NR; ++i) T::advance(at[i], n);
    }

    // Starts the stream at chunk 0 of `rows`.
    __device__ __forceinline__ void prime(const typename T::Row (&rows)[NR], uint32_t c_end) {
        const uint32_t last = c_end - 1;
#pragma unroll
        for (int i = 0; i < NR; ++i) at[i] = rows[i];
#pragma unroll
        for (int p = 0; p < PF; ++p) {
            const uint32_t c = static_cast<uint32_t>(p) < last ? static_cast<uint32_t>(p) : last;
#pragma unroll
            for (int i = 0; i < NR; ++i) buf[p][i] = T::load(at[i], c);
        }
    }

    // Chunks [c0, c1) against the LDS tile that starts at block tile_b0; c0
    // is the stream's position.
    __device__ __forceinline__ void run(uint32_t c0, uint32_t c1, uint32_t c_end, uint32_t blocks,
                                        uint32_t tile_b0, uint32_t nb_tile, const float *lds, uint32_t l,
                                        float (&t)[NR]) {
        const uint32_t full_end = blocks / T::kPerChunk; // chunks [0, full_end) hold kPerChunk blocks
        const uint32_t last = c_end - 1;
        const uint32_t cf = c1 < full_end ? c1 : full_end;
        uint32_t c = c0;
        if constexpr (kPipe) {
            typename T::XHalf xa, xb;
            if (c + kSlots <= cf) T::read_half(xa, lds, nb_tile, c * T::kPerChunk - tile_b0, 0, l);
            // LDS reads relative to the pass's first block; the pass's last
            // chunk reads the next chunk's first half only when one follows
            const float4 *xst = reinterpret_cast<const float4 *>(lds) + l;
            const float *s8t = lds + nb_tile * 32 + l;
            if (U > 1)
                for (; c + kSlots * U <= cf; c += kSlots * U) {
                    const uint32_t b = c * T::kPerChunk - tile_b0;
                    const float4 *xs0 = xst + b * 8;
                    const float *s80 = s8t + b * 8;
                    const uint32_t kend = c + kSlots * U < cf ? kSlots * U * T::kPerChunk : (kSlots * U - 1) * T::kPerChunk;
#pragma unroll
                    for (int u = 0; u < U; ++u) {
#pragma unroll
                        for (int p = 0; p < kSlots; ++p) {
                            const uint32_t k = u * kSlots + p;
                            const uint32_t kn = k + 1 < kSlots * U ? (k + 1) * T::kPerChunk : kend;
                            pipe_step(buf[p], buf[(p + PF) % kSlots], k + PF, xs0, s80, k * T::kPerChunk, kn,
                                               t, xa, xb);
                        }
                    }
                    advance(kSlots * U);
                }
            for (; c + kSlots <= cf; c += kSlots) {
                const uint32_t b = c * T::kPerChunk - tile_b0;
                const float4 *xs0 = xst + b * 8;
                const float *s80 = s8t + b * 8;
                const uint32_t kend = c + kSlots < cf ? kSlots * T::kPerChunk : (kSlots - 1) * T::kPerChunk;
#pragma unroll
                for (int p = 0; p < kSlots; ++p) {
                    const uint32_t kn = p + 1 < kSlots ? (p + 1) * T::kPerChunk : kend;
                    pipe_step(buf[p], buf[(p + PF) % kSlots], p + PF, xs0, s80, p * T::kPerChunk, kn, t, xa,
                                       xb);
                }
                advance(kSlots);
            }
        }
        // steady state: U whole rings of full chunks per pass, one basic block
        if (!kPipe && U > 1)
            for (; c + kSlots * U <= cf; c += kSlots * U) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
#pragma unroll
                    for (int p = 0; p < kSlots; ++p) {
                        const uint32_t cc = c + u * kSlots + p;
#pragma unroll
                        for (int i = 0; i < NR; ++i)
                            buf[(p + PF) % kSlots][i] = T::load(at[i], u * kSlots + p + PF);
                        __builtin_amdgcn_sched_barrier(0);
                        chain_step<T, NR, true>(buf[p], lds, nb_tile, cc * T::kPerChunk - tile_b0,
                                                   T::kPerChunk, l, t);
                    }
                }
                advance(kSlots * U);
            }
        for (; !kPipe && c + kSlots <= cf; c += kSlots) {
#pragma unroll
            for (int p = 0; p < kSlots; ++p) {
                const uint32_t cc = c + p;
#pragma unroll
                for (int i = 0; i < NR; ++i) buf[(p + PF) % kSlots][i] = T::load(at[i], p + PF);
                // the scheduler would otherwise sink loads whose data is used
                // late in a step down to that use, emptying the prefetch ring
                __builtin_amdgcn_sched_barrier(0);
                chain_step<T, NR, true>(buf[p], lds, nb_tile, cc * T::kPerChunk - tile_b0, T::kPerChunk, l, t);
            }
            advance(kSlots);
        }
        // the rest of the tile (fewer than kSlots chunks, the last may be
        // partial); its requests stop at the row's last chunk
#pragma unroll
        for (int p = 0; p < kSlots; ++p) {
            const uint32_t cc = c + p;
            if (cc >= c1) break;
            const uint32_t nxt = cc + PF < last ? cc + PF : last;
#pragma unroll
            for (int i = 0; i < NR; ++i) buf[(p + PF) % kSlots][i] = T::load(at[i], nxt - c);
            const uint32_t b = cc * T::kPerChunk;
            if (cc < full_end)
                chain_step<T, NR, true>(buf[p], lds, nb_tile, b - tile_b0, T::kPerChunk, l, t);
            else
                chain_step<T, NR, false>(buf[p], lds, nb_tile, b - tile_b0, blocks - b, l, t);
        }
        if (c1 > c) advance(c1 - c);
    }
};

// Blocks per LDS tile: the whole row when it fits in `budget_floats` of LDS,
// else a whole number of `align`-chunk groups (at least one group).
template <class T>
__host__ __device__ inline uint32_t tile_blocks_for(uint32_t blocks, uint32_t budget_floats,
                                                    uint32_t align = 1) {
    const uint32_t whole = (blocks + T::kPerChunk - 1) / T::kPerChunk * T::kPerChunk;
    if (whole * T::kLdsFloatsPerBlock <= budget_floats) return whole;
    const uint32_t unit = T::kPerChunk * align;
    uint32_t tb = budget_floats / T::kLdsFloatsPerBlock;
    tb = tb / unit * unit;
    if (tb == 0) tb = unit;
    return tb < whole ? tb : whole;
}

} // namespace fmx
